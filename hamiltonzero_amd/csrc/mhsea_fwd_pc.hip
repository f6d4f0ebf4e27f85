// Producer/consumer forward / forward+tangent / tangent-only MHSEA kernel for float32
// storage and N <= 64 (every key of a (walker, head) fits one LDS tile).
//
// A workgroup is four waves: one producer and three consumers (roles by SIMD: pc_role). A
// fixed grid of workgroups walks the (walker, head) items; workgroup L takes items L, L+G,
// L+2G, ... and processes them in "periods", one item per period. In period k
//   - the consumers compute item k from LDS buffer k%2: each owns one 16-query tile of the
//     compacted query list and runs S^T = K Q^T, the exact softmax (all keys in one tile)
//     and O^T += V^T P^T on the fp32 matrix cores (v_mfma_f32_16x16x4_f32), with the
//     tangent products dS^T = Kt Q^T + K Qt^T, A^T = V^T (P o dS)^T, C^T = Vt^T P^T;
//   - the producer gathers item k+1's physical key rows (K, Kt, V, Vt) from HBM into
//     LDS buffer (k+1)%2 (all 16-byte reads of the item in flight at once, one wait, then
//     swizzled LDS writes), zero-fills the rows of the last partial 16-key tile, writes its
//     item's share of the walker's masked output rows (exact zeros, lse = -1e4 + log N;
//     every head of a site in one contiguous run) and reads item k+2's mask row.
// A single s_barrier ends a period. The producer publishes each item's compacted site
// list in one of four LDS slots two periods ahead, so the consumers can prefetch their
// query fragments one item ahead into registers. Consumers alternate two register sets
// (the loop is unrolled by two), so no register copy forces an early wait.
//
// vmcnt on gfx950 counts loads and stores together and in order: waiting for a load also
// waits for every older memory operation. Every consumer load and store is therefore
// unconditional — lanes without a valid row address a buffer resource past its last
// record, which reads 0 and drops stores — so the compiler's waits are exact counts and
// the wait for item k's query fragments never waits for item k-1's output stores. The
// producer never computes, so its own waits (vmcnt(0) once per period) stall nobody.
//
// Key rows are stored unpadded (D floats per row) with the 16-byte chunks of row r XOR-
// swizzled by (r / rows_per_128B) mod chunks_per_row, which keeps the consumers' K reads
// (16 rows x one chunk) and V reads (4 rows x 16 floats) free of LDS bank conflicts at
// D >= 32.
#include <atomic>
#include <type_traits>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kProducerWave = 3;
constexpr int kSlots = 4;
constexpr int kSlotBytes = 144;  // int16 perm[64], int32 n_phys at byte 128
constexpr int kRoleBytes = 132;  // slot 0: one byte per wave for the role exchange (below)
constexpr int kDmaBytes = 1024;  // bytes one 16-byte-per-lane wave instruction moves

// D = 32 (not the tangent-only kernel): the two 16-row tiles of O^T (and A^T, C^T) cover the
// features d = 2 i + dt (i = tile row, dt = tile) instead of 16 dt + i, so a lane's two V
// values of a contraction step (features 2 c, 2 c + 1) are one 8-byte LDS read instead of two
// 4-byte reads, and a lane's eight outputs are the contiguous features 8 g .. 8 g + 7. (While
// the partner wave's products run, an LDS read instruction costs a wave ~80 cycles whatever
// its width: c2 89.5 -> 88.7 us, the gated c2 shape 89.3 -> 88.0 us, the forward-only kernel
// of the two-launch route 0.4% faster on MI355X; the tangent-only kernel, whose given out
// rows then load as eight floats, measured 1% slower and keeps 4-byte reads.)
template <int D, int T, bool GIVEN_LSE>
constexpr bool pc_pair_d() {
  return D == 32 && !GIVEN_LSE;
}

template <int D, int T>
struct PcShape {
  static constexpr int NT = 2 + 2 * T;  // K, Kt[T], V, Vt[T]
  static constexpr int ROWB = D * 4;
  static constexpr int CHUNKS = D / 4;  // 16-byte chunks per row
  static constexpr int TILE = 64 * ROWB;
  static constexpr int BUF = NT * TILE;
  static constexpr int LDS = 2 * BUF + kSlots * kSlotBytes;
  static constexpr int DG = D / 4;
  static constexpr int DT = (D + 15) / 16;
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int C4 = D / 4;
};

// Chunk swizzle of key row r: the 16-byte chunk c of row r sits at chunk position
// c ^ swz(r). With x = r mod 16, swz = ((x >> 2) & 3) | ((x & 1) << 2), cut to the chunks
// of a row. It is a bijection on {x : x mod 4 in {0, 1}} and on {x : x mod 4 in {2, 3}}
// (the rows that eight lanes of a K read touch together) and flips bit 2 between rows
// 4m and 4m+1, 4m+2 and 4m+3 (the row pairs of a V read), so neither read pattern
// conflicts on the 32 LDS banks for D >= 32.
// Row staging of the bias (mode 2 below): a consumer wave loads its 16 query rows whole and
// gathers its keys from them through LDS, one region per tensor (e, e_t[t]). Row cq of a
// region sits at cq * kERowF floats (64 keys and a pad that keeps rows 16-byte aligned).
// Rows of the compacted layout hold the keys in the item's key order, so they are staged
// with the keys of every 16-key block permuted (key 16 q + 4 r + u at 16 q + 4 u + r): a
// lane's four keys of a key tile are then one 16-byte read instead of four 4-byte reads.
// While the partner wave's products run, an LDS read instruction costs a wave ~80 cycles
// whatever its width (MI355X), so this takes the gated trunk call from 286 to 244 us.
// Served where two workgroups per CU still fit (D = 8; D = 16 with T <= 1; D = 32 with
// T = 0); sharing one region between the tensors costs more than it saves (measured at
// D = 32, T = 1: 139 against 137 us).
template <int D, int T>
struct PcEStage {
  static constexpr int kERowF = 68;
  static constexpr int kRegion = 16 * kERowF * 4;
  static constexpr int BYTES = 3 * (1 + T) * kRegion;  // three consumer waves
  static constexpr bool OK = PcShape<D, T>::LDS + BYTES <= 80 * 1024;
};

template <int D>
__device__ __forceinline__ int swz(int r) {
  return ((((r >> 2) & 3) | ((r & 1) << 2))) & (PcShape<D, 0>::CHUNKS - 1);
}

// Byte offset of 16-byte chunk c of key row r inside a tile.
template <int D>
__device__ __forceinline__ int swz_off(int r, int c) {
  return r * PcShape<D, 0>::ROWB + ((c ^ swz<D>(r)) << 4);
}

// Inside a 16-key tile the S^T rows are a transposed 4x4 arrangement of the keys: S^T row
// 4g + r holds key 4r + g. A lane's C-layout values r = 0..3 then hold keys 4r + g, so
// the P.V products of contraction step r cover keys 4r..4r+3, and a partial last tile
// (n mod 16 keys) skips the steps whose four keys are all padding.
__device__ __forceinline__ int srow_key(int row) { return 4 * (row & 3) + (row >> 2); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}

// Output rows are written once and not read again by this kernel: non-temporal stores (the
// nt cache-policy bit; same bytes). On MI355X at [1024, 64, 8, 32]: 0-1.3% faster without a
// bias, 4% faster with one (the bias rows then keep more of the caches).
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, int voff, float a, float b,
                                           float c, float d) {
  constexpr int kNonTemporal = 2;
  const u32x4_t v = {__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)};
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, kNonTemporal);
}

// The producer's zero rows keep the default cache policy: non-temporal stores there made the
// c2 shape 1.5% slower on MI355X.
__device__ __forceinline__ void zero_row4(void* base, int64_t off) {
  *reinterpret_cast<float4*>(static_cast<float*>(base) + off) = make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, int voff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
}

__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, int voff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0]+[15:14], expcnt[6:4], lgkmcnt[11:8]).
constexpr int kWaitLgkm0 = 0xC07F;
constexpr int kWaitAll0 = 0x0070;

__device__ __forceinline__ void wg_barrier() {
  compiler_fence();
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

// Compacted sites of one walker, lane-resident: lane j holds the j-th physical site
// (ascending), then the masked sites (ascending).
struct PcSites {
  int perm;
  int n_phys;
};

__device__ __forceinline__ PcSites pc_sites(uint32_t mbyte, int N) {
  const int lane = threadIdx.x & 63;
  const bool on = lane < N && mbyte != 0;
  const uint64_t bal = __ballot(on);
  PcSites st;
  st.n_phys = __popcll(bal);
  const int below = __popcll(bal & ((uint64_t(1) << lane) - 1));
  const int pos = on ? below : (lane < N ? st.n_phys + (lane - below) : lane);
  st.perm = __builtin_amdgcn_ds_permute(pos << 2, lane);
  return st;
}

// Key / query lists from the site list (mask semantics of include/hz_mhsea.h): under the
// square mask both are the physical sites; under the key mask the queries are all sites,
// and so are the keys when no site is physical.
__device__ __forceinline__ int pc_nk(int n_phys, bool km, int N) { return (km && n_phys == 0) ? N : n_phys; }
__device__ __forceinline__ int pc_nq(int n_phys, bool km, int N) { return km ? N : n_phys; }

// Items of one workgroup: units first, first + stride, ...; a unit is a (walker, head), or
// under the gated head collapse (half = H/2 > 0) a (walker, head pair) taken as two
// consecutive items, the gate head hp (even k) and then the value head hp + H/2 (odd k).
struct ItemSeq {
  uint32_t first, stride, nitems, H, half;
  __device__ __forceinline__ uint32_t item(int k) const { return first + static_cast<uint32_t>(k) * stride; }
  __device__ __forceinline__ void bh(int k, int& b, int& h) const {
    if (half != 0) {
      const uint32_t u = item(k >> 1);
      const uint32_t bq = u / half;
      b = static_cast<int>(bq);
      h = static_cast<int>(u - bq * half) + (k & 1) * static_cast<int>(half);
      return;
    }
    const uint32_t it = item(k);
    const uint32_t bq = it / H;
    b = static_cast<int>(bq);
    h = static_cast<int>(it - bq * H);
  }
};

// ------------------------------------------------------------------------------------
// Producer (role 3)
// ------------------------------------------------------------------------------------
template <int D, int T, bool GIVEN_LSE, bool GATED>
__device__ __forceinline__ void pc_producer(const FwdParams& p, char* lds, const ItemSeq& seq, int cnt) {
  using Sh = PcShape<D, T>;
  const int lane = threadIdx.x & 63;
  const int N = p.N, H = p.H;
  const bool km = p.key_mask != 0;
  const MaskReader mreader(p.mask, static_cast<int64_t>(p.B) * N);
  char* const slots = lds + 2 * Sh::BUF;

  auto write_slot = [&](int k, const PcSites& st) {
    char* s = slots + (k % kSlots) * kSlotBytes;
    reinterpret_cast<int16_t*>(s)[lane] = static_cast<int16_t>(st.perm);
    if (lane == 0) reinterpret_cast<int*>(s + 128)[0] = st.n_phys;
  };

  auto zero_rows = [&](char* tile, int r0, int r1) {
    const int n = (r1 - r0) * Sh::CHUNKS;
    for (int i = lane; i < n; i += 64) {
      const int r = r0 + i / Sh::CHUNKS;
      *reinterpret_cast<float4*>(tile + r * Sh::ROWB + (i % Sh::CHUNKS) * 16) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };

  // Item k's key tiles travel in two steps one period apart: load() issues every 16-byte
  // global read of the item's physical key rows into registers (one wave instruction per
  // 1 KiB of a tile), and a period later, after one wait, store() writes them to LDS. So
  // the load latency of an item overlaps a whole period of the consumers' work.
  // Instruction j of a tile covers tile bytes [1024 j, 1024 j + 1024); lane l holds the
  // 16 bytes at 1024 j + 16 l, i.e. chunk position pch of row r_j, which comes from the
  // row's swizzled source chunk. The per-lane byte offsets inside the walker's slice are
  // computed once per item (one batch of ds_bpermute); each tensor then reads from a
  // scalar base address. A null tangent stages zeros.
  constexpr int RPI = kDmaBytes / Sh::ROWB;  // rows per instruction
  constexpr int NJ = 64 / RPI;               // instructions per full 64-row tile
  float4 stage[Sh::NT][NJ];
  const int r0 = lane * 16 / Sh::ROWB;
  auto load = [&](int k, const PcSites& st) {
    int b, h;
    seq.bh(k, b, h);
    const int nk = pc_nk(st.n_phys, km, N);
    const int kperm = (km && st.n_phys == 0) ? lane : st.perm;
    const int pch = (lane * 16 % Sh::ROWB) >> 4;
    uint32_t off[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int r = j * RPI + r0;
      const int site = __shfl(kperm, r, 64);
      const int c = pch ^ swz<D>(r);
      off[j] = static_cast<uint32_t>(((site * H + h) * D) * 4 + c * 16);
    }
    const int64_t wofs = static_cast<int64_t>(b) * N * H * D;  // walker offset, elements
#pragma unroll
    for (int x = 0; x < Sh::NT; ++x) {
      const bool is_t = (x >= 1 && x <= T) || x > T + 1;
      const bool is_v = x > T;
      const int t = is_v ? x - T - 2 : x - 1;
      const void* src0 = is_v ? (is_t ? p.vt : p.v) : (is_t ? p.kt : p.k);
      const void* src = src0 != nullptr ? src0 : p.k;
      const char* wbase = reinterpret_cast<const char*>(static_cast<const float*>(src) +
                                                        (is_t && src0 != nullptr ? t * p.t_stride : 0) + wofs);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j * RPI < nk && j * RPI + r0 < nk) v = *reinterpret_cast<const float4*>(wbase + off[j]);
        stage[x][j] = src0 != nullptr ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto store = [&](int k, const PcSites& st) {
    const int nk = pc_nk(st.n_phys, km, N);
    const int nkpad = (nk + 15) & ~15;
    char* buf = lds + (k & 1) * Sh::BUF;
#pragma unroll
    for (int x = 0; x < Sh::NT; ++x) {
      char* tile = buf + x * Sh::TILE;
      zero_rows(tile, nk, nkpad);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (j * RPI < nk && j * RPI + r0 < nk)
          *reinterpret_cast<float4*>(tile + j * kDmaBytes + lane * 16) = stage[x][j];
      }
    }
  };

  // Rows of masked queries (square mask): exact zeros, lse = -1e4 + log N. Item (b, h) writes
  // the masked sites i = h, h + H, h + 2H, ... of walker b (i-th in the site list after the
  // physical ones) for every head at once, so each site's [H, D] rows (1 KB at c2's shape)
  // leave as one contiguous run; the walker's H items cover every masked site once. Writing
  // each item's own 128-byte row of every masked site instead (the same bytes, scattered at
  // a 1 KB stride) made the c2 step 2.6% slower (91.1 against 88.7 us). Under the gated
  // collapse the value-head items (odd k) write y's [H/2, D] site rows, pair hp taking the
  // sites i = hp, hp + H/2, ...
  auto masked_rows = [&](int k, const PcSites& st) {
    if (km) return;
    if (GATED && (k & 1) == 0) return;
    int b, h;
    seq.bh(k, b, h);
    const int nmask = N - st.n_phys;
    const int hs = GATED ? H / 2 : H;  // heads per site row of the output
    const int hi = GATED ? h - hs : h;  // this item's share: sites hi, hi + hs, ...
    const int F = hs * Sh::C4;          // float4 per site row
    const int nmine = nmask > hi ? (nmask - hi + hs - 1) / hs : 0;
    const int64_t tstride = GATED ? p.y_tstride : p.t_stride;
    for (int si = 0; si < nmine; ++si) {
      const int s = __builtin_amdgcn_readlane(st.perm, (st.n_phys + hi + si * hs) & 63);
      const int64_t base = (static_cast<int64_t>(b) * N + s) * hs * D;
      for (int w = lane; w < F; w += 64) {
        if constexpr (!GIVEN_LSE) zero_row4(p.out, base + w * 4);
#pragma unroll
        for (int t = 0; t < T; ++t) zero_row4(p.tout, t * tstride + base + w * 4);
      }
      if (!GATED && !GIVEN_LSE && p.lse != nullptr)
        for (int hh = lane; hh < H; hh += 64) p.lse[(static_cast<int64_t>(b) * N + s) * H + hh] = p.masked_lse;
    }
  };

  auto mask_byte = [&](int k) -> uint32_t {
    int b, h;
    seq.bh(k < cnt ? k : 0, b, h);
    return mreader.byte(b, N, lane);
  };

  // ---- prologue: item 0 in LDS, item 1's sites published and its rows in flight --------
  PcSites cur = pc_sites(mask_byte(0), N);
  write_slot(0, cur);
  load(0, cur);
  uint32_t m = mask_byte(1);
  masked_rows(0, cur);
  __builtin_amdgcn_s_waitcnt(kWaitAll0);
  store(0, cur);
  cur = pc_sites(m, N);  // item 1
  if (cnt > 1) {
    write_slot(1, cur);
    load(1, cur);
    masked_rows(1, cur);
  }
  m = mask_byte(2);
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  wg_barrier();

  for (int k = 0; k < cnt; ++k) {
    // period k: the consumers work on item k. Item k+1's rows (in flight since period
    // k-1) go to LDS, item k+2's sites are published and its rows start loading.
    __builtin_amdgcn_s_waitcnt(kWaitAll0);
    if (k + 1 < cnt) store(k + 1, cur);
    cur = pc_sites(m, N);  // item k+2
    if (k + 2 < cnt) {
      write_slot(k + 2, cur);
      load(k + 2, cur);
      masked_rows(k + 2, cur);
    }
    m = mask_byte(k + 3);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    wg_barrier();
  }
  __builtin_amdgcn_s_waitcnt(kWaitAll0);
}

// ------------------------------------------------------------------------------------
// Consumers (roles 0-2)
// ------------------------------------------------------------------------------------

// One consumer's per-item state: where its query rows are, and their fragments (loaded
// one item ahead).
template <int D, int T>
struct QSet {
  using Sh = PcShape<D, T>;
  float qf[Sh::DG];
  float qtf[Sh::TT][Sh::DG];
  float lse_in;
  float oin[Sh::DT][4];
  int b, h, n_phys, qsite;  // qsite: site of this lane's query (any in-range site if invalid)
};

// DG consecutive floats at byte offset voff of buffer r (16- or 8-byte loads).
template <int DG>
__device__ __forceinline__ void buf_frag(__amdgpu_buffer_rsrc_t r, int voff, float* dst) {
  if constexpr (DG >= 4) {
#pragma unroll
    for (int s = 0; s < DG; s += 4) {
      const u32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 4 * s, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[s + i] = __uint_as_float(x[i]);
    }
  } else {
#pragma unroll
    for (int s = 0; s < DG; s += 2) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, voff + 4 * s, 0, 0);
      dst[s] = __uint_as_float(x[0]);
      dst[s + 1] = __uint_as_float(x[1]);
    }
  }
}

// Query fragments of one 16-query tile of item (b, h): lane (g, c) takes floats
// g*DG .. g*DG+DG-1 of query row c of the tile. Every address is a 32-bit offset into the
// walker's slice of the tensor (b and h are uniform over the wave, so the descriptors are
// scalar); a tangent-free call reads from an empty descriptor, which yields zeros.
template <int D, int T, bool GIVEN_LSE>
__device__ __forceinline__ void pc_load_q(const FwdParams& p, QSet<D, T>& qs, int b, int h, int n_phys,
                                          const int16_t* slot_perm, int tile) {
  using Sh = PcShape<D, T>;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int N = p.N, H = p.H;
  const bool km = p.key_mask != 0;
  const int jq = tile * 16 + c;
  const int nq = pc_nq(n_phys, km, N);
  const int s_raw = km ? jq : static_cast<int>(slot_perm[jq & 63]);
  const int site = (jq < nq) ? s_raw : 0;  // always an in-range row
  // b and h are wave-uniform but may reach here through branches the compiler cannot
  // prove uniform; readfirstlane keeps the descriptors below in scalar registers.
  b = __builtin_amdgcn_readfirstlane(b);
  h = __builtin_amdgcn_readfirstlane(h);
  qs.b = b;
  qs.h = h;
  qs.n_phys = n_phys;
  qs.qsite = site;
  const int64_t wrow = static_cast<int64_t>(N) * H * D;  // floats per walker
  const int wbytes = static_cast<int>(wrow * 4);
  const int row = (site * H + h) * D;
  const int qoff = (row + g * Sh::DG) * 4;
  buf_frag<Sh::DG>(make_rsrc(static_cast<const float*>(p.q) + b * wrow, wbytes), qoff, qs.qf);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float* qt = p.qt != nullptr ? static_cast<const float*>(p.qt) + t * p.t_stride + b * wrow
                                      : static_cast<const float*>(p.q);
    buf_frag<Sh::DG>(make_rsrc(qt, p.qt != nullptr ? wbytes : 0), qoff, qs.qtf[t]);
  }
  if constexpr (GIVEN_LSE) {
    const __amdgpu_buffer_rsrc_t l_rs = make_rsrc(p.lse_in + static_cast<int64_t>(b) * N * H, N * H * 4);
    qs.lse_in = buf_load1(l_rs, (site * H + h) * 4);
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(static_cast<const float*>(p.out_in) + b * wrow, wbytes);
#pragma unroll
    for (int dt = 0; dt < Sh::DT; ++dt) {
      const int d0 = (D % 16 == 0) ? dt * 16 + 4 * g : min(dt * 16 + 4 * g, D - 4);
      buf_frag<4>(o_rs, (row + d0) * 4, qs.oin[dt]);
    }
  }
}

// Forces the compiler to materialise v here (and so to wait for its load, if any),
// without emitting an instruction.
__device__ __forceinline__ void settle(float& v) { asm volatile("" : "+v"(v)); }

template <int D, int T, bool GIVEN_LSE>
__device__ __forceinline__ void settle_q(QSet<D, T>& qs) {
  using Sh = PcShape<D, T>;
#pragma unroll
  for (int s = 0; s < Sh::DG; ++s) {
    settle(qs.qf[s]);
#pragma unroll
    for (int t = 0; t < T; ++t) settle(qs.qtf[t][s]);
  }
  if constexpr (GIVEN_LSE) {
    settle(qs.lse_in);
#pragma unroll
    for (int dt = 0; dt < Sh::DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) settle(qs.oin[dt][r]);
  }
}

// Compute one 16-query tile of the item described by qs from the key tiles in buf, with
// NJ = ceil(n_keys / 16) key tiles (a compile-time count, so every loop is unrolled
// without branches and the scheduler can interleave the tiles' loads and products).
// pf() issues the next item's query prefetch; it runs after this tile's own global loads
// (bias) are issued, so waiting for those never waits for the prefetch. sq() settles
// the prefetch before this tile's stores, so the next period never waits for them.
// Gate terms of one 16-query tile, carried in registers from the gate head's item to the
// value head's (the next item of the same workgroup: same tile, same lane).
template <int D, int T>
struct GateRegs {
  float s[PcShape<D, T>::DT][4];                         // sigma(g)
  float d[PcShape<D, T>::TT][PcShape<D, T>::DT][4];      // sigma(g) (1 - sigma(g)) gdot[t]
};

// ROLE 0: plain item (out, lse, tout). Gated head collapse (out = y, tout = its tangents,
// layout [B, N, H/2, D]): ROLE 1, the gate head g, leaves sigma(g) and sigma'(g) gdot in gr
// and writes nothing; ROLE 2, the value head v of the same pair, writes
// y = sigma(g) v, ydot = sigma'(g) gdot v + sigma(g) vdot.
// Bias mode EM: 0 none; 1 one 4-byte load per score (any layout of e); 2 the tile's query
// rows loaded whole (a query's keys contiguous, 16-byte-aligned rows) and gathered through
// the wave's LDS regions at estage.
template <int D, int T, bool GIVEN_LSE, int EM, int NJ, int ROLE, class PF, class SQ>
__device__ __forceinline__ void pc_tile(const FwdParams& p, const char* buf, const int16_t* slot_perm,
                                        const QSet<D, T>& qs, int tile, PF&& pf, SQ&& sq, GateRegs<D, T>& gr,
                                        float* estage) {
  using Sh = PcShape<D, T>;
  constexpr bool HAS_E = EM != 0;
  constexpr bool ROWS = EM == 2;
  constexpr int DG = Sh::DG, DT = Sh::DT, TT = Sh::TT;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int N = p.N, H = p.H;
  const bool km = p.key_mask != 0;
  const int b = __builtin_amdgcn_readfirstlane(qs.b), h = __builtin_amdgcn_readfirstlane(qs.h);
  const int nk = pc_nk(qs.n_phys, km, N);
  const int nq = pc_nq(qs.n_phys, km, N);
  const bool key_all = km && qs.n_phys == 0;
  const int jq = tile * 16 + c;
  const bool qvalid = jq < nq;
  const int qsite = qs.qsite;
  constexpr bool kPairD = pc_pair_d<D, T, GIVEN_LSE>();

  // ---- bias (and its tangents) for this lane's 4 NJ scores: issued first -------------
  float ev[NJ][4];
  float etv[TT][NJ][4];
  float4 erow[ROWS ? T + 1 : 1][4];
  // The compacted layout holds row jq of the item's query order at h * N * ceil4(N) +
  // jq * ceil4(nk), keys in the item's key order (no gather through the site list).
  const bool cmp = p.e_compact != 0;
  const int nk4 = (nk + 3) & ~3;
  const int eblk = N * ((N + 3) & ~3);
  if constexpr (HAS_E) {
    const int64_t wstride = cmp ? static_cast<int64_t>(H) * eblk : static_cast<int64_t>(N) * N * H;
    const int64_t ebytes = wstride * 4;
    const __amdgpu_buffer_rsrc_t e_rs = make_rsrc(
        p.e != nullptr ? static_cast<const float*>(p.e) + b * wstride : nullptr, p.e != nullptr ? ebytes : 0);
    auto et_rsrc = [&](int t) {
      return make_rsrc(p.et != nullptr ? static_cast<const float*>(p.et) + t * p.et_stride + b * wstride : nullptr,
                       p.et != nullptr ? ebytes : 0);
    };
    const int e_oob = static_cast<int>(ebytes);
    if constexpr (ROWS) {
      // load i: rows 4i + g of the tile (query tile*16 + 4i + g), the lane's 16-byte chunk c
      // (keys 4c..4c+3); rows of queries past the item's last are not read
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int cq = 4 * i + g;
        const int qs_i = __shfl(qsite, cq, 64);
        const bool ok = tile * 16 + cq < nq && 4 * c < (cmp ? nk : N);
        const int row = cmp ? h * eblk + (tile * 16 + cq) * nk4 : static_cast<int>(qs_i * p.e_sq + h * p.e_sh);
        const int off = ok ? row * 4 + 16 * c : e_oob;
        erow[0][i] = buf_load4(e_rs, off);
#pragma unroll
        for (int t = 0; t < T; ++t) erow[1 + t][i] = buf_load4(et_rsrc(t), off);
      }
    } else {
      const int e_row = cmp ? h * eblk + jq * nk4 : static_cast<int>(qsite * p.e_sq + h * p.e_sh);
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = jt * 16 + 4 * r + g;
          const int ks = cmp ? j : (key_all ? j : static_cast<int>(slot_perm[j & 63])) * static_cast<int>(p.e_sk);
          const int eo = (j < nk && qvalid) ? (e_row + ks) * 4 : e_oob;
          ev[jt][r] = buf_load1(e_rs, eo);
#pragma unroll
          for (int t = 0; t < T; ++t) etv[t][jt][r] = buf_load1(et_rsrc(t), eo);
        }
    }
  }
  static_assert(ROLE == 0 || !GIVEN_LSE, "the gated collapse computes the forward");
  pf();

  // Scores are formed in base 2: log2(e) rides on the query scale, so S^T and dS^T leave
  // the matrix cores already multiplied by it; the tangent epilogue takes ln(2) back.
  const float qscale = qvalid ? p.scale * kLog2e : 0.f;
  const float qtscale = p.qt != nullptr ? qscale : 0.f;
  float qf[DG], qtf[TT][DG];
#pragma unroll
  for (int s = 0; s < DG; ++s) {
    qf[s] = qs.qf[s] * qscale;
#pragma unroll
    for (int t = 0; t < T; ++t) qtf[t][s] = qs.qtf[t][s] * qtscale;
  }

  const char* K0 = buf;                        // K, then Kt[t] at +(1+t) tiles
  const char* V0 = buf + (T + 1) * Sh::TILE;   // V, then Vt[t] at +(1+t) tiles

  // ---- S^T and dS^T -------------------------------------------------------------------
  // Every key row of this item's tiles is read up front (the compiler fence keeps the
  // reads here), then the three product chains run tile-interleaved, so consecutive
  // matrix-core instructions never depend on each other.
  const int krow = srow_key(c);
  float kv[NJ][DG];
  float ktv[NJ][TT][DG];
  if constexpr (DG >= 4) {
#pragma unroll
    for (int u = 0; u < DG / 4; ++u)
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt) {
        const int off = swz_off<D>(jt * 16 + krow, g * (DG / 4) + u);
        const float4 x = *reinterpret_cast<const float4*>(K0 + off);
        kv[jt][4 * u] = x.x;
        kv[jt][4 * u + 1] = x.y;
        kv[jt][4 * u + 2] = x.z;
        kv[jt][4 * u + 3] = x.w;
      }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int u = 0; u < DG / 4; ++u)
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) {
          const int off = swz_off<D>(jt * 16 + krow, g * (DG / 4) + u);
          const float4 y = *reinterpret_cast<const float4*>(K0 + (1 + t) * Sh::TILE + off);
          ktv[jt][t][4 * u] = y.x;
          ktv[jt][t][4 * u + 1] = y.y;
          ktv[jt][t][4 * u + 2] = y.z;
          ktv[jt][t][4 * u + 3] = y.w;
        }
  } else {  // D = 8: two floats per lane, half a chunk
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
      const int off = swz_off<D>(jt * 16 + krow, g >> 1) + (g & 1) * 8;
      const float2 x = *reinterpret_cast<const float2*>(K0 + off);
      kv[jt][0] = x.x;
      kv[jt][1] = x.y;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float2 y = *reinterpret_cast<const float2*>(K0 + (1 + t) * Sh::TILE + off);
        ktv[jt][t][0] = y.x;
        ktv[jt][t][1] = y.y;
      }
    }
  }
  compiler_fence();
  v4f sc[NJ];
  v4f ds[TT][NJ];
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt) {
    sc[jt] = zero4();
#pragma unroll
    for (int t = 0; t < T; ++t) ds[t][jt] = zero4();
  }
#pragma unroll
  for (int s = 0; s < DG; ++s)
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) sc[jt] = mfma16x4(kv[jt][s], qf[s], sc[jt]);
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int s = 0; s < DG; ++s)
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt) ds[t][jt] = mfma16x4(ktv[jt][t][s], qf[s], ds[t][jt]);
#pragma unroll
    for (int s = 0; s < DG; ++s)
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt) ds[t][jt] = mfma16x4(kv[jt][s], qtf[t][s], ds[t][jt]);
  }

  // ---- row-staged bias: the rows go to LDS while the matrix cores work on S -----------
  constexpr int kRF = PcEStage<D, T>::kERowF;
  if constexpr (ROWS) {
    if (cmp) {
      // compacted rows: key 16 q + 4 r + u of a staged row at 16 q + 4 u + r, so a lane's
      // four keys of one key tile (4 r + g, r = 0..3) are one 16-byte read below
#pragma unroll
      for (int x = 0; x <= T; ++x)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float* const w = estage + (x * 16 + 4 * i + g) * kRF + 16 * (c >> 2) + (c & 3);
          w[0] = erow[x][i].x;
          w[4] = erow[x][i].y;
          w[8] = erow[x][i].z;
          w[12] = erow[x][i].w;
        }
    } else {
#pragma unroll
      for (int x = 0; x <= T; ++x)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<float4*>(estage + (x * 16 + 4 * i + g) * kRF + 4 * c) = erow[x][i];
    }
  }

  // ---- V and Vt rows for the products, read while the matrix cores finish S -----------
  const bool colok = D % 16 == 0 || c < D;
  const int vcol = (D % 16 == 0) ? c : min(c, D - 1);
  float va[NJ][4][DT];
  float vta[NJ][TT][4][DT];
  if constexpr (kPairD) {
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int off = swz_off<D>(jt * 16 + 4 * r + g, c >> 1) + (c & 1) * 8;
        const float2 x = *reinterpret_cast<const float2*>(V0 + off);
        va[jt][r][0] = x.x;
        va[jt][r][1] = x.y;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float2 y = *reinterpret_cast<const float2*>(V0 + (1 + t) * Sh::TILE + off);
          vta[jt][t][r][0] = y.x;
          vta[jt][t][r][1] = y.y;
        }
      }
  } else {
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int col = dt * 16 + vcol;
        const int off = swz_off<D>(jt * 16 + 4 * r + g, col >> 2) + (col & 3) * 4;
        va[jt][r][dt] = *reinterpret_cast<const float*>(V0 + off);
#pragma unroll
        for (int t = 0; t < T; ++t) vta[jt][t][r][dt] = *reinterpret_cast<const float*>(V0 + (1 + t) * Sh::TILE + off);
      }
  }
  compiler_fence();

  // ---- row-staged bias: this lane's keys from the staged rows (the wave reads only what
  // it wrote, and its LDS accesses complete in order) ----------------------------------
  if constexpr (ROWS) {
    if (cmp) {
#pragma unroll
      for (int x = 0; x <= T; ++x) {
        const float* const rg = estage + x * 16 * kRF + c * kRF + 4 * g;
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) {
          const float4 v = *reinterpret_cast<const float4*>(rg + 16 * jt);
          const float vr[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (x == 0)
              ev[jt][r] = vr[r];
            else
              etv[x - 1][jt][r] = vr[r];
          }
        }
      }
    } else {
#pragma unroll
      for (int x = 0; x <= T; ++x) {
        const float* const rg = estage + x * 16 * kRF;
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = jt * 16 + 4 * r + g;
            const int ks = key_all ? j : static_cast<int>(slot_perm[j & 63]);
            const float val = rg[c * kRF + ks];
            if (x == 0)
              ev[jt][r] = val;
            else
              etv[x - 1][jt][r] = val;
          }
      }
    }
  }

  // ---- bias, validity (only the last key tile can hold padding), max ----------------
  float mx = -INFINITY;
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = jt * 16 + 4 * r + g;
      const bool valid = jt < NJ - 1 || j < nk;
      float sv = sc[jt][r];
      if constexpr (HAS_E) {
        sv = fmaf(ev[jt][r], kLog2e, sv);
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][jt][r] = fmaf(etv[t][jt][r], kLog2e, ds[t][jt][r]);
      }
      sc[jt][r] = valid ? sv : -INFINITY;
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t][jt][r] = valid ? ds[t][jt][r] : 0.f;
      mx = fmaxf(mx, sc[jt][r]);
    }
  }

  float lsum = 0.f;
  if constexpr (GIVEN_LSE) {
    const float lse2 = qs.lse_in * kLog2e;
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[jt][r] = lse_weight(sc[jt][r] - lse2);
  } else {
    mx = group_max(mx);
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[jt][r] = fast_exp2(sc[jt][r] - mx);
        lsum += sc[jt][r];
      }
  }
  float mu[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    mu[t] = 0.f;
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
      ds[t][jt] *= sc[jt];
      mu[t] += (ds[t][jt][0] + ds[t][jt][1]) + (ds[t][jt][2] + ds[t][jt][3]);
    }
  }

  // ---- O^T, A^T, C^T: step r of tile jt contracts keys jt*16 + 4r + (0..3); steps of
  // the last tile whose four keys are all padding are skipped ----------------------------
  const bool colmask = !colok;
  v4f o[DT];
  v4f at[TT][DT];
  v4f ct[TT][DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    o[dt] = zero4();
#pragma unroll
    for (int t = 0; t < T; ++t) at[t][dt] = ct[t][dt] = zero4();
  }
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (jt < NJ - 1 || r == 0 || jt * 16 + 4 * r < nk) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const float vv = colmask ? 0.f : va[jt][r][dt];
          if constexpr (!GIVEN_LSE) o[dt] = mfma16x4(vv, sc[jt][r], o[dt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            at[t][dt] = mfma16x4(vv, ds[t][jt][r], at[t][dt]);
            ct[t][dt] = mfma16x4(colmask ? 0.f : vta[jt][t][r][dt], sc[jt][r], ct[t][dt]);
          }
        }
      }
    }
  }

  float inv = 1.f, ltot = 0.f;
  if constexpr (!GIVEN_LSE) {
    ltot = group_sum(lsum);
    inv = __builtin_amdgcn_rcpf(ltot);  // ltot >= 1: the maximum key contributes 2^0
  }
  // A^T and mu carry the log2(e) of dS^T; ln(2) folds into their scale factors.
  const float inv_ln2 = inv * kLn2;
  float mut[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) mut[t] = group_sum(mu[t]) * inv_ln2;

  float ov[DT][4];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) ov[dt][r] = GIVEN_LSE ? qs.oin[dt][r] : o[dt][r] * inv;
  sq();
  // Store u (u < DT) writes features sd0(u) .. sd0(u) + 3; its m-th value is element
  // (sdt(u, m), sr(u, m)) of a lane's [DT][4] outputs.
  auto sd0 = [&](int u) { return kPairD ? 8 * g + 4 * u : u * 16 + 4 * g; };
  auto sdt = [&](int u, int m) { return kPairD ? (m & 1) : u; };
  auto sr = [&](int u, int m) { return kPairD ? 2 * u + (m >> 1) : m; };

  // ---- stores: unconditional, invalid lanes past the walker's last record ------------
  if constexpr (ROLE == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sg = __builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * ov[dt][r]));
        gr.s[dt][r] = sg;
#pragma unroll
        for (int t = 0; t < T; ++t)
          gr.d[t][dt][r] = sg * (1.f - sg) * fmaf(-mut[t], ov[dt][r], fmaf(at[t][dt][r], inv_ln2, ct[t][dt][r] * inv));
      }
    return;
  }
  if constexpr (ROLE == 2) {
    const int hh = H / 2;
    const int64_t ywrow = static_cast<int64_t>(N) * hh * D;  // floats of y per walker
    const int ybytes = static_cast<int>(ywrow * 4);
    const int ybase = (qsite * hh + (h - hh)) * D;
    auto yoff = [&](int u) {
      const int d0 = sd0(u);
      return (qvalid && (D % 16 == 0 || d0 < D)) ? (ybase + d0) * 4 : ybytes;
    };
    const __amdgpu_buffer_rsrc_t y_rs = make_rsrc(static_cast<float*>(p.out) + b * ywrow, ybytes);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      float yv[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) yv[m] = gr.s[sdt(u, m)][sr(u, m)] * ov[sdt(u, m)][sr(u, m)];
      buf_store4(y_rs, yoff(u), yv[0], yv[1], yv[2], yv[3]);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const __amdgpu_buffer_rsrc_t t_rs = make_rsrc(static_cast<float*>(p.tout) + t * p.y_tstride + b * ywrow, ybytes);
#pragma unroll
      for (int u = 0; u < DT; ++u) {
        float tv[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int dt = sdt(u, m), r = sr(u, m);
          const float od = fmaf(-mut[t], ov[dt][r], fmaf(at[t][dt][r], inv_ln2, ct[t][dt][r] * inv));
          tv[m] = fmaf(gr.d[t][dt][r], ov[dt][r], gr.s[dt][r] * od);
        }
        buf_store4(t_rs, yoff(u), tv[0], tv[1], tv[2], tv[3]);
      }
    }
    return;
  }
  const int64_t wrow = static_cast<int64_t>(N) * H * D;  // floats per walker
  const int obytes = static_cast<int>(wrow * 4);
  const int obase = (qsite * H + h) * D;
  if constexpr (!GIVEN_LSE) {
    const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(static_cast<float*>(p.out) + b * wrow, obytes);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      const int d0 = sd0(u);
      const int voff = (qvalid && (D % 16 == 0 || d0 < D)) ? (obase + d0) * 4 : obytes;
      buf_store4(o_rs, voff, ov[sdt(u, 0)][sr(u, 0)], ov[sdt(u, 1)][sr(u, 1)], ov[sdt(u, 2)][sr(u, 2)],
                 ov[sdt(u, 3)][sr(u, 3)]);
    }
    const int lbytes = N * H * 4;
    const __amdgpu_buffer_rsrc_t l_rs =
        make_rsrc(p.lse != nullptr ? p.lse + static_cast<int64_t>(b) * N * H : nullptr, p.lse != nullptr ? lbytes : 0);
    const int lvoff = (qvalid && g == 0) ? (qsite * H + h) * 4 : lbytes;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint((mx + log2f(ltot)) * kLn2), l_rs, lvoff, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const __amdgpu_buffer_rsrc_t t_rs = make_rsrc(static_cast<float*>(p.tout) + t * p.t_stride + b * wrow, obytes);
#pragma unroll
    for (int u = 0; u < DT; ++u) {
      const int d0 = sd0(u);
      const int voff = (qvalid && (D % 16 == 0 || d0 < D)) ? (obase + d0) * 4 : obytes;
      float tv[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int dt = sdt(u, m), r = sr(u, m);
        tv[m] = fmaf(-mut[t], ov[dt][r], fmaf(at[t][dt][r], inv_ln2, ct[t][dt][r] * inv));
      }
      buf_store4(t_rs, voff, tv[0], tv[1], tv[2], tv[3]);
    }
  }
}

// ---- remainder tile of at most four queries ------------------------------------------
// An item's last query tile often holds only a few queries (36 sites: 16 + 16 + 4). The
// 16x16x4 products of pc_tile would spend 12 of their 16 query columns on padding; here
// v_mfma_f32_4x4x1_16b_f32 (sixteen independent 4x4 outer products per instruction, the same
// flops per cycle) does the tile's work at a third of the matrix-core time.
//   S^T: one instruction per feature d; lane l supplies A = K[key l][d] and B = Q[query
//   l & 3][d], so lane 4m + j accumulates the scores of keys 4m .. 4m+3 (registers 0-3) for
//   query j. The four query rows reach every lane through a small LDS region (written from
//   the query fragments, read back as 16-byte rows). The softmax reduces over the 16 lanes of a
//   query (lane bits 2-5).
//   O^T = V^T P^T, A^T, C^T: block b = 8 part + dg covers features 4dg .. 4dg+3; the keys are
//   cut into two parts of 4 H4 (H4 = ceil(nk / 8) groups of 4), and in step (m, r) block b
//   takes key 4 (part H4 + m) + r: lane l supplies A = V[key][l mod 32] and B = P[query
//   l & 3][key]. The weights go through the same LDS region, so one 16-byte read gives a lane
//   the four keys of its steps (m, 0..3) (gathering them by ds_bpermute, one per step, made the
//   c2 step 1.5% slower). Lane 32 part + 4dg + j then holds features 4dg .. 4dg+3 of query j for
//   its part; the parts are added across lane bit 5. Keys nk .. 8 H4 - 1 read rows the
//   producer zero-fills (8 H4 <= the 16-row padded count) and carry P = 0.
// Served for D = 32, the plain forward (+ tangents) without bias; the LDS region holds
// (1 + T) x (4 query rows + 4 x 64 weights) floats, one per workgroup (one remainder tile per
// item).
__device__ __forceinline__ v4f mfma4x4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// Rotation by n lanes inside each row of 16 lanes (DPP row_ror).
template <int n>
__device__ __forceinline__ float row_ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + n, 0xF, 0xF, false));
}
// Max / sum over the 16 lanes with the same lane & 3.
__device__ __forceinline__ float query_max(float x) {
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  return group_max(x);
}
__device__ __forceinline__ float query_sum(float x) {
  x += row_ror<4>(x);
  x += row_ror<8>(x);
  return group_sum(x);
}

template <int D, int T, class PF, class SQ>
__device__ __forceinline__ void pc_tile_rem4(const FwdParams& p, const char* buf, const QSet<D, T>& qs, int tile,
                                             PF&& pf, SQ&& sq, float* rl) {
  static_assert(D == 32, "four-query remainder tile: D = 32");
  using Sh = PcShape<D, T>;
  constexpr int DG = Sh::DG, TT = Sh::TT;
  const int lane = threadIdx.x & 63;
  const int j = lane & 3;
  const int N = p.N, H = p.H;
  const bool km = p.key_mask != 0;
  const int b = __builtin_amdgcn_readfirstlane(qs.b), h = __builtin_amdgcn_readfirstlane(qs.h);
  const int nk = pc_nk(qs.n_phys, km, N);
  const int nq = pc_nq(qs.n_phys, km, N);
  const bool qvalid = tile * 16 + j < nq;
  const int qsite = __shfl(qs.qsite, j, 64);
  pf();

  const char* K0 = buf;
  const char* V0 = buf + (T + 1) * Sh::TILE;

  // ---- S^T and dS^T: key row `lane` against the four queries --------------------------
  float kv[D], ktv[TT][D];
#pragma unroll
  for (int c = 0; c < D / 4; ++c) {
    const int off = swz_off<D>(lane, c);
    const float4 x = *reinterpret_cast<const float4*>(K0 + off);
    kv[4 * c] = x.x;
    kv[4 * c + 1] = x.y;
    kv[4 * c + 2] = x.z;
    kv[4 * c + 3] = x.w;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float4 y = *reinterpret_cast<const float4*>(K0 + (1 + t) * Sh::TILE + off);
      ktv[t][4 * c] = y.x;
      ktv[t][4 * c + 1] = y.y;
      ktv[t][4 * c + 2] = y.z;
      ktv[t][4 * c + 3] = y.w;
    }
  }
  // the four query rows (and tangents) through LDS: lanes (g, c < 4) write their fragments,
  // every lane reads its query's row (the wave's LDS accesses complete in order)
  {
    const int g = lane >> 4, c = lane & 15;
    if (c < 4) {
#pragma unroll
      for (int s4 = 0; s4 < DG; s4 += 4) {
        *reinterpret_cast<float4*>(rl + c * D + g * DG + s4) =
            make_float4(qs.qf[s4], qs.qf[s4 + 1], qs.qf[s4 + 2], qs.qf[s4 + 3]);
#pragma unroll
        for (int t = 0; t < T; ++t)
          *reinterpret_cast<float4*>(rl + (1 + t) * 4 * D + c * D + g * DG + s4) =
              make_float4(qs.qtf[t][s4], qs.qtf[t][s4 + 1], qs.qtf[t][s4 + 2], qs.qtf[t][s4 + 3]);
      }
    }
  }
  float qrow[D], qtrow[TT][D];
#pragma unroll
  for (int d4 = 0; d4 < D; d4 += 4) {
    const float4 x = *reinterpret_cast<const float4*>(rl + j * D + d4);
    qrow[d4] = x.x;
    qrow[d4 + 1] = x.y;
    qrow[d4 + 2] = x.z;
    qrow[d4 + 3] = x.w;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float4 y = *reinterpret_cast<const float4*>(rl + (1 + t) * 4 * D + j * D + d4);
      qtrow[t][d4] = y.x;
      qtrow[t][d4 + 1] = y.y;
      qtrow[t][d4 + 2] = y.z;
      qtrow[t][d4 + 3] = y.w;
    }
  }
  v4f sc = zero4();
  v4f ds[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) ds[t] = zero4();
#pragma unroll
  for (int d = 0; d < D; ++d) {
    sc = mfma4x4(kv[d], qrow[d], sc);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      ds[t] = mfma4x4(ktv[t][d], qrow[d], ds[t]);
      ds[t] = mfma4x4(kv[d], qtrow[t][d], ds[t]);
    }
  }

  // ---- scale (log2 e rides on it), validity, exact softmax over the item's keys --------
  const float qscale = qvalid ? p.scale * kLog2e : 0.f;
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const bool valid = 4 * (lane >> 2) + r < nk;
    sc[r] = valid ? sc[r] * qscale : -INFINITY;
#pragma unroll
    for (int t = 0; t < T; ++t) ds[t][r] = valid ? ds[t][r] * qscale : 0.f;
    mx = fmaxf(mx, sc[r]);
  }
  mx = query_max(mx);
  float lsum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    sc[r] = fast_exp2(sc[r] - mx);
    lsum += sc[r];
  }
  float mu[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    ds[t] *= sc;
    mu[t] = (ds[t][0] + ds[t][1]) + (ds[t][2] + ds[t][3]);
  }

  // ---- O^T, A^T, C^T ---------------------------------------------------------------------
  const int part = lane >> 5;
  const int h4 = (nk + 7) >> 3;
  const int dcol = lane & 31;
  // weights through LDS: lane 4m + j holds P[j][4m .. 4m + 3] (and P o dS): one 16-byte write
  // each, then one 16-byte read per key group gives a lane its four keys of a step
  float* const pl = rl + (1 + T) * 4 * D;  // [(1 + T)][4 queries][64 keys]
  *reinterpret_cast<v4f*>(pl + j * 64 + 4 * (lane >> 2)) = sc;
#pragma unroll
  for (int t = 0; t < T; ++t) *reinterpret_cast<v4f*>(pl + (1 + t) * 256 + j * 64 + 4 * (lane >> 2)) = ds[t];
  v4f o = zero4();
  v4f at[TT], ct[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) at[t] = ct[t] = zero4();
  for (int m = 0; m < h4; ++m) {
    const int grp = part * h4 + m;
    const v4f p4 = *reinterpret_cast<const v4f*>(pl + j * 64 + 4 * grp);
    v4f d4[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) d4[t] = *reinterpret_cast<const v4f*>(pl + (1 + t) * 256 + j * 64 + 4 * grp);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int off = swz_off<D>(4 * grp + r, dcol >> 2) + (dcol & 3) * 4;
      const float vv = *reinterpret_cast<const float*>(V0 + off);
      o = mfma4x4(vv, p4[r], o);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float vt = *reinterpret_cast<const float*>(V0 + (1 + t) * Sh::TILE + off);
        at[t] = mfma4x4(vv, d4[t][r], at[t]);
        ct[t] = mfma4x4(vt, p4[r], ct[t]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    o[r] = xor32_pair_sum(o[r]);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      at[t][r] = xor32_pair_sum(at[t][r]);
      ct[t][r] = xor32_pair_sum(ct[t][r]);
    }
  }

  const float ltot = query_sum(lsum);
  const float inv = __builtin_amdgcn_rcpf(ltot);  // ltot >= 1: the maximum key contributes 2^0
  const float inv_ln2 = inv * kLn2;
  float mut[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) mut[t] = query_sum(mu[t]) * inv_ln2;
  float ov[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) ov[r] = o[r] * inv;
  sq();

  // ---- stores: lanes 0-31 (part 0) write features 4 dg .. 4 dg + 3 of query j ------------
  const int64_t wrow = static_cast<int64_t>(N) * H * D;
  const int obytes = static_cast<int>(wrow * 4);
  const int obase = (qsite * H + h) * D;
  const int voff = (qvalid && part == 0) ? (obase + 4 * (lane >> 2)) * 4 : obytes;
  const __amdgpu_buffer_rsrc_t o_rs = make_rsrc(static_cast<float*>(p.out) + b * wrow, obytes);
  buf_store4(o_rs, voff, ov[0], ov[1], ov[2], ov[3]);
  const int lbytes = N * H * 4;
  const __amdgpu_buffer_rsrc_t l_rs =
      make_rsrc(p.lse != nullptr ? p.lse + static_cast<int64_t>(b) * N * H : nullptr, p.lse != nullptr ? lbytes : 0);
  const int lvoff = (qvalid && lane < 4) ? (qsite * H + h) * 4 : lbytes;
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint((mx + log2f(ltot)) * kLn2), l_rs, lvoff, 0, 0);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const __amdgpu_buffer_rsrc_t t_rs = make_rsrc(static_cast<float*>(p.tout) + t * p.t_stride + b * wrow, obytes);
    float tv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) tv[r] = fmaf(-mut[t], ov[r], fmaf(at[t][r], inv_ln2, ct[t][r] * inv));
    buf_store4(t_rs, voff, tv[0], tv[1], tv[2], tv[3]);
  }
}

template <int D, int T, bool GIVEN_LSE, int EM, bool GATED>
__device__ __forceinline__ void pc_consumer(const FwdParams& p, char* lds, const ItemSeq& seq, int cnt, int wave) {
  using Sh = PcShape<D, T>;
  float* const estage = EM == 2 ? reinterpret_cast<float*>(lds + 2 * Sh::BUF + kSlots * kSlotBytes) +
                                      wave * (1 + T) * (PcEStage<D, T>::kRegion / 4)
                                : nullptr;
  const int N = p.N;
  const bool km = p.key_mask != 0;
  const char* const slots = lds + 2 * Sh::BUF;
  // the four-query remainder tile's LDS region (one per workgroup: one remainder tile per item)
  float* const rem_lds = reinterpret_cast<float*>(lds + Sh::LDS + (EM == 2 ? PcEStage<D, T>::BYTES : 0));
  auto slot_perm = [&](int k) { return reinterpret_cast<const int16_t*>(slots + (k % kSlots) * kSlotBytes); };
  auto slot_n = [&](int k) { return reinterpret_cast<const int*>(slots + (k % kSlots) * kSlotBytes + 128)[0]; };

  // Prefetch item k's query fragments (item k-1's when k is past the end, which keeps
  // the number of loads per period fixed).
  auto prefetch = [&](QSet<D, T>& qs, const QSet<D, T>& prev, int k) {
    if (k < cnt) {
      int b, h;
      seq.bh(k, b, h);
      pc_load_q<D, T, GIVEN_LSE>(p, qs, b, h, slot_n(k), slot_perm(k), wave);
    } else {
      pc_load_q<D, T, GIVEN_LSE>(p, qs, prev.b, prev.h, 0, slot_perm(k - 1), wave);
      qs.n_phys = prev.n_phys;
    }
  };

  // Item k with this wave's query fragments qs; the next item's go into nq_set.
  // gate terms of this wave's tile and of the fourth tile (consumer 0), gated collapse only
  GateRegs<D, T> gm, gx;
  auto compute = [&](auto role, const QSet<D, T>& qs, QSet<D, T>& nx, int k) {
    constexpr int R = decltype(role)::value;
    const char* buf = lds + (k & 1) * Sh::BUF;
    const int nq = pc_nq(qs.n_phys, km, N);
    const int nk = pc_nk(qs.n_phys, km, N);
    auto pf = [&]() { prefetch(nx, qs, k + 1); };
    auto sq = [&]() { settle_q<D, T, GIVEN_LSE>(nx); };
    const int16_t* sp = slot_perm(k);
    // Remainder tiles of at most four queries take the 4x4-block path where it is built.
    constexpr bool kRem4 = D == 32 && !GIVEN_LSE && EM == 0 && R == 0;
    if (kRem4 && wave * 16 < nq && nq - wave * 16 <= 4) {
      if constexpr (kRem4) pc_tile_rem4<D, T>(p, buf, qs, wave, pf, sq, rem_lds);
    } else if (wave * 16 < nq) {
      switch ((nk + 15) >> 4) {
        case 1: pc_tile<D, T, GIVEN_LSE, EM, 1, R>(p, buf, sp, qs, wave, pf, sq, gm, estage); break;
        case 2: pc_tile<D, T, GIVEN_LSE, EM, 2, R>(p, buf, sp, qs, wave, pf, sq, gm, estage); break;
        case 3: pc_tile<D, T, GIVEN_LSE, EM, 3, R>(p, buf, sp, qs, wave, pf, sq, gm, estage); break;
        default: pc_tile<D, T, GIVEN_LSE, EM, 4, R>(p, buf, sp, qs, wave, pf, sq, gm, estage); break;
      }
    } else {
      pf();
      sq();
    }
    // A fourth query tile (n > 48) goes to consumer 0, with its fragments loaded here.
    // The tile count must be the item's own: padding is only masked in the last key tile.
    if (wave == 0 && 3 * 16 < nq) {
      QSet<D, T> q3;
      pc_load_q<D, T, GIVEN_LSE>(p, q3, qs.b, qs.h, qs.n_phys, sp, 3);
      if (kRem4 && nq - 3 * 16 <= 4) {
        if constexpr (kRem4) pc_tile_rem4<D, T>(p, buf, q3, 3, [] {}, [] {}, rem_lds);
      } else {
        switch ((nk + 15) >> 4) {
          case 1: pc_tile<D, T, GIVEN_LSE, EM, 1, R>(p, buf, sp, q3, 3, [] {}, [] {}, gx, estage); break;
          case 2: pc_tile<D, T, GIVEN_LSE, EM, 2, R>(p, buf, sp, q3, 3, [] {}, [] {}, gx, estage); break;
          case 3: pc_tile<D, T, GIVEN_LSE, EM, 3, R>(p, buf, sp, q3, 3, [] {}, [] {}, gx, estage); break;
          default: pc_tile<D, T, GIVEN_LSE, EM, 4, R>(p, buf, sp, q3, 3, [] {}, [] {}, gx, estage); break;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  };

  QSet<D, T> qa, qb;
  wg_barrier();  // item 0 ready, item 1's sites published
  {
    int b, h;
    seq.bh(0, b, h);
    pc_load_q<D, T, GIVEN_LSE>(p, qa, b, h, slot_n(0), slot_perm(0), wave);
  }
  // Gated: cnt is even, so item k (even) is the gate head and k + 1 the value head.
  for (int k = 0; k < cnt; k += 2) {
    compute(std::integral_constant<int, GATED ? 1 : 0>{}, qa, qb, k);
    wg_barrier();
    if (k + 1 >= cnt) break;
    compute(std::integral_constant<int, GATED ? 2 : 0>{}, qb, qa, k + 1);
    wg_barrier();
  }
}

// Roles by SIMD. The hardware spreads a workgroup's four waves over the CU's four SIMDs in an
// order that differs between the two workgroups sharing the CU (recorded from HW_ID on MI355X:
// waves 0-3 of one on SIMDs 2, 1, 3, 0, of the other on 1, 3, 0, 2), so roles taken from the
// wave index put a producer beside a consumer on two SIMDs. Roles here are the ranks of
// (SIMD, wave index) within the workgroup (a permutation of 0-3 whatever the placement): the
// wave on the highest SIMD produces, so both workgroups' producers share one SIMD and every
// consumer shares its SIMD with the other workgroup's consumer of the same query tile. Without
// a bias, a producer's loads, LDS stores and waits beside a consumer cost that consumer more
// than a second consumer does (MI355X, same box: c2 91.9 against 95.4 us, the forward of the
// two-launch route 125.3 against 132.8, the gated c2 shape unchanged). With a bias the
// consumers stream the bias rows themselves and the wave-index roles are faster (c2e 120.1
// against 124.1 us, the gated trunk shape 290 against 303), so they keep those. The ranks go
// through one byte per wave in slot 0 (bytes the site lists never use) before the first
// barrier.
__device__ __forceinline__ int pc_role(char* xch) {
  const int w = threadIdx.x >> 6;
  constexpr int kHwIdAll = (31 << 11) | 4;  // s_getreg: HW_REG_HW_ID, bits 0-31
  const int simd = static_cast<int>((__builtin_amdgcn_s_getreg(kHwIdAll) >> 4) & 3);
  const int key = (simd << 2) | w;
  if ((threadIdx.x & 63) == 0) xch[w] = static_cast<char>(key);
  __syncthreads();
  int role = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) role += xch[i] < key;
  return __builtin_amdgcn_readfirstlane(role);
}

template <int D, int T, bool GIVEN_LSE, int EM, bool GATED>
__global__ void __launch_bounds__(256, 2) mhsea_fwd_pc_kernel(const FwdParams p) {
  using Sh = PcShape<D, T>;
  extern __shared__ float4 smem4[];
  char* const lds = reinterpret_cast<char*>(smem4);
  const uint32_t half = GATED ? static_cast<uint32_t>(p.H) / 2 : 0u;
  const uint32_t nunits = static_cast<uint32_t>(p.B) * (GATED ? half : static_cast<uint32_t>(p.H));
  const uint32_t G = gridDim.x;
  const uint32_t L = static_cast<uint32_t>(xcd_logical_block(blockIdx.x, G));
  if (L >= nunits) return;  // workgroup-uniform
  const ItemSeq seq{L, G, nunits, static_cast<uint32_t>(p.H), half};
  const int cnt = static_cast<int>((nunits - L + G - 1) / G) * (GATED ? 2 : 1);
  const int role = EM == 0 ? pc_role(lds + 2 * Sh::BUF + kRoleBytes) : static_cast<int>(threadIdx.x >> 6);
  if (role == kProducerWave)
    pc_producer<D, T, GIVEN_LSE, GATED>(p, lds, seq, cnt);
  else
    pc_consumer<D, T, GIVEN_LSE, EM, GATED>(p, lds, seq, cnt, role);
  (void)Sh::LDS;
}

template <int D, int T, bool GIVEN_LSE, int EM, bool GATED>
hipError_t launch_pc_t(const FwdParams& p, hipStream_t stream) {
  using Sh = PcShape<D, T>;
  static_assert(EM != 2 || PcEStage<D, T>::OK, "two workgroups per CU");
  auto kern = mhsea_fwd_pc_kernel<D, T, GIVEN_LSE, EM, GATED>;
  constexpr bool kRem4Lds = D == 32 && !GIVEN_LSE && EM == 0 && !GATED;
  const size_t lds = Sh::LDS + (EM == 2 ? PcEStage<D, T>::BYTES : 0) + (kRem4Lds ? (1 + T) * (4 * D + 256) * 4 : 0);
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  // occupancy of this instantiation, computed once; relaxed atomics keep concurrent
  // first calls from several host threads free of data races
  static std::atomic<int> per_cu_cache{0};
  int per_cu = per_cu_cache.load(std::memory_order_relaxed);
  if (per_cu == 0) {
    int n = 0;
    hipError_t err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kern), 256, lds);
    if (err != hipSuccess) return err;
    per_cu = n > 0 ? n : 1;
    per_cu_cache.store(per_cu, std::memory_order_relaxed);
  }
  int cus = 0;
  hipError_t err = device_cu_count(&cus);
  if (err != hipSuccess) return err;
  const int64_t nunits = static_cast<int64_t>(p.B) * (GATED ? p.H / 2 : p.H);
  int64_t grid = static_cast<int64_t>(cus) * per_cu;
  if (grid > nunits) grid = nunits;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(256), lds, stream, p);
  return hipGetLastError();
}

// Shapes served: two workgroups per CU must fit their double-buffered key tiles in LDS.
template <int D, int T>
constexpr bool pc_shape_ok() {
  return PcShape<D, T>::LDS <= 80 * 1024;
}

// Bias rows can be staged whole when a query's keys are contiguous and every row starts on a
// 16-byte boundary (the [B, N, H, N] layout with N a multiple of 4, or the compacted layout;
// aligned base pointers).
bool e_rows_ok(const FwdParams& p) {
  auto aligned = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  // compacted rows start at multiples of four floats whatever N
  if (p.e_compact) return p.et_stride % 4 == 0 && aligned(p.e) && aligned(p.et);
  return p.e_sk == 1 && p.e_sq % 4 == 0 && p.e_sh % 4 == 0 && p.N % 4 == 0 && p.et_stride % 4 == 0 &&
         aligned(p.e) && aligned(p.et);
}

template <int D, int T, bool GIVEN_LSE, bool GATED>
hipError_t launch_pc_em(const FwdParams& p, hipStream_t stream) {
  if (p.e == nullptr && p.et == nullptr) return launch_pc_t<D, T, GIVEN_LSE, 0, GATED>(p, stream);
  if constexpr (PcEStage<D, T>::OK) {
    if (e_rows_ok(p)) return launch_pc_t<D, T, GIVEN_LSE, 2, GATED>(p, stream);
  }
  return launch_pc_t<D, T, GIVEN_LSE, 1, GATED>(p, stream);
}

template <int D, int T, bool GIVEN_LSE>
hipError_t dispatch_e(const FwdParams& p, hipStream_t stream) {
  if constexpr (pc_shape_ok<D, T>()) {
    if constexpr (!GIVEN_LSE) {
      if (p.gated) return launch_pc_em<D, T, false, true>(p, stream);
    } else {
      if (p.gated) return hipErrorInvalidValue;
    }
    return launch_pc_em<D, T, GIVEN_LSE, false>(p, stream);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t dispatch_t(const FwdParams& p, int T, bool given_lse, hipStream_t stream) {
  if (given_lse) {
    if (T == 1) return dispatch_e<D, 1, true>(p, stream);
    if (T == 2) return dispatch_e<D, 2, true>(p, stream);
    return hipErrorInvalidValue;
  }
  if (T == 0) return dispatch_e<D, 0, false>(p, stream);
  if (T == 1) return dispatch_e<D, 1, false>(p, stream);
  if (T == 2) return dispatch_e<D, 2, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool pc_fwd_supported(int N, int H, int D, int T, int dtype) {
  if (dtype != 0 || N > 64 || T > 2) return false;
  // Per-walker buffer resources: the walker's bias and output slices must stay below 2 GiB.
  if (static_cast<int64_t>(N) * N * H * 4 >= (int64_t(1) << 31)) return false;
  if (static_cast<int64_t>(N) * H * D * 4 >= (int64_t(1) << 31)) return false;
  switch (D) {
    case 8: return pc_shape_ok<8, 0>() && (T < 1 || pc_shape_ok<8, 1>()) && (T < 2 || pc_shape_ok<8, 2>());
    case 16: return (T < 1 || pc_shape_ok<16, 1>()) && (T < 2 || pc_shape_ok<16, 2>());
    case 32: return (T < 1 || pc_shape_ok<32, 1>()) && (T < 2 || pc_shape_ok<32, 2>());
    default: return false;  // D = 64: the key operands of a tile no longer fit the registers
  }
}

hipError_t launch_fwd_pc(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream) {
  switch (D) {
    case 8: return dispatch_t<8>(p, T, given_lse, stream);
    case 16: return dispatch_t<16>(p, T, given_lse, stream);
    case 32: return dispatch_t<32>(p, T, given_lse, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hz
