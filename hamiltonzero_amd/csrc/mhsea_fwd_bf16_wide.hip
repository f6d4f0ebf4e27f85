// bfloat16 forward / forward+tangent MHSEA kernel for large N at head dimension 64 without
// an edge bias: 32-query waves on v_mfma_f32_32x32x16_bf16, one wave per SIMD.
//
// Work decomposition: a 256-thread workgroup (4 waves) owns one (walker, head) and 128
// consecutive compacted queries, 32 per wave. Keys stream through LDS in chunks of 32
// compacted keys, each chunk staged once for the workgroup.
//
// Why 32 x 32 tiles: one v_mfma_f32_32x32x16_bf16 does twice the work of a 16x16x32 product
// for the same 1 KiB operand read from LDS, so the LDS reads per product halve and each K or
// V operand feeds the primal and both tangent products. The price is registers: the
// accumulators (out and T tangent outputs, 32 queries x 64 columns each), a chunk's scores,
// two chunks' bf16 weights, the query fragments and two staging sets take ~460 registers, so
// each SIMD runs one wave with the unified register file (architectural and accumulation
// registers), and the wave hides its own latencies by software pipelining.
//
// Per chunk i a wave runs: S(i), the score products S^T = K Q^T and dS^T = Kt Q^T + K Qt^T;
// SM(i), the online softmax of S(i); PV(i), O^T += V^T P^T and A^T += V^T (s P o dS)^T +
// Vt^T P^T. Iteration i runs SM(i) on the vector ALU interleaved (scheduling-group barriers)
// with the products of PV(i-1) and the global reads of the chunks two ahead, the weights
// of chunks i-1 and i living in two register sets; then S(i+1), interleaved with the LDS
// writes of the staged chunks. One workgroup barrier per iteration.
//
// Staging: K-like chunks (K, Kt[t]) and V-like chunks (V, Vt[t]) have two LDS buffers each;
// chunk j lives in buffer j mod 2. Iteration i issues the global reads of K(i+3) and V(i+1)
// into the staging registers of parity i mod 2 and writes K(i+2) and V(i), read in
// iteration i-1, into the buffers of parity i mod 2. K(j) is read in iteration j-1, V(j) in
// iteration j+1, so every write goes to a buffer whose last reader finished before the
// previous barrier. Every thread stages one 16-byte piece of one row per tensor and kind.
//
// Matrix-core layout of v_mfma_f32_32x32x16_bf16, lane l = 32 hh + c (hh = l / 32):
//   A operand: lane supplies A[row c][k 8 hh .. 8 hh + 7]
//   B operand: lane supplies B[k 8 hh .. 8 hh + 7][col c]
//   C/D:       lane holds element i = 0..15 at C[row 8 (i / 4) + 4 hh + i % 4][col c]
// S^T[key][query]: A = the chunk's K rows (row-major in LDS, rows padded to 72 bf16 so the
// 16 rows of a read phase hit distinct banks), B = the wave's query fragments (registers).
// A lane's scores are 16 keys of one query; k-step s of the P.V products contracts keys
// kappa(s, hh, j) = 16 s + 8 (j / 4) + 4 hh + j % 4, which are exactly the lane's score
// elements 8 s + j, so the B operand is the lane's own weights rounded to bf16. V-like tiles
// stay row-major ([key][d], rows padded to 96 bf16 so the transposing reads below are free
// of bank conflicts); the A operand V^T[d][8 keys] comes from two ds_read_b64_tr_b16.
//
// Online softmax with a lazy rescale: the base m of a query row only moves when the chunk
// maximum exceeds it by more than 8 (base 2). The rescale of the accumulators for chunk i
// runs after PV(i-1) has been added (the products of i-1 are relative to the old base);
// SM(i)'s partial sums are added after the rescale. The normaliser and the tangent row sums
// are summed from the bf16-rounded weights the products use.
//
// Scope: D = 64, T in {0, 1, 2}, no bias, the forward variants (not the tangent-only one
// from a given lse), scale > 0. bf16_large_fwd serves the rest.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kD = 64;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kQW = 32;            // queries per wave
constexpr int kQB = kQW * kWaves;  // queries per workgroup
constexpr int kKC = 32;            // keys per chunk
constexpr int kKLD = kD + 8;       // K-like row, bf16 (144 bytes)
constexpr int kVLD = kD + 32;      // V-like row, bf16 (192 bytes)
constexpr int kKTile = kKC * kKLD;  // bf16 elements of one K-like tile
constexpr int kVTile = kKC * kVLD;  // bf16 elements of one V-like tile
constexpr float kRescale = 8.f;
// Products and operand reads of one PV step (T tangents), and the vector instructions the
// scheduler places after each product while the softmax runs.
template <int T>
constexpr int kPvProducts = 4 * (1 + 2 * T);
template <int T>
constexpr int kPvReads = 8 * (1 + T);  // two transposing reads per operand
template <int T>
constexpr int kStageLoads = 2 * (1 + T);  // one K-like and one V-like row piece per tensor
constexpr int kSmValuPerProduct = 5;

static_assert((kKLD * 2) % 16 == 0 && (kVLD * 2) % 16 == 0, "16-byte aligned LDS rows");

template <int T>
struct WShape {
  static constexpr int NX = 1 + T;
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int kKBuf = NX * kKTile;
  static constexpr int kVBuf = NX * kVTile;
  // two K-like and two V-like buffers, then scratch ints, the mask bytes and the site list
  static constexpr int kElems = 2 * kKBuf + 2 * kVBuf;
  static_assert(kWaves * NX * kQW * kKLD <= kElems, "the output staging fits over the key buffers");
  static size_t lds_bytes(int N) {
    const size_t n16 = (static_cast<size_t>(N) + 15) & ~size_t(15);
    return static_cast<size_t>(kElems) * 2 + 64 + n16 + 2 * n16;
  }
};

__device__ __forceinline__ v16f mfma32(bf16x8 a, bf16x8 b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ v16f zero16() { return v16f{}; }
// Materialises x here (an empty asm that reads and writes it): pins a value's computation
// before this point, which the IR optimiser would otherwise sink towards its first use.
__device__ __forceinline__ void settle(bf16x8& x) {
  uint4 u = __builtin_bit_cast(uint4, x);
  asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
  x = __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ void settle(float& x) { asm volatile("" : "+v"(x)); }
// acc + the sum of the eight bf16 values of x (v_dot2_f32_bf16 against ones, two per
// instruction): the normaliser and the tangent row sums are formed from exactly the rounded
// weights the products use.
__device__ __forceinline__ float sum8(bf16x8 x, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const uint4 u = __builtin_bit_cast(uint4, x);
  const bf16x2 one = __builtin_bit_cast(bf16x2, 0x3f803f80u);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.x), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.y), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.z), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.w), one, acc, false);
  return acc;
}
// acc *= alpha for an accumulator tile kept in accumulation registers: each element is
// read into a vector register, scaled and written back in place. Written out so the
// compiler does not move the tile into vector registers around the (rarely taken) rescale
// branch on every chunk.
__device__ __forceinline__ void scale_acc(v16f& acc, float alpha) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float x = acc[e];
    float tmp;
    asm volatile(
        "v_accvgpr_read_b32 %1, %0\n\t"
        "v_mul_f32_e32 %1, %2, %1\n\t"
        "v_accvgpr_write_b32 %0, %1"
        : "+a"(x), "=&v"(tmp)
        : "v"(alpha));
    acc[e] = x;
  }
}
// Elements 8 s .. 8 s + 7 of a score tile as bf16 (element j of the result = x[8 s + j]).
__device__ __forceinline__ bf16x8 pack_half(const v16f& x, int s) {
  uint4 u;
  u.x = pack2_bf16(x[8 * s + 0], x[8 * s + 1]);
  u.y = pack2_bf16(x[8 * s + 2], x[8 * s + 3]);
  u.z = pack2_bf16(x[8 * s + 4], x[8 * s + 5]);
  u.w = pack2_bf16(x[8 * s + 6], x[8 * s + 7]);
  return as_bf16x8(u);
}

// Site compaction of one walker's mask: idx[0 .. count) = the physical sites in ascending
// order, mask_s = the mask bytes; returns count to every thread. Rounds of 4 sites per
// thread (all mask reads of a round in flight together); a thread's exclusive prefix within
// its wave comes from the three bit planes of its count (0..4) by ballot.
__device__ __forceinline__ int compact_sites(const uint8_t* __restrict__ mask_row, int N, int16_t* __restrict__ idx,
                                             uint8_t* __restrict__ mask_s, int* __restrict__ scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const uint64_t below = (uint64_t(1) << lane) - 1;
  int total = 0;
  for (int base = 0; base < N; base += 4 * kThreads) {
    uint8_t m[4];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = base + 4 * tid + j;
      m[j] = pos < N ? mask_row[pos] : 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = base + 4 * tid + j;
      if (pos < N) mask_s[pos] = m[j];
      cnt += m[j] != 0 ? 1 : 0;
    }
    const uint64_t b0 = __ballot(cnt & 1), b1 = __ballot(cnt & 2), b2 = __ballot(cnt & 4);
    const int excl = __popcll(b0 & below) + 2 * __popcll(b1 & below) + 4 * __popcll(b2 & below);
    if (lane == 0) scratch[wave] = __popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2);
    __syncthreads();
    int at = total + excl;
    for (int w = 0; w < wave; ++w) at += scratch[w];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (m[j] != 0) idx[at++] = static_cast<int16_t>(base + 4 * tid + j);
    for (int w = 0; w < kWaves; ++w) total += scratch[w];
    __syncthreads();
  }
  return total;
}

// UNIT: scale == 1 (the reference passes pre-scaled queries), which drops the tangent-scale
// multiply from the softmax.
template <int T, bool UNIT>
__global__ void __launch_bounds__(kThreads, 1) mhsea_fwd_bf16_wide_kernel(const FwdParams p) {
  using Sh = WShape<T>;
  constexpr int NX = Sh::NX, TT = Sh::TT;

  extern __shared__ float4 smem4[];
  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* const kbuf = lds;                   // [2][NX][kKC][kKLD]
  uint16_t* const vbuf = lds + 2 * Sh::kKBuf;   // [2][NX][kKC][kVLD]
  int* const scratch = reinterpret_cast<int*>(lds + Sh::kElems);
  const int n16 = (p.N + 15) & ~15;
  uint8_t* const mask_s = reinterpret_cast<uint8_t*>(scratch + 16);
  int16_t* const idx = reinterpret_cast<int16_t*>(mask_s + n16);

  const int N = p.N, H = p.H;
  const int nblk = (N + kQB - 1) / kQB;
  const int64_t nwg = static_cast<int64_t>(p.B) * H * nblk;
  const int64_t lb = xcd_logical_block(blockIdx.x, nwg);
  const int blk = static_cast<int>(lb % nblk);
  const int h = static_cast<int>((lb / nblk) % H);
  const int b = static_cast<int>(lb / (static_cast<int64_t>(nblk) * H));

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hh = lane >> 5;
  const int c = lane & 31;

  const int n_phys = compact_sites(p.mask + static_cast<int64_t>(b) * N, N, idx, mask_s, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int nc = (nk + kKC - 1) / kKC;
  if (key_all) {  // every site is a key: the identity site list
    for (int j = tid; j < N; j += kThreads) idx[j] = static_cast<int16_t>(j);
    __syncthreads();
  }

  if (blk * kQB < nq && nc > 0) {
    // ---- staging: buffer resources over the walker's slice of each tensor ----------------
    // Rows past the last key and null tangents read zeros (offsets past the last record,
    // an empty resource) without memory traffic.
    const int64_t wel = static_cast<int64_t>(N) * H * kD;
    const int wbytes = static_cast<int>(wel * 2);
    auto rsrc = [&](const void* base, int64_t eoff, bool ok) {
      return __builtin_amdgcn_make_buffer_rsrc(
          ok ? const_cast<uint16_t*>(static_cast<const uint16_t*>(base) + eoff) : nullptr, static_cast<short>(0),
          ok ? wbytes : 0, 0x00020000);
    };
    __amdgpu_buffer_rsrc_t kr[NX], vr[NX];
#pragma unroll
    for (int x = 0; x < NX; ++x) {
      const int64_t woff = b * wel + (x > 0 ? (x - 1) * p.t_stride : 0);
      kr[x] = rsrc(x == 0 ? p.k : p.kt, woff, x == 0 || p.kt != nullptr);
      vr[x] = rsrc(x == 0 ? p.v : p.vt, woff, x == 0 || p.vt != nullptr);
    }
    const int rowstride = H * kD * 2;
    const int hoff = h * kD * 2;
    auto bload = [&](const __amdgpu_buffer_rsrc_t& r, int off) -> uint4 {
      typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
      const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      return make_uint4(u.x, u.y, u.z, u.w);
    };
    // Staging item of this thread: row srow of the chunk, 16-byte column scol, one per
    // tensor of each kind; K-like and V-like tiles are both row-major.
    const int srow = tid >> 3, scol = tid & 7;

    // Byte offsets of this thread's rows of K(kck) and V(kcv) (site-list reads), then the
    // loads themselves: split so the site lookups can run ahead of the products.
    // The site-list reads are unconditional (clamped index) and materialised by an empty
    // asm: otherwise the compiler sinks each into the select that uses it, behind a branch.
    auto site_reads = [&](int kck, int kcv, int& sk, int& sv) {
      sk = idx[min(kck + srow, N - 1)];
      sv = idx[min(kcv + srow, N - 1)];
    };
    auto site_offsets = [&](int kck, int kcv, int sk, int sv, int& ko, int& vo) {
      asm volatile("" : "+v"(sk), "+v"(sv));
      const int jk = kck + srow, jv = kcv + srow;
      ko = jk < nk ? sk * rowstride + hoff + scol * 16 : wbytes;
      vo = jv < nk ? sv * rowstride + hoff + scol * 16 : wbytes;
    };
    auto stage_offsets = [&](int kck, int kcv, int& ko, int& vo) {
      int sk, sv;
      site_reads(kck, kcv, sk, sv);
      site_offsets(kck, kcv, sk, sv, ko, vo);
    };
    auto stage_issue = [&](int ko, int vo, uint4(&rk)[NX], uint4(&rv)[NX]) {
#pragma unroll
      for (int x = 0; x < NX; ++x) {
        rk[x] = bload(kr[x], ko);
        rv[x] = bload(vr[x], vo);
      }
    };
    auto stage_loads = [&](int kck, int kcv, uint4(&rk)[NX], uint4(&rv)[NX]) {
      int ko, vo;
      stage_offsets(kck, kcv, ko, vo);
      stage_issue(ko, vo, rk, rv);
    };
    auto kstore = [&](int buf, const uint4(&rk)[NX]) {
#pragma unroll
      for (int x = 0; x < NX; ++x)
        *reinterpret_cast<uint4*>(kbuf + buf * Sh::kKBuf + x * kKTile + srow * kKLD + scol * 8) = rk[x];
    };
    auto vstore = [&](int buf, const uint4(&rv)[NX]) {
#pragma unroll
      for (int x = 0; x < NX; ++x)
        *reinterpret_cast<uint4*>(vbuf + buf * Sh::kVBuf + x * kVTile + srow * kVLD + scol * 8) = rv[x];
    };

    // ---- this wave's queries: B-operand fragments, lane (hh, c) holds q[32 s' .. ] -------
    const int q0 = blk * kQB + wave * kQW;
    const bool qvalid = q0 + c < nq;
    const int qsite = qvalid ? (p.key_mask ? (q0 + c) : idx[q0 + c]) : -1;
    const int qload = qvalid ? qsite : 0;
    bf16x8 qf[4], qtf[TT][4];
    {
      const int64_t qoff = bnhd(b, qload, h, N, H, kD) + 8 * hh;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qoff + 16 * s));
#pragma unroll
        for (int t = 0; t < T; ++t)
          qtf[t][s] = p.qt != nullptr
                          ? as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.qt) + t * p.t_stride + qoff + 16 * s))
                          : bf16x8{};
      }
    }
    const float s2scale = UNIT ? kLog2e : p.scale * kLog2e;
    const float stscale = UNIT ? 1.f : p.scale;

    v16f o[2], ac[TT][2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      o[dt] = zero16();
#pragma unroll
      for (int t = 0; t < T; ++t) ac[t][dt] = zero16();
    }
    float m2 = -INFINITY, lsum = 0.f;
    float mu[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) mu[t] = 0.f;

    // Scores of one chunk; two sets (A, B) of bf16 weights and two of staging registers,
    // used alternately.
    v16f sc, ds[TT];
    bf16x8 pA[2], pB[2], pdA[TT][2], pdB[TT][2];
    uint4 rkA[NX], rvA[NX], rkB[NX], rvB[NX];

    // ---- S(j): scores of the chunk in K-like buffer kb ----------------------------------
    auto s_products = [&](const uint16_t* kb, v16f& sc, v16f(&ds)[TT]) {
      sc = zero16();
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t] = zero16();
      const uint16_t* const kp = kb + c * kKLD + 8 * hh;
      // Order per k-step: Kt Q^T of every tangent, K Q^T, K Qt^T of every tangent, so two
      // products into one accumulator are never adjacent.
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(kp + 16 * s));
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const bf16x8 ktf = as_bf16x8(*reinterpret_cast<const uint4*>(kp + (1 + t) * kKTile + 16 * s));
          ds[t] = mfma32(ktf, qf[s], ds[t]);
        }
        sc = mfma32(kf, qf[s], sc);
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t] = mfma32(kf, qtf[t][s], ds[t]);
      }
    };
    // ---- PV(j): products of chunk j's weights with the V-like buffer vb -----------------
    // The A operand V^T[32 dt + c][kappa(s, hh, 0..7)] comes from the row-major tile by two
    // transposing reads (ds_read_b64_tr_b16): within each 16-lane group g, lane 16 g + 4 j + q
    // addresses row 16 s + 8 h2 + 4 (g / 2) + j at column 32 dt + 16 (g % 2) + 4 q, and lane
    // 16 g + m receives element m % 4 of the rows of lanes 16 g + 4 j + m / 4, j = 0..3, i.e.
    // column 32 dt + c of keys kappa(s, hh, 4 h2 + j).
    const int trg = lane >> 4, trm = lane & 15;
    const int trbase = (4 * (trg >> 1) + (trm >> 2)) * kVLD + 16 * (trg & 1) + 4 * (trm & 3);
    auto vfrag = [&](const uint16_t* vt, int dt, int s) -> bf16x8 {
      typedef short v4s __attribute__((ext_vector_type(4)));
      const uint16_t* const p0 = vt + trbase + (16 * s) * kVLD + 32 * dt;
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p0));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p0 + 8 * kVLD));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      return as_bf16x8(make_uint4(l2.x, l2.y, h2.x, h2.y));
    };
    // Order per k-step: V^T P^T of both column tiles, V^T (P o dS)^T of every tangent and
    // tile, then Vt^T P^T of every tangent and tile, so two products into one accumulator
    // are never adjacent.
    auto pv_products = [&](const uint16_t* vb, const bf16x8(&pw)[2], const bf16x8(&pdw)[TT][2]) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8 vf[2];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          vf[dt] = vfrag(vb, dt, s);
          o[dt] = mfma32(vf[dt], pw[s], o[dt]);
        }
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) ac[t][dt] = mfma32(vf[dt], pdw[t][s], ac[t][dt]);
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) ac[t][dt] = mfma32(vfrag(vb + (1 + t) * kVTile, dt, s), pw[s], ac[t][dt]);
      }
    };

    // ---- one pipeline iteration i (parity PAR = i mod 2) ----------------------------------
    // SM(i) turns the scores of chunk i into weights (set PAR) while the matrix cores run
    // PV(i-1) on the other set and the global reads of K(i+3) and V(i+1) go out into the
    // staging set PAR; then S(i+1) refills the score registers while K(i+2) and V(i),
    // read in iteration i-1 (staging set 1 - PAR), are written into the buffers of parity PAR.
    // MASKED: the chunk may hold padding keys (only the last one does; it is peeled off).
    // Scheduling barriers keep the phases in this order: without them the compiler hoists
    // S(i+1) above the softmax, which keeps two chunks' scores live.
    // ko, vo: byte offsets of this thread's staging rows of K(i+3) and V(i+1)
    int ko, vo;
    auto iteration = [&](auto par, auto masked, int i, bf16x8(&pw)[2], bf16x8(&pdw)[TT][2], const bf16x8(&pwp)[2],
                         const bf16x8(&pdwp)[TT][2], uint4(&rkl)[NX], uint4(&rvl)[NX], const uint4(&rkw)[NX],
                         const uint4(&rvw)[NX]) {
      constexpr int PAR = decltype(par)::value;
      constexpr bool MASKED = decltype(masked)::value;
      // prelude: validity of the last chunk, chunk maximum, base update
      if constexpr (MASKED) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = i * kKC + 8 * (e >> 2) + 4 * hh + (e & 3);
          if (key >= nk) sc[e] = -INFINITY;
        }
      }
      float mx = sc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sc[e]);
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      mx *= s2scale;
      const bool need = mx > m2 + kRescale;  // also true for the first chunk (m2 = -inf)
      const bool resc = __any(need);
      float alpha = 1.f;
      if (resc) {
        const float mnew = need ? mx : m2;
        alpha = fast_exp2(m2 - mnew);  // 0 on the first chunk
        m2 = mnew;
      }

      __builtin_amdgcn_sched_barrier(0);
      // SM(i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pe = fast_exp2(fmaf(sc[e], s2scale, -m2));
        sc[e] = pe;
        const float ps = UNIT ? pe : pe * stscale;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][e] *= ps;
      }
      float ls = 0.f;
      float muc[TT];
#pragma unroll
      for (int t = 0; t < T; ++t) muc[t] = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        pw[s] = pack_half(sc, s);
        ls = sum8(pw[s], ls);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          pdw[t][s] = pack_half(ds[t], s);
          muc[t] = sum8(pdw[t][s], muc[t]);
        }
      }
      // PV(i-1), its products interleaved with the softmax and the staging reads of K(i+3)
      // and V(i+1) (into the staging set of parity PAR): the site-list reads first, then per
      // product one operand read, one global read while any are left, and a run of vector
      // instructions
      stage_issue(ko, vo, rkl, rvl);
      pv_products(vbuf + (1 - PAR) * Sh::kVBuf, pwp, pdwp);
      constexpr int kL = kStageLoads<T>, kP = kPvProducts<T>;
      static_assert(kPvReads<T> == 4 + kP && kL <= kP, "read / load groups per product");
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the first two operands
#pragma unroll
      for (int k = 0; k < kL; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // product
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  // LDS read
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                  // global read
        __builtin_amdgcn_sched_group_barrier(0x002, kSmValuPerProduct, 0);  // vector ALU
      }
#pragma unroll
      for (int k = kL; k < kP; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, kSmValuPerProduct, 0);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        settle(pw[s]);
#pragma unroll
        for (int t = 0; t < T; ++t) settle(pdw[t][s]);
      }
      settle(ls);
#pragma unroll
      for (int t = 0; t < T; ++t) settle(muc[t]);
      __builtin_amdgcn_sched_barrier(0);
      // S(i+1), with the LDS writes of K(i+2) and V(i) (loaded in iteration i-1) into the
      // buffers of parity PAR between its products; the site lookups for iteration i+1's
      // staging reads go out first and are materialised last (an empty asm, a scheduling
      // boundary), so their LDS latency is hidden
      int sk, sv;
      site_reads((i + 4) * kKC, (i + 2) * kKC, sk, sv);
      s_products(kbuf + (1 - PAR) * Sh::kKBuf, sc, ds);
      kstore(PAR, rkw);
      vstore(PAR, rvw);
      site_offsets((i + 4) * kKC, (i + 2) * kKC, sk, sv, ko, vo);

      // postlude: rescale (after PV(i-1)), then SM(i)'s sums
      if (resc) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          scale_acc(o[dt], alpha);
#pragma unroll
          for (int t = 0; t < T; ++t) scale_acc(ac[t][dt], alpha);
        }
        lsum *= alpha;
#pragma unroll
        for (int t = 0; t < T; ++t) mu[t] *= alpha;
      }
      lsum += ls;
#pragma unroll
      for (int t = 0; t < T; ++t) mu[t] += muc[t];
      __syncthreads();
    };

    // ---- prologue: K(0), K(1) in LDS; zero weights and V rows for PV(-1); K(2) and V(0)
    // in flight; S(0) in the score registers ---------------------------------------------
    stage_loads(0, 0, rkA, rvA);
    stage_loads(kKC, 0, rkB, rvB);
    kstore(0, rkA);
    kstore(1, rkB);
    for (int e = tid; e < Sh::kVBuf / 8; e += kThreads)
      reinterpret_cast<uint4*>(vbuf + Sh::kVBuf)[e] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      pB[s] = bf16x8{};
#pragma unroll
      for (int t = 0; t < T; ++t) pdB[t][s] = bf16x8{};
    }
    stage_loads(2 * kKC, 0, rkB, rvB);
    stage_offsets(3 * kKC, kKC, ko, vo);
    __syncthreads();
    s_products(kbuf, sc, ds);
    __syncthreads();  // K(0)'s buffer is rewritten in iteration 0

    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using Full = std::integral_constant<bool, false>;
    using Part = std::integral_constant<bool, true>;
    // chunks 0 .. nc - 2 are full; the last one is peeled (partial unless nk % 32 == 0)
    int i = 0;
#pragma clang loop unroll(disable)
    for (; i + 2 < nc; i += 2) {
      iteration(P0{}, Full{}, i, pA, pdA, pB, pdB, rkA, rvA, rkB, rvB);
      iteration(P1{}, Full{}, i + 1, pB, pdB, pA, pdA, rkB, rvB, rkA, rvA);
    }
    if (i + 1 < nc) {  // i = nc - 2: one full chunk of parity 0, then the last of parity 1
      iteration(P0{}, Full{}, i, pA, pdA, pB, pdB, rkA, rvA, rkB, rvB);
      iteration(P1{}, Part{}, i + 1, pB, pdB, pA, pdA, rkB, rvB, rkA, rvA);
    } else {  // i = nc - 1, parity 0
      iteration(P0{}, Part{}, i, pA, pdA, pB, pdB, rkA, rvA, rkB, rvB);
    }
    // epilogue: PV(nc - 1)
    if (((nc - 1) & 1) == 0)
      pv_products(vbuf, pA, pdA);
    else
      pv_products(vbuf + Sh::kVBuf, pB, pdB);

    // ---- normalisation and stores -----------------------------------------------------
    // Each wave stages its 32 rows of out and the tangent outputs (bf16) in LDS, over the
    // staging buffers (free after the barrier), then writes every query row as eight
    // 16-byte pieces, whole 128-byte rows per instruction.
    const float ltot = xor32_pair_sum(lsum);
    const float inv = 1.f / ltot;
    float mut[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) mut[t] = xor32_pair_sum(mu[t]) * inv;
    if (qvalid && hh == 0 && p.lse != nullptr)
      p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] = (m2 + log2f(ltot)) * kLn2;
    __syncthreads();
    uint16_t* const ot = lds + wave * (NX * kQW * kKLD);  // [NX][32 queries][kKLD]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * dt + 8 * a + 4 * hh;
        float o4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o4[r] = o[dt][4 * a + r] * inv;
        *reinterpret_cast<uint2*>(ot + c * kKLD + d0) = make_uint2(pack2_bf16(o4[0], o4[1]), pack2_bf16(o4[2], o4[3]));
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float tv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) tv[r] = fmaf(ac[t][dt][4 * a + r], inv, -mut[t] * o4[r]);
          *reinterpret_cast<uint2*>(ot + (1 + t) * kQW * kKLD + c * kKLD + d0) =
              make_uint2(pack2_bf16(tv[0], tv[1]), pack2_bf16(tv[2], tv[3]));
        }
      }
    // the wave reads back only what it wrote (LDS accesses of one wave complete in order)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int piece = lane + 64 * u;
      const int q = piece >> 3, col = piece & 7;
      if (q0 + q < nq) {
        const int site = p.key_mask ? q0 + q : idx[q0 + q];
        const int64_t off = bnhd(b, site, h, N, H, kD) + col * 8;
#pragma unroll
        for (int x = 0; x < NX; ++x) {
          const uint4 v = *reinterpret_cast<const uint4*>(ot + x * kQW * kKLD + q * kKLD + col * 8);
          uint16_t* const dst = x == 0 ? static_cast<uint16_t*>(p.out) : static_cast<uint16_t*>(p.tout) + (x - 1) * p.t_stride;
          *reinterpret_cast<uint4*>(dst + off) = v;
        }
      }
    }
  }

  // rows of masked sites in this block's site range (square mask): zeros, lse = -1e4 + log N.
  // Each wave takes 32 rows; a wave whose rows are all physical stores nothing.
  if (!p.key_mask) {
    const int r0 = blk * kQB + wave * kQW;
    const int rl = r0 + (lane & 31);
    const uint64_t masked = __ballot(lane < 32 && rl < N && mask_s[rl] == 0);
    if (masked != 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int piece = lane + 64 * u;
        const int q = piece >> 3, col = piece & 7;
        if ((masked >> q) & 1) {
          const int64_t off = bnhd(b, r0 + q, h, N, H, kD) + col * 8;
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + off) = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
          for (int t = 0; t < T; ++t)
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.tout) + t * p.t_stride + off) = make_uint4(0u, 0u, 0u, 0u);
          if (col == 0 && p.lse != nullptr) p.lse[(static_cast<int64_t>(b) * N + r0 + q) * H + h] = p.masked_lse;
        }
      }
    }
  }
}

template <int T, bool UNIT>
hipError_t launch_t(const FwdParams& p, hipStream_t stream) {
  using Sh = WShape<T>;
  const int nblk = (p.N + kQB - 1) / kQB;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = Sh::lds_bytes(p.N);
  auto kern = mhsea_fwd_bf16_wide_kernel<T, UNIT>;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

}  // namespace

bool bf16_wide_fwd_supported(const FwdParams& p, int D, bool given_lse) {
  const int64_t wbytes = static_cast<int64_t>(p.N) * p.H * D * 2;
  return D == kD && !given_lse && p.e == nullptr && p.et == nullptr && p.scale > 0.f && p.scale < INFINITY &&
         p.N > 128 && wbytes < (int64_t(1) << 31) && WShape<2>::lds_bytes(p.N) <= 160 * 1024 && p.gated == 0;
}

hipError_t launch_fwd_bf16_wide(const FwdParams& p, int T, hipStream_t stream) {
  const bool unit = p.scale == 1.f;
  if (T == 0) return unit ? launch_t<0, true>(p, stream) : launch_t<0, false>(p, stream);
  if (T == 1) return unit ? launch_t<1, true>(p, stream) : launch_t<1, false>(p, stream);
  if (T == 2) return unit ? launch_t<2, true>(p, stream) : launch_t<2, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace hz
