// bfloat16 forward / forward+tangent / tangent-only MHSEA kernel for large N (N > 128,
// D in {32, 64}), bfloat16 storage, fp32 softmax and accumulation.
//
// Work decomposition: one 512-thread workgroup (8 waves) owns one (walker, head) and 128
// consecutive compacted queries; each wave owns 16 of them. Keys are streamed through LDS
// in chunks of 64 compacted keys, each staged once for all 128 queries.
//
// Per wave, chunk i takes three steps: S(i), the score products (matrix cores); SM(i), the
// online softmax (vector ALU and transcendental unit); PV(i), the P.V products (matrix
// cores). The eight waves form two groups, one wave of each per SIMD (assigned at start
// from the hardware wave id), and run a ping-pong schedule of phases, one workgroup
// barrier per phase:
//   phase 2i   : group 0 runs PV(i-1) and S(i);  group 1 runs SM(i-1) and its staging
//   phase 2i+1 : group 1 runs PV(i-1) and S(i);  group 0 runs SM(i) and its staging
// so on every SIMD one wave feeds the matrix cores while the other runs its softmax and
// moves chunk data, and the wave in its matrix phase runs at raised priority so its
// products issue first.
//
// K-like tensors (K, Kt[t]) and V-like tensors (V, Vt[t]) have separate triple buffers:
// K(j) is read in phases 2j and 2j+1, V(j) in phases 2j+2 and 2j+3. In its softmax phase
// of step i a wave writes its items of K(i+2) and V(i+1) from registers to LDS (buffers
// last read at least one barrier earlier) and issues the global reads of K(i+3) and V(i+2),
// which have two phases to arrive.
//
// LDS layout: K and Kt[t] row-major ([key][d], D bf16 per row) with the 16-byte chunks of
// row r XOR-swizzled by r mod (D / 8), so the 16 rows x one chunk of an operand read hit
// distinct banks; V and Vt[t] transposed ([d][key'], rows padded to 72 bf16), with the
// keys of each 32-key pair block reordered so that the eight keys one lane feeds to a P.V
// product (below) are adjacent: key 16h + 4g + r of the block sits at position
// 8g + 4h + r, and the operand is one 16-byte read. The transposition happens in registers:
// a thread loads 4 consecutive keys x 8 columns (four 16-byte reads) and writes 8 columns
// x 4 keys with v_perm_b32 and eight 8-byte LDS writes. With 72-element rows (144 bytes)
// eight lanes of a P.V operand read (8 rows, one 16-byte run each) cover all 32 banks.
//
// Products run on v_mfma_f32_16x16x32_bf16 (bf16 operands, fp32 accumulation), in the
// transposed orientation S^T = K Q^T, O^T += V^T P^T of the other kernels:
//   S^T[key 16 jt + 4g + r][query c] = sum_s K[16 jt + c][32 s + 8g .. +8] . Q[c][32 s + 8g .. +8]
//   O^T[d 16 dt + 4g + r][query c] += sum over key pairs (2p, 2p+1) of
//       V^T[16 dt + c][kappa(g, i)] . P[c][kappa(g, i)],  kappa(g, i) = 16 (2p + i/4) + 4g + i%4
// so the B operand of the P.V product is the lane's own softmax weights of two key tiles,
// rounded to bf16.
//
// Online softmax with a lazy rescale: the exponent base m of a query row only moves when
// the chunk maximum exceeds it by more than 8 (base 2), and the accumulators are rescaled
// only then (a wave-uniform branch); weights exp2(s - m) stay <= 256, and out = O / l,
// lse = (m + log2 l) ln 2 are exact for any base.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kQB = 16 * kWaves;  // queries per workgroup
constexpr int kKC = 64;           // keys per chunk
constexpr float kRescale = 8.f;   // lazy-rescale threshold (base-2 exponent)

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ bf16x8 pack8(v4f a, v4f b) {
  uint4 u;
  u.x = pack2_bf16(a[0], a[1]);
  u.y = pack2_bf16(a[2], a[3]);
  u.z = pack2_bf16(b[0], b[1]);
  u.w = pack2_bf16(b[2], b[3]);
  return as_bf16x8(u);
}
// Forces the compiler to materialise x here (waiting for its load, if any), without
// emitting an instruction.
__device__ __forceinline__ void settle_bf16x8(bf16x8& x) {
  uint4 u = __builtin_bit_cast(uint4, x);
  asm volatile("" : "+v"(u.x), "+v"(u.y), "+v"(u.z), "+v"(u.w));
  x = __builtin_bit_cast(bf16x8, u);
}
// Word w of a uint4.
__device__ __forceinline__ uint32_t word(const uint4& u, int w) { return w == 0 ? u.x : w == 1 ? u.y : w == 2 ? u.z : u.w; }

template <int D, int T>
struct LShape {
  static constexpr int LDR = D;       // row-major row, bf16 (chunks swizzled)
  static constexpr int LDT = 72;      // transposed row (64 keys + 8), bf16
  static constexpr int NS = D / 32;
  static constexpr int DT = D / 16;
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int C8 = D / 8;    // 16-byte chunks of a row
  static constexpr int NX = 1 + T;    // tensors of each kind (K-like, V-like)
  static constexpr int kRow = kKC * LDR;  // elements of one row-major tile
  static constexpr int kTr = D * LDT;     // elements of one transposed tile
  static constexpr int kBuf = NX * (kRow + kTr);  // elements of one buffer
  // Staging work per chunk: K-like 16-byte items, V-like 4-key x 8-column units.
  static constexpr int kKItems = NX * kKC * C8;
  static constexpr int kKPer = (kKItems + kThreads - 1) / kThreads;
  static constexpr int kVUnits = NX * (kKC / 4) * C8;
  static constexpr int kVPer = (kVUnits + kThreads - 1) / kThreads;
  static constexpr int kNBuf = 3;     // buffers of each kind
  static size_t lds_bytes(int N) {
    const size_t n16 = (static_cast<size_t>(N) + 15) & ~size_t(15);
    return static_cast<size_t>(kNBuf * kBuf) * 2 + 64 + n16 + 2 * n16;
  }
};

// HW_ID register (id 4, all 32 bits); the SIMD of the wave is bits 5:4.
constexpr int kHwIdReg = 4 | (31 << 11);

template <int D, int T, bool GIVEN_LSE, bool HAS_E>
__global__ void __launch_bounds__(kThreads, 1) mhsea_fwd_bf16_large_kernel(const FwdParams p) {
  using Sh = LShape<D, T>;
  constexpr int LDR = Sh::LDR, LDT = Sh::LDT, NS = Sh::NS, DT = Sh::DT, TT = Sh::TT, C8 = Sh::C8, NX = Sh::NX;
  constexpr int NJT = kKC / 16;
  static_assert(Sh::kKItems % 64 == 0 && Sh::kVUnits % 64 == 0, "staging items must split into whole waves");

  extern __shared__ float4 smem4[];
  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* const kbuf = lds;                               // [3][NX][kKC][LDR]
  uint16_t* const vbuf = lds + Sh::kNBuf * NX * Sh::kRow;   // [3][NX][D][LDT]
  int* const scratch = reinterpret_cast<int*>(lds + Sh::kNBuf * Sh::kBuf);
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
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;

  // SIMD of each wave, published by the barriers of the mask compaction.
  if (lane == 0) scratch[8 + wave] = static_cast<int>((__builtin_amdgcn_s_getreg(kHwIdReg) >> 4) & 3);
  const int n_phys = compact_mask_wg<kWaves>(p.mask + static_cast<int64_t>(b) * N, N, idx, mask_s, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int nchunks = (nk + kKC - 1) / kKC;
  // Group: 0 for the first wave (by index) on its SIMD, 1 for the second. Any placement
  // gives correct results; one wave of each group per SIMD gives the overlap.
  int grp = 0;
  {
    const int mine = scratch[8 + wave];
    for (int w = 0; w < wave; ++w) grp += scratch[8 + w] == mine ? 1 : 0;
    grp = __builtin_amdgcn_readfirstlane(grp & 1);
  }

  // Staging reads go through buffer resources over the walker's slice of each tensor: a
  // 32-bit byte offset per key row, zeros for padding keys (offsets past the last record)
  // and for a null tangent (an empty resource).
  const int64_t wel = static_cast<int64_t>(N) * H * D;  // elements per walker slice
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
  // resource x of an array, x wave-uniform (scalar selects, no waterfall over lanes)
  auto pick = [&](const __amdgpu_buffer_rsrc_t* r, int x) -> __amdgpu_buffer_rsrc_t {
    if constexpr (NX == 1) return r[0];
    if constexpr (NX == 2) return x == 0 ? r[0] : r[1];
    return x == 0 ? r[0] : (x == 1 ? r[1] : r[2]);
  };
  const int rowstride = H * D * 2;  // bytes between sites
  const int hoff = h * D * 2;
  auto site_of = [&](int j) { return key_all ? j : static_cast<int>(idx[j]); };
  auto bload = [&](const __amdgpu_buffer_rsrc_t& r, int off) -> uint4 {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(u.x, u.y, u.z, u.w);
  };

  // ---- chunk staging: global -> registers (load), registers -> LDS buffer (store) -----
  // A thread's staging items sit at the same place of every chunk, so their tensor (one
  // per wave: 64 divides the items of a tensor), descriptor, row and column are fixed for
  // the whole workgroup; per chunk only the rows' site offsets are looked up. Loads are
  // unconditional: rows past the last key, chunks past the last one and the items of
  // waves past the last item (wave-uniform) read past the buffer's last record, which
  // yields zeros without memory traffic; only the LDS writes of missing items are skipped.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  __amdgpu_buffer_rsrc_t krs[Sh::kKPer], vrs[Sh::kVPer];
  int krow[Sh::kKPer], kcol[Sh::kKPer], vkey[Sh::kVPer], vcol[Sh::kVPer];
#pragma unroll
  for (int u = 0; u < Sh::kKPer; ++u) {
    const int it = tid + u * kThreads;
    const int x = (wv * 64 + u * kThreads) / (kKC * C8);  // wave-uniform
    krs[u] = pick(kr, min(x, NX - 1));
    const int rem = it % (kKC * C8);
    krow[u] = rem / C8;
    kcol[u] = (rem % C8) * 16;
  }
#pragma unroll
  for (int u = 0; u < Sh::kVPer; ++u) {
    const int it = tid + u * kThreads;
    const int x = (wv * 64 + u * kThreads) / ((kKC / 4) * C8);  // wave-uniform
    vrs[u] = pick(vr, min(x, NX - 1));
    const int rem = it % ((kKC / 4) * C8);
    vkey[u] = 4 * (rem % (kKC / 4));
    vcol[u] = (rem / (kKC / 4)) * 16;
  }
  auto kitem = [&](int u) { return Sh::kKItems % kThreads == 0 || wv * 64 + u * kThreads < Sh::kKItems; };
  auto vunit = [&](int u) { return Sh::kVUnits % kThreads == 0 || wv * 64 + u * kThreads < Sh::kVUnits; };
  uint4 rk[Sh::kKPer];
  uint4 rv[Sh::kVPer][4];
  // Staging reads of K(kck) and V(kcv): every site-list read is issued before the first
  // is used (clamped index, so unconditional), then each is materialised by an empty asm
  // (without it the compiler sinks each read into the select that uses it, one LDS wait
  // per read), then the global loads go out.
  auto stage_loads = [&](int kck, int kcv) {
    int sk[Sh::kKPer], sv[Sh::kVPer][4];
#pragma unroll
    for (int u = 0; u < Sh::kKPer; ++u) sk[u] = idx[min(kck + krow[u], N - 1)];
#pragma unroll
    for (int u = 0; u < Sh::kVPer; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[u][i] = idx[min(kcv + vkey[u] + i, N - 1)];
#pragma unroll
    for (int u = 0; u < Sh::kKPer; ++u) asm volatile("" : "+v"(sk[u]));
#pragma unroll
    for (int u = 0; u < Sh::kVPer; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(sv[u][i]));
    auto off = [&](int j, int sj, int col, bool mine) {
      return (j < nk && mine) ? (key_all ? j : sj) * rowstride + hoff + col : wbytes;
    };
#pragma unroll
    for (int u = 0; u < Sh::kKPer; ++u) rk[u] = bload(krs[u], off(kck + krow[u], sk[u], kcol[u], kitem(u)));
#pragma unroll
    for (int u = 0; u < Sh::kVPer; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) rv[u][i] = bload(vrs[u], off(kcv + vkey[u] + i, sv[u][i], vcol[u], vunit(u)));
  };
  auto kstore = [&](int buf, const uint4(&src)[Sh::kKPer]) {
    uint16_t* const base = kbuf + buf * NX * Sh::kRow;
#pragma unroll
    for (int u = 0; u < Sh::kKPer; ++u) {
      if (kitem(u)) {
        const int it = tid + u * kThreads;
        const int x = it / (kKC * C8);
        const int rem = it % (kKC * C8);
        const int row = rem / C8;
        *reinterpret_cast<uint4*>(base + x * Sh::kRow + row * LDR + (((rem % C8) ^ (row & (C8 - 1))) * 8)) = src[u];
      }
    }
  };
  auto vstore = [&](int buf) {
    uint16_t* const base = vbuf + buf * NX * Sh::kTr;
#pragma unroll
    for (int u = 0; u < Sh::kVPer; ++u) {
      if (vunit(u)) {
        const int it = tid + u * kThreads;
        const int x = it / ((kKC / 4) * C8);
        const int rem = it % ((kKC / 4) * C8);
        const int kg = rem % (kKC / 4), dg = rem / (kKC / 4);
        // key group kg (keys 4kg .. 4kg+3) of pair block kg / 8 goes to position
        // 8 (kg mod 4) + 4 ((kg / 4) mod 2) of the block
        uint16_t* const tr = base + x * Sh::kTr + (dg * 8) * LDT + 32 * (kg >> 3) + 8 * (kg & 3) + 4 * ((kg >> 2) & 1);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          // columns 2w (low halves) and 2w + 1 (high halves) of the four keys
          uint2 ev, od;
          ev.x = __builtin_amdgcn_perm(word(rv[u][1], w), word(rv[u][0], w), 0x05040100u);
          ev.y = __builtin_amdgcn_perm(word(rv[u][3], w), word(rv[u][2], w), 0x05040100u);
          od.x = __builtin_amdgcn_perm(word(rv[u][1], w), word(rv[u][0], w), 0x07060302u);
          od.y = __builtin_amdgcn_perm(word(rv[u][3], w), word(rv[u][2], w), 0x07060302u);
          *reinterpret_cast<uint2*>(tr + (2 * w) * LDT) = ev;
          *reinterpret_cast<uint2*>(tr + (2 * w + 1) * LDT) = od;
        }
      }
    }
  };

  // ---- this wave's queries -------------------------------------------------------------
  const int q0 = blk * kQB + wave * 16;
  const bool active = q0 < nq;
  const bool qvalid = q0 + c < nq;
  const int qsite = qvalid ? (p.key_mask ? (q0 + c) : idx[q0 + c]) : -1;
  const int qload = qvalid ? qsite : 0;
  bf16x8 qf[NS], qtf[TT][NS];
  {
    const int64_t qoff = bnhd(b, qload, h, N, H, D) + 8 * g;
    const uint16_t* qt = p.qt != nullptr ? static_cast<const uint16_t*>(p.qt) : static_cast<const uint16_t*>(p.q);
    const int64_t qts = p.qt != nullptr ? p.t_stride : 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qoff + 32 * s));
#pragma unroll
      for (int t = 0; t < T; ++t)
        qtf[t][s] = p.qt != nullptr ? as_bf16x8(*reinterpret_cast<const uint4*>(qt + t * qts + qoff + 32 * s)) : bf16x8{};
    }
  }
  const float sscale = p.scale;
  const float stscale = p.scale;  // a null qt gives zero fragments: dS = Kt Q^T alone
  const float s2scale = sscale * kLog2e;
  float lse2 = 0.f;
  if constexpr (GIVEN_LSE) lse2 = p.lse_in[(static_cast<int64_t>(b) * N + qload) * H + h] * kLog2e;
  const int64_t e_row = static_cast<int64_t>(b) * N * N * H + static_cast<int64_t>(qload) * p.e_sq +
                        static_cast<int64_t>(h) * p.e_sh;

  v4f o[DT], at[TT][DT], ct[TT][DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    o[dt] = zero4();
#pragma unroll
    for (int t = 0; t < T; ++t) at[t][dt] = ct[t][dt] = zero4();
  }
  float m2 = -INFINITY, lsum = 0.f;
  float mu[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) mu[t] = 0.f;

  // Scores of the current chunk (S(i) -> SM(i)) and the bf16 weights of the last
  // softmaxed one (SM(i) -> PV(i)).
  v4f sc[NJT], ds[TT][NJT];
  bf16x8 pw[NJT / 2], pdw[TT][NJT / 2];

  // ---- S(i): S^T and dS^T of chunk i ---------------------------------------------------
  // Every key tile is multiplied, also past the last key: padding rows are staged as
  // zeros and their scores are masked in SM, so the chunk's code has no branches.
  auto s_step = [&](int buf) {
    const uint16_t* const Kb = kbuf + buf * NX * Sh::kRow;
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      sc[jt] = zero4();
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t][jt] = zero4();
      const int row = jt * 16 + c;
      const uint16_t* krow_p = Kb + row * LDR;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int ch = ((4 * s + g) ^ (row & (C8 - 1))) * 8;
        const bf16x8 kv = as_bf16x8(*reinterpret_cast<const uint4*>(krow_p + ch));
        sc[jt] = mfma_bf16(kv, qf[s], sc[jt]);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const bf16x8 ktv = as_bf16x8(*reinterpret_cast<const uint4*>(krow_p + (1 + t) * Sh::kRow + ch));
          ds[t][jt] = mfma_bf16(ktv, qf[s], ds[t][jt]);
          ds[t][jt] = mfma_bf16(kv, qtf[t][s], ds[t][jt]);
        }
      }
    }
  };

  // ---- SM(i): online softmax of chunk i, bf16 weights for PV(i) -------------------------
  auto sm_step = [&](int i) {
    const int kc = i * kKC;
    // Base-2 scores. A full chunk (every key physical) needs no validity selects and keeps
    // the raw products, scaled inside the exponent (smul); the other path stores masked
    // base-2 scores (smul = 1). Without a bias the tangent scores stay unscaled here:
    // P o dS is linear in the scale, which is applied once to A and mu at the end.
    float mx = -INFINITY;
    const bool full = kc + kKC <= nk;
    float smul = 1.f;
    if (!HAS_E && full) {
      smul = s2scale;
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[jt][r] * s2scale);
    } else {
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = kc + jt * 16 + 4 * g + r;
          const bool valid = j < nk;
          float sv = sc[jt][r];
          if constexpr (HAS_E) {
            sv *= sscale;
#pragma unroll
            for (int t = 0; t < T; ++t) ds[t][jt][r] *= stscale;
            if (valid) {
              const int64_t eo = e_row + static_cast<int64_t>(site_of(j)) * p.e_sk;
              if (p.e != nullptr) sv += load1<BF16>(p.e, eo);
              if (p.et != nullptr) {
#pragma unroll
                for (int t = 0; t < T; ++t) ds[t][jt][r] += load1<BF16>(p.et, t * p.et_stride + eo);
              }
            }
            sv *= kLog2e;
          } else {
            sv *= s2scale;
          }
          sc[jt][r] = valid ? sv : -INFINITY;
#pragma unroll
          for (int t = 0; t < T; ++t) ds[t][jt][r] = valid ? ds[t][jt][r] : 0.f;
          mx = fmaxf(mx, sc[jt][r]);
        }
      }
    }

    if constexpr (GIVEN_LSE) {
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[jt][r] = lse_weight(fmaf(sc[jt][r], smul, -lse2));
    } else {
      mx = group_max(mx);
      const bool need = mx > m2 + kRescale;  // also true for the first chunk (m2 = -inf)
      if (__any(need)) {
        const float mnew = need ? mx : m2;
        const float alpha = fast_exp2(m2 - mnew);  // 1 where unchanged, 0 on the first chunk
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          o[dt] *= alpha;
#pragma unroll
          for (int t = 0; t < T; ++t) {
            at[t][dt] *= alpha;
            ct[t][dt] *= alpha;
          }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) mu[t] *= alpha;
        m2 = mnew;
      }
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[jt][r] = fast_exp2(fmaf(sc[jt][r], smul, -m2));
          lsum += sc[jt][r];
        }
    }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) {
        ds[t][jt] *= sc[jt];
        mu[t] += (ds[t][jt][0] + ds[t][jt][1]) + (ds[t][jt][2] + ds[t][jt][3]);
      }
#pragma unroll
    for (int pp = 0; pp < NJT / 2; ++pp) {
      pw[pp] = pack8(sc[2 * pp], sc[2 * pp + 1]);
#pragma unroll
      for (int t = 0; t < T; ++t) pdw[t][pp] = pack8(ds[t][2 * pp], ds[t][2 * pp + 1]);
    }
  };

  // ---- PV(i): P.V products of chunk i over key pairs -------------------------------------
  // Padding keys carry weight 0 against zero rows of V, so every pair is multiplied.
  auto pv_step = [&](int buf) {
    const uint16_t* const Vb = vbuf + buf * NX * Sh::kTr;
#pragma unroll
    for (int pp = 0; pp < NJT / 2; ++pp) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* vrow = Vb + (dt * 16 + c) * LDT + pp * 32 + 8 * g;
        const bf16x8 vv = as_bf16x8(*reinterpret_cast<const uint4*>(vrow));
        if constexpr (!GIVEN_LSE) o[dt] = mfma_bf16(vv, pw[pp], o[dt]);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          at[t][dt] = mfma_bf16(vv, pdw[t][pp], at[t][dt]);
          const bf16x8 vtv = as_bf16x8(*reinterpret_cast<const uint4*>(vrow + (1 + t) * Sh::kTr));
          ct[t][dt] = mfma_bf16(vtv, pw[pp], ct[t][dt]);
        }
      }
    }
  };

  // ---- pipeline: prologue, then the ping-pong phases -------------------------------------
  // Before phase 0: K(0), K(1) and V(0) in LDS, K(2) and V(1) in registers.
  // K(1) goes into a second register set so that its reads overlap those of K(0), V(0).
  if (nchunks > 0) {
    stage_loads(0, 0);
    uint4 rk1[Sh::kKPer];
    {
      int sk[Sh::kKPer];
#pragma unroll
      for (int u = 0; u < Sh::kKPer; ++u) sk[u] = idx[min(kKC + krow[u], N - 1)];
#pragma unroll
      for (int u = 0; u < Sh::kKPer; ++u) {
        const int j = kKC + krow[u];
        rk1[u] = bload(krs[u], (j < nk && kitem(u)) ? (key_all ? j : sk[u]) * rowstride + hoff + kcol[u] : wbytes);
      }
    }
    kstore(0, rk);
    vstore(0);
    kstore(1, rk1);
    stage_loads(2 * kKC, kKC);
  }
  // Wait for the query fragments here (they precede the staging reads, which the stores
  // above have waited for): left pending into the loop, the compiler's merged wait state
  // at their first use would also cover the staging reads in flight.
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    settle_bf16x8(qf[s]);
#pragma unroll
    for (int t = 0; t < T; ++t) settle_bf16x8(qtf[t][s]);
  }
  asm volatile("" : "+v"(lse2));
  __syncthreads();

  // Each wave runs pairs (matrix phase of step i, barrier, softmax phase of step i,
  // barrier) for i = 0..nchunks; group 1 starts one barrier late and group 0 ends one
  // barrier late, so both pass the same number of barriers and stay one phase apart.
  // Staging past the last chunk moves zero chunks into buffers nobody reads again, so the
  // phases have no branches around their memory operations.
  if (nchunks > 0) {
    if (grp == 1) __syncthreads();
    int bi = 0;  // i mod 3
#pragma clang loop unroll(disable)
    for (int i = 0; i <= nchunks; ++i) {
      const int bprev = bi == 0 ? 2 : bi - 1;  // (i - 1) mod 3 = (i + 2) mod 3
      const int bnext = bi == 2 ? 0 : bi + 1;  // (i + 1) mod 3
      __builtin_amdgcn_s_setprio(1);
      if (active && i >= 1) pv_step(bprev);
      if (active && i < nchunks) s_step(bi);
      __builtin_amdgcn_s_setprio(0);
      __syncthreads();
      if (active && i < nchunks) sm_step(i);
      kstore(bprev, rk);
      vstore(bnext);
      stage_loads((i + 3) * kKC, (i + 2) * kKC);
      __syncthreads();
      bi = bnext;
    }
    if (grp == 0) __syncthreads();
  }

  if (active) {
    float inv = 1.f, l2tot = 0.f;
    if constexpr (!GIVEN_LSE) {
      l2tot = group_sum(lsum);
      inv = 1.f / l2tot;
    }
    float mut[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) mut[t] = group_sum(mu[t]) * inv;
    if constexpr (!HAS_E) {
      // the tangent scale, deferred from the scores (see above)
#pragma unroll
      for (int t = 0; t < T; ++t) {
        mut[t] *= stscale;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) at[t][dt] *= stscale;
      }
    }
    if (qvalid) {
      const int64_t obase = bnhd(b, qsite, h, N, H, D);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        float o4[4];
        if constexpr (!GIVEN_LSE) {
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] = o[dt][r] * inv;
          store4<BF16>(p.out, obase + d0, o4[0], o4[1], o4[2], o4[3]);
        } else {
          const float4 x = load4<BF16>(p.out_in, obase + d0);
          o4[0] = x.x;
          o4[1] = x.y;
          o4[2] = x.z;
          o4[3] = x.w;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float tv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) tv[r] = (at[t][dt][r] + ct[t][dt][r]) * inv - mut[t] * o4[r];
          store4<BF16>(p.tout, t * p.t_stride + obase + d0, tv[0], tv[1], tv[2], tv[3]);
        }
      }
      if constexpr (!GIVEN_LSE) {
        if (g == 0 && p.lse != nullptr)
          p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] = (m2 + log2f(l2tot)) * kLn2;
      }
    }
  }

  // rows of masked sites in this block's site range (square mask): zeros, lse = -1e4 + log N
  if (!p.key_mask) {
    constexpr int C4 = D / 4;
    const int r0 = blk * kQB;
    for (int it = tid; it < kQB * C4; it += kThreads) {
      const int r = r0 + it / C4;
      const int c4 = it % C4;
      if (r < N && mask_s[r] == 0) {
        const int64_t off = bnhd(b, r, h, N, H, D) + c4 * 4;
        if constexpr (!GIVEN_LSE) store4<BF16>(p.out, off, 0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < T; ++t) store4<BF16>(p.tout, t * p.t_stride + off, 0.f, 0.f, 0.f, 0.f);
        if (!GIVEN_LSE && c4 == 0 && p.lse != nullptr)
          p.lse[(static_cast<int64_t>(b) * N + r) * H + h] = p.masked_lse;
      }
    }
  }
}

template <int D, int T, bool GIVEN_LSE, bool HAS_E>
hipError_t launch_t(const FwdParams& p, hipStream_t stream) {
  using Sh = LShape<D, T>;
  const int nblk = (p.N + kQB - 1) / kQB;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = Sh::lds_bytes(p.N);
  auto kern = mhsea_fwd_bf16_large_kernel<D, T, GIVEN_LSE, HAS_E>;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

template <int D, int T, bool GIVEN_LSE>
hipError_t dispatch_e(const FwdParams& p, hipStream_t stream) {
  if (p.e != nullptr || p.et != nullptr) return launch_t<D, T, GIVEN_LSE, true>(p, stream);
  return launch_t<D, T, GIVEN_LSE, false>(p, stream);
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

bool bf16_large_fwd_supported(int N, int D) {
  // LDS: two buffers plus the walker's mask and site list must fit 160 KiB.
  return N > 128 && (D == 32 || D == 64) && (D == 32 ? LShape<32, 2>::lds_bytes(N) : LShape<64, 2>::lds_bytes(N)) <= 160 * 1024;
}

hipError_t launch_fwd_bf16_large(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream) {
  if (D == 32) return dispatch_t<32>(p, T, given_lse, stream);
  if (D == 64) return dispatch_t<64>(p, T, given_lse, stream);
  return hipErrorInvalidValue;
}

}  // namespace hz
