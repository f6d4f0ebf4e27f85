// bfloat16 forward / forward+tangent MHSEA kernel for large N at head dimension 64 without
// an edge bias: 32-query tiles on v_mfma_f32_32x32x16_bf16, each tile served by a pair of
// waves with split roles.
//
// Work decomposition: a 512-thread workgroup (8 waves) owns one (walker, head) and 128
// consecutive compacted queries, four tiles of 32. Tile p is served by score wave p and value
// wave p + 4 (the hardware places waves w and w + 4 on one SIMD, so each SIMD holds one
// pair; any placement gives the same results). Keys stream through LDS in chunks of 32
// compacted keys, each chunk staged once for the workgroup.
//
// Roles, per 32-key chunk i:
//   score wave: S(i), the score products S^T = K Q^T and dS^T = Kt Q^T + K Qt^T, then the
//     online softmax; it writes the chunk's bf16 weights P and s P o dS and the rescale
//     factor of its queries to LDS (each lane exactly the operand its partner lane reads)
//     and keeps the normaliser l and the tangent row sums mu;
//   value wave: the rescale and the P.V products O^T += V^T P^T, A^T += V^T (s P o dS)^T +
//     Vt^T P^T of the previous chunk, the staging of K-like and V-like chunks, and at the
//     end the normalised outputs.
// The two waves of a SIMD interleave in hardware: the softmax of one tile runs on the vector
// ALU while the other wave's products run on the matrix cores. A score wave keeps the query
// fragments and one chunk's scores (~190 registers), a value wave the accumulators and the
// staging registers (~200), so two waves fit a SIMD. One workgroup barrier per chunk.
//
// Pipeline, iteration i: score waves run the softmax of chunk i (scores computed in iteration
// i-1) interleaved with the products of S(i+1) (K buffer (i+1) mod 3) and write W(i) (weights
// and rescale factors) into weight buffer i mod 2; value waves apply W(i-1) to V(i-1) (weight
// and V buffers (i-1) mod 2), write K(i+2) into K buffer (i+2) mod 3 and V(i) into V buffer
// i mod 2 (both read from HBM in iteration i-1), and issue the reads of K(i+3) and V(i+1). Every write goes to a buffer whose last reader finished before the
// previous barrier: K(i+2) replaces K(i-1) (read in iteration i-1), V(i) replaces V(i-2)
// and W(i) replaces W(i-2) (both read in iteration i-1).
//
// Matrix-core layout of v_mfma_f32_32x32x16_bf16, lane l = 32 hh + c (hh = l / 32):
//   A operand: lane supplies A[row c][k 8 hh .. 8 hh + 7]
//   B operand: lane supplies B[k 8 hh .. 8 hh + 7][col c]
//   C/D:       lane holds element i = 0..15 at C[row 8 (i / 4) + 4 hh + i % 4][col c]
// S^T[key][query]: A = the chunk's K rows (row-major, rows padded to 72 bf16), B = the query
// fragments. A lane's scores are 16 keys of one query; k-step s of the P.V products contracts
// keys kappa(s, hh, j) = 16 s + 8 (j / 4) + 4 hh + j % 4, the lane's score elements 8 s + j,
// so the B operand of the value wave's lane is the score wave's same lane's weights. V tiles
// are row-major (rows padded to 96 bf16) and the A operand V^T[d][8 keys] comes from two
// transposing reads (ds_read_b64_tr_b16).
//
// Online softmax with a lazy rescale: the base m of a query row only moves when the chunk
// maximum exceeds it by more than 8 (base 2); the value wave rescales its accumulators by
// alpha = 2^(m_old - m_new) before adding the chunk's products. l and mu are summed from the
// bf16-rounded weights the products use.
//
// Scope: D = 64, T in {0, 1, 2}, no bias, the forward variants, scale > 0.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kD = 64;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kPairs = 4;
constexpr int kQW = 32;              // queries per tile (wave pair)
constexpr int kQB = kQW * kPairs;    // queries per workgroup
constexpr int kKC = 32;              // keys per chunk
constexpr int kKLD = kD + 8;         // K-like row, bf16 (144 bytes)
constexpr int kVLD = kD + 32;        // V-like row, bf16 (192 bytes)
constexpr int kKTile = kKC * kKLD;
constexpr int kVTile = kKC * kVLD;
constexpr float kRescale = 8.f;

template <int T>
struct SShape {
  static constexpr int NX = 1 + T;
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int kKBuf = NX * kKTile;
  static constexpr int kVBuf = NX * kVTile;
  // weights of one tile and chunk: NX sets x 2 k-steps x 64 lanes x 8 bf16
  static constexpr int kWTile = NX * 2 * 64 * 8;
  static constexpr int kWBuf = kPairs * kWTile;
  // bf16 elements: 3 K buffers, 2 V buffers, 2 weight buffers
  static constexpr int kElems = 3 * kKBuf + 2 * kVBuf + 2 * kWBuf;
  // floats after that: rescale factors [2][pairs][32], final l and mu [pairs][1 + T][32]
  static constexpr int kFloats = 2 * kPairs * kQW + kPairs * (1 + T) * kQW;
  static_assert(kPairs * NX * kQW * kKLD <= 3 * kKBuf + 2 * kVBuf, "output staging fits over the key buffers");
  static size_t lds_bytes(int N) {
    const size_t n16 = (static_cast<size_t>(N) + 15) & ~size_t(15);
    return static_cast<size_t>(kElems) * 2 + static_cast<size_t>(kFloats) * 4 + 64 + n16 + 2 * n16;
  }
};

__device__ __forceinline__ v16f mfma32(bf16x8 a, bf16x8 b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ v16f zero16() { return v16f{}; }
// acc + the sum of the eight bf16 values of x (v_dot2_f32_bf16 against ones).
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
// Elements 8 s .. 8 s + 7 of a score tile as bf16 (element j of the result = x[8 s + j]).
__device__ __forceinline__ bf16x8 pack_half(const v16f& x, int s) {
  uint4 u;
  u.x = pack2_bf16(x[8 * s + 0], x[8 * s + 1]);
  u.y = pack2_bf16(x[8 * s + 2], x[8 * s + 3]);
  u.z = pack2_bf16(x[8 * s + 4], x[8 * s + 5]);
  u.w = pack2_bf16(x[8 * s + 6], x[8 * s + 7]);
  return as_bf16x8(u);
}

// Site compaction (4 sites per thread per round; exclusive prefix from bit-plane ballots).
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

template <int T, bool UNIT>
__global__ void __launch_bounds__(kThreads, 1) mhsea_fwd_bf16_ws_kernel(const FwdParams p) {
  using Sh = SShape<T>;
  constexpr int NX = Sh::NX, TT = Sh::TT;

  extern __shared__ float4 smem4[];
  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* const kbuf = lds;                                  // [3][NX][kKC][kKLD]
  uint16_t* const vbuf = kbuf + 3 * Sh::kKBuf;                 // [2][NX][kKC][kVLD]
  uint16_t* const wbuf = vbuf + 2 * Sh::kVBuf;                 // [2][pairs][NX][2][64][8]
  float* const abuf = reinterpret_cast<float*>(lds + Sh::kElems);  // [2][pairs][32]
  float* const fbuf = abuf + 2 * kPairs * kQW;                     // [pairs][1 + T][32]
  int* const scratch = reinterpret_cast<int*>(fbuf + kPairs * (1 + T) * kQW);
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
  const bool scorer = wave < kPairs;
  const int pair = scorer ? wave : wave - kPairs;

  const int n_phys = compact_sites(p.mask + static_cast<int64_t>(b) * N, N, idx, mask_s, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int nc = (nk + kKC - 1) / kKC;
  if (key_all) {  // every site is a key: the identity site list
    for (int j = tid; j < N; j += kThreads) idx[j] = static_cast<int16_t>(j);
    __syncthreads();
  }

  const int q0 = blk * kQB + pair * kQW;
  const bool qvalid = q0 + c < nq;
  const int qsite = qvalid ? (p.key_mask ? (q0 + c) : idx[q0 + c]) : -1;

  if (blk * kQB < nq && nc > 0) {
    // ---- staging (value waves): buffer resources over the walker's slice of each tensor --
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
    // a value-wave thread stages one 16-byte piece (row srow, column scol) per tensor and kind
    const int vt_id = tid - kPairs * 64;  // 0..255 in value waves
    const int srow = (vt_id & 255) >> 3, scol = vt_id & 7;
    auto stage_offsets = [&](int kck, int kcv, int& ko, int& vo) {
      const int jk = kck + srow, jv = kcv + srow;
      int sk = idx[min(jk, N - 1)];
      int sv = idx[min(jv, N - 1)];
      asm volatile("" : "+v"(sk), "+v"(sv));
      ko = jk < nk ? sk * rowstride + hoff + scol * 16 : wbytes;
      vo = jv < nk ? sv * rowstride + hoff + scol * 16 : wbytes;
    };
    auto stage_loads = [&](int kck, int kcv, uint4(&rk)[NX], uint4(&rv)[NX]) {
      int ko, vo;
      stage_offsets(kck, kcv, ko, vo);
#pragma unroll
      for (int x = 0; x < NX; ++x) {
        rk[x] = bload(kr[x], ko);
        rv[x] = bload(vr[x], vo);
      }
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

    uint16_t* const wtile0 = wbuf + pair * Sh::kWTile + lane * 8;  // + buf * kWBuf + (x * 2 + s) * 512
    float* const atile0 = abuf + pair * kQW;                          // + buf * pairs * 32
    const float s2scale = UNIT ? kLog2e : p.scale * kLog2e;
    const float stscale = UNIT ? 1.f : p.scale;

    if (scorer) {
      // ================================ score wave ======================================
      bf16x8 qf[4], qtf[TT][4];
      {
        const int64_t qoff = bnhd(b, qvalid ? qsite : 0, h, N, H, kD) + 8 * hh;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qoff + 16 * s));
#pragma unroll
          for (int t = 0; t < T; ++t)
            qtf[t][s] = p.qt != nullptr ? as_bf16x8(*reinterpret_cast<const uint4*>(
                                              static_cast<const uint16_t*>(p.qt) + t * p.t_stride + qoff + 16 * s))
                                        : bf16x8{};
        }
      }
      float m2 = -INFINITY, lsum = 0.f;
      float mu[TT];
#pragma unroll
      for (int t = 0; t < T; ++t) mu[t] = 0.f;
      // S(j) into (sc, ds) from K buffer j mod 3; the order per k-step keeps products into
      // one accumulator apart
      auto s_products = [&](int j, v16f& sc, v16f(&ds)[TT]) {
        const uint16_t* const kp = kbuf + (j % 3) * Sh::kKBuf + c * kKLD + 8 * hh;
        sc = zero16();
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t] = zero16();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 kf = as_bf16x8(*reinterpret_cast<const uint4*>(kp + 16 * s));
#pragma unroll
          for (int t = 0; t < T; ++t)
            ds[t] = mfma32(as_bf16x8(*reinterpret_cast<const uint4*>(kp + (1 + t) * kKTile + 16 * s)), qf[s], ds[t]);
          sc = mfma32(kf, qf[s], sc);
#pragma unroll
          for (int t = 0; t < T; ++t) ds[t] = mfma32(kf, qtf[t][s], ds[t]);
        }
      };
      // The softmax of chunk i (scores in sc, ds) with the products of S(i+1) (into scn, dsn,
      // K(i+1) staged since the last barrier) interleaved between its vector instructions.
      auto step = [&](int i, v16f& sc, v16f(&ds)[TT], v16f& scn, v16f(&dsn)[TT]) {
        // validity (only the last chunk holds padding keys), chunk maximum, base update
        if (i == nc - 1 && (nk & (kKC - 1)) != 0) {
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
        float alpha = 1.f;
        if (__any(need)) {
          const float mnew = need ? mx : m2;
          alpha = fast_exp2(m2 - mnew);  // 0 on the first chunk
          m2 = mnew;
        }
        __builtin_amdgcn_sched_barrier(0);
        s_products(i + 1, scn, dsn);
        // softmax weights, bf16, written where the partner lane reads them
        uint16_t* const wt = wtile0 + (i & 1) * Sh::kWBuf;
        float ls = 0.f, muc[TT];
#pragma unroll
        for (int t = 0; t < T; ++t) muc[t] = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float pe = fast_exp2(fmaf(sc[e], s2scale, -m2));
          sc[e] = pe;
          const float ps = UNIT ? pe : pe * stscale;
#pragma unroll
          for (int t = 0; t < T; ++t) ds[t][e] *= ps;
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 pw = pack_half(sc, s);
          ls = sum8(pw, ls);
          *reinterpret_cast<uint4*>(wt + s * 512) = __builtin_bit_cast(uint4, pw);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const bf16x8 pdw = pack_half(ds[t], s);
            muc[t] = sum8(pdw, muc[t]);
            *reinterpret_cast<uint4*>(wt + ((1 + t) * 2 + s) * 512) = __builtin_bit_cast(uint4, pdw);
          }
        }
        if (hh == 0) atile0[(i & 1) * kPairs * kQW + c] = alpha;
        // one product, then a run of vector instructions; the operand reads go out early
        constexpr int kR = 4 * NX, kP = 4 * (1 + 2 * T);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int k = 0; k < kR - 4; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
#pragma unroll
        for (int k = kR - 4; k < kP; ++k) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        lsum = fmaf(lsum, alpha, ls);
#pragma unroll
        for (int t = 0; t < T; ++t) mu[t] = fmaf(mu[t], alpha, muc[t]);
        __syncthreads();
      };
      v16f sA, sB, dA[TT], dB[TT];
      __syncthreads();  // prologue: K(0), K(1) staged by the value waves
      s_products(0, sA, dA);
      int i = 0;
#pragma clang loop unroll(disable)
      for (; i + 1 < nc; i += 2) {
        step(i, sA, dA, sB, dB);
        step(i + 1, sB, dB, sA, dA);
      }
      if (i < nc) step(i, sA, dA, sB, dB);
      // normaliser and tangent row sums for the value wave; lse
      // (the cross-half sums run with every lane active; only the writes are per half)
      const float ltot = xor32_pair_sum(lsum);
      float mut[TT];
#pragma unroll
      for (int t = 0; t < T; ++t) mut[t] = xor32_pair_sum(mu[t]);
      if (hh == 0) {
        fbuf[pair * (1 + T) * kQW + c] = ltot;
#pragma unroll
        for (int t = 0; t < T; ++t) fbuf[(pair * (1 + T) + 1 + t) * kQW + c] = mut[t];
      }
      if (qvalid && hh == 0 && p.lse != nullptr)
        p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] = (m2 + log2f(ltot)) * kLn2;
      __syncthreads();  // l and mu published; the value waves are past their last V reads
    } else {
      // ================================ value wave ======================================
      v16f o[2], ac[TT][2];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        o[dt] = zero16();
#pragma unroll
        for (int t = 0; t < T; ++t) ac[t][dt] = zero16();
      }
      // transposing reads of the V^T operand: lane 16 g + 4 j + q addresses row
      // 16 s + 8 h2 + 4 (g / 2) + j, column 32 dt + 16 (g % 2) + 4 q of the row-major tile
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
      // rescale, then the products of chunk j (weights in buffer j mod 2, V in buffer j mod 2)
      auto pv_step = [&](int j) {
        const float alpha = atile0[(j & 1) * kPairs * kQW + c];
        if (__any(alpha != 1.f)) {
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            o[dt] *= alpha;
#pragma unroll
            for (int t = 0; t < T; ++t) ac[t][dt] *= alpha;
          }
        }
        const uint16_t* const wt = wtile0 + (j & 1) * Sh::kWBuf;
        const uint16_t* const vb = vbuf + (j & 1) * Sh::kVBuf;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x8 pw = as_bf16x8(*reinterpret_cast<const uint4*>(wt + s * 512));
          bf16x8 pdw[TT];
#pragma unroll
          for (int t = 0; t < T; ++t) pdw[t] = as_bf16x8(*reinterpret_cast<const uint4*>(wt + ((1 + t) * 2 + s) * 512));
          bf16x8 vf[2];
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            vf[dt] = vfrag(vb, dt, s);
            o[dt] = mfma32(vf[dt], pw, o[dt]);
          }
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) ac[t][dt] = mfma32(vf[dt], pdw[t], ac[t][dt]);
#pragma unroll
          for (int t = 0; t < T; ++t)
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) ac[t][dt] = mfma32(vfrag(vb + (1 + t) * kVTile, dt, s), pw, ac[t][dt]);
        }
      };

      // prologue: K(0), K(1) into K buffers 0, 1; K(2) and V(0) in flight
      uint4 rk[NX], rv[NX];
      {
        uint4 rk1[NX], rv1[NX];
        stage_loads(0, 0, rk, rv);
        stage_loads(kKC, 0, rk1, rv1);
        kstore(0, rk);
        kstore(1, rk1);
      }
      stage_loads(2 * kKC, 0, rk, rv);
      __syncthreads();
      for (int i = 0; i < nc; ++i) {
        // site ids of this iteration's staging rows, read ahead of the products so their LDS
        // latency hides under them
        const int jk = (i + 3) * kKC + srow, jv = (i + 1) * kKC + srow;
        int sk = idx[min(jk, N - 1)];
        int sv = idx[min(jv, N - 1)];
        if (i > 0) pv_step(i - 1);
        // K(i+2) into K buffer (i+2) mod 3 (last read: K(i-1), in iteration i-1), V(i) into
        // V buffer i mod 2 (last read: V(i-2), in iteration i-1), then the next reads
        kstore((i + 2) % 3, rk);
        vstore(i & 1, rv);
        asm volatile("" : "+v"(sk), "+v"(sv));
        const int ko = jk < nk ? sk * rowstride + hoff + scol * 16 : wbytes;
        const int vo = jv < nk ? sv * rowstride + hoff + scol * 16 : wbytes;
#pragma unroll
        for (int x = 0; x < NX; ++x) {
          rk[x] = bload(kr[x], ko);
          rv[x] = bload(vr[x], vo);
        }
        __syncthreads();
      }
      pv_step(nc - 1);
      __syncthreads();  // every value wave is past its V reads; the score waves published l, mu

      // ---- normalisation and stores: stage rows in LDS (over the K/V buffers), then whole
      // 128-byte rows per store
      const float ltot = fbuf[pair * (1 + T) * kQW + c];
      const float inv = 1.f / ltot;
      float mut[TT];
#pragma unroll
      for (int t = 0; t < T; ++t) mut[t] = fbuf[(pair * (1 + T) + 1 + t) * kQW + c] * inv;
      uint16_t* const ot = lds + pair * (NX * kQW * kKLD);  // [NX][32 queries][kKLD]
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
            uint16_t* const dst =
                x == 0 ? static_cast<uint16_t*>(p.out) : static_cast<uint16_t*>(p.tout) + (x - 1) * p.t_stride;
            *reinterpret_cast<uint4*>(dst + off) = v;
          }
        }
      }
    }
  }

  // rows of masked sites in this block's site range (square mask): zeros, lse = -1e4 + log N;
  // the score waves take 32 rows each
  if (!p.key_mask && scorer) {
    const int r0 = blk * kQB + pair * kQW;
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
  using Sh = SShape<T>;
  const int nblk = (p.N + kQB - 1) / kQB;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = Sh::lds_bytes(p.N);
  auto kern = mhsea_fwd_bf16_ws_kernel<T, UNIT>;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(kThreads), lds, stream, p);
  return hipGetLastError();
}

}  // namespace

bool bf16_ws_fwd_supported(const FwdParams& p, int D, bool given_lse) {
  const int64_t wbytes = static_cast<int64_t>(p.N) * p.H * D * 2;
  return D == kD && !given_lse && p.e == nullptr && p.et == nullptr && p.scale > 0.f && p.scale < INFINITY &&
         p.N > 128 && wbytes < (int64_t(1) << 31) && SShape<2>::lds_bytes(p.N) <= 160 * 1024 && p.gated == 0;
}

hipError_t launch_fwd_bf16_ws(const FwdParams& p, int T, hipStream_t stream) {
  const bool unit = p.scale == 1.f;
  if (T == 0) return unit ? launch_t<0, true>(p, stream) : launch_t<0, false>(p, stream);
  if (T == 1) return unit ? launch_t<1, true>(p, stream) : launch_t<1, false>(p, stream);
  if (T == 2) return unit ? launch_t<2, true>(p, stream) : launch_t<2, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace hz
