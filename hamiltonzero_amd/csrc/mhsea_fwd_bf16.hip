// bfloat16 matrix-core forward / forward+tangent / tangent-only MHSEA kernel (any N,
// D in {32, 64}, bfloat16 storage).
//
// Products run on v_mfma_f32_16x16x32_bf16 (bf16 operands, fp32 accumulation); the
// softmax and every reduction stay in fp32. Layout per wave (16 queries, lane = 16 g + c):
//   S^T[key 16jt + 4g + r][query c] = sum over 32-wide d blocks s of
//        K[16jt + c][32s + 8g .. +8] . Q[c][32s + 8g .. +8]        (8 bf16 per lane)
//   O^T[d 16dt + 4g + r][query c] += sum over key pairs (2p, 2p+1) of
//        V^T[16dt + c][keys kappa(g,i)] . P[c][kappa(g,i)],  kappa(g,i) = 16(2p + i/4) + 4g + i%4
// The B operand of the P.V product is the lane's own softmax weights of two key tiles (the
// C layout of S^T), rounded to bf16; V and the tangent values are staged transposed in LDS
// so a lane reads its 8 keys as two 8-byte runs. The contraction index of one instruction may
// be any permutation as long as A and B agree, which is what kappa expresses.
//
// Work decomposition and mask handling follow the fp32 streaming kernel: workgroup = (walker,
// head, 64 compacted queries); keys streamed through LDS in chunks of 64 with a register
// prefetch of the next chunk; online softmax across chunks; masked query rows written as
// zeros with lse = -1e4 + log N.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }


// keep ? u : 0, component-wise (a select of whole HIP vector structs would go through
// private memory).
__device__ __forceinline__ uint4 keep4(bool keep, const uint4& u) {
  return make_uint4(keep ? u.x : 0u, keep ? u.y : 0u, keep ? u.z : 0u, keep ? u.w : 0u);
}

// Element e (0..7) of eight bf16 packed in a uint4, as its 16-bit pattern.
__device__ __forceinline__ uint16_t bf16_at(const uint4& u, int e) {
  const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// 8 fp32 weights (4 of key tile 2p, 4 of key tile 2p+1) as one bf16x8 operand.
__device__ __forceinline__ bf16x8 pack8(v4f a, v4f b) {
  uint4 u;
  u.x = pack2_bf16(a[0], a[1]);
  u.y = pack2_bf16(a[2], a[3]);
  u.z = pack2_bf16(b[0], b[1]);
  u.w = pack2_bf16(b[2], b[3]);
  return as_bf16x8(u);
}

template <int D, int T>
struct Bf16Shape {
  static constexpr int KC = 64;           // keys per chunk
  static constexpr int LDR = D + 8;       // row-major tile row, bf16 elements (16 B pad)
  static constexpr int LDT = KC + 8;      // transposed tile row, bf16 elements
  static constexpr int NS = D / 32;       // 32-wide d blocks
  static constexpr int DT = D / 16;       // 16-row tiles of O^T
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int kRowTile = KC * LDR;   // K, Kt (row-major), elements
  static constexpr int kTrTile = D * LDT;      // V^T, Vt^T, elements
  static constexpr int kC8 = D / 8;           // 8-element (16 B) chunks of one row
  static constexpr int kItems = KC * kC8;     // 16 B items of one tensor chunk
  static constexpr int kPerThread = (kItems + 255) / 256;
  // V staging at D = 64: one item = rows (2p, 2p+1) of one 8-column chunk, written transposed
  // as 32-bit (row pair) words, so a wave's 32 pairs x 2 chunks cover 64 distinct LDS banks
  // (one row per item and 16-bit writes put 8 lanes on each bank). At D = 32 the pairs would
  // leave half of the threads without V items, so V is staged like K, one row per item.
  static constexpr bool kPairV = D == 64;
  static constexpr int kPairItems = (KC / 2) * kC8;
  static constexpr int kPairPer = kPairV ? (kPairItems + 255) / 256 : 1;
  static size_t lds_bytes(int N) {
    const size_t n16 = (static_cast<size_t>(N) + 15) & ~size_t(15);
    return static_cast<size_t>((1 + T) * kRowTile + (1 + T) * kTrTile) * 2 + 16 + n16 + 2 * n16;
  }
};

template <int D, int T, bool GIVEN_LSE, bool HAS_E, bool MULTI>
__global__ void __launch_bounds__(256, ((D == 64 && T > 0) ? 2 : 3)) mhsea_fwd_bf16_kernel(const FwdParams p) {
  using Sh = Bf16Shape<D, T>;
  constexpr int KC = Sh::KC, LDR = Sh::LDR, LDT = Sh::LDT, NS = Sh::NS, DT = Sh::DT, TT = Sh::TT;
  constexpr int NPT = Sh::kPerThread, C8 = Sh::kC8;
  constexpr int NJT = KC / 16;

  extern __shared__ float4 smem4[];
  uint16_t* const Kr = reinterpret_cast<uint16_t*>(smem4);         // K rows
  uint16_t* const Ktr = Kr + Sh::kRowTile;                           // Kt[t] rows
  uint16_t* const Vtr = Ktr + T * Sh::kRowTile;                      // V^T
  uint16_t* const Vttr = Vtr + Sh::kTrTile;                          // Vt[t]^T
  int* const scratch = reinterpret_cast<int*>(Vttr + T * Sh::kTrTile);
  const int n16 = (p.N + 15) & ~15;
  uint8_t* const mask_s = reinterpret_cast<uint8_t*>(scratch + 4);
  int16_t* const idx = reinterpret_cast<int16_t*>(mask_s + n16);

  const int N = p.N, H = p.H;
  const int nblk = (N + 63) >> 6;
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

  const int n_phys = compact_mask_lds(p.mask + static_cast<int64_t>(b) * N, N, idx, mask_s, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;

  const bool has_kt = p.kt != nullptr, has_vt = p.vt != nullptr, has_qt = p.qt != nullptr;
  const void* const ktp = has_kt ? p.kt : p.k;
  const void* const vtp = has_vt ? p.vt : p.v;
  const void* const qtp = has_qt ? p.qt : p.q;
  const int64_t kts = has_kt ? p.t_stride : 0, vts = has_vt ? p.t_stride : 0;
  const int64_t qts = has_qt ? p.t_stride : 0;

  // ---- key chunk staging: global (16 B of one row per item) -> registers -> LDS ---------
  constexpr int NPP = Sh::kPairPer;
  uint4 ck[NPT], ckt[TT][NPT];
  // V (and Vt): [pair item][row of the pair] at D = 64, [row item][0] otherwise
  uint4 cv[Sh::kPairV ? NPP : NPT][2], cvt[TT][Sh::kPairV ? NPP : NPT][2];
  auto chunk_load = [&](int kc) {
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int it = tid + u * 256;
      const int j = kc + it / C8;
      const bool ok = (Sh::kItems % 256 == 0 || it < Sh::kItems) && j < nk;
      const int n = ok ? (key_all ? j : idx[j]) : 0;
      const int64_t off = bnhd(b, n, h, N, H, D) + (it % C8) * 8;
      ck[u] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.k) + off);
#pragma unroll
      for (int t = 0; t < T; ++t)
        ckt[t][u] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(ktp) + t * kts + off);
      if constexpr (!Sh::kPairV) {
        cv[u][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.v) + off);
#pragma unroll
        for (int t = 0; t < T; ++t)
          cvt[t][u][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(vtp) + t * vts + off);
      }
    }
    if constexpr (Sh::kPairV) {
#pragma unroll
    for (int u = 0; u < NPP; ++u) {
      const int pi = tid + u * 256;
      const bool live = Sh::kPairItems % 256 == 0 || pi < Sh::kPairItems;
      const int pr = pi % 32;
      const int kk = live ? pi / 32 : 0;  // 8-column chunk (in range also for idle threads)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int j = kc + 2 * pr + h2;
        const bool ok = live && j < nk;
        const int n = ok ? (key_all ? j : idx[j]) : 0;
        const int64_t off = bnhd(b, n, h, N, H, D) + kk * 8;
        cv[u][h2] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.v) + off);
#pragma unroll
        for (int t = 0; t < T; ++t)
          cvt[t][u][h2] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(vtp) + t * vts + off);
      }
    }
    }
  };
  auto chunk_store = [&](int kc) {
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int it = tid + u * 256;
      if (Sh::kItems % 256 == 0 || it < Sh::kItems) {
        const int r = it / C8;
        const int c8 = (it % C8) * 8;
        const bool ok = kc + r < nk;
        *reinterpret_cast<uint4*>(Kr + r * LDR + c8) = keep4(ok, ck[u]);
#pragma unroll
        for (int t = 0; t < T; ++t)
          *reinterpret_cast<uint4*>(Ktr + t * Sh::kRowTile + r * LDR + c8) = keep4(ok && has_kt, ckt[t][u]);
        if constexpr (!Sh::kPairV) {
          const uint4 vv = keep4(ok, cv[u][0]);
#pragma unroll
          for (int e = 0; e < 8; ++e) Vtr[(c8 + e) * LDT + r] = bf16_at(vv, e);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const uint4 tv = keep4(ok && has_vt, cvt[t][u][0]);
#pragma unroll
            for (int e = 0; e < 8; ++e) Vttr[t * Sh::kTrTile + (c8 + e) * LDT + r] = bf16_at(tv, e);
          }
        }
      }
    }
    if constexpr (Sh::kPairV) {
#pragma unroll
    for (int u = 0; u < NPP; ++u) {
      const int pi = tid + u * 256;
      if (Sh::kPairItems % 256 == 0 || pi < Sh::kPairItems) {
        const int r0 = 2 * (pi % 32);
        const int c8 = (pi / 32) * 8;
        const bool ok0 = kc + r0 < nk, ok1 = kc + r0 + 1 < nk;
        const uint4 v0 = keep4(ok0, cv[u][0]), v1 = keep4(ok1, cv[u][1]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t*>(Vtr + (c8 + e) * LDT + r0) =
              bf16_at(v0, e) | (static_cast<uint32_t>(bf16_at(v1, e)) << 16);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint4 t0 = keep4(ok0 && has_vt, cvt[t][u][0]), t1 = keep4(ok1 && has_vt, cvt[t][u][1]);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            *reinterpret_cast<uint32_t*>(Vttr + t * Sh::kTrTile + (c8 + e) * LDT + r0) =
                bf16_at(t0, e) | (static_cast<uint32_t>(bf16_at(t1, e)) << 16);
        }
      }
    }
    }
  };

  chunk_load(0);

  const int q0 = blk * 64 + wave * 16;
  const bool active = q0 < nq;
  const bool qvalid = q0 + c < nq;
  const int qsite = qvalid ? (p.key_mask ? (q0 + c) : idx[q0 + c]) : -1;
  const int qload = qvalid ? qsite : 0;

  // Query fragments, bf16, B-operand layout: lane (g, c) holds q[qsite][32 s + 8 g .. +8].
  bf16x8 qf[NS], qtf[TT][NS];
  {
    const int64_t qoff = bnhd(b, qload, h, N, H, D) + 8 * g;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) + qoff + 32 * s));
#pragma unroll
      for (int t = 0; t < T; ++t)
        qtf[t][s] = has_qt ? as_bf16x8(*reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(qtp) + t * qts + qoff + 32 * s))
                           : bf16x8{};
    }
  }
  // Padding query lanes only produce values that are never stored; the scale is applied to
  // the fp32 scores (exact in the product, no extra rounding of q). A null qt contributes
  // zero fragments, so dS = Kt Q^T alone keeps its scale.
  const float sscale = p.scale;
  const float stscale = p.scale;
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

  for (int kc = 0; kc < nk; kc += KC) {
    if (kc > 0) __syncthreads();
    chunk_store(kc);
    __syncthreads();
    if constexpr (MULTI) {
      if (kc + KC < nk) chunk_load(kc + KC);
    }
    if (!active) continue;

    const int jn = min(KC, nk - kc);
    const int njt = (jn + 15) >> 4;
    v4f sc[NJT], ds[TT][NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      sc[jt] = zero4();
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t][jt] = zero4();
      if (jt < njt) {
        const uint16_t* krow = Kr + (jt * 16 + c) * LDR + 8 * g;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bf16x8 kv = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 32 * s));
          sc[jt] = mfma_bf16(kv, qf[s], sc[jt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const uint16_t* ktrow = Ktr + t * Sh::kRowTile + (jt * 16 + c) * LDR + 8 * g;
            const bf16x8 ktv = as_bf16x8(*reinterpret_cast<const uint4*>(ktrow + 32 * s));
            ds[t][jt] = mfma_bf16(ktv, qf[s], ds[t][jt]);
            ds[t][jt] = mfma_bf16(kv, qtf[t][s], ds[t][jt]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    float mx = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = kc + jt * 16 + 4 * g + r;
        const bool valid = jt < njt && j < nk;
        float sv = sc[jt][r] * sscale;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][jt][r] *= stscale;
        if constexpr (HAS_E) {
          if (valid) {
            const int64_t eo = e_row + static_cast<int64_t>(key_all ? j : idx[j]) * p.e_sk;
            if (p.e != nullptr) sv += load1<BF16>(p.e, eo);
            if (p.et != nullptr) {
#pragma unroll
              for (int t = 0; t < T; ++t) ds[t][jt][r] += load1<BF16>(p.et, t * p.et_stride + eo);
            }
          }
        }
        sc[jt][r] = valid ? sv * kLog2e : -INFINITY;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][jt][r] = valid ? ds[t][jt][r] : 0.f;
        mx = fmaxf(mx, sc[jt][r]);
      }
    }

    if constexpr (GIVEN_LSE) {
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[jt][r] = lse_weight(sc[jt][r] - lse2);
    } else {
      const float mnew = fmaxf(m2, group_max(mx));
      if (MULTI && kc > 0) {
        const float alpha = fast_exp2(m2 - mnew);
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
      }
      m2 = mnew;
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[jt][r] = fast_exp2(sc[jt][r] - m2);
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

    // ---- P.V products over key pairs ------------------------------------------------
#pragma unroll
    for (int pp = 0; pp < NJT / 2; ++pp) {
      if (2 * pp < njt) {
        const bf16x8 pw = pack8(sc[2 * pp], sc[2 * pp + 1]);
        bf16x8 pdw[TT];
#pragma unroll
        for (int t = 0; t < T; ++t) pdw[t] = pack8(ds[t][2 * pp], ds[t][2 * pp + 1]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const uint16_t* vrow = Vtr + (dt * 16 + c) * LDT + pp * 32 + 4 * g;
          uint4 va;
          const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
          const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
          va.x = lo.x;
          va.y = lo.y;
          va.z = hi.x;
          va.w = hi.y;
          const bf16x8 vv = as_bf16x8(va);
          if constexpr (!GIVEN_LSE) o[dt] = mfma_bf16(vv, pw, o[dt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            at[t][dt] = mfma_bf16(vv, pdw[t], at[t][dt]);
            const uint16_t* trow = Vttr + t * Sh::kTrTile + (dt * 16 + c) * LDT + pp * 32 + 4 * g;
            uint4 ta;
            const uint2 tl = *reinterpret_cast<const uint2*>(trow);
            const uint2 th = *reinterpret_cast<const uint2*>(trow + 16);
            ta.x = tl.x;
            ta.y = tl.y;
            ta.z = th.x;
            ta.w = th.y;
            ct[t][dt] = mfma_bf16(as_bf16x8(ta), pw, ct[t][dt]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
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

  if (!p.key_mask) {
    constexpr int C4 = D / 4;
    const int r0 = blk * 64;
    for (int it = tid; it < 64 * C4; it += 256) {
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
  using Sh = Bf16Shape<D, T>;
  const int nblk = (p.N + 63) / 64;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = Sh::lds_bytes(p.N);
  auto kern = p.N > Sh::KC ? mhsea_fwd_bf16_kernel<D, T, GIVEN_LSE, HAS_E, true>
                           : mhsea_fwd_bf16_kernel<D, T, GIVEN_LSE, HAS_E, false>;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(256), lds, stream, p);
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

bool bf16_fwd_supported(int D) { return D == 32 || D == 64; }

hipError_t launch_fwd_bf16(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream) {
  if (D == 32) return dispatch_t<32>(p, T, given_lse, stream);
  if (D == 64) return dispatch_t<64>(p, T, given_lse, stream);
  return hipErrorInvalidValue;
}

}  // namespace hz
