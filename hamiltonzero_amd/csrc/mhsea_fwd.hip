// Forward, fused forward+tangent, and tangent-only MHSEA kernels for gfx950.
//
// Work decomposition. One 256-thread workgroup (4 waves) owns one (walker b, head h,
// block of 64 query rows). The walker's mask is compacted into the ascending list of
// physical sites; queries and keys are taken from that list, so padded (virtual) sites
// cost neither bytes nor matrix-core cycles. This is exact: under the reference's square
// mask an invalid pair has score -1e4 (mhsea.py:18-25), whose softmax weight
// exp(-1e4 - lse) is 0 in float32, and masked query rows are overwritten by zeros
// (mhsea_tuned.py:91, mhsea_tuned_jvp.py:90).
//
// Each wave owns 16 query rows and works in the transposed orientation
//   S^T(16 keys x 16 queries) = K . Q^T,    O^T(d x queries) += V^T . P^T
// so that the query index is always lane % 16: the row statistics of the online softmax
// (running max, normaliser, tangent mean) stay lane-local, and the matrix-core output
// layout of S^T is directly the B operand of the P.V product (no LDS round trip for P).
// Keys (and the tangent keys / values) are staged in LDS in chunks of KC rows and shared
// by the 4 waves.
//
// Tangent (forward-mode) algebra, per query row i, with P_ij = softmax_j(S_ij):
//   dS_ij = scale (qt_i . k_j + q_i . kt_j) + et_ij                (mhsea_tuned_jvp.py:69-74)
//   tout_i = sum_j P_ij dS_ij v_j + sum_j P_ij vt_j - (sum_j P_ij dS_ij) out_i   (:76-89)
// The three sums are accumulated with the same online rescaling as out_i, so one pass
// over the keys produces the primal and all T tangents.
#include <atomic>
#include <type_traits>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

template <int D, int T>
struct FwdShape {
  static constexpr int KC = (D == 64 && T > 0) ? 32 : 64;  // key rows per LDS chunk
  static constexpr int LD = D + 4;                         // padded LDS row, floats
  static constexpr int DG = D / 4;   // contraction values per lane group in K.Q^T
  static constexpr int DT = (D + 15) / 16;  // 16-row tiles of O^T
  static constexpr int C4 = D / 4;          // float4 columns of one row
  static constexpr int NT = 2 + 2 * T;      // staged tensors: K, V, Kt[T], Vt[T]
  static constexpr int TT = T > 0 ? T : 1;
  static constexpr int kTileFloats = KC * LD;
  static constexpr int kItems = KC * C4;                 // float4 items per tensor chunk
  static constexpr int kPerThread = (kItems + 255) / 256;
  static size_t lds_bytes(int N) {
    const size_t n16 = (static_cast<size_t>(N) + 15) & ~size_t(15);
    return static_cast<size_t>(NT) * kTileFloats * 4 + 16 + n16 /*mask*/ + 2 * n16 /*idx*/;
  }
};

template <int DG, class S>
__device__ __forceinline__ void load_row_frag(const void* base, int64_t off, float* dst) {
  if constexpr (DG >= 4) {
#pragma unroll
    for (int s = 0; s < DG; s += 4) {
      const float4 x = load4<S>(base, off + s);
      dst[s] = x.x;
      dst[s + 1] = x.y;
      dst[s + 2] = x.z;
      dst[s + 3] = x.w;
    }
  } else {
    const float2 x = load2<S>(base, off);
    dst[0] = x.x;
    dst[1] = x.y;
  }
}

// Issue the global loads of key rows [kc, kc + KC) of the compacted list into registers
// (K, V and the tangent keys / values). Every load is unconditional from an in-bounds row
// (site 0 stands in for padding) so that all of them are in flight before the first wait;
// padding is zeroed when the chunk is written to LDS.
template <int D, int T, class S, int NPT, int TT>
__device__ __forceinline__ void chunk_load(float4 (&ck)[NPT], float4 (&cv)[NPT],
                                           float4 (&ckt)[TT][NPT], float4 (&cvt)[TT][NPT],
                                           const FwdParams& p, int b, int h, int kc, int nk,
                                           bool key_all, const int16_t* idx, const void* ktp,
                                           int64_t kts, const void* vtp, int64_t vts) {
  using Sh = FwdShape<D, T>;
#pragma unroll
  for (int u = 0; u < Sh::kPerThread; ++u) {
    const int it = threadIdx.x + u * 256;
    const int j = kc + it / Sh::C4;
    const bool ok = (Sh::kItems % 256 == 0 || it < Sh::kItems) && j < nk;
    const int n = ok ? (key_all ? j : idx[j]) : 0;
    const int64_t off = bnhd(b, n, h, p.N, p.H, D) + (it % Sh::C4) * 4;
    ck[u] = load4<S>(p.k, off);
    cv[u] = load4<S>(p.v, off);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      ckt[t][u] = load4<S>(ktp, t * kts + off);
      cvt[t][u] = load4<S>(vtp, t * vts + off);
    }
  }
}

__device__ __forceinline__ void put4(float* dst, float4 x, bool keep) {
  *reinterpret_cast<float4*>(dst) =
      make_float4(keep ? x.x : 0.f, keep ? x.y : 0.f, keep ? x.z : 0.f, keep ? x.w : 0.f);
}

template <int D, int T, int NPT, int TT>
__device__ __forceinline__ void chunk_store(const float4 (&ck)[NPT], const float4 (&cv)[NPT],
                                            const float4 (&ckt)[TT][NPT], const float4 (&cvt)[TT][NPT],
                                            float* Ks, int kc, int nk, bool has_kt, bool has_vt) {
  using Sh = FwdShape<D, T>;
#pragma unroll
  for (int u = 0; u < Sh::kPerThread; ++u) {
    const int it = threadIdx.x + u * 256;
    if (Sh::kItems % 256 == 0 || it < Sh::kItems) {
      const int r = it / Sh::C4;
      const bool ok = kc + r < nk;
      const int so = r * Sh::LD + (it % Sh::C4) * 4;
      put4(Ks + so, ck[u], ok);
      put4(Ks + Sh::kTileFloats + so, cv[u], ok);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        put4(Ks + (2 + t) * Sh::kTileFloats + so, ckt[t][u], ok && has_kt);
        put4(Ks + (2 + T + t) * Sh::kTileFloats + so, cvt[t][u], ok && has_vt);
      }
    }
  }
}

// MULTI: N > KC, so keys arrive in several chunks (register prefetch of the next chunk,
// online rescaling between chunks); otherwise the single chunk holds every key.
// GATED (fp32, no given lse): the grid runs over head pairs; a workgroup computes the gate
// head h0 and then the value head h0 + H/2 of the same query block in two passes, keeping
// sigma(g) and sigma'(g) gdot of its rows in registers between them, and writes only the
// collapse y = sigma(g) v and ydot = sigma'(g) gdot v + sigma(g) vdot ([B, N, H/2, D]).
template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S, bool MULTI, bool GATED>
__global__ void __launch_bounds__(256, ((D == 64 && T > 0) || (D == 32 && T == 2) || (GATED && D >= 32)) ? 2 : 3)
    mhsea_fwd_kernel(const FwdParams p) {
  static_assert(!GATED || (!GIVEN_LSE && std::is_same<S, F32>::value), "the gated collapse is float32, no given lse");
  using Sh = FwdShape<D, T>;
  constexpr int KC = Sh::KC, LD = Sh::LD, DG = Sh::DG, DT = Sh::DT, C4 = Sh::C4, TT = Sh::TT;
  constexpr int NJT = KC / 16;  // 16-key tiles per chunk

  extern __shared__ float4 smem4[];
  float* const Ks = reinterpret_cast<float*>(smem4);
  float* const Vs = Ks + Sh::kTileFloats;
  float* const Kts = Vs + Sh::kTileFloats;
  float* const Vts = Kts + T * Sh::kTileFloats;
  int* const scratch = reinterpret_cast<int*>(Ks + Sh::NT * Sh::kTileFloats);
  const int n16 = (p.N + 15) & ~15;
  uint8_t* const mask_s = reinterpret_cast<uint8_t*>(scratch + 4);
  int16_t* const idx = reinterpret_cast<int16_t*>(mask_s + n16);

  const int N = p.N, H = p.H;
  const int HG = GATED ? H / 2 : H;  // heads of the grid (head pairs when gated)
  const int nblk = (N + 63) >> 6;
  const int64_t nwg = static_cast<int64_t>(p.B) * HG * nblk;
  const int64_t lb = xcd_logical_block(blockIdx.x, nwg);
  const int blk = static_cast<int>(lb % nblk);
  const int h0 = static_cast<int>((lb / nblk) % HG);
  const int b = static_cast<int>(lb / (static_cast<int64_t>(nblk) * HG));

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;

  const int n_phys = compact_mask_lds(p.mask + static_cast<int64_t>(b) * N, N, idx, mask_s, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;

  // A null tangent pointer is replaced by its primal (always readable); the values are
  // discarded when written to LDS / registers.
  const bool has_kt = p.kt != nullptr, has_vt = p.vt != nullptr, has_qt = p.qt != nullptr;
  const void* const ktp = has_kt ? p.kt : p.k;
  const void* const vtp = has_vt ? p.vt : p.v;
  const void* const qtp = has_qt ? p.qt : p.q;
  const int64_t kts = has_kt ? p.t_stride : 0, vts = has_vt ? p.t_stride : 0;
  const int64_t qts = has_qt ? p.t_stride : 0;

  const int q0 = blk * 64 + wave * 16;
  const bool active = q0 < nq;  // wave-uniform
  const bool qvalid = q0 + c < nq;
  const int qsite = qvalid ? (p.key_mask ? (q0 + c) : idx[q0 + c]) : -1;
  const int qload = qvalid ? qsite : 0;
  const float qscale = qvalid ? p.scale : 0.f;
  const float qtscale = has_qt ? qscale : 0.f;
  constexpr int NPT = Sh::kPerThread;
  float gs[DT][4], gd[TT][DT][4];  // gated: sigma(g), sigma'(g) gdot[t] of this lane's row

#pragma unroll 1
  for (int pass = 0; pass < (GATED ? 2 : 1); ++pass) {
  const int h = h0 + pass * HG;  // gated: the gate head, then the value head
  if (pass > 0) __syncthreads();  // every wave is done with the gate head's last chunk

  // ---- issue every global load of the prologue before the first wait ---------------
  float4 ck[NPT], cv[NPT], ckt[TT][NPT], cvt[TT][NPT];
  chunk_load<D, T, S, NPT, TT>(ck, cv, ckt, cvt, p, b, h, 0, nk, key_all, idx, ktp, kts, vtp, vts);

  // Query fragment in B-operand layout: lane (g, c) holds q[qsite][g*DG .. g*DG+DG).
  float qf[DG];
  float qtf[TT][DG];
  float lse2 = 0.f;
  const int64_t qoff = bnhd(b, qload, h, N, H, D) + g * DG;
  load_row_frag<DG, S>(p.q, qoff, qf);
#pragma unroll
  for (int t = 0; t < T; ++t) load_row_frag<DG, S>(qtp, t * qts + qoff, qtf[t]);
  if constexpr (GIVEN_LSE) lse2 = p.lse_in[(static_cast<int64_t>(b) * N + qload) * H + h] * kLog2e;
#pragma unroll
  for (int s = 0; s < DG; ++s) {
    qf[s] *= qscale;
#pragma unroll
    for (int t = 0; t < T; ++t) qtf[t][s] *= qtscale;
  }
  const int64_t e_row = static_cast<int64_t>(b) * N * N * H + static_cast<int64_t>(qload) * p.e_sq +
                        static_cast<int64_t>(h) * p.e_sh;

  v4f o[DT];
  v4f at[TT][DT];
  v4f ct[TT][DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    o[dt] = zero4();
#pragma unroll
    for (int t = 0; t < T; ++t) {
      at[t][dt] = zero4();
      ct[t][dt] = zero4();
    }
  }
  float m2 = -INFINITY;  // running max of the base-2 scores (uniform over a lane column)
  float lsum = 0.f;      // this lane's share of the softmax normaliser
  float mu[TT];
#pragma unroll
  for (int t = 0; t < T; ++t) mu[t] = 0.f;

  for (int kc = 0; kc < nk; kc += KC) {
    if (kc > 0) __syncthreads();  // every wave is done with the previous chunk
    chunk_store<D, T, NPT, TT>(ck, cv, ckt, cvt, Ks, kc, nk, has_kt, has_vt);
    __syncthreads();
    if constexpr (MULTI) {
      if (kc + KC < nk)
        chunk_load<D, T, S, NPT, TT>(ck, cv, ckt, cvt, p, b, h, kc + KC, nk, key_all, idx, ktp, kts, vtp, vts);
    }
    if (!active) continue;

    // The whole chunk at once: scores of every 16-key tile, one max, one rescale of the
    // accumulators per chunk (none for the first), then the P.V products.
    const int jn = min(KC, nk - kc);
    const int njt = (jn + 15) >> 4;
    v4f sc[NJT];
    v4f ds[TT][NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      sc[jt] = zero4();
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t][jt] = zero4();
    }
    // One tile at a time (the scheduling fences keep the next tile's LDS reads from being
    // hoisted, which would multiply the live registers).
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      if (jt < njt) {
        const float* krow = Ks + (jt * 16 + c) * LD + g * DG;
#pragma unroll
        for (int s = 0; s < DG; ++s) {
          const float kv = krow[s];
          sc[jt] = mfma16x4(kv, qf[s], sc[jt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            const float ktv = krow[(2 + t) * Sh::kTileFloats + s];
            ds[t][jt] = mfma16x4(ktv, qf[s], ds[t][jt]);
            ds[t][jt] = mfma16x4(kv, qtf[t][s], ds[t][jt]);
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
        float sv = sc[jt][r];
        if constexpr (HAS_E) {
          if (valid) {
            const int64_t eo = e_row + static_cast<int64_t>(key_all ? j : idx[j]) * p.e_sk;
            if (p.e != nullptr) sv += load1<S>(p.e, eo);
            if (p.et != nullptr) {
#pragma unroll
              for (int t = 0; t < T; ++t) ds[t][jt][r] += load1<S>(p.et, t * p.et_stride + eo);
            }
          }
        }
        sc[jt][r] = valid ? sv * kLog2e : -INFINITY;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][jt][r] = valid ? ds[t][jt][r] : 0.f;
        mx = fmaxf(mx, sc[jt][r]);
      }
    }

    // sc becomes the (unnormalised) softmax weight in place.
    if constexpr (GIVEN_LSE) {
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[jt][r] = lse_weight(sc[jt][r] - lse2);
    } else {
      // Lazy rescale: a row's base m2 only moves when the chunk maximum exceeds it by more
      // than 8 (base 2), so most chunks skip the rescale of the 4 DT (1 + 2 T) accumulators
      // (weights stay below 2^8; the first chunk sets m2, which starts at -inf).
      const float cmax = group_max(mx);
      const bool need = cmax > m2 + 8.f;
      if (__any(need)) {  // wave-uniform
        const float mnew = need ? cmax : m2;
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
      }
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sc[jt][r] = fast_exp2(sc[jt][r] - m2);
          lsum += sc[jt][r];
        }
    }
    // ds becomes P o dS in place.
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) {
        ds[t][jt] *= sc[jt];
        mu[t] += (ds[t][jt][0] + ds[t][jt][1]) + (ds[t][jt][2] + ds[t][jt][3]);
      }

    // ---- O^T += V^T P^T ;  A^T += V^T (P o dS)^T ;  C^T += Vt^T P^T ------------------
    // Per 4-key step, every V (and Vt) operand of the step is read before its products, so
    // the LDS latency is paid once per step rather than once per product pair.
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      if (jt < njt) {
        // contraction step r takes keys r, r + 4, r + 8, r + 12 of the tile: in a partial
        // last tile the steps from its key count on hold padding only (weight 0) and are skipped
        const int jrem = jn - jt * 16;  // wave-uniform
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r > 0 && r >= jrem) break;
          const int row = jt * 16 + 4 * g + r;
          float va[DT], vta[TT][DT];
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = dt * 16 + c;
            va[dt] = (D % 16 == 0 || col < D) ? Vs[row * LD + col] : 0.f;
#pragma unroll
            for (int t = 0; t < T; ++t)
              vta[t][dt] = (D % 16 == 0 || col < D) ? Vts[t * Sh::kTileFloats + row * LD + col] : 0.f;
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            if constexpr (!GIVEN_LSE) o[dt] = mfma16x4(va[dt], sc[jt][r], o[dt]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
              at[t][dt] = mfma16x4(va[dt], ds[t][jt][r], at[t][dt]);
              ct[t][dt] = mfma16x4(vta[t][dt], sc[jt][r], ct[t][dt]);
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if (active) {
    float inv = 1.f;
    float l2tot = 0.f;
    if constexpr (!GIVEN_LSE) {
      l2tot = group_sum(lsum);
      inv = 1.f / l2tot;
    }
    float mut[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) mut[t] = group_sum(mu[t]) * inv;
    if (GATED && qvalid) {
      const int64_t ybase = (static_cast<int64_t>(b) * N + qsite) * HG * D + static_cast<int64_t>(h0) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        if (D % 16 != 0 && d0 >= D) continue;
        float ov[4], tv[TT][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ov[r] = o[dt][r] * inv;
#pragma unroll
          for (int t = 0; t < T; ++t) tv[t][r] = (at[t][dt][r] + ct[t][dt][r]) * inv - mut[t] * ov[r];
        }
        if (pass == 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float sg = __builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * ov[r]));
            gs[dt][r] = sg;
#pragma unroll
            for (int t = 0; t < T; ++t) gd[t][dt][r] = sg * (1.f - sg) * tv[t][r];
          }
        } else {
          store4<F32>(p.out, ybase + d0, gs[dt][0] * ov[0], gs[dt][1] * ov[1], gs[dt][2] * ov[2], gs[dt][3] * ov[3]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            float yd[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) yd[r] = gd[t][dt][r] * ov[r] + gs[dt][r] * tv[t][r];
            store4<F32>(p.tout, t * p.y_tstride + ybase + d0, yd[0], yd[1], yd[2], yd[3]);
          }
        }
      }
    } else if (qvalid) {
      const int64_t obase = bnhd(b, qsite, h, N, H, D);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        if (D % 16 != 0 && d0 >= D) continue;
        float o4[4];
        if constexpr (!GIVEN_LSE) {
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] = o[dt][r] * inv;
          store4<S>(p.out, obase + d0, o4[0], o4[1], o4[2], o4[3]);
        } else {
          const float4 x = load4<S>(p.out_in, obase + d0);
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
          store4<S>(p.tout, t * p.t_stride + obase + d0, tv[0], tv[1], tv[2], tv[3]);
        }
      }
      if constexpr (!GIVEN_LSE) {
        if (g == 0 && p.lse != nullptr)
          p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] = (m2 + log2f(l2tot)) * kLn2;
      }
    }
  }
  }  // pass

  // Rows of masked queries (square mask only) are exact zeros; lse takes the value the
  // reference's all -1e4 row produces, -1e4 + log(N). Decided from the LDS copy of the
  // mask, after the compute so these stores never delay a load.
  if (GATED && !p.key_mask) {
    const int r0 = blk * 64;
    for (int it = tid; it < 64 * C4; it += 256) {
      const int r = r0 + it / C4;
      const int c4 = it % C4;
      if (r < N && mask_s[r] == 0) {
        const int64_t off = (static_cast<int64_t>(b) * N + r) * HG * D + static_cast<int64_t>(h0) * D + c4 * 4;
        store4<F32>(p.out, off, 0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < T; ++t) store4<F32>(p.tout, t * p.y_tstride + off, 0.f, 0.f, 0.f, 0.f);
      }
    }
  } else if (!p.key_mask) {
    const int h = h0;
    const int r0 = blk * 64;
    for (int it = tid; it < 64 * C4; it += 256) {
      const int r = r0 + it / C4;
      const int c4 = it % C4;
      if (r < N && mask_s[r] == 0) {
        const int64_t off = bnhd(b, r, h, N, H, D) + c4 * 4;
        if constexpr (!GIVEN_LSE) store4<S>(p.out, off, 0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < T; ++t) store4<S>(p.tout, t * p.t_stride + off, 0.f, 0.f, 0.f, 0.f);
        if (!GIVEN_LSE && c4 == 0 && p.lse != nullptr)
          p.lse[(static_cast<int64_t>(b) * N + r) * H + h] = p.masked_lse;
      }
    }
  }
}

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S, bool GATED = false>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const int nblk = (p.N + 63) / 64;
  const int64_t nwg = static_cast<int64_t>(p.B) * (GATED ? p.H / 2 : p.H) * nblk;
  const size_t lds = FwdShape<D, T>::lds_bytes(p.N);
  auto kern = p.N > FwdShape<D, T>::KC ? mhsea_fwd_kernel<D, T, GIVEN_LSE, HAS_E, S, true, GATED>
                                       : mhsea_fwd_kernel<D, T, GIVEN_LSE, HAS_E, S, false, GATED>;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(256), lds, stream, p);
  return hipGetLastError();
}

template <int D, int T, bool GIVEN_LSE, class S>
hipError_t dispatch_e(const FwdParams& p, hipStream_t stream) {
  if (p.e != nullptr) return launch_fwd_t<D, T, GIVEN_LSE, true, S>(p, stream);
  return launch_fwd_t<D, T, GIVEN_LSE, false, S>(p, stream);
}

template <int D, class S>
hipError_t dispatch_t(const FwdParams& p, int T, bool given_lse, hipStream_t stream) {
  if (given_lse) {
    if (T == 1) return dispatch_e<D, 1, true, S>(p, stream);
    if (T == 2) return dispatch_e<D, 2, true, S>(p, stream);
    return hipErrorInvalidValue;
  }
  if (T == 0) return dispatch_e<D, 0, false, S>(p, stream);
  if (T == 1) return dispatch_e<D, 1, false, S>(p, stream);
  if (T == 2) return dispatch_e<D, 2, false, S>(p, stream);
  return hipErrorInvalidValue;
}

template <int D>
hipError_t dispatch_gated(const FwdParams& p, int T, hipStream_t stream) {
  const bool e = p.e != nullptr;
  if (T == 0) return e ? launch_fwd_t<D, 0, false, true, F32, true>(p, stream) : launch_fwd_t<D, 0, false, false, F32, true>(p, stream);
  if (T == 1) return e ? launch_fwd_t<D, 1, false, true, F32, true>(p, stream) : launch_fwd_t<D, 1, false, false, F32, true>(p, stream);
  if constexpr (D < 32) {  // two directions per launch only where their gate terms fit the registers
    if (T == 2) return e ? launch_fwd_t<D, 2, false, true, F32, true>(p, stream) : launch_fwd_t<D, 2, false, false, F32, true>(p, stream);
  }
  return hipErrorInvalidValue;
}

template <class S>
hipError_t dispatch_d(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream) {
  switch (D) {
    case 8: return dispatch_t<8, S>(p, T, given_lse, stream);
    case 16: return dispatch_t<16, S>(p, T, given_lse, stream);
    case 32: return dispatch_t<32, S>(p, T, given_lse, stream);
    case 64: return dispatch_t<64, S>(p, T, given_lse, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t device_cu_count(int* cus) {
  // per-device cache; relaxed atomics keep concurrent calls from several host threads free
  // of data races (every writer stores the same value)
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices] = {};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *cus = c;
      return hipSuccess;
    }
  }
  int n = 0;
  err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (err != hipSuccess) return err;
  if (dev >= 0 && dev < kMaxDevices) cached[dev].store(n, std::memory_order_relaxed);
  *cus = n;
  return hipSuccess;
}

hipError_t launch_fwd_gated_generic(const FwdParams& p, int D, int T, hipStream_t stream) {
  switch (D) {
    case 8: return dispatch_gated<8>(p, T, stream);
    case 16: return dispatch_gated<16>(p, T, stream);
    case 32: return dispatch_gated<32>(p, T, stream);
    case 64: return dispatch_gated<64>(p, T, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                      hipStream_t stream) {
  if (p.e_compact)  // the compacted bias layout is read by the producer/consumer kernel only
    return pc_fwd_supported(p.N, p.H, D, T, dtype) ? launch_fwd_pc(p, D, T, given_lse, stream) : hipErrorInvalidValue;
  if (!p.force_generic) {
    if (dtype == 1 && bf16_ws_fwd_supported(p, D, given_lse)) return launch_fwd_bf16_ws(p, T, stream);
    if (dtype == 1 && bf16_large_fwd_supported(p.N, D)) return launch_fwd_bf16_large(p, D, T, given_lse, stream);
    if (dtype == 1 && bf16_fwd_supported(D)) return launch_fwd_bf16(p, D, T, given_lse, stream);
    if (small_fwd_supported(p.N, D, T)) return launch_fwd_small(p, D, T, given_lse, dtype, stream);
    if (pc_fwd_supported(p.N, p.H, D, T, dtype)) return launch_fwd_pc(p, D, T, given_lse, stream);
    if (stream_fwd_supported(p.N, D, T, dtype)) return launch_fwd_stream(p, D, T, given_lse, dtype, stream);
  }
  if (dtype == 1) return dispatch_d<BF16>(p, D, T, given_lse, stream);
  return dispatch_d<F32>(p, D, T, given_lse, stream);
}

}  // namespace hz
