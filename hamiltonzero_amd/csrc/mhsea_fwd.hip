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
  static constexpr int NT = 2 + 2 * T;      // staged tensors: K, V, Kt[T], Vt[T]
  static constexpr int kTileFloats = KC * LD;
  static size_t lds_bytes(int N) {
    return static_cast<size_t>(NT) * kTileFloats * 4 + 8 * 4 + ((static_cast<size_t>(N) * 2 + 15) & ~size_t(15));
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

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S>
__global__ void __launch_bounds__(256) mhsea_fwd_kernel(const FwdParams p) {
  using Sh = FwdShape<D, T>;
  constexpr int KC = Sh::KC, LD = Sh::LD, DG = Sh::DG, DT = Sh::DT;
  constexpr int C4 = D / 4;

  extern __shared__ float4 smem4[];
  float* const Ks = reinterpret_cast<float*>(smem4);
  float* const Vs = Ks + Sh::kTileFloats;
  float* const Kts = Vs + Sh::kTileFloats;
  float* const Vts = Kts + T * Sh::kTileFloats;
  int* const scratch = reinterpret_cast<int*>(Ks + Sh::NT * Sh::kTileFloats);
  int16_t* const idx = reinterpret_cast<int16_t*>(scratch + 8);

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

  const uint8_t* mrow = p.mask + static_cast<int64_t>(b) * N;
  const int n_phys = compact_mask(mrow, N, idx, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;

  // Rows of masked queries (square mask only) are exact zeros; lse takes the value the
  // reference's all -1e4 row produces, -1e4 + log(N).
  if (!p.key_mask) {
    const int r0 = blk * 64;
    for (int it = tid; it < 64 * C4; it += 256) {
      const int r = r0 + it / C4;
      const int c4 = it % C4;
      if (r < N && mrow[r] == 0) {
        const int64_t off = bnhd(b, r, h, N, H, D) + c4 * 4;
        if constexpr (!GIVEN_LSE) store4<S>(p.out, off, 0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < T; ++t) store4<S>(p.tout, t * p.t_stride + off, 0.f, 0.f, 0.f, 0.f);
        if (!GIVEN_LSE && c4 == 0 && p.lse != nullptr)
          p.lse[(static_cast<int64_t>(b) * N + r) * H + h] = p.masked_lse;
      }
    }
  }

  const int q0 = blk * 64 + wave * 16;
  const bool active = q0 < nq;  // wave-uniform
  int qsite = -1;
  if (q0 + c < nq) qsite = p.key_mask ? (q0 + c) : idx[q0 + c];

  // Query fragment in B-operand layout: lane (g, c) holds q[qsite][g*DG .. g*DG+DG).
  float qf[DG];
  float qtf[T > 0 ? T : 1][DG];
  float lse2 = 0.f;
#pragma unroll
  for (int s = 0; s < DG; ++s) qf[s] = 0.f;
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int s = 0; s < DG; ++s) qtf[t][s] = 0.f;
  if (qsite >= 0) {
    const int64_t off = bnhd(b, qsite, h, N, H, D) + g * DG;
    load_row_frag<DG, S>(p.q, off, qf);
#pragma unroll
    for (int s = 0; s < DG; ++s) qf[s] *= p.scale;
    if (p.qt != nullptr) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        load_row_frag<DG, S>(p.qt, t * p.t_stride + off, qtf[t]);
#pragma unroll
        for (int s = 0; s < DG; ++s) qtf[t][s] *= p.scale;
      }
    }
    if constexpr (GIVEN_LSE) lse2 = p.lse_in[(static_cast<int64_t>(b) * N + qsite) * H + h] * kLog2e;
  }
  const int64_t e_row = static_cast<int64_t>(b) * N * N * H +
                        static_cast<int64_t>(qsite < 0 ? 0 : qsite) * p.e_sq +
                        static_cast<int64_t>(h) * p.e_sh;

  v4f o[DT];
  v4f at[T > 0 ? T : 1][DT];
  v4f ct[T > 0 ? T : 1][DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    o[dt] = zero4();
#pragma unroll
    for (int t = 0; t < T; ++t) {
      at[t][dt] = zero4();
      ct[t][dt] = zero4();
    }
  }
  float m2 = -INFINITY;  // running max of the base-2 scores
  float lsum = 0.f;      // this lane's share of the softmax normaliser
  float mu[T > 0 ? T : 1];
#pragma unroll
  for (int t = 0; t < T; ++t) mu[t] = 0.f;

  for (int kc = 0; kc < nk; kc += KC) {
    __syncthreads();  // previous chunk fully consumed
    for (int it = tid; it < KC * C4; it += 256) {
      const int r = it / C4;
      const int c4 = it % C4;
      const int j = kc + r;
      float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
      float4 ktx[T > 0 ? T : 1], vtx[T > 0 ? T : 1];
#pragma unroll
      for (int t = 0; t < T; ++t) ktx[t] = vtx[t] = kx;
      if (j < nk) {
        const int n = key_all ? j : idx[j];
        const int64_t off = bnhd(b, n, h, N, H, D) + c4 * 4;
        kx = load4<S>(p.k, off);
        vx = load4<S>(p.v, off);
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (p.kt != nullptr) ktx[t] = load4<S>(p.kt, t * p.t_stride + off);
          if (p.vt != nullptr) vtx[t] = load4<S>(p.vt, t * p.t_stride + off);
        }
      }
      const int so = r * LD + c4 * 4;
      *reinterpret_cast<float4*>(Ks + so) = kx;
      *reinterpret_cast<float4*>(Vs + so) = vx;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        *reinterpret_cast<float4*>(Kts + t * Sh::kTileFloats + so) = ktx[t];
        *reinterpret_cast<float4*>(Vts + t * Sh::kTileFloats + so) = vtx[t];
      }
    }
    __syncthreads();
    if (!active) continue;

    const int jn = min(KC, nk - kc);
    for (int jt = 0; jt * 16 < jn; ++jt) {
      // ---- scores S^T[key 4g+r][query c] and their tangents -------------------------
      const float* krow = Ks + (jt * 16 + c) * LD + g * DG;
      v4f sc = zero4();
#pragma unroll
      for (int s = 0; s < DG; ++s) sc = mfma16x4(krow[s], qf[s], sc);
      v4f ds[T > 0 ? T : 1];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float* ktrow = Kts + t * Sh::kTileFloats + (jt * 16 + c) * LD + g * DG;
        ds[t] = zero4();
#pragma unroll
        for (int s = 0; s < DG; ++s) {
          ds[t] = mfma16x4(ktrow[s], qf[s], ds[t]);
          ds[t] = mfma16x4(krow[s], qtf[t][s], ds[t]);
        }
      }

      float s2[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = kc + jt * 16 + 4 * g + r;
        const bool valid = j < nk;
        float sv = sc[r];
        if (HAS_E || p.et != nullptr) {
          if (valid && qsite >= 0) {
            const int n = key_all ? j : idx[j];
            const int64_t eo = e_row + static_cast<int64_t>(n) * p.e_sk;
            if constexpr (HAS_E) sv += load1<S>(p.e, eo);
            if (p.et != nullptr) {
#pragma unroll
              for (int t = 0; t < T; ++t) ds[t][r] += load1<S>(p.et, t * p.et_stride + eo);
            }
          }
        }
        s2[r] = valid ? sv * kLog2e : -INFINITY;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][r] = valid ? ds[t][r] : 0.f;
      }

      // ---- softmax weights --------------------------------------------------------
      float pr[4];
      if constexpr (GIVEN_LSE) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = exp2f(s2[r] - lse2);
      } else {
        const float mx = group_max(fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3])));
        const float mnew = fmaxf(m2, mx);
        const float alpha = exp2f(m2 - mnew);
        m2 = mnew;
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = exp2f(s2[r] - mnew);
        lsum = lsum * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
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
      float pds[T > 0 ? T : 1][4];
#pragma unroll
      for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pds[t][r] = pr[r] * ds[t][r];
        mu[t] += (pds[t][0] + pds[t][1]) + (pds[t][2] + pds[t][3]);
      }

      // ---- O^T += V^T P^T ;  A^T += V^T (P o dS)^T ;  C^T += Vt^T P^T ----------------
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int col = dt * 16 + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = jt * 16 + 4 * g + r;
          const float va = (D % 16 == 0 || col < D) ? Vs[row * LD + col] : 0.f;
          if constexpr (!GIVEN_LSE) o[dt] = mfma16x4(va, pr[r], o[dt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            at[t][dt] = mfma16x4(va, pds[t][r], at[t][dt]);
            const float vta =
                (D % 16 == 0 || col < D) ? Vts[t * Sh::kTileFloats + row * LD + col] : 0.f;
            ct[t][dt] = mfma16x4(vta, pr[r], ct[t][dt]);
          }
        }
      }
    }
  }

  if (!active) return;
  float inv = 1.f;
  float l2tot = 0.f;
  if constexpr (!GIVEN_LSE) {
    l2tot = group_sum(lsum);
    inv = 1.f / l2tot;
  }
  float mut[T > 0 ? T : 1];
#pragma unroll
  for (int t = 0; t < T; ++t) mut[t] = group_sum(mu[t]) * inv;
  if (qsite < 0) return;

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

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S>
hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  const int nblk = (p.N + 63) / 64;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = FwdShape<D, T>::lds_bytes(p.N);
  auto kern = mhsea_fwd_kernel<D, T, GIVEN_LSE, HAS_E, S>;
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

hipError_t launch_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                      hipStream_t stream) {
  if (dtype == 1) return dispatch_d<BF16>(p, D, T, given_lse, stream);
  return dispatch_d<F32>(p, D, T, given_lse, stream);
}

}  // namespace hz
