// Reverse-mode (VJP) MHSEA kernels for gfx950.
//
// Cotangent algebra (custom_gradients.py:249-285 and :307-347), per walker and head, over
// valid (query i, key j) pairs:
//   P_ij    = exp(S_ij - lse_i),        S = scale Q K^T + E
//   dP_ij   = dout_i . v_j
//   delta_i = out_i . dout_i            (sum_columns(o * o_vjp))
//   dS_ij   = P_ij (dP_ij - delta_i)
//   dq_i = scale sum_j dS_ij k_j,  dk_j = scale sum_i dS_ij q_i,  dv_j = sum_i P_ij dout_i,
//   de_ij = dS_ij.
// Two kernels, as the dq-side and dk/dv-side reductions run over different indices and
// the library stays free of atomics (deterministic):
//  * mhsea_bwd_q_kernel: workgroup = (walker, head, 64 compacted queries); each wave owns
//    16 queries in the transposed orientation S^T = K Q^T (query = lane % 16), streams
//    key chunks through LDS and accumulates dq^T = K^T dS^T; writes de.
//  * mhsea_bwd_kv_kernel: workgroup = (walker, head, 64 compacted keys); each wave owns
//    16 keys in the orientation S = Q K^T (key = lane % 16), streams query chunks (q,
//    dout, lse, delta) through LDS and accumulates dv^T = dout^T P and dk^T = Q^T dS.
// Both take queries and keys from the compacted list of physical sites, like the
// forward; rows of masked sites are written as exact zeros.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

template <int D>
struct BwdShape {
  static constexpr int KC = 64;  // rows per LDS chunk
  static constexpr int LD = D + 4;
  static constexpr int DG = D / 4;
  static constexpr int DT = (D + 15) / 16;
  static constexpr int kTileFloats = KC * LD;
  static size_t lds_bytes(int N) {
    // two row tiles + two per-row vectors + scratch + compacted index list
    return static_cast<size_t>(2 * kTileFloats + 2 * KC) * 4 + 8 * 4 +
           ((static_cast<size_t>(N) * 2 + 15) & ~size_t(15));
  }
};

template <int DG, class S>
__device__ __forceinline__ void load_frag(const void* base, int64_t off, float* dst) {
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

__device__ __forceinline__ void decode_block(const BwdParams& p, int& b, int& h, int& blk) {
  const int nblk = (p.N + 63) >> 6;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const int64_t lb = xcd_logical_block(blockIdx.x, nwg);
  blk = static_cast<int>(lb % nblk);
  h = static_cast<int>((lb / nblk) % p.H);
  b = static_cast<int>(lb / (static_cast<int64_t>(nblk) * p.H));
}

// ------------------------------------------------------------------------------------
// dq and de
// ------------------------------------------------------------------------------------
template <int D, bool HAS_E, class S>
__global__ void __launch_bounds__(256) mhsea_bwd_q_kernel(const BwdParams p) {
  using Sh = BwdShape<D>;
  constexpr int KC = Sh::KC, LD = Sh::LD, DG = Sh::DG, DT = Sh::DT;
  constexpr int C4 = D / 4;

  extern __shared__ float4 smem4[];
  float* const Ks = reinterpret_cast<float*>(smem4);
  float* const Vs = Ks + Sh::kTileFloats;
  int* const scratch = reinterpret_cast<int*>(Vs + Sh::kTileFloats + 2 * KC);
  int16_t* const idx = reinterpret_cast<int16_t*>(scratch + 8);

  const int N = p.N, H = p.H;
  int b, h, blk;
  decode_block(p, b, h, blk);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;

  const uint8_t* mrow = p.mask + static_cast<int64_t>(b) * N;
  const int n_phys = compact_mask(mrow, N, idx, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int64_t e_walker = static_cast<int64_t>(b) * N * N * H + static_cast<int64_t>(h) * p.e_sh;

  // Zeros: dq rows of masked queries; de at every invalid (query, key) pair of the
  // workgroup's own 64 original query rows.
  {
    const int r0 = blk * 64;
    if (!p.key_mask) {
      for (int it = tid; it < 64 * C4; it += 256) {
        const int r = r0 + it / C4;
        if (r < N && mrow[r] == 0)
          store4<S>(p.dq, bnhd(b, r, h, N, H, D) + (it % C4) * 4, 0.f, 0.f, 0.f, 0.f);
      }
    }
    if (p.de != nullptr) {
      const int rows = min(64, N - r0);
      for (int it = tid; it < rows * N; it += 256) {
        const int r = r0 + it / N;
        const int j = it % N;
        const bool valid = key_all || ((p.key_mask || mrow[r] != 0) && mrow[j] != 0);
        if (!valid) store1<S>(p.de, e_walker + static_cast<int64_t>(r) * p.e_sq + j * p.e_sk, 0.f);
      }
    }
  }

  const int q0 = blk * 64 + wave * 16;
  const bool active = q0 < nq;
  int qsite = -1;
  if (q0 + c < nq) qsite = p.key_mask ? (q0 + c) : idx[q0 + c];

  float qf[DG], gf[DG];
  float delta = 0.f, lse2 = 0.f;
#pragma unroll
  for (int s = 0; s < DG; ++s) qf[s] = gf[s] = 0.f;
  if (qsite >= 0) {
    const int64_t off = bnhd(b, qsite, h, N, H, D) + g * DG;
    float of[DG];
    load_frag<DG, S>(p.q, off, qf);
    load_frag<DG, S>(p.dout, off, gf);
    load_frag<DG, S>(p.out, off, of);
#pragma unroll
    for (int s = 0; s < DG; ++s) {
      qf[s] *= p.scale;
      delta += of[s] * gf[s];
    }
    lse2 = p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] * kLog2e;
  }
  delta = group_sum(delta);  // all lanes of the wave take part
  const int64_t e_row = e_walker + static_cast<int64_t>(qsite < 0 ? 0 : qsite) * p.e_sq;

  v4f dqa[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqa[dt] = zero4();

  for (int kc = 0; kc < nk; kc += KC) {
    __syncthreads();
    for (int it = tid; it < KC * C4; it += 256) {
      const int r = it / C4, c4 = it % C4, j = kc + r;
      float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
      if (j < nk) {
        const int n = key_all ? j : idx[j];
        const int64_t off = bnhd(b, n, h, N, H, D) + c4 * 4;
        kx = load4<S>(p.k, off);
        vx = load4<S>(p.v, off);
      }
      *reinterpret_cast<float4*>(Ks + r * LD + c4 * 4) = kx;
      *reinterpret_cast<float4*>(Vs + r * LD + c4 * 4) = vx;
    }
    __syncthreads();
    if (!active) continue;

    const int jn = min(KC, nk - kc);
    for (int jt = 0; jt * 16 < jn; ++jt) {
      const float* krow = Ks + (jt * 16 + c) * LD + g * DG;
      const float* vrow = Vs + (jt * 16 + c) * LD + g * DG;
      v4f sc = zero4(), dp = zero4();
#pragma unroll
      for (int s = 0; s < DG; ++s) {
        sc = mfma16x4(krow[s], qf[s], sc);  // S^T[key][query]
        dp = mfma16x4(vrow[s], gf[s], dp);  // dP^T[key][query]
      }
      float dsv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = kc + jt * 16 + 4 * g + r;
        const bool valid = (j < nk) && qsite >= 0;
        float sv = sc[r];
        int n = 0;
        if (valid) {
          n = key_all ? j : idx[j];
          if constexpr (HAS_E) sv += load1<S>(p.e, e_row + static_cast<int64_t>(n) * p.e_sk);
        }
        const float pv = valid ? clamp01(exp2f(sv * kLog2e - lse2)) : 0.f;
        dsv[r] = pv * (dp[r] - delta);
        if (valid && p.de != nullptr) store1<S>(p.de, e_row + static_cast<int64_t>(n) * p.e_sk, dsv[r]);
      }
      // dq^T[d][query] += K^T[d][key] dS^T[key][query]
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int col = dt * 16 + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = jt * 16 + 4 * g + r;
          const float ka = (D % 16 == 0 || col < D) ? Ks[row * LD + col] : 0.f;
          dqa[dt] = mfma16x4(ka, dsv[r], dqa[dt]);
        }
      }
    }
  }
  if (!active || qsite < 0) return;
  const int64_t obase = bnhd(b, qsite, h, N, H, D);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d0 = dt * 16 + 4 * g;
    if (D % 16 != 0 && d0 >= D) continue;
    store4<S>(p.dq, obase + d0, dqa[dt][0] * p.scale, dqa[dt][1] * p.scale,
              dqa[dt][2] * p.scale, dqa[dt][3] * p.scale);
  }
}

// ------------------------------------------------------------------------------------
// dk and dv
// ------------------------------------------------------------------------------------
template <int D, bool HAS_E, class S>
__global__ void __launch_bounds__(256) mhsea_bwd_kv_kernel(const BwdParams p) {
  using Sh = BwdShape<D>;
  constexpr int KC = Sh::KC, LD = Sh::LD, DG = Sh::DG, DT = Sh::DT;
  constexpr int C4 = D / 4;

  extern __shared__ float4 smem4[];
  float* const Qs = reinterpret_cast<float*>(smem4);  // scale * q rows
  float* const Gs = Qs + Sh::kTileFloats;              // dout rows
  float* const L2s = Gs + Sh::kTileFloats;             // lse * log2(e), +inf for padding
  float* const Dls = L2s + KC;                         // delta
  int* const scratch = reinterpret_cast<int*>(Dls + KC);
  int16_t* const idx = reinterpret_cast<int16_t*>(scratch + 8);

  const int N = p.N, H = p.H;
  int b, h, blk;
  decode_block(p, b, h, blk);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, c = lane & 15;

  const uint8_t* mrow = p.mask + static_cast<int64_t>(b) * N;
  const int n_phys = compact_mask(mrow, N, idx, scratch);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int64_t e_walker = static_cast<int64_t>(b) * N * N * H + static_cast<int64_t>(h) * p.e_sh;

  // Zeros: dk, dv rows of masked keys among the workgroup's 64 original rows.
  if (!key_all) {
    const int r0 = blk * 64;
    for (int it = tid; it < 64 * C4; it += 256) {
      const int r = r0 + it / C4;
      if (r < N && mrow[r] == 0) {
        const int64_t off = bnhd(b, r, h, N, H, D) + (it % C4) * 4;
        store4<S>(p.dk, off, 0.f, 0.f, 0.f, 0.f);
        store4<S>(p.dv, off, 0.f, 0.f, 0.f, 0.f);
      }
    }
  }

  const int k0 = blk * 64 + wave * 16;
  const bool active = k0 < nk;
  int ksite = -1;
  if (k0 + c < nk) ksite = key_all ? (k0 + c) : idx[k0 + c];

  float kf[DG], vf[DG];
#pragma unroll
  for (int s = 0; s < DG; ++s) kf[s] = vf[s] = 0.f;
  if (ksite >= 0) {
    const int64_t off = bnhd(b, ksite, h, N, H, D) + g * DG;
    load_frag<DG, S>(p.k, off, kf);
    load_frag<DG, S>(p.v, off, vf);
  }

  v4f dka[DT], dva[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dka[dt] = dva[dt] = zero4();

  for (int qc = 0; qc < nq; qc += KC) {
    __syncthreads();
    for (int it = tid; it < KC * C4; it += 256) {
      const int r = it / C4, c4 = it % C4, i = qc + r;
      float4 qx = make_float4(0.f, 0.f, 0.f, 0.f), gx = qx, ox = qx;
      if (i < nq) {
        const int n = p.key_mask ? i : idx[i];
        const int64_t off = bnhd(b, n, h, N, H, D) + c4 * 4;
        qx = load4<S>(p.q, off);
        gx = load4<S>(p.dout, off);
        ox = load4<S>(p.out, off);
        qx.x *= p.scale;
        qx.y *= p.scale;
        qx.z *= p.scale;
        qx.w *= p.scale;
      }
      *reinterpret_cast<float4*>(Qs + r * LD + c4 * 4) = qx;
      *reinterpret_cast<float4*>(Gs + r * LD + c4 * 4) = gx;
      // delta_i: the C4 threads of one row are consecutive lanes of one wave.
      float part = (ox.x * gx.x + ox.y * gx.y) + (ox.z * gx.z + ox.w * gx.w);
#pragma unroll
      for (int w = 1; w < C4; w <<= 1) part += __shfl_xor(part, w, 64);
      if (c4 == 0) {
        Dls[r] = part;
        L2s[r] = (i < nq) ? p.lse[(static_cast<int64_t>(b) * N + (p.key_mask ? i : idx[i])) * H + h] * kLog2e
                          : INFINITY;
      }
    }
    __syncthreads();
    if (!active) continue;

    const int in_ = min(KC, nq - qc);
    for (int itile = 0; itile * 16 < in_; ++itile) {
      const float* qrow = Qs + (itile * 16 + c) * LD + g * DG;
      const float* grow = Gs + (itile * 16 + c) * LD + g * DG;
      v4f sc = zero4(), dp = zero4();
#pragma unroll
      for (int s = 0; s < DG; ++s) {
        sc = mfma16x4(qrow[s], kf[s], sc);  // S[query 4g+r][key c]
        dp = mfma16x4(grow[s], vf[s], dp);  // dP[query][key]
      }
      float pv[4], dsv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int il = itile * 16 + 4 * g + r;
        float sv = sc[r];
        const bool valid = (qc + il < nq) && ksite >= 0;
        if constexpr (HAS_E) {
          if (valid) {
            const int qn = p.key_mask ? (qc + il) : idx[qc + il];
            sv += load1<S>(p.e, e_walker + static_cast<int64_t>(qn) * p.e_sq +
                                    static_cast<int64_t>(ksite) * p.e_sk);
          }
        }
        pv[r] = valid ? clamp01(exp2f(sv * kLog2e - L2s[il])) : 0.f;
        dsv[r] = pv[r] * (dp[r] - Dls[il]);
      }
      // dv^T[d][key] += dout^T[d][query] P[query][key];  dk^T += (scale q)^T dS
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int col = dt * 16 + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = itile * 16 + 4 * g + r;
          const bool in_d = (D % 16 == 0 || col < D);
          const float ga = in_d ? Gs[row * LD + col] : 0.f;
          const float qa = in_d ? Qs[row * LD + col] : 0.f;
          dva[dt] = mfma16x4(ga, pv[r], dva[dt]);
          dka[dt] = mfma16x4(qa, dsv[r], dka[dt]);
        }
      }
    }
  }
  if (!active || ksite < 0) return;
  const int64_t obase = bnhd(b, ksite, h, N, H, D);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d0 = dt * 16 + 4 * g;
    if (D % 16 != 0 && d0 >= D) continue;
    store4<S>(p.dk, obase + d0, dka[dt][0], dka[dt][1], dka[dt][2], dka[dt][3]);
    store4<S>(p.dv, obase + d0, dva[dt][0], dva[dt][1], dva[dt][2], dva[dt][3]);
  }
}

template <class K>
hipError_t launch_with_lds(K kern, int64_t nwg, size_t lds, const BwdParams& p,
                           hipStream_t stream) {
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(256), lds, stream, p);
  return hipGetLastError();
}

template <int D, bool HAS_E, class S>
hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
  const int nblk = (p.N + 63) / 64;
  const int64_t nwg = static_cast<int64_t>(p.B) * p.H * nblk;
  const size_t lds = BwdShape<D>::lds_bytes(p.N);
  hipError_t err = launch_with_lds(mhsea_bwd_q_kernel<D, HAS_E, S>, nwg, lds, p, stream);
  if (err != hipSuccess) return err;
  return launch_with_lds(mhsea_bwd_kv_kernel<D, HAS_E, S>, nwg, lds, p, stream);
}

template <int D, class S>
hipError_t dispatch_e(const BwdParams& p, hipStream_t stream) {
  if (p.e != nullptr) return launch_bwd_t<D, true, S>(p, stream);
  return launch_bwd_t<D, false, S>(p, stream);
}

template <class S>
hipError_t dispatch_d(const BwdParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 8: return dispatch_e<8, S>(p, stream);
    case 16: return dispatch_e<16, S>(p, stream);
    case 32: return dispatch_e<32, S>(p, stream);
    case 64: return dispatch_e<64, S>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_bwd(const BwdParams& p, int D, int dtype, hipStream_t stream) {
  if (!p.force_generic) {
    if (dtype == 1 && bf16_bwd_supported(p.N, p.H, D)) return launch_bwd_bf16(p, D, stream);
    if (stream_bwd_supported(p.N)) return launch_bwd_stream(p, D, dtype, stream);
  }
  if (dtype == 1) return dispatch_d<BF16>(p, D, stream);
  return dispatch_d<F32>(p, D, stream);
}

}  // namespace hz
