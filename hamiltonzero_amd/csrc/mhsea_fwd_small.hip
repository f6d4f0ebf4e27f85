// Register-resident forward / forward+tangent / tangent-only MHSEA kernel for N <= 64.
//
// One wave owns one (walker b, head h); the four waves of a workgroup are independent
// (no LDS, no barriers). The walker's mask (at most 64 sites) is compacted with one
// ballot and one ds_permute into a lane-resident permutation "perm": lane j holds the
// j-th physical site for j < n_phys, then the masked sites. Every key operand of the
// (walker, head) — K and Kt in the A-operand layout of S^T = K Q^T, V and Vt in the
// A-operand layout of O^T = V^T P^T — is loaded once into registers; the wave then
// sweeps its query tiles of 16 rows. With all keys resident the softmax is exact (no
// online rescaling): P = exp(S - max) / sum, as in the reference kernel (mhsea.py:26-28).
//
// Matrix-core layout (v_mfma_f32_16x16x4_f32), lane = 16 g + c:
//   S^T[key 16kt + 4g + r][query c]   = sum_s K[16kt + c][g DG + s] * Q[c][g DG + s]
//   O^T[d 16dt + 4g + r'][query c]   += sum_r V[16kt + 4g + r][16dt + c] * P[c][16kt + 4g + r]
// so the C layout of S^T is directly the B operand of the P.V products.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

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

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S, int NKT>
__global__ void __launch_bounds__(256, 2) mhsea_fwd_small_kernel(const FwdParams p) {
  constexpr int DG = D / 4;
  constexpr int DT = (D + 15) / 16;
  constexpr int C4 = D / 4;
  constexpr int TT = T > 0 ? T : 1;

  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (wid >= static_cast<int64_t>(p.B) * p.H) return;  // wave-uniform
  const int N = p.N, H = p.H;
  const int b = static_cast<int>(wid / H);
  const int h = static_cast<int>(wid % H);

  // ---- mask compaction: perm = physical sites (ascending), then masked sites --------
  const uint8_t* mrow = p.mask + static_cast<int64_t>(b) * N;
  const bool on = lane < N && mrow[lane] != 0;
  const uint64_t bal = __ballot(on);
  const int n_phys = __popcll(bal);
  const int below = __popcll(bal & ((uint64_t(1) << lane) - 1));
  const int pos = on ? below : (lane < N ? n_phys + (lane - below) : lane);
  const int perm = __builtin_amdgcn_ds_permute(pos << 2, lane);
  const bool key_all = p.key_mask && n_phys == 0;
  const int nk = key_all ? N : n_phys;
  const int nq = p.key_mask ? N : n_phys;
  const int kperm = key_all ? lane : perm;
  const int qperm = p.key_mask ? lane : perm;
  const int nkt = (nk + 15) >> 4;

  // ---- zero rows of masked queries (square mask) ----------------------------------
  if (!p.key_mask) {
    const int nmask = N - n_phys;
    for (int base = 0; base < nmask * C4; base += 64) {
      const int it = base + lane;
      const int site = __shfl(perm, (n_phys + it / C4) & 63, 64);
      if (it < nmask * C4) {
        const int64_t off = bnhd(b, site, h, N, H, D) + (it % C4) * 4;
        if constexpr (!GIVEN_LSE) store4<S>(p.out, off, 0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < T; ++t) store4<S>(p.tout, t * p.t_stride + off, 0.f, 0.f, 0.f, 0.f);
      }
    }
    if (!GIVEN_LSE && p.lse != nullptr && lane < N && !on)
      p.lse[(static_cast<int64_t>(b) * N + lane) * H + h] = p.masked_lse;
  }

  // ---- key operands in registers --------------------------------------------------
  float fk[NKT][DG];
  float fkt[TT][NKT][DG];
  float fv[NKT][DT][4];
  float fvt[TT][NKT][DT][4];
  int ksite[HAS_E ? NKT : 1][4];  // site of key 16kt + 4g + r (-1 if padding)
  // Loads are unconditional from a clamped in-bounds row (site 0 for padding keys) and
  // padding lanes are zeroed afterwards; a null tangent pointer is replaced by its
  // primal (always readable) and the loaded values discarded. No per-lane branches.
  const bool has_kt = p.kt != nullptr, has_vt = p.vt != nullptr;
  const void* const ktp = has_kt ? p.kt : p.k;
  const void* const vtp = has_vt ? p.vt : p.v;
  const int64_t kts = has_kt ? p.t_stride : 0;
  const int64_t vts = has_vt ? p.t_stride : 0;
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) {
    const int j = kt * 16 + c;
    const bool valid = j < nk;
    const int sj = __shfl(kperm, j & 63, 64);
    const int site = valid ? sj : 0;
    const int64_t off = bnhd(b, site, h, N, H, D) + g * DG;
    load_frag<DG, S>(p.k, off, fk[kt]);
#pragma unroll
    for (int t = 0; t < T; ++t) load_frag<DG, S>(ktp, t * kts + off, fkt[t][kt]);
#pragma unroll
    for (int s = 0; s < DG; ++s) {
      fk[kt][s] = valid ? fk[kt][s] : 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t) fkt[t][kt][s] = (valid && has_kt) ? fkt[t][kt][s] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j2 = kt * 16 + 4 * g + r;
      const bool valid2 = j2 < nk;
      const int sj2 = __shfl(kperm, j2 & 63, 64);
      const int site2 = valid2 ? sj2 : 0;
      if constexpr (HAS_E) ksite[kt][r] = valid2 ? site2 : -1;
      const int64_t roff = bnhd(b, site2, h, N, H, D);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int col = (D % 16 == 0) ? dt * 16 + c : min(dt * 16 + c, D - 1);
        const bool ok = valid2 && (D % 16 == 0 || dt * 16 + c < D);
        const float x = load1<S>(p.v, roff + col);
        fv[kt][dt][r] = ok ? x : 0.f;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float y = load1<S>(vtp, t * vts + roff + col);
          fvt[t][kt][dt][r] = (ok && has_vt) ? y : 0.f;
        }
      }
    }
  }

  // ---- sweep the query tiles -------------------------------------------------------
  const int nqt = (nq + 15) >> 4;
  for (int qt = 0; qt < nqt; ++qt) {
    const int jq = qt * 16 + c;
    const int qs = __shfl(qperm, jq & 63, 64);
    const bool qvalid = jq < nq;
    const int qsite = qvalid ? qs : -1;
    const int qload = qvalid ? qs : 0;  // in-bounds row for the unconditional loads
    const float qscale = qvalid ? p.scale : 0.f;

    float qf[DG];
    float qtf[TT][DG];
    const int64_t qoff = bnhd(b, qload, h, N, H, D) + g * DG;
    load_frag<DG, S>(p.q, qoff, qf);
#pragma unroll
    for (int s = 0; s < DG; ++s) qf[s] *= qscale;
    const float qtscale = p.qt != nullptr ? qscale : 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      load_frag<DG, S>(p.qt != nullptr ? p.qt : p.q, (p.qt != nullptr ? t * p.t_stride : 0) + qoff, qtf[t]);
#pragma unroll
      for (int s = 0; s < DG; ++s) qtf[t][s] = p.qt != nullptr ? qtf[t][s] * qtscale : 0.f;
    }
    float lse2 = 0.f;
    if constexpr (GIVEN_LSE) lse2 = p.lse_in[(static_cast<int64_t>(b) * N + qload) * H + h] * kLog2e;

    // S^T and its tangents, one 16x16 tile per key tile; independent chains interleaved.
    v4f st[NKT];
    v4f ds[TT][NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      st[kt] = zero4();
#pragma unroll
      for (int t = 0; t < T; ++t) ds[t][kt] = zero4();
    }
#pragma unroll
    for (int s = 0; s < DG; ++s) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        if (kt < nkt) {
          st[kt] = mfma16x4(fk[kt][s], qf[s], st[kt]);
#pragma unroll
          for (int t = 0; t < T; ++t) {
            ds[t][kt] = mfma16x4(fkt[t][kt][s], qf[s], ds[t][kt]);
            ds[t][kt] = mfma16x4(fk[kt][s], qtf[t][s], ds[t][kt]);
          }
        }
      }
    }

    // bias, validity, base-2 scores
    const int64_t e_row = static_cast<int64_t>(b) * N * N * H +
                          static_cast<int64_t>(qsite < 0 ? 0 : qsite) * p.e_sq +
                          static_cast<int64_t>(h) * p.e_sh;
    // st becomes the base-2 score, then the softmax weight, in place.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = kt * 16 + 4 * g + r < nk;
        float sv = st[kt][r];
        if constexpr (HAS_E) {
          if (valid && qsite >= 0) {
            const int64_t eo = e_row + static_cast<int64_t>(ksite[kt][r]) * p.e_sk;
            if (p.e != nullptr) sv += load1<S>(p.e, eo);
            if (p.et != nullptr) {
#pragma unroll
              for (int t = 0; t < T; ++t) ds[t][kt][r] += load1<S>(p.et, t * p.et_stride + eo);
            }
          }
        }
        st[kt][r] = valid ? sv * kLog2e : -INFINITY;
#pragma unroll
        for (int t = 0; t < T; ++t) ds[t][kt][r] = valid ? ds[t][kt][r] : 0.f;
        mx = fmaxf(mx, st[kt][r]);
      }
    }

    // softmax weights
    float lsum = 0.f;
    if constexpr (GIVEN_LSE) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) st[kt][r] = clamp01(exp2f(st[kt][r] - lse2));
    } else {
      mx = group_max(mx);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          st[kt][r] = exp2f(st[kt][r] - mx);
          lsum += st[kt][r];
        }
      lsum = group_sum(lsum);
      const float inv = 1.f / lsum;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) st[kt] *= inv;
    }
    // ds becomes P o dS in place; mu = rowsum(P o dS)
    float mu[TT];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      mu[t] = 0.f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        ds[t][kt] *= st[kt];
        mu[t] += (ds[t][kt][0] + ds[t][kt][1]) + (ds[t][kt][2] + ds[t][kt][3]);
      }
      mu[t] = group_sum(mu[t]);
    }

    // O^T, A^T = V^T (P o dS)^T, C^T = Vt^T P^T
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
    for (int kt = 0; kt < NKT; ++kt) {
      if (kt < nkt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            if constexpr (!GIVEN_LSE) o[dt] = mfma16x4(fv[kt][dt][r], st[kt][r], o[dt]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
              at[t][dt] = mfma16x4(fv[kt][dt][r], ds[t][kt][r], at[t][dt]);
              ct[t][dt] = mfma16x4(fvt[t][kt][dt][r], st[kt][r], ct[t][dt]);
            }
          }
        }
      }
    }

    if (qsite < 0) continue;
    const int64_t obase = bnhd(b, qsite, h, N, H, D);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = dt * 16 + 4 * g;
      if (D % 16 != 0 && d0 >= D) continue;
      float o4[4];
      if constexpr (!GIVEN_LSE) {
#pragma unroll
        for (int r = 0; r < 4; ++r) o4[r] = o[dt][r];
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
        for (int r = 0; r < 4; ++r) tv[r] = at[t][dt][r] + ct[t][dt][r] - mu[t] * o4[r];
        store4<S>(p.tout, t * p.t_stride + obase + d0, tv[0], tv[1], tv[2], tv[3]);
      }
    }
    if constexpr (!GIVEN_LSE) {
      if (g == 0 && p.lse != nullptr)
        p.lse[(static_cast<int64_t>(b) * N + qsite) * H + h] = (mx + log2f(lsum)) * kLn2;
    }
  }
}

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S, int NKT>
hipError_t launch_small_t(const FwdParams& p, hipStream_t stream) {
  const int64_t waves = static_cast<int64_t>(p.B) * p.H;
  const int64_t nwg = (waves + 3) / 4;
  hipLaunchKernelGGL((mhsea_fwd_small_kernel<D, T, GIVEN_LSE, HAS_E, S, NKT>),
                     dim3(static_cast<unsigned>(nwg)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int D, int T, bool GIVEN_LSE, bool HAS_E, class S>
hipError_t dispatch_nkt(const FwdParams& p, hipStream_t stream) {
  const int nkt = (p.N + 15) / 16;
  if constexpr (SmallFits<D, T>::kMaxKeyTiles >= 1) {
    if (nkt == 1) return launch_small_t<D, T, GIVEN_LSE, HAS_E, S, 1>(p, stream);
  }
  if constexpr (SmallFits<D, T>::kMaxKeyTiles >= 2) {
    if (nkt == 2) return launch_small_t<D, T, GIVEN_LSE, HAS_E, S, 2>(p, stream);
  }
  // small_fwd_supported admits N <= 32, i.e. at most two key tiles; wider instantiations
  // would be unreachable (and do not fit the register budget without spilling).
  return hipErrorInvalidValue;
}

template <int D, int T, bool GIVEN_LSE, class S>
hipError_t dispatch_e(const FwdParams& p, hipStream_t stream) {
  if (p.e != nullptr || p.et != nullptr) return dispatch_nkt<D, T, GIVEN_LSE, true, S>(p, stream);
  return dispatch_nkt<D, T, GIVEN_LSE, false, S>(p, stream);
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

bool small_fwd_supported(int N, int D, int T) {
  // Above 32 sites the resident key operands leave too few registers for two waves per
  // SIMD; the LDS-streaming kernel serves those shapes.
  if (N > 32) return false;
  const int nkt = (N + 15) / 16;
  return nkt <= small_max_key_tiles(D, T);
}

hipError_t launch_fwd_small(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                            hipStream_t stream) {
  if (dtype == 1) return dispatch_d<BF16>(p, D, T, given_lse, stream);
  return dispatch_d<F32>(p, D, T, given_lse, stream);
}

}  // namespace hz
