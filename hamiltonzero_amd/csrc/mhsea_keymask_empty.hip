// Walkers with no physical site under the additive key mask (HZ_FLAG_KEY_MASK).
//
// reference_edge_attention adds the key penalty in float32
// (src/hamiltonzero/model/pallas_attention.py:34-35): a masked key's logit is
// fl32(s - 1e9), a multiple of 64 (the float32 spacing at 1e9). While one key of a walker
// is physical this only means that masked keys get weight exactly 0, which the main
// kernels implement by never reading masked keys. When NO key is physical, the reference's
// softmax runs over the rounded logits of every key — uniform weights whenever all
// |s| < 32 — and the main kernels' softmax over the unrounded s would differ. These
// kernels run after the main kernels of a key-mask call and rewrite the results of exactly
// those walkers:
//     s'  = fl32(fl32(s - 1e9) + 1e9)     (s rounded as the reference rounds it, shifted
//                                          back by the constant 1e9, which softmax ignores)
//     P   = softmax_j(s'),  lse = log-sum-exp_j(s')   (lse relative to that shift)
// and the tangent / cotangent formulas of the main kernels with this P. The derivative of
// the penalty is 1 under autodiff, so dS keeps its usual form.
//
// One thread per (query or key) row; a 64-thread workgroup serves one walker's block of 64
// rows and loops over the heads (over the head pairs in the gated collapse), so a launch is
// B * ceil(N / 64) workgroups whatever H is. A workgroup whose walker has a physical site
// exits at once (one pass over the walker's mask bytes), so a call without empty walkers
// costs one small launch. Plain fp32 loops: this serves a degenerate input, not a throughput path.
#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

constexpr int kRows = 64;  // rows per workgroup (one wave)
constexpr float kPenalty = 1e9f;

// fl32(fl32(s - 1e9) + 1e9). The empty asm keeps the compiler from folding the pair.
__device__ __forceinline__ float penalised(float s) {
  float t = s - kPenalty;
  asm volatile("" : "+v"(t));
  return t + kPenalty;
}

// True for every thread iff walker b has no physical site.
__device__ __forceinline__ bool walker_empty(const uint8_t* __restrict__ mask, int b, int N) {
  const uint8_t* row = mask + static_cast<int64_t>(b) * N;
  int any = 0;
  for (int j = threadIdx.x; j < N; j += kRows) any |= row[j] != 0;
  return !__syncthreads_or(any);
}

template <class S, int D>
__device__ __forceinline__ void load_row(float (&x)[D], const void* base, int64_t off) {
#pragma unroll
  for (int d = 0; d < D; ++d) x[d] = load1<S>(base, off + d);
}

template <class S, int D>
__device__ __forceinline__ float dot_row(const float (&x)[D], const void* base, int64_t off) {
  float acc = 0.f;
#pragma unroll
  for (int d = 0; d < D; ++d) acc = fmaf(x[d], load1<S>(base, off + d), acc);
  return acc;
}

struct Walker {
  int b, N, H, D;
  __device__ int64_t row(int n, int h) const { return ((static_cast<int64_t>(b) * N + n) * H + h) * D; }
};

// Logit s'_ij of query i, key j, head h (the query row qi is already in registers).
template <class S, int D>
__device__ __forceinline__ float logit(const FwdParams& p, const Walker& w, const float (&qi)[D], int i,
                                       int j, int h) {
  float s = p.scale * dot_row<S, D>(qi, p.k, w.row(j, h));
  if (p.e != nullptr) {
    const int64_t eoff = static_cast<int64_t>(w.b) * w.N * w.N * w.H + i * p.e_sq + h * p.e_sh + j * p.e_sk;
    s += load1<S>(p.e, eoff);
  }
  return penalised(s);
}

// lse of row i (natural log).
template <class S, int D>
__device__ float row_lse(const FwdParams& p, const Walker& w, const float (&qi)[D], int i, int h) {
  float m = -INFINITY;
  for (int j = 0; j < w.N; ++j) m = fmaxf(m, logit<S, D>(p, w, qi, i, j, h));
  float l = 0.f;
  for (int j = 0; j < w.N; ++j) l += expf(logit<S, D>(p, w, qi, i, j, h) - m);
  return m + logf(l);
}

// out row i = sum_j P_ij v_j.
template <class S, int D>
__device__ void row_out(const FwdParams& p, const Walker& w, const float (&qi)[D], int i, int h, float lse,
                        float (&o)[D]) {
#pragma unroll
  for (int d = 0; d < D; ++d) o[d] = 0.f;
  for (int j = 0; j < w.N; ++j) {
    const float pj = expf(logit<S, D>(p, w, qi, i, j, h) - lse);
    const int64_t vo = w.row(j, h);
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] = fmaf(pj, load1<S>(p.v, vo + d), o[d]);
  }
}

// Tangent row i of direction t: sum_j P_ij (dS_ij v_j + vt_j) - (sum_j P_ij dS_ij) out_i,
// dS_ij = scale (qt_i . k_j + q_i . kt_j) + et_ij.
template <class S, int D>
__device__ void row_tangent(const FwdParams& p, const Walker& w, const float (&qi)[D], int i, int h, int t,
                            float lse, const float (&o)[D], float (&to)[D]) {
  float qti[D];
  const int64_t tq = static_cast<int64_t>(t) * p.t_stride;
  if (p.qt != nullptr) {
    load_row<S, D>(qti, p.qt, tq + w.row(i, h));
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d) qti[d] = 0.f;
  }
#pragma unroll
  for (int d = 0; d < D; ++d) to[d] = 0.f;
  float mean = 0.f;
  for (int j = 0; j < w.N; ++j) {
    const float pj = expf(logit<S, D>(p, w, qi, i, j, h) - lse);
    const int64_t kj = w.row(j, h);
    float ds = 0.f;
    if (p.qt != nullptr) ds = dot_row<S, D>(qti, p.k, kj);
    if (p.kt != nullptr) ds += dot_row<S, D>(qi, p.kt, tq + kj);
    ds *= p.scale;
    if (p.et != nullptr) {
      const int64_t eoff = static_cast<int64_t>(t) * p.et_stride +
                           static_cast<int64_t>(w.b) * w.N * w.N * w.H + i * p.e_sq + h * p.e_sh + j * p.e_sk;
      ds += load1<S>(p.et, eoff);
    }
    const float pds = pj * ds;
    mean += pds;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      float a = pds * load1<S>(p.v, kj + d);
      if (p.vt != nullptr) a = fmaf(pj, load1<S>(p.vt, tq + kj + d), a);
      to[d] += a;
    }
  }
#pragma unroll
  for (int d = 0; d < D; ++d) to[d] = fmaf(-mean, o[d], to[d]);
}

// Forward / tangent of empty walkers. given_lse: read out_in / lse_in (the tangent-only
// call) instead of computing them. T directions, all written here.
template <class S, int D>
__global__ __launch_bounds__(kRows) void keymask_empty_fwd_kernel(FwdParams p, int T, int given_lse) {
  const int nrb = (p.N + kRows - 1) / kRows;
  const int b = blockIdx.x / nrb;
  if (!walker_empty(p.mask, b, p.N)) return;
  const int i = (blockIdx.x % nrb) * kRows + threadIdx.x;
  if (i >= p.N) return;
  const Walker w{b, p.N, p.H, D};
  for (int h = 0; h < p.H; ++h) {
    float qi[D], o[D], to[D];
    load_row<S, D>(qi, p.q, w.row(i, h));
    const int64_t lrow = (static_cast<int64_t>(b) * p.N + i) * p.H + h;
    float lse;
    if (given_lse) {
      lse = p.lse_in[lrow];
      load_row<S, D>(o, p.out_in, w.row(i, h));
    } else {
      lse = row_lse<S, D>(p, w, qi, i, h);
      row_out<S, D>(p, w, qi, i, h, lse, o);
#pragma unroll
      for (int d = 0; d < D; ++d) store1<S>(p.out, w.row(i, h) + d, o[d]);
      if (p.lse != nullptr) p.lse[lrow] = lse;
    }
    for (int t = 0; t < T; ++t) {
      row_tangent<S, D>(p, w, qi, i, h, t, lse, o, to);
      const int64_t to_off = static_cast<int64_t>(t) * p.t_stride + w.row(i, h);
#pragma unroll
      for (int d = 0; d < D; ++d) store1<S>(p.tout, to_off + d, to[d]);
    }
  }
}

// The gated head collapse of empty walkers: y = sigmoid(g) v and its tangents, g = out of
// head h, v = out of head h + H/2 (float32 only).
template <int D>
__global__ __launch_bounds__(kRows) void keymask_empty_gated_kernel(FwdParams p, int T) {
  const int nrb = (p.N + kRows - 1) / kRows;
  const int b = blockIdx.x / nrb;
  if (!walker_empty(p.mask, b, p.N)) return;
  const int i = (blockIdx.x % nrb) * kRows + threadIdx.x;
  if (i >= p.N) return;
  const Walker w{b, p.N, p.H, D};
  const int hh = p.H / 2;
  float* y = static_cast<float*>(p.out);
  float* ty = static_cast<float*>(p.tout);
  for (int h = 0; h < hh; ++h) {
    float qg[D], qv[D], og[D], ov[D], tg[D], tv[D];
    load_row<F32, D>(qg, p.q, w.row(i, h));
    load_row<F32, D>(qv, p.q, w.row(i, h + hh));
    const float lg = row_lse<F32, D>(p, w, qg, i, h);
    const float lv = row_lse<F32, D>(p, w, qv, i, h + hh);
    row_out<F32, D>(p, w, qg, i, h, lg, og);
    row_out<F32, D>(p, w, qv, i, h + hh, lv, ov);
    const int64_t yrow = ((static_cast<int64_t>(b) * p.N + i) * hh + h) * D;
#pragma unroll
    for (int d = 0; d < D; ++d) y[yrow + d] = ov[d] / (1.f + expf(-og[d]));
    for (int t = 0; t < T; ++t) {
      row_tangent<F32, D>(p, w, qg, i, h, t, lg, og, tg);
      row_tangent<F32, D>(p, w, qv, i, h + hh, t, lv, ov, tv);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const float sg = 1.f / (1.f + expf(-og[d]));
        ty[static_cast<int64_t>(t) * p.y_tstride + yrow + d] = sg * (1.f - sg) * tg[d] * ov[d] + sg * tv[d];
      }
    }
  }
}

// Cotangents of empty walkers. Workgroups of the first half own query rows (dq, de), of the
// second half key rows (dk, dv):
//     dS_ij = P_ij (dout_i . v_j - out_i . dout_i),  dq_i = scale sum_j dS_ij k_j,  de_ij = dS_ij,
//     dk_j = scale sum_i dS_ij q_i,  dv_j = sum_i P_ij dout_i,   P_ij = exp(s'_ij - lse_i).
template <class S, int D>
__global__ __launch_bounds__(kRows) void keymask_empty_bwd_kernel(BwdParams p) {
  const int nrb = (p.N + kRows - 1) / kRows;
  const int per_role = p.B * nrb;
  const bool key_role = static_cast<int>(blockIdx.x) >= per_role;
  const int blk = key_role ? blockIdx.x - per_role : blockIdx.x;
  const int b = blk / nrb;
  if (!walker_empty(p.mask, b, p.N)) return;
  const int r = (blk % nrb) * kRows + threadIdx.x;
  if (r >= p.N) return;
  const Walker w{b, p.N, p.H, D};
  const int64_t ebase = static_cast<int64_t>(b) * p.N * p.N * p.H;
  FwdParams f{};  // the logit helper's view of the primal operands
  f.k = p.k;
  f.e = p.e;
  f.scale = p.scale;
  f.e_sq = p.e_sq;
  f.e_sh = p.e_sh;
  f.e_sk = p.e_sk;
  for (int h = 0; h < p.H; ++h) {
    float acc[D], acc2[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = acc2[d] = 0.f;
    if (!key_role) {
      const int i = r;
      float qi[D], gi[D];
      load_row<S, D>(qi, p.q, w.row(i, h));
      load_row<S, D>(gi, p.dout, w.row(i, h));
      const float lse = p.lse[(static_cast<int64_t>(b) * p.N + i) * p.H + h];
      const float delta = dot_row<S, D>(gi, p.out, w.row(i, h));
      for (int j = 0; j < p.N; ++j) {
        const float pj = expf(logit<S, D>(f, w, qi, i, j, h) - lse);
        const float ds = pj * (dot_row<S, D>(gi, p.v, w.row(j, h)) - delta);
        const int64_t kj = w.row(j, h);
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = fmaf(ds, load1<S>(p.k, kj + d), acc[d]);
        if (p.de != nullptr) store1<S>(p.de, ebase + i * p.e_sq + h * p.e_sh + j * p.e_sk, ds);
      }
#pragma unroll
      for (int d = 0; d < D; ++d) store1<S>(p.dq, w.row(i, h) + d, p.scale * acc[d]);
    } else {
      const int j = r;
      for (int i = 0; i < p.N; ++i) {
        float qi[D], gi[D];
        load_row<S, D>(qi, p.q, w.row(i, h));
        load_row<S, D>(gi, p.dout, w.row(i, h));
        const float lse = p.lse[(static_cast<int64_t>(b) * p.N + i) * p.H + h];
        const float delta = dot_row<S, D>(gi, p.out, w.row(i, h));
        const float pj = expf(logit<S, D>(f, w, qi, i, j, h) - lse);
        const float ds = pj * (dot_row<S, D>(gi, p.v, w.row(j, h)) - delta);
#pragma unroll
        for (int d = 0; d < D; ++d) {
          acc[d] = fmaf(ds, qi[d], acc[d]);
          acc2[d] = fmaf(pj, gi[d], acc2[d]);
        }
      }
#pragma unroll
      for (int d = 0; d < D; ++d) {
        store1<S>(p.dk, w.row(j, h) + d, p.scale * acc[d]);
        store1<S>(p.dv, w.row(j, h) + d, acc2[d]);
      }
    }
  }
}

template <class S>
hipError_t fwd_for(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(p.B * ((p.N + kRows - 1) / kRows));
  switch (D) {
    case 8: keymask_empty_fwd_kernel<S, 8><<<grid, kRows, 0, stream>>>(p, T, given_lse); break;
    case 16: keymask_empty_fwd_kernel<S, 16><<<grid, kRows, 0, stream>>>(p, T, given_lse); break;
    case 32: keymask_empty_fwd_kernel<S, 32><<<grid, kRows, 0, stream>>>(p, T, given_lse); break;
    case 64: keymask_empty_fwd_kernel<S, 64><<<grid, kRows, 0, stream>>>(p, T, given_lse); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <class S>
hipError_t bwd_for(const BwdParams& p, int D, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(2 * p.B * ((p.N + kRows - 1) / kRows));
  switch (D) {
    case 8: keymask_empty_bwd_kernel<S, 8><<<grid, kRows, 0, stream>>>(p); break;
    case 16: keymask_empty_bwd_kernel<S, 16><<<grid, kRows, 0, stream>>>(p); break;
    case 32: keymask_empty_bwd_kernel<S, 32><<<grid, kRows, 0, stream>>>(p); break;
    case 64: keymask_empty_bwd_kernel<S, 64><<<grid, kRows, 0, stream>>>(p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_keymask_empty_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                                    hipStream_t stream) {
  if (p.gated) {
    const unsigned grid = static_cast<unsigned>(p.B * ((p.N + kRows - 1) / kRows));
    switch (D) {
      case 8: keymask_empty_gated_kernel<8><<<grid, kRows, 0, stream>>>(p, T); break;
      case 16: keymask_empty_gated_kernel<16><<<grid, kRows, 0, stream>>>(p, T); break;
      case 32: keymask_empty_gated_kernel<32><<<grid, kRows, 0, stream>>>(p, T); break;
      case 64: keymask_empty_gated_kernel<64><<<grid, kRows, 0, stream>>>(p, T); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  return dtype == 1 ? fwd_for<BF16>(p, D, T, given_lse, stream) : fwd_for<F32>(p, D, T, given_lse, stream);
}

hipError_t launch_keymask_empty_bwd(const BwdParams& p, int D, int dtype, hipStream_t stream) {
  return dtype == 1 ? bwd_for<BF16>(p, D, stream) : bwd_for<F32>(p, D, stream);
}

}  // namespace hz
