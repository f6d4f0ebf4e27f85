// C ABI of the MHSEA kernels: argument validation, error reporting and dispatch.
// Every check runs on the host before anything is enqueued, so an invalid call never
// reaches the GPU.
#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "../../include/hz_executor.h"
#include "../../include/hz_pair_bias.h"
#include "../../include/hz_mhsea.h"
#include "mhsea_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return HZ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shared validation of the dimensions and flags (mirrors the shape assertions of
// _validate_primals, mhsea_tuned.py:29-50, and the head-dim set of pallas_attention.py:13).
int check_dims(int64_t B, int64_t N, int64_t H, int64_t D, int dtype, int flags, bool compact_ok = false) {
  if (B < 1 || H < 1) return fail(HZ_EINVAL, "B and H must be >= 1, got B=%lld H=%lld", (long long)B, (long long)H);
  if (N < 1 || N > HZ_MAX_N)
    return fail(HZ_EINVAL, "N must be in [1, %d], got %lld", HZ_MAX_N, (long long)N);
  if (D != 8 && D != 16 && D != 32 && D != 64)
    return fail(HZ_EINVAL, "head dimension must be one of [8, 16, 32, 64], got %lld", (long long)D);
  if (dtype != HZ_DTYPE_F32 && dtype != HZ_DTYPE_BF16)
    return fail(HZ_EINVAL, "dtype must be HZ_DTYPE_F32 (0) or HZ_DTYPE_BF16 (1), got %d", dtype);
  if (flags & ~(HZ_FLAG_KEY_MASK | HZ_FLAG_E_QKH | HZ_FLAG_GENERIC | HZ_FLAG_E_COMPACT))
    return fail(HZ_EINVAL, "unknown flag bits 0x%x", flags);
  if ((flags & HZ_FLAG_E_COMPACT) && !compact_ok)
    return fail(HZ_EINVAL, "HZ_FLAG_E_COMPACT is read by the forward family only (fwd, jvp, fwd_jvp, fwd_jvp_gated)");
  const int64_t nwg = B * H * ((N + 63) / 64);
  if (nwg > 0x7fffffffLL) return fail(HZ_EINVAL, "B*H*ceil(N/64) = %lld exceeds the grid limit", (long long)nwg);
  if (B * N > 0x7fffffffLL)
    return fail(HZ_EINVAL, "B*N = %lld exceeds the supported mask size", (long long)(B * N));
  if (B * N * H * N > (int64_t(1) << 46))
    return fail(HZ_EINVAL, "B*N*H*N = %lld exceeds the supported tensor size", (long long)(B * N * H * N));
  return HZ_OK;
}

// The compacted bias layout is read by the N <= 64 producer/consumer kernel only: square
// mask, float32, the kernel's shapes (with tangents, in passes of one direction where two
// do not fit it).
int check_compact(int64_t N, int64_t H, int64_t D, int dtype, int flags, int64_t T) {
  if (!(flags & HZ_FLAG_E_COMPACT)) return HZ_OK;
  if (flags & (HZ_FLAG_KEY_MASK | HZ_FLAG_E_QKH | HZ_FLAG_GENERIC))
    return fail(HZ_EINVAL, "HZ_FLAG_E_COMPACT excludes HZ_FLAG_KEY_MASK, HZ_FLAG_E_QKH and HZ_FLAG_GENERIC");
  const int t = T > 0 ? 1 : 0;
  if (dtype != HZ_DTYPE_F32 || !hz::pc_fwd_supported(static_cast<int>(N), static_cast<int>(H), static_cast<int>(D), t, dtype))
    return fail(HZ_EINVAL, "HZ_FLAG_E_COMPACT needs float32, N <= 64 and D in [8, 16, 32] (N=%lld, D=%lld)",
                (long long)N, (long long)D);
  return HZ_OK;
}

#define HZ_REQUIRE(ptr)                                                     \
  do {                                                                      \
    if ((ptr) == nullptr) return fail(HZ_ENULL, "%s must not be NULL", #ptr); \
    if (!aligned16(ptr)) return fail(HZ_EALIGN, "%s must be 16-byte aligned", #ptr); \
  } while (0)

#define HZ_OPTIONAL(ptr)                                                    \
  do {                                                                      \
    if ((ptr) != nullptr && !aligned16(ptr))                                \
      return fail(HZ_EALIGN, "%s must be 16-byte aligned", #ptr);           \
  } while (0)

void set_e_strides(int64_t N, int64_t H, int flags, int64_t& sq, int64_t& sh, int64_t& sk) {
  if (flags & HZ_FLAG_E_QKH) {  // [B, Nq, Nk, H]
    sq = N * H;
    sk = H;
    sh = 1;
  } else {  // [B, Nq, H, Nk]
    sq = H * N;
    sh = N;
    sk = 1;
  }
}

size_t elem_bytes(int dtype) { return dtype == HZ_DTYPE_BF16 ? 2 : 4; }

int launched(hipError_t err) {
  if (err != hipSuccess) return fail(HZ_ELAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

hz::FwdParams fwd_params(const void* q, const void* k, const void* e, const void* v,
                         const uint8_t* mask, int64_t B, int64_t N, int64_t H, int64_t D,
                         float scale, int flags) {
  hz::FwdParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.e = e;
  p.mask = mask;
  p.B = static_cast<int>(B);
  p.N = static_cast<int>(N);
  p.H = static_cast<int>(H);
  p.t_stride = B * N * H * D;
  p.et_stride = B * N * H * N;
  set_e_strides(N, H, flags, p.e_sq, p.e_sh, p.e_sk);
  if (flags & HZ_FLAG_E_COMPACT) {
    p.e_compact = 1;
    p.et_stride = B * H * N * ((N + 3) & ~int64_t(3));
  }
  p.scale = scale;
  p.key_mask = (flags & HZ_FLAG_KEY_MASK) ? 1 : 0;
  p.masked_lse = -10000.0f + std::log(static_cast<float>(N));
  p.force_generic = (flags & HZ_FLAG_GENERIC) ? 1 : 0;
  return p;
}

// Runs the forward / tangent family over all T directions in groups of at most two
// (the kernels are specialised for T in {0, 1, 2}); the primal is written by the first
// group only.
int run_tangent_groups(hz::FwdParams p, int64_t D, int64_t T, bool given_lse, int dtype,
                       hipStream_t stream, void* tout, const void* qt, const void* kt,
                       const void* et, const void* vt) {
  const size_t eb = elem_bytes(dtype);
  const int64_t ts = p.t_stride, es = p.et_stride;
  void* const out0 = p.out;
  float* const lse0 = p.lse;
  // groups of two directions; one where the compacted bias layout's kernel takes only one
  const int64_t tg = (p.e_compact && !hz::pc_fwd_supported(p.N, p.H, static_cast<int>(D), 2, dtype)) ? 1 : 2;
  for (int64_t t0 = 0; t0 < T; t0 += tg) {
    const int tn = static_cast<int>(T - t0 < tg ? T - t0 : tg);
    auto shift = [&](const void* base, int64_t stride) -> const void* {
      return base == nullptr ? nullptr : static_cast<const char*>(base) + t0 * stride * eb;
    };
    p.qt = shift(qt, ts);
    p.kt = shift(kt, ts);
    p.vt = shift(vt, ts);
    p.et = shift(et, es);
    p.tout = static_cast<char*>(tout) + t0 * ts * eb;
    if (!given_lse && t0 > 0) {
      // Later groups rewrite identical primal values; point them at the same buffers so
      // the call never needs scratch memory.
      p.out = out0;
      p.lse = lse0;
    }
    hipError_t err = hz::launch_fwd(p, static_cast<int>(D), tn, given_lse, dtype, stream);
    if (err != hipSuccess) return launched(err);
  }
  return ok();
}

// Tangent operands of all T directions (the bases; the groups above shift them).
void set_tangents(hz::FwdParams& p, void* tout, const void* qt, const void* kt, const void* et,
                  const void* vt) {
  p.tout = tout;
  p.qt = qt;
  p.kt = kt;
  p.et = et;
  p.vt = vt;
}

// Key-mask calls: rewrite the walkers without a physical site (the reference's float32
// penalty, include/hz_mhsea.h); a no-op launch-free return in the square-mask mode.
int keymask_empty_fwd(const hz::FwdParams& p, int64_t D, int64_t T, bool given_lse, int dtype,
                      hipStream_t stream) {
  if (!p.key_mask) return ok();
  return launched(hz::launch_keymask_empty_fwd(p, static_cast<int>(D), static_cast<int>(T), given_lse, dtype, stream));
}

// Shared by the rectangular entry points: shape checks of noncausal_bias_mha
// (pallas_mha.py:101-118) and _validate_rectangular_attention_inputs
// (sequence_parallel.py:13-47), on C sizes, then the launch.
int rect_attention(hipStream_t stream, const float* q, const float* k, const float* v, const float* bias,
                   const uint8_t* key_mask, float* out, int64_t B, int64_t Nq, int64_t Nk, int64_t H, int64_t D,
                   float scale, bool gated) {
  if (B < 1 || H < 1) return fail(HZ_EINVAL, "B and H must be >= 1, got B=%lld H=%lld", (long long)B, (long long)H);
  if (Nq < 1 || Nk < 1)
    return fail(HZ_EINVAL, "query and key sequence lengths must both be positive, got Nq=%lld Nk=%lld",
                (long long)Nq, (long long)Nk);
  if (Nq > HZ_MAX_N || Nk > HZ_MAX_N)
    return fail(HZ_EINVAL, "Nq and Nk must be <= %d, got Nq=%lld Nk=%lld", HZ_MAX_N, (long long)Nq, (long long)Nk);
  if (D != 8 && D != 16 && D != 32 && D != 64)
    return fail(HZ_EINVAL, "head dimension must be one of [8, 16, 32, 64], got %lld", (long long)D);
  if (B * ((Nq + 63) / 64) * H > 0x7fffffffLL) return fail(HZ_EINVAL, "B*ceil(Nq/64)*H exceeds the grid limit");
  if (B * Nk > 0x7fffffffLL) return fail(HZ_EINVAL, "B*Nk = %lld exceeds the supported mask size", (long long)(B * Nk));
  if (B * Nq * Nk * H > (int64_t(1) << 46))
    return fail(HZ_EINVAL, "B*Nq*Nk*H = %lld exceeds the supported tensor size", (long long)(B * Nq * Nk * H));
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  HZ_REQUIRE(out);
  HZ_OPTIONAL(bias);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::RectParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.bias = bias;
  p.key_mask = key_mask;
  p.out = out;
  p.B = static_cast<int>(B);
  p.Nq = static_cast<int>(Nq);
  p.Nk = static_cast<int>(Nk);
  p.H = static_cast<int>(H);
  p.scale = scale;
  p.gated = gated ? 1 : 0;
  return launched(hz::launch_rect_fwd(p, static_cast<int>(D), stream));
}

}  // namespace

extern "C" {

int hz_version(void) { return HZ_MHSEA_VERSION; }

const char* hz_last_error(void) { return g_err; }

int hz_mhsea_fwd(hipStream_t stream, const void* q, const void* k, const void* e,
                 const void* v, const uint8_t* mask, void* out, float* lse, int64_t B,
                 int64_t N, int64_t H, int64_t D, int dtype, float scale, int flags) {
  if (int rc = check_dims(B, N, H, D, dtype, flags, true)) return rc;
  if (int rc = check_compact(N, H, D, dtype, flags, 0)) return rc;
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  if (mask == nullptr) return fail(HZ_ENULL, "mask must not be NULL");
  HZ_REQUIRE(out);
  HZ_OPTIONAL(e);
  HZ_OPTIONAL(lse);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::FwdParams p = fwd_params(q, k, e, v, mask, B, N, H, D, scale, flags);
  p.out = out;
  p.lse = lse;
  if (int rc = launched(hz::launch_fwd(p, static_cast<int>(D), 0, false, dtype, stream))) return rc;
  return keymask_empty_fwd(p, D, 0, false, dtype, stream);
}

int hz_mhsea_jvp(hipStream_t stream, const void* q, const void* k, const void* e,
                 const void* v, const uint8_t* mask, const void* out, const float* lse,
                 const void* qt, const void* kt, const void* et, const void* vt, int64_t T,
                 void* tout, int64_t B, int64_t N, int64_t H, int64_t D, int dtype,
                 float scale, int flags) {
  if (int rc = check_dims(B, N, H, D, dtype, flags, true)) return rc;
  if (T < 1 || T > 4096) return fail(HZ_EINVAL, "T must be in [1, 4096], got %lld", (long long)T);
  if (int rc = check_compact(N, H, D, dtype, flags, T)) return rc;
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  if (mask == nullptr) return fail(HZ_ENULL, "mask must not be NULL");
  HZ_REQUIRE(out);
  HZ_REQUIRE(lse);
  HZ_REQUIRE(tout);
  HZ_OPTIONAL(e);
  HZ_OPTIONAL(qt);
  HZ_OPTIONAL(kt);
  HZ_OPTIONAL(et);
  HZ_OPTIONAL(vt);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::FwdParams p = fwd_params(q, k, e, v, mask, B, N, H, D, scale, flags);
  p.out_in = out;
  p.lse_in = lse;
  if (int rc = run_tangent_groups(p, D, T, true, dtype, stream, tout, qt, kt, et, vt)) return rc;
  set_tangents(p, tout, qt, kt, et, vt);
  return keymask_empty_fwd(p, D, T, true, dtype, stream);
}

int hz_mhsea_fwd_jvp(hipStream_t stream, const void* q, const void* k, const void* e,
                     const void* v, const uint8_t* mask, const void* qt, const void* kt,
                     const void* et, const void* vt, int64_t T, void* out, float* lse,
                     void* tout, int64_t B, int64_t N, int64_t H, int64_t D, int dtype,
                     float scale, int flags) {
  if (int rc = check_dims(B, N, H, D, dtype, flags, true)) return rc;
  if (T < 1 || T > 4096) return fail(HZ_EINVAL, "T must be in [1, 4096], got %lld", (long long)T);
  if (int rc = check_compact(N, H, D, dtype, flags, T)) return rc;
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  if (mask == nullptr) return fail(HZ_ENULL, "mask must not be NULL");
  HZ_REQUIRE(out);
  HZ_REQUIRE(tout);
  HZ_OPTIONAL(e);
  HZ_OPTIONAL(lse);
  HZ_OPTIONAL(qt);
  HZ_OPTIONAL(kt);
  HZ_OPTIONAL(et);
  HZ_OPTIONAL(vt);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::FwdParams p = fwd_params(q, k, e, v, mask, B, N, H, D, scale, flags);
  p.out = out;
  p.lse = lse;
  if (int rc = run_tangent_groups(p, D, T, false, dtype, stream, tout, qt, kt, et, vt)) return rc;
  set_tangents(p, tout, qt, kt, et, vt);
  return keymask_empty_fwd(p, D, T, false, dtype, stream);
}

int hz_mhsea_fwd_jvp_gated(hipStream_t stream, const void* q, const void* k, const void* e,
                           const void* v, const uint8_t* mask, const void* qt, const void* kt,
                           const void* et, const void* vt, int64_t T, void* y, void* ty,
                           int64_t B, int64_t N, int64_t H, int64_t D, float scale, int flags) {
  if (int rc = check_dims(B, N, H, D, HZ_DTYPE_F32, flags, true)) return rc;
  if (T < 0 || T > 2) return fail(HZ_EINVAL, "T must be in [0, 2] for the gated collapse, got %lld", (long long)T);
  if (int rc = check_compact(N, H, D, HZ_DTYPE_F32, flags, T)) return rc;
  if (H % 2 != 0) return fail(HZ_EINVAL, "the gated collapse pairs head h with h + H/2: H must be even, got %lld", (long long)H);
  // The producer/consumer kernel where it serves the shape (fp32, N <= 64, D <= 32), in
  // passes of its tangent variants; otherwise (and with HZ_FLAG_GENERIC) the LDS-streaming
  // kernel, every direction in one launch.
  auto served = [&](int t) {
    return !(flags & HZ_FLAG_GENERIC) &&
           hz::pc_fwd_supported(static_cast<int>(N), static_cast<int>(H), static_cast<int>(D), t, HZ_DTYPE_F32);
  };
  const bool use_pc = served(T < 1 ? 0 : 1);
  // (the LDS-streaming kernel carries the gate terms of two directions in registers below
  // D = 32; from D = 32 one direction per pass keeps it free of spills)
  const int64_t tpass = use_pc ? (served(2) ? 2 : 1) : (D >= 32 ? 1 : 2);
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  if (mask == nullptr) return fail(HZ_ENULL, "mask must not be NULL");
  HZ_REQUIRE(y);
  if (T > 0) HZ_REQUIRE(ty);
  HZ_OPTIONAL(e);
  HZ_OPTIONAL(qt);
  HZ_OPTIONAL(kt);
  HZ_OPTIONAL(et);
  HZ_OPTIONAL(vt);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::FwdParams p = fwd_params(q, k, e, v, mask, B, N, H, D, scale, flags);
  p.out = y;
  p.lse = nullptr;
  p.gated = 1;
  p.y_tstride = B * N * (H / 2) * D;
  auto launch = [&](int t) {
    return use_pc ? hz::launch_fwd_pc(p, static_cast<int>(D), t, false, stream)
                  : hz::launch_fwd_gated_generic(p, static_cast<int>(D), t, stream);
  };
  if (T == 0) {
    if (int rc = launched(launch(0))) return rc;
    return keymask_empty_fwd(p, D, 0, false, HZ_DTYPE_F32, stream);
  }
  // Later passes rewrite identical y values, so the call needs no scratch memory.
  const int64_t ts = p.t_stride, es = p.et_stride;
  auto shift = [](const void* base, int64_t off) -> const void* {
    return base == nullptr ? nullptr : static_cast<const float*>(base) + off;
  };
  for (int64_t t0 = 0; t0 < T; t0 += tpass) {
    const int64_t tn = T - t0 < tpass ? T - t0 : tpass;
    p.qt = shift(qt, t0 * ts);
    p.kt = shift(kt, t0 * ts);
    p.vt = shift(vt, t0 * ts);
    p.et = shift(et, t0 * es);
    p.tout = static_cast<float*>(ty) + t0 * p.y_tstride;
    hipError_t err = launch(static_cast<int>(tn));
    if (err != hipSuccess) return launched(err);
  }
  set_tangents(p, ty, qt, kt, et, vt);
  return keymask_empty_fwd(p, D, T, false, HZ_DTYPE_F32, stream);
}

int hz_mhsea_bwd(hipStream_t stream, const void* q, const void* k, const void* e,
                 const void* v, const uint8_t* mask, const float* lse, const void* out,
                 const void* dout, void* dq, void* dk, void* de, void* dv, int64_t B,
                 int64_t N, int64_t H, int64_t D, int dtype, float scale, int flags) {
  if (int rc = check_dims(B, N, H, D, dtype, flags)) return rc;
  HZ_REQUIRE(q);
  HZ_REQUIRE(k);
  HZ_REQUIRE(v);
  if (mask == nullptr) return fail(HZ_ENULL, "mask must not be NULL");
  HZ_REQUIRE(lse);
  HZ_REQUIRE(out);
  HZ_REQUIRE(dout);
  HZ_REQUIRE(dq);
  HZ_REQUIRE(dk);
  HZ_REQUIRE(dv);
  HZ_OPTIONAL(e);
  HZ_OPTIONAL(de);
  if (!std::isfinite(scale)) return fail(HZ_EINVAL, "scale must be finite");
  hz::BwdParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.e = e;
  p.mask = mask;
  p.lse = lse;
  p.out = out;
  p.dout = dout;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.de = de;
  p.B = static_cast<int>(B);
  p.N = static_cast<int>(N);
  p.H = static_cast<int>(H);
  set_e_strides(N, H, flags, p.e_sq, p.e_sh, p.e_sk);
  p.scale = scale;
  p.key_mask = (flags & HZ_FLAG_KEY_MASK) ? 1 : 0;
  p.force_generic = (flags & HZ_FLAG_GENERIC) ? 1 : 0;
  if (int rc = launched(hz::launch_bwd(p, static_cast<int>(D), dtype, stream))) return rc;
  if (!p.key_mask) return ok();
  return launched(hz::launch_keymask_empty_bwd(p, static_cast<int>(D), dtype, stream));
}

int hz_rect_attention_fwd(hipStream_t stream, const float* q, const float* k, const float* v,
                          const float* bias, const uint8_t* key_mask, float* out, int64_t B,
                          int64_t Nq, int64_t Nk, int64_t H, int64_t D, float scale) {
  return rect_attention(stream, q, k, v, bias, key_mask, out, B, Nq, Nk, H, D, scale, false);
}

int hz_rect_attention_fwd_gated(hipStream_t stream, const float* q, const float* k, const float* v,
                                const float* bias, const uint8_t* key_mask, float* y, int64_t B,
                                int64_t Nq, int64_t Nk, int64_t H, int64_t D, float scale) {
  if (H % 2 != 0)
    return fail(HZ_EINVAL, "the gated collapse pairs head h with h + H/2: H must be even, got %lld", (long long)H);
  return rect_attention(stream, q, k, v, bias, key_mask, y, B, Nq, Nk, H, D, scale, true);
}

int hz_pair_mlp_bias(hipStream_t stream, const float* edge, const float* edge_t, const float* extra,
                     const float* extra_t, const uint8_t* mask, const float* w_in, const float* b_in,
                     const float* norm_w, const float* w_1, const float* b_1, const float* w_2, const float* b_2,
                     const float* out_norm_w, const float* w_out, const float* b_out, const float* alibi_slopes,
                     float* e, float* e_t, int64_t B, int64_t Nq, int64_t Nk, int64_t C, int64_t hidden, int64_t H,
                     int64_t n_blocks, int64_t T, int64_t row_offset, float inner_gain, float eps, float bias_div,
                     int flags) {
  if (B < 1 || Nq < 1 || Nk < 1 || Nq > HZ_MAX_N || Nk > HZ_MAX_N)
    return fail(HZ_EINVAL, "B must be >= 1 and Nq, Nk in [1, %d]", HZ_MAX_N);
  if (C != 32 && C != 64 && C != 96 && C != 128)
    return fail(HZ_EINVAL, "C = %lld: edge channels must be 32, 64, 96 or 128", (long long)C);
  if (hidden != 32 && hidden != 64 && hidden != 128)
    return fail(HZ_EINVAL, "hidden = %lld: the bias MLP's hidden width must be 32, 64 or 128", (long long)hidden);
  if (H != 16 && H != 32) return fail(HZ_EINVAL, "H = %lld: heads must be 16 or 32", (long long)H);
  if (n_blocks < 1 || n_blocks > hz::pair_mlp_max_blocks(static_cast<int>(hidden)))
    return fail(HZ_EINVAL, "n_blocks = %lld: must be in [1, %d] at hidden width %lld", (long long)n_blocks,
                hz::pair_mlp_max_blocks(static_cast<int>(hidden)), (long long)hidden);
  if (T != 0 && T != 1) return fail(HZ_EINVAL, "T = %lld: T must be 0 or 1", (long long)T);
  if (flags & ~(HZ_FLAG_KEY_MASK | HZ_FLAG_E_QKH)) return fail(HZ_EINVAL, "unknown flag bits 0x%x", flags);
  if (mask != nullptr && !(flags & HZ_FLAG_KEY_MASK) && Nq != Nk)
    return fail(HZ_EINVAL, "a square (query and key) mask needs Nq == Nk, got Nq=%lld Nk=%lld; pass HZ_FLAG_KEY_MASK",
                (long long)Nq, (long long)Nk);
  if (row_offset < 0 || row_offset + Nq > 0x7fffffffLL) return fail(HZ_EINVAL, "row_offset must be >= 0 and fit int32");
  if (B * Nq * Nk > (int64_t(1) << 40)) return fail(HZ_EINVAL, "B*Nq*Nk exceeds the supported size");
  if (!std::isfinite(inner_gain) || !std::isfinite(eps) || eps < 0.0f || !std::isfinite(bias_div) || bias_div == 0.0f)
    return fail(HZ_EINVAL, "inner_gain and bias_div must be finite (bias_div nonzero), eps finite and >= 0");
  HZ_REQUIRE(edge);
  HZ_OPTIONAL(mask);
  HZ_REQUIRE(w_in);
  HZ_REQUIRE(b_in);
  HZ_REQUIRE(norm_w);
  HZ_REQUIRE(w_1);
  HZ_REQUIRE(b_1);
  HZ_REQUIRE(w_2);
  HZ_REQUIRE(b_2);
  HZ_REQUIRE(out_norm_w);
  HZ_REQUIRE(w_out);
  HZ_REQUIRE(b_out);
  HZ_OPTIONAL(alibi_slopes);
  HZ_REQUIRE(e);
  if (T == 1) {
    HZ_REQUIRE(edge_t);
    HZ_REQUIRE(e_t);
    if (extra != nullptr && extra_t == nullptr) return fail(HZ_ENULL, "extra_t must not be NULL when extra is given and T = 1");
  }
  if ((reinterpret_cast<uintptr_t>(extra) | reinterpret_cast<uintptr_t>(extra_t)) & 3u)
    return fail(HZ_EALIGN, "extra and extra_t must be 4-byte aligned");
  hz::PairMlpParams p{};
  p.edge = edge;
  p.edge_t = T == 1 ? edge_t : nullptr;
  p.extra = extra;
  p.extra_t = T == 1 ? extra_t : nullptr;
  p.mask = mask;
  p.w_in = w_in;
  p.b_in = b_in;
  p.norm_w = norm_w;
  p.w_1 = w_1;
  p.b_1 = b_1;
  p.w_2 = w_2;
  p.b_2 = b_2;
  p.out_norm_w = out_norm_w;
  p.w_out = w_out;
  p.b_out = b_out;
  p.slopes = alibi_slopes;
  p.e = e;
  p.e_t = T == 1 ? e_t : nullptr;
  p.B = B;
  p.Nq = static_cast<int>(Nq);
  p.Nk = static_cast<int>(Nk);
  p.n_blocks = static_cast<int>(n_blocks);
  p.row_offset = static_cast<int>(row_offset);
  if (flags & HZ_FLAG_E_QKH) {  // [B, Nq, Nk, H]
    p.e_sq = Nk * H;
    p.e_sk = H;
    p.e_sh = 1;
  } else {  // [B, Nq, H, Nk]
    p.e_sq = H * Nk;
    p.e_sh = Nk;
    p.e_sk = 1;
  }
  p.gain = inner_gain;
  p.eps = eps;
  p.div = bias_div;
  p.key_mask = (flags & HZ_FLAG_KEY_MASK) != 0;
  return launched(hz::launch_pair_mlp_bias(p, static_cast<int>(C), static_cast<int>(hidden), static_cast<int>(H),
                                           T == 1, stream));
}

int hz_quadrilinear_merge(hipStream_t stream, const float* T, const float* u_a, const float* u_b, float* out,
                          int64_t M, int64_t G, int64_t R) {
  if (R != 32) return fail(HZ_EINVAL, "the merge rank R must be 32, got %lld", (long long)R);
  if (M < 1 || G < 1) return fail(HZ_EINVAL, "M and G must be >= 1, got M=%lld G=%lld", (long long)M, (long long)G);
  if (G > 65535) return fail(HZ_EINVAL, "G = %lld exceeds the grid limit", (long long)G);
  if ((M + 255) / 256 > 0x7fffffffLL) return fail(HZ_EINVAL, "M = %lld exceeds the grid limit", (long long)M);
  HZ_REQUIRE(T);
  HZ_REQUIRE(u_a);
  HZ_REQUIRE(u_b);
  HZ_REQUIRE(out);
  return launched(hz::launch_quadrilinear_merge(T, u_a, u_b, out, M, static_cast<int>(G), G * R, stream));
}

int hz_factorized_apply(hipStream_t stream, const float* x, const float* V, const float* h, const float* U,
                        const float* residual, float* y, float* workspace, int64_t M, int64_t d_in, int64_t R,
                        int64_t d_out, int64_t h_rows) {
  if (M < 1 || d_in < 1 || R < 1 || d_out < 1 || h_rows < 1)
    return fail(HZ_EINVAL, "M, d_in, R, d_out and h_rows must be >= 1");
  if (d_in > 0x7fffffffLL || R > 0x7fffffffLL || d_out > 0x7fffffffLL || h_rows > 0x7fffffffLL)
    return fail(HZ_EINVAL, "dimensions exceed the 32-bit range");
  if ((M + 127) / 128 > 65535) return fail(HZ_EINVAL, "M = %lld exceeds the grid limit", (long long)M);
  HZ_REQUIRE(x);
  HZ_REQUIRE(V);
  HZ_REQUIRE(h);
  HZ_REQUIRE(U);
  HZ_REQUIRE(y);
  HZ_REQUIRE(workspace);
  HZ_OPTIONAL(residual);
  return launched(hz::launch_factorized_apply(x, V, h, U, residual, y, workspace, M, static_cast<int>(d_in),
                                              static_cast<int>(R), static_cast<int>(d_out), static_cast<int>(h_rows),
                                              stream));
}

int hz_factorized_apply_noalloc(hipStream_t stream, const float* x, const float* V, const float* h, const float* U,
                                const float* residual, float* y, int64_t M, int64_t d_in, int64_t R, int64_t d_out,
                                int64_t h_rows) {
  if (M < 1 || d_in < 1 || R < 1 || d_out < 1 || h_rows < 1)
    return fail(HZ_EINVAL, "M, d_in, R, d_out and h_rows must be >= 1");
  if (d_in > 0x7fffffffLL || d_out > 0x7fffffffLL || h_rows > 0x7fffffffLL)
    return fail(HZ_EINVAL, "dimensions exceed the 32-bit range");
  if (R > hz::kApplyScratchMaxRank)
    return fail(HZ_EINVAL,
                "R = %lld exceeds the no-alloc workspace: R <= %lld (its %lld MiB device array holds 128 rows of "
                "R floats); use hz_factorized_apply with a caller-owned workspace",
                (long long)R, (long long)hz::kApplyScratchMaxRank, (long long)(hz::kApplyScratchFloats * 4 >> 20));
  if ((M + 127) / 128 > 65535) return fail(HZ_EINVAL, "M = %lld exceeds the grid limit", (long long)M);
  HZ_REQUIRE(x);
  HZ_REQUIRE(V);
  HZ_REQUIRE(h);
  HZ_REQUIRE(U);
  HZ_REQUIRE(y);
  HZ_OPTIONAL(residual);
  return launched(hz::launch_factorized_apply_noalloc(x, V, h, U, residual, y, M, static_cast<int>(d_in),
                                                      static_cast<int>(R), static_cast<int>(d_out),
                                                      static_cast<int>(h_rows), stream));
}

int hz_pair_bias(hipStream_t stream, const float* edge, const float* edge_t, const uint8_t* mask, const float* ln_w,
                 const float* w_in, const float* b_in, const float* w_1, const float* b_1, const float* w_2,
                 const float* b_2, const float* w_out, const float* b_out, float* e, float* e_t, int64_t B, int64_t N,
                 int64_t C, int64_t hidden, int64_t H, int64_t T, float inner_gain, float eps, float bias_div,
                 int flags) {
  if (B < 1 || N < 1 || N > HZ_MAX_N) return fail(HZ_EINVAL, "B must be >= 1 and N in [1, %d]", HZ_MAX_N);
  if (C != 32 && C != 64 && C != 96 && C != 128) return fail(HZ_EINVAL, "C = %lld: edge channels must be 32, 64, 96 or 128", (long long)C);
  if (hidden != 64) return fail(HZ_EINVAL, "hidden = %lld: the bias MLP's hidden width must be 64", (long long)hidden);
  if (H != 16 && H != 32 && H != 64) return fail(HZ_EINVAL, "H = %lld: heads must be 16, 32 or 64", (long long)H);
  if (T != 0 && T != 1) return fail(HZ_EINVAL, "T = %lld: T must be 0 or 1", (long long)T);
  if (flags & ~(HZ_FLAG_KEY_MASK | HZ_FLAG_E_QKH | HZ_FLAG_E_COMPACT)) return fail(HZ_EINVAL, "unknown flag bits 0x%x", flags);
  if ((flags & HZ_FLAG_E_COMPACT) && (flags & (HZ_FLAG_KEY_MASK | HZ_FLAG_E_QKH)))
    return fail(HZ_EINVAL, "HZ_FLAG_E_COMPACT excludes HZ_FLAG_KEY_MASK and HZ_FLAG_E_QKH");
  if ((flags & HZ_FLAG_E_COMPACT) && mask != nullptr && N > 256)
    return fail(HZ_EINVAL, "HZ_FLAG_E_COMPACT with a mask needs N <= 256, got %lld", (long long)N);
  if (!std::isfinite(inner_gain) || !std::isfinite(eps) || eps < 0.0f || !std::isfinite(bias_div) || bias_div == 0.0f)
    return fail(HZ_EINVAL, "inner_gain and bias_div must be finite (bias_div nonzero), eps finite and >= 0");
  HZ_REQUIRE(edge);
  HZ_OPTIONAL(mask);
  HZ_REQUIRE(ln_w);
  HZ_REQUIRE(w_in);
  HZ_REQUIRE(b_in);
  HZ_REQUIRE(w_1);
  HZ_REQUIRE(b_1);
  HZ_REQUIRE(w_2);
  HZ_REQUIRE(b_2);
  HZ_REQUIRE(w_out);
  HZ_REQUIRE(b_out);
  HZ_REQUIRE(e);
  if (T == 1) {
    HZ_REQUIRE(edge_t);
    HZ_REQUIRE(e_t);
  }
  hz::PairBiasParams p{};
  p.edge = edge;
  p.edge_t = T == 1 ? edge_t : nullptr;
  p.mask = mask;
  p.ln_w = ln_w;
  p.w_in = w_in;
  p.b_in = b_in;
  p.w_1 = w_1;
  p.b_1 = b_1;
  p.w_2 = w_2;
  p.b_2 = b_2;
  p.w_out = w_out;
  p.b_out = b_out;
  p.e = e;
  p.e_t = T == 1 ? e_t : nullptr;
  p.B = B;
  p.N = static_cast<int>(N);
  set_e_strides(N, H, flags, p.e_sq, p.e_sh, p.e_sk);
  if (flags & HZ_FLAG_E_COMPACT) p.e_blk = N * ((N + 3) & ~int64_t(3));
  p.gain = inner_gain;
  p.eps = eps;
  p.div = bias_div;
  p.key_mask = (flags & HZ_FLAG_KEY_MASK) != 0;
  return launched(hz::launch_pair_bias(p, static_cast<int>(C), static_cast<int>(H), T == 1, stream));
}

int64_t hz_compiled_wavefunction_workspace(int64_t B, int64_t n_sites, int64_t d_z, int64_t R_leaf, int64_t d_m,
                                           int64_t R_merge, int64_t R_out) {
  if (B < 1 || n_sites < 1 || d_z < 1 || R_leaf < 1 || d_m < 1 || R_merge < 1 || R_out < 1) return -1;
  return hz::compiled_wavefunction_workspace_bytes(B, n_sites, d_z, R_leaf, d_m, R_merge, R_out);
}

int hz_compiled_wavefunction(hipStream_t stream, const float* q, const float* q_weight, const float* leaf_V,
                             const float* leaf_U, const float* leaf_h, const float* merge_T, const float* merge_V,
                             const float* merge_U, const float* merge_h, const uint8_t* opcodes, const float* readout_V,
                             const float* readout_U, const float* readout_h, float* log_abs, float* phase,
                             void* workspace, int64_t workspace_bytes, int64_t B, int64_t n_sites, int64_t d_q,
                             int64_t d_z, int64_t R_leaf, int64_t G, int64_t d_r, int64_t R_merge, int64_t R_out,
                             float merge_eps) {
  if (B < 1 || n_sites < 1 || d_q < 1 || d_z < 1 || R_leaf < 1 || G < 1 || R_merge < 1 || R_out < 1)
    return fail(HZ_EINVAL, "B, n_sites, d_q, d_z, R_leaf, G, R_merge and R_out must be >= 1");
  if (n_sites & (n_sites - 1)) return fail(HZ_EINVAL, "n_sites must be a power of two, got %lld", (long long)n_sites);
  if (d_r != 32) return fail(HZ_EINVAL, "d_r = %lld: the merge tensor's rank must be 32", (long long)d_r);
  const int64_t d_m = G * d_r;
  if (d_m > hz::kRowMaxFloats)
    return fail(HZ_EINVAL, "carrier width G * d_r = %lld exceeds %d", (long long)d_m, hz::kRowMaxFloats);
  if (n_sites > 0x7fffffffLL || d_q > 0x7fffffffLL || d_z > 0x7fffffffLL || R_leaf > 0x7fffffffLL ||
      R_merge > 0x7fffffffLL || R_out > 0x7fffffffLL)
    return fail(HZ_EINVAL, "dimensions exceed the 32-bit range");
  if ((B * n_sites + 127) / 128 > 65535 || (B * n_sites + 255) / 256 > 0x7fffffffLL)
    return fail(HZ_EINVAL, "B * n_sites = %lld exceeds the grid limit", (long long)(B * n_sites));
  if (!std::isfinite(merge_eps) || merge_eps < 0.0f) return fail(HZ_EINVAL, "merge_eps must be finite and >= 0");
  const int64_t need = hz::compiled_wavefunction_workspace_bytes(B, n_sites, d_z, R_leaf, d_m, R_merge, R_out);
  if (workspace_bytes < need)
    return fail(HZ_EINVAL, "workspace_bytes = %lld, need %lld (hz_compiled_wavefunction_workspace)",
                (long long)workspace_bytes, (long long)need);
  HZ_REQUIRE(q);
  HZ_REQUIRE(q_weight);
  HZ_REQUIRE(leaf_V);
  HZ_REQUIRE(leaf_U);
  HZ_REQUIRE(leaf_h);
  if (n_sites > 1) {  // one site: no merge level, so no merge operand is read
    HZ_REQUIRE(merge_T);
    HZ_REQUIRE(merge_V);
    HZ_REQUIRE(merge_U);
    HZ_REQUIRE(merge_h);
    HZ_REQUIRE(opcodes);
  }
  HZ_REQUIRE(readout_V);
  HZ_REQUIRE(readout_U);
  HZ_REQUIRE(readout_h);
  HZ_REQUIRE(log_abs);
  HZ_REQUIRE(phase);
  HZ_REQUIRE(workspace);
  hz::WaveFnParams p{};
  p.q = q;
  p.q_weight = q_weight;
  p.leaf_V = leaf_V;
  p.leaf_U = leaf_U;
  p.leaf_h = leaf_h;
  p.merge_T = merge_T;
  p.merge_V = merge_V;
  p.merge_U = merge_U;
  p.merge_h = merge_h;
  p.opcodes = opcodes;
  p.readout_V = readout_V;
  p.readout_U = readout_U;
  p.readout_h = readout_h;
  p.log_abs = log_abs;
  p.phase = phase;
  p.workspace = static_cast<float*>(workspace);
  p.B = B;
  p.n = static_cast<int>(n_sites);
  p.d_q = static_cast<int>(d_q);
  p.d_z = static_cast<int>(d_z);
  p.r_leaf = static_cast<int>(R_leaf);
  p.d_m = static_cast<int>(d_m);
  p.r_merge = static_cast<int>(R_merge);
  p.r_out = static_cast<int>(R_out);
  p.merge_eps = merge_eps;
  return launched(hz::launch_compiled_wavefunction(p, stream));
}

int hz_gated_out_proj(hipStream_t stream, const float* y, const float* ty, const float* w_o, const uint8_t* mask,
                      float* delta, float* delta_t, int64_t B, int64_t N, int64_t d_attn, int64_t d_e, int64_t T) {
  if (B < 1 || N < 1 || d_attn < 1 || d_e < 1) return fail(HZ_EINVAL, "B, N, d_attn and d_e must be >= 1");
  if (T < 0 || T > 3) return fail(HZ_EINVAL, "T must be in [0, 3], got %lld", (long long)T);
  if (d_attn > 0x7fffffffLL || d_e > 0x7fffffffLL) return fail(HZ_EINVAL, "dimensions exceed the 32-bit range");
  const int64_t M = B * N;
  if ((M + 127) / 128 > 65535) return fail(HZ_EINVAL, "B * N = %lld exceeds the grid limit", (long long)M);
  HZ_REQUIRE(y);
  HZ_REQUIRE(w_o);
  HZ_OPTIONAL(mask);
  HZ_REQUIRE(delta);
  if (T > 0) {
    HZ_REQUIRE(ty);
    HZ_REQUIRE(delta_t);
  }
  if (int rc = launched(hz::launch_out_proj(y, w_o, mask, delta, M, static_cast<int>(d_attn), static_cast<int>(d_e),
                                            stream)))
    return rc;
  for (int64_t t = 0; t < T; ++t)
    if (int rc = launched(hz::launch_out_proj(ty + t * M * d_attn, w_o, mask, delta_t + t * M * d_e, M,
                                              static_cast<int>(d_attn), static_cast<int>(d_e), stream)))
      return rc;
  return 0;
}

int hz_mhsea_bwd_gated(hipStream_t stream, const void* q, const void* k, const void* e, const void* v,
                       const uint8_t* mask, const float* lse, const void* out, const float* dy, void* dq, void* dk,
                       void* de, void* dv, float* dout_work, int64_t B, int64_t N, int64_t H, int64_t D, float scale,
                       int flags) {
  if (int rc = check_dims(B, N, H, D, HZ_DTYPE_F32, flags)) return rc;
  if (H % 2 != 0) return fail(HZ_EINVAL, "the gated collapse pairs head h with h + H/2: H must be even, got %lld", (long long)H);
  HZ_REQUIRE(out);
  HZ_REQUIRE(dy);
  HZ_REQUIRE(dout_work);
  if (int rc = launched(hz::launch_gate_collapse_bwd(static_cast<const float*>(out), dy, dout_work, B * N,
                                                     static_cast<int>(H), static_cast<int>(D), stream)))
    return rc;
  return hz_mhsea_bwd(stream, q, k, e, v, mask, lse, out, dout_work, dq, dk, de, dv, B, N, H, D, HZ_DTYPE_F32, scale,
                      flags);
}

}  // extern "C"
