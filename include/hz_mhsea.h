/*
 * hz_mhsea.h — C ABI of the MI355X (gfx950) MHSEA attention kernels.
 *
 * MHSEA = masked, edge-biased multi-head self attention:
 *     S   = scale * Q K^T + E            (per walker b, head h)
 *     P   = softmax_k(S)                 restricted to valid (query, key) pairs
 *     out = P V
 * together with its forward-mode tangent (JVP) and reverse-mode cotangent (VJP).
 *
 * This header replaces the reference's Pallas primitives
 *   mhsea_tuned_ad_p      (src/hamiltonzero/model/_pallas_attn/mhsea_tuned.py:72-174)
 *   mhsea_tuned_ad_lin_p  (src/hamiltonzero/model/_pallas_attn/mhsea_tuned.py:175-240)
 *   mhsea_full_ad_p / _lin_p (src/hamiltonzero/model/_pallas_attn/mhsea_full_ad.py:32-185)
 * and the jnp op reference_edge_attention
 *   (src/hamiltonzero/model/pallas_attention.py:22-37).
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - All tensor pointers are DEVICE pointers, row-major, C-contiguous.
 *      q, k, v, out, dq, dk, dv, dout : [B, N, H, D]   ("sites-major", as the
 *                                        reference BlockSpecs in _pallas_attn/utils.py:21-36)
 *      tangents qt, kt, vt, tout       : [T, B, N, H, D]   (T tangent directions)
 *      e, de                           : [B, N, H, N]  (query, head, key)  default, or
 *                                        [B, N, N, H]  with HZ_FLAG_E_QKH (op-level layout,
 *                                        pallas_attention.py:45, so no transpose pass)
 *      et                              : [T, <layout of e>]
 *      e (compact, HZ_FLAG_E_COMPACT)  : [B, H, N, N4], N4 = N rounded up to a multiple of 4:
 *                                        block (b, h) holds the bias of the n x n physical
 *                                        pairs of walker b (n = its physical site count,
 *                                        sites in ascending order on both sides) as n rows
 *                                        of stride n4 = n rounded up to 4, i.e. entry
 *                                        (i, j) at i * n4 + j; the rest is never read.
 *                                        The forward family reads only these n * n4 floats
 *                                        per (walker, head). hz_pair_bias writes it.
 *      mask                            : [B, N] uint8 (0 = padded/virtual site, else physical)
 *      lse                             : [B, N, H] float32 (natural log-sum-exp per query row)
 *  - dtype: HZ_DTYPE_F32 (all float tensors float32) or HZ_DTYPE_BF16 (q, k, v, e, all
 *    tangents/cotangents and float outputs are bfloat16; lse is always float32; every
 *    reduction and the softmax run in float32).
 *  - D must be 8, 16, 32 or 64 (the reference's supported head dims,
 *    pallas_attention.py:13).  1 <= N <= HZ_MAX_N.  B, H >= 1.
 *  - Optional pointers (documented per call) may be NULL: a NULL bias / bias tangent means
 *    zero, a NULL tangent means a zero tangent (ad.instantiate_zeros, mhsea_tuned.py:107-110).
 *  - scale multiplies Q K^T before the bias is added. The primitives take pre-scaled Q and
 *    pass scale = 1 (mhsea.py:14-31); the op-level wrapper passes D^-1/2 (pallas_attention.py:31).
 *  - Mask semantics (flags):
 *      default ("square", the primitive, mhsea.py:18-25 + mhsea_tuned.py:91):
 *          a (query i, key j) pair is valid iff mask[i] && mask[j]; scores of invalid
 *          pairs are -1e4 (utils.py:51-52). Rows of masked queries are written as exact
 *          zeros in out / tout / dq, and their lse is -1e4 + log(N).
 *      HZ_FLAG_KEY_MASK (reference_edge_attention, pallas_attention.py:34-36):
 *          only keys are masked (additive -1e9); every query row is computed. The
 *          reference adds the penalty in float32, so a masked key's logit is fl32(s - 1e9),
 *          a multiple of 64. While a walker has a physical key, masked keys get weight
 *          exactly 0 (and are never read). If NO key of a walker is physical, every key is
 *          used with the logit fl32(fl32(s - 1e9) + 1e9) — the reference's rounded value
 *          shifted back by the constant 1e9, which softmax ignores — so all |s| < 32 give
 *          uniform weights (out = mean of the walker's value rows), as in the reference;
 *          that walker's lse is relative to the shift. Tangents and cotangents use the
 *          same weights (the penalty's derivative is 1, as under autodiff).
 *          One intended difference on non-finite inputs: a NaN / Inf in a masked key's
 *          k, v or bias reaches the reference's output (0 * NaN), not this library's.
 *  - Every call is enqueue-only on `stream` (no host synchronisation), allocates nothing,
 *    fully overwrites its outputs (including masked rows), and is deterministic
 *    (no atomics). Calls on distinct output buffers are re-entrant.
 *  - Return value: 0 on success, otherwise an HZ_E* code; hz_last_error() then returns a
 *    thread-local message. Argument errors are detected on the host before any GPU work.
 */
#ifndef HZ_MHSEA_H
#define HZ_MHSEA_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HZ_MHSEA_VERSION 100 /* 1.0.0 */
#define HZ_MAX_N 16384

enum hz_dtype { HZ_DTYPE_F32 = 0, HZ_DTYPE_BF16 = 1 };

enum hz_flags {
  HZ_FLAG_KEY_MASK = 1, /* reference_edge_attention masking instead of the square mask */
  HZ_FLAG_E_QKH = 2,    /* e / et / de are [B, N(query), N(key), H] */
  HZ_FLAG_GENERIC = 4,  /* always use the LDS-streaming kernels (testing / comparison) */
  /* e / et in the compacted physical-pair layout (above). Square mask only (not with
     HZ_FLAG_KEY_MASK), float32, and only where the N <= 64 producer/consumer kernel serves
     the shape (N <= 64, D in {8, 16, 32}); accepted by hz_mhsea_fwd, hz_mhsea_jvp,
     hz_mhsea_fwd_jvp and hz_mhsea_fwd_jvp_gated, refused (HZ_EINVAL) elsewhere. */
  HZ_FLAG_E_COMPACT = 8
};

enum hz_status {
  HZ_OK = 0,
  HZ_EINVAL = 1,   /* bad dimension, dtype, flag or T */
  HZ_ENULL = 2,    /* a required pointer is NULL */
  HZ_EALIGN = 3,   /* a tensor pointer is not 16-byte aligned */
  HZ_ELAUNCH = 4   /* the HIP runtime rejected a kernel launch */
};

/* Library version (HZ_MHSEA_VERSION). */
int hz_version(void);

/* Message for the last non-zero status returned on this thread ("" if none). */
const char* hz_last_error(void);

/*
 * Forward. Replaces mhsea_tuned_ad_p's impl (_outer_impl, mhsea_tuned.py:76-92 ->
 * mhsea_forward, custom_gradients.py:24-75 -> mhsea_kernel, mhsea.py:11-31).
 * Writes out [B,N,H,D] and, if lse != NULL, lse [B,N,H].
 * Optional: e (NULL = no bias), lse.
 */
int hz_mhsea_fwd(hipStream_t stream,
                 const void* q, const void* k, const void* e, const void* v,
                 const uint8_t* mask,
                 void* out, float* lse,
                 int64_t B, int64_t N, int64_t H, int64_t D,
                 int dtype, float scale, int flags);

/*
 * Tangent of the forward given its primal outputs. Replaces mhsea_tuned_ad_lin_p's impl
 * (_inner_impl, mhsea_tuned.py:179-198 -> mhsea_tangent_pallas,
 * mhsea_tuned_jvp.py:104-222), with the same 11 operands in the same order plus a native
 * tangent axis T (the reference instead broadcasts the primals T times,
 * mhsea_tuned.py:144-148):
 *     tout[t] = P(dS_t) V + P vt[t] - rowsum(P o dS_t) out,    P = exp(S - lse)
 *     dS_t    = scale (qt[t] K^T + Q kt[t]^T) + et[t]           (valid pairs, else 0)
 * Required: q, k, v, mask, out, lse, tout. Optional: e, qt, kt, et, vt. T >= 1.
 */
int hz_mhsea_jvp(hipStream_t stream,
                 const void* q, const void* k, const void* e, const void* v,
                 const uint8_t* mask, const void* out, const float* lse,
                 const void* qt, const void* kt, const void* et, const void* vt,
                 int64_t T, void* tout,
                 int64_t B, int64_t N, int64_t H, int64_t D,
                 int dtype, float scale, int flags);

/*
 * Fused forward + T tangents in one pass (P is formed once per tile and shared by all
 * tangents). Same results as hz_mhsea_fwd followed by hz_mhsea_jvp, i.e. as the
 * reference's _outer_jvp (mhsea_tuned.py:104-118), without the round trip of out/lse
 * through HBM. Required: q, k, v, mask, out, tout. Optional: e, lse, qt, kt, et, vt.
 */
int hz_mhsea_fwd_jvp(hipStream_t stream,
                     const void* q, const void* k, const void* e, const void* v,
                     const uint8_t* mask,
                     const void* qt, const void* kt, const void* et, const void* vt,
                     int64_t T,
                     void* out, float* lse, void* tout,
                     int64_t B, int64_t N, int64_t H, int64_t D,
                     int dtype, float scale, int flags);

/*
 * Fused forward + T tangents with the trunk's sigmoid-gate head collapse in the epilogue.
 * Replaces the caller-side code after the attention call in trunk.py:134-137
 *     gate = out[:, :H/2], value = out[:, H/2:], y = sigmoid(gate) * value
 * together with its forward-mode tangent
 *     ydot[t] = sigmoid(gate) (1 - sigmoid(gate)) gatedot[t] * value + sigmoid(gate) valuedot[t]
 * where out and tout[t] are what hz_mhsea_fwd_jvp computes. Head h < H/2 is the gate of
 * head h + H/2. Writes y [B, N, H/2, D] and ty [T, B, N, H/2, D] (masked query rows 0);
 * out, lse and the per-head tangents never reach memory.
 * Served shapes: fp32, any N <= HZ_MAX_N and D, H even, 0 <= T <= 2 (N <= 64 and D <= 32 on
 * the producer/consumer kernel, at D = 32 two directions as two passes; otherwise, and with
 * HZ_FLAG_GENERIC, on the LDS-streaming kernel, which computes the gate head and then the
 * value head of each query block in one workgroup). Required: q, k, v, mask, y, and ty when T >= 1.
 * Optional: e, qt, kt, et, vt (tangent strides B*N*H*D; ty's stride is B*N*(H/2)*D).
 */
int hz_mhsea_fwd_jvp_gated(hipStream_t stream,
                           const void* q, const void* k, const void* e, const void* v,
                           const uint8_t* mask,
                           const void* qt, const void* kt, const void* et, const void* vt,
                           int64_t T, void* y, void* ty,
                           int64_t B, int64_t N, int64_t H, int64_t D,
                           float scale, int flags);

/*
 * Output projection of the attention block after the gate collapse, and its tangents.
 * Replaces the trunk's W_O (src/hamiltonzero/model/trunk.py:138-144) and the tree's w_o with
 * its site mask (model/tree.py:1479-1488: proposal = mask_q * (out_flat @ w_o)):
 *     delta[b, i, :]    = (y[b, i, :] W_o) * (mask[b, i] != 0)        (mask NULL: no factor)
 *     delta_t[t, b, i]  = (ty[t, b, i, :] W_o) * (mask[b, i] != 0)
 * y [B, N, d_attn] is hz_mhsea_fwd_jvp_gated's y [B, N, H/2, D] read as rows (d_attn =
 * H/2 * D), ty [T, B, N, d_attn]; W_o [d_attn, d_e] (BiasFreeLinear, [in, out]); float32,
 * fp32 matrix cores. T in [0, 3]. With a mask (d_attn and d_e multiples of 4), rows with
 * mask 0 are written as zeros without being read or multiplied, so only the physical rows
 * cost matrix work; they equal the formula above for finite y (a NaN or Inf in a masked row
 * of y does not reach delta).
 */
int hz_gated_out_proj(hipStream_t stream, const float* y, const float* ty, const float* w_o, const uint8_t* mask,
                      float* delta, float* delta_t, int64_t B, int64_t N, int64_t d_attn, int64_t d_e, int64_t T);

/*
 * Reverse mode: cotangents of (q, k, e, v) for the upstream cotangent dout. Replaces the
 * transpose rule _inner_transpose (mhsea_tuned.py:206-221 -> mhsea_backward,
 * custom_gradients.py:78-228 -> mhsea_q_vjp_kernel :231-285, mhsea_kv_vjp_kernel
 * :288-347):
 *     dP = dout V^T,  delta = rowsum(out o dout),  dS = P o (dP - delta)  (valid pairs)
 *     dq = scale dS K,  dk = scale dS^T Q,  dv = P^T dout,  de = dS
 * Required: q, k, v, mask, lse, out, dout, dq, dk, dv. Optional: e, de (NULL = not
 * requested). Rows of masked sites are exact zeros in dq, dk, dv and de.
 */
int hz_mhsea_bwd(hipStream_t stream,
                 const void* q, const void* k, const void* e, const void* v,
                 const uint8_t* mask, const float* lse, const void* out, const void* dout,
                 void* dq, void* dk, void* de, void* dv,
                 int64_t B, int64_t N, int64_t H, int64_t D,
                 int dtype, float scale, int flags);

/*
 * Reverse mode of the gated head collapse (hz_mhsea_fwd_jvp_gated's y = sigmoid(g) v):
 * cotangents of (q, k, e, v) for the cotangent dy [B, N, H/2, D] of y. Replaces the reverse
 * pass JAX derives for the trunk's attention call followed by trunk.py:134-137 (the
 * collapse's VJP, then _inner_transpose, mhsea_tuned.py:206-221):
 *     dout[:, :, h]       = dy[:, :, h] v sigmoid(g) (1 - sigmoid(g)),   g = out[:, :, h]
 *     dout[:, :, h + H/2] = dy[:, :, h] sigmoid(g),                      v = out[:, :, h + H/2]
 * then exactly hz_mhsea_bwd on dout. out [B, N, H, D] and lse are the attention's primal
 * outputs (hz_mhsea_fwd); dout_work [B, N, H, D] is caller-owned scratch that receives dout.
 * float32 only; H even; other operands and semantics as hz_mhsea_bwd.
 */
int hz_mhsea_bwd_gated(hipStream_t stream,
                       const void* q, const void* k, const void* e, const void* v,
                       const uint8_t* mask, const float* lse, const void* out, const float* dy,
                       void* dq, void* dk, void* de, void* dv, float* dout_work,
                       int64_t B, int64_t N, int64_t H, int64_t D, float scale, int flags);

/*
 * Rectangular attention with a dense pair bias, forward only (the large-N evaluation
 * path). Replaces noncausal_bias_mha (src/hamiltonzero/evaluation/pallas_mha.py:92-161,
 * kernel :43-89) and its wrapper pallas_rectangular_edge_attention
 * (src/hamiltonzero/evaluation/sequence_parallel.py:59-90):
 *     out[b,i,h] = sum_j softmax_j(scale q[b,i,h].k[b,j,h] + bias'[b,i,j,h]) v[b,j,h]
 *     bias'      = key_mask[b,j] ? bias[b,i,j,h] : -1e30      (sequence_parallel.py:79-83)
 * Layouts: q, out [B, Nq, H, D]; k, v [B, Nk, H, D]; bias [B, Nq, Nk, H] (heads innermost,
 * the reference's [batch, query, key, heads], pallas_mha.py:111); key_mask [B, Nk] uint8.
 * Nq and Nk are independent (a sequence-parallel rank's local queries against all keys).
 * float32 only, as the reference (sequence_parallel.py:42-47). noncausal_bias_mha is
 * scale = 1 with key_mask = NULL; the wrapper is scale = D^-1/2 with its mask.
 * Optional: bias (NULL = zero), key_mask (NULL = every key physical). If no key of a
 * system is physical every score is -1e30 and out is the mean of all Nk value rows, as in
 * the reference's float32 arithmetic. 1 <= Nq, Nk <= HZ_MAX_N; D in {8, 16, 32, 64}.
 */
int hz_rect_attention_fwd(hipStream_t stream,
                          const float* q, const float* k, const float* v,
                          const float* bias, const uint8_t* key_mask, float* out,
                          int64_t B, int64_t Nq, int64_t Nk, int64_t H, int64_t D,
                          float scale);

/*
 * hz_rect_attention_fwd with the large-N caller's head collapse fused into its epilogue.
 * Replaces, in _sequence_level_edge_attention (src/hamiltonzero/evaluation/
 * sequence_trunk.py:973-981), pallas_rectangular_edge_attention followed by
 *     out = sigmoid(out[:, :n_heads]) * out[:, n_heads:]
 * (n_heads = H / 2, the kernel's H = 2 n_heads heads): writes only
 *     y [B, Nq, H/2, D] = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:]
 * with out as hz_rect_attention_fwd defines it (same operands, layouts, mask and scale);
 * the attention output itself never reaches memory. H must be even. The caller's W_O with
 * the row mask (sequence_trunk.py:982-984) is hz_gated_out_proj on y.
 */
int hz_rect_attention_fwd_gated(hipStream_t stream,
                                const float* q, const float* k, const float* v,
                                const float* bias, const uint8_t* key_mask, float* y,
                                int64_t B, int64_t Nq, int64_t Nk, int64_t H, int64_t D,
                                float scale);

#ifdef __cplusplus
}
#endif

#endif /* HZ_MHSEA_H */
