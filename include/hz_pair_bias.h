/*
 * hz_pair_bias.h — C ABI of the trunk attention's coupling-bias producer on MI355X (gfx950).
 *
 * Replaces the producer of the attention bias inside MultiHeadEvenAttention.__call__
 * (src/hamiltonzero/model/trunk.py:89-105): ln_edge (eqx-style RMS, odd_ops.py:183-215,
 * model/tree.py:339-375), bias_mlp (UnnormalizedMLP with one block, odd_ops.py:279-316) and
 * the division by sqrt(d_head), per site pair (i, j) of every walker:
 *
 *     y    = x * (ln_w * rsqrt(mean(x^2) + eps))                x = edge[b, i, j, :]
 *     h0   = y W_in + b_in
 *     h1   = h0 + inner_gain * (silu(h0 W_1 + b_1) W_2 + b_2)
 *     e    = (h1 W_out + b_out) / bias_div
 *
 * and, with T = 1, its forward-mode derivative e_t along edge_t (parameters held fixed), as
 * jax.jvp of the reference would give. The output goes straight into the attention's bias
 * layout (hz_mhsea.h: [B, N, H, N], or [B, N, N, H] with HZ_FLAG_E_QKH, the reference's
 * coup_bias layout), so hz_mhsea_fwd_jvp / hz_mhsea_fwd_jvp_gated read it with no transpose.
 * All arithmetic is float32 with float32 accumulation (the reference's compute dtype,
 * model/fp32.py:7-8), on the matrix cores.
 *
 * Operands (device pointers, row-major, float32, 16-byte aligned):
 *   edge [B, N, N, C], edge_t [B, N, N, C] (T = 1) or NULL (T = 0), mask [B, N] uint8 or NULL,
 *   ln_w [C], w_in [C, hidden], b_in [hidden], w_1 / w_2 [hidden, hidden], b_1 / b_2
 *   [hidden], w_out [hidden, H], b_out [H]; e (and e_t) in the attention's bias layout.
 * Sizes: C in {32, 64, 96, 128} (edge_channels, config.py:28: 96), hidden = 64
 * (trunk_attention_bias_hidden_dim, config.py:31), H in {16, 32, 64} (2 n_heads: 32),
 * 1 <= N <= HZ_MAX_N, B >= 1, T in {0, 1}. inner_gain = n_layers^-1/2 (trunk.py:61),
 * eps = 1e-5 (odd_ops.py:185), bias_div = sqrt(d_head) (trunk.py:103-105).
 *
 * HZ_FLAG_E_COMPACT (hz_mhsea.h): e / e_t in the compacted physical-pair layout [B, H, N,
 * ceil4(N)] that the N <= 64 forward family reads with the same flag — pair (i, j) of the
 * walker's ascending physical-site list at i * ceil4(n) + j of head h's block, so the rows are
 * contiguous and hold only the pairs the attention reads. Square mask only (not with
 * HZ_FLAG_KEY_MASK or HZ_FLAG_E_QKH); with a mask, N <= 256; with mask == NULL every site
 * counts as physical.
 *
 * Mask: with mask != NULL and N <= 256 only the pairs the attention reads are computed and
 * written — keys with mask[j] != 0, and queries with mask[i] != 0 unless HZ_FLAG_KEY_MASK
 * (whose attention computes every query row); in key-mask mode a walker with no physical
 * site gets every pair (the key-mask attention then uses every key). Other entries of e /
 * e_t are left untouched. With mask == NULL (or N > 256) every pair is computed, which is
 * the reference's full coup_bias.
 *
 * Enqueue-only on `stream`, nothing allocated, deterministic; 0 or an HZ_E* status with
 * hz_last_error() (argument errors are found on the host before any GPU work).
 */
#ifndef HZ_PAIR_BIAS_H
#define HZ_PAIR_BIAS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

int hz_pair_bias(hipStream_t stream, const float* edge, const float* edge_t, const uint8_t* mask, const float* ln_w,
                 const float* w_in, const float* b_in, const float* w_1, const float* b_1, const float* w_2,
                 const float* b_2, const float* w_out, const float* b_out, float* e, float* e_t, int64_t B, int64_t N,
                 int64_t C, int64_t hidden, int64_t H, int64_t T, float inner_gain, float eps, float bias_div,
                 int flags);

/*
 * The MLP-class pair-bias producer, with the LCA-ALiBi term. Replaces the coupling-bias
 * computation of the tree's LevelEdgeAttn (src/hamiltonzero/model/tree.py:1392-1456), of the
 * readout context's _attend (model/readout_leaf_context.py:694-712) and of the large-N
 * sequence trunk (evaluation/sequence_trunk.py:962-972, _pair_mlp_tiled + lca_alibi_bias):
 * bias_mlp is the normalised MLP (model/odd_ops.py:218-276: in_proj, n_blocks residual blocks
 * each with an RMS norm before its first Linear, an RMS norm before out_proj), per pair
 *
 *     h    = x W_in[:C] + xe W_in[C] + b_in          x = edge[b, i, j, :], xe = extra[b, i, j]
 *     h   += inner_gain * (silu(rms_k(h) W_1[k] + b_1[k]) W_2[k] + b_2[k])   for k < n_blocks
 *     e    = (rms_out(h) W_out + b_out) / bias_div - slope[h] * lca(row_offset + i, j)
 *     rms_k(h) = h * norm_w[k] * rsqrt(mean(h^2) + eps)           (_RMS, odd_ops.py:183-215)
 *     lca(p, q) = min(bit length of p ^ q, 13)    (lca_level, readout_leaf_context.py:140-148)
 *
 * and, with T = 1, its forward-mode derivative e_t along (edge_t, extra_t) (parameters fixed;
 * the ALiBi term is constant). The readout concatenates [edge_n, direction] as the MLP input
 * (readout_leaf_context.py:694): pass direction as `extra` and W_in with C + 1 rows. The tree
 * adds the ALiBi term with positions 0..n-1 on both sides (tree.py:1448-1451, only when
 * level_idx is given: pass alibi_slopes = NULL otherwise); the large-N trunk with the global
 * row index of its local query rows (sequence_trunk.py:964-971: row_offset).
 * slopes = lca_fixed_slopes(H) (readout_leaf_context.py:151-154) or any [H] vector.
 *
 * Operands (device pointers, float32, 16-byte aligned except extra / extra_t): edge / edge_t
 * [B, Nq, Nk, C]; extra / extra_t [B, Nq, Nk] or NULL; mask [B, Nk] uint8 or NULL; w_in
 * [C (+1 with extra), hidden]; b_in [hidden]; norm_w [n_blocks, hidden]; w_1 / w_2
 * [n_blocks, hidden, hidden]; b_1 / b_2 [n_blocks, hidden]; out_norm_w [hidden]; w_out
 * [hidden, H]; b_out [H]; alibi_slopes [H] or NULL; e (and e_t) [B, Nq, H, Nk], or
 * [B, Nq, Nk, H] with HZ_FLAG_E_QKH (the reference's layout; the rectangular attention's).
 * Sizes: C in {32, 64, 96, 128}; hidden in {32, 64, 128} (level_edge_bias_mlp_dim 128,
 * readout_context_bias_dim 32, config.py:82,80); H in {16, 32}; n_blocks 1 or 2 (1 at hidden
 * 128); T in {0, 1}. Mask as hz_pair_bias (keys and, without HZ_FLAG_KEY_MASK, queries; a
 * square mask needs Nq == Nk): with Nk <= 256 only the pairs the attention reads are written,
 * beyond that every pair is computed.
 *
 * Enqueue-only, nothing allocated, deterministic; 0 or an HZ_E* status with hz_last_error().
 */
int hz_pair_mlp_bias(hipStream_t stream, const float* edge, const float* edge_t, const float* extra,
                     const float* extra_t, const uint8_t* mask, const float* w_in, const float* b_in,
                     const float* norm_w, const float* w_1, const float* b_1, const float* w_2, const float* b_2,
                     const float* out_norm_w, const float* w_out, const float* b_out, const float* alibi_slopes,
                     float* e, float* e_t, int64_t B, int64_t Nq, int64_t Nk, int64_t C, int64_t hidden, int64_t H,
                     int64_t n_blocks, int64_t T, int64_t row_offset, float inner_gain, float eps, float bias_div,
                     int flags);

#ifdef __cplusplus
}
#endif

#endif /* HZ_PAIR_BIAS_H */
