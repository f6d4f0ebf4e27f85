/*
 * hz_executor.h — C ABI of the compiled per-walker executor's products on MI355X (gfx950).
 *
 * The compiled executor (src/hamiltonzero/compiled/execute.py:80-125,
 * compiled/model.py:140-168) evaluates the wavefunction of every walker as a tree: a leaf
 * factorized apply, then per level a quadrilinear merge of node pairs followed by a residual
 * factorized apply, then a readout factorized apply. These entry points run those two
 * products for all walkers and nodes of a call at once (rows = walkers x nodes, nodes
 * innermost), and hz_compiled_wavefunction runs the whole tree. Conventions as in hz_mhsea.h:
 * device pointers, row-major, float32 (the reference computes this path in float32:
 * odd_dtype = jnp.float32, execute.py:25,41), enqueue-only on `stream`, nothing allocated,
 * deterministic, 0 or an HZ_E* status with hz_last_error().
 */
#ifndef HZ_EXECUTOR_H
#define HZ_EXECUTOR_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Quadrilinear merge. Replaces quadrilinear_merge_p's impl
 * (src/hamiltonzero/model/_custom_lap_primitives.py:36-50) and
 * _compiled_quadrilinear_merge (src/hamiltonzero/compiled/execute.py:34-52):
 *     out[m, i R + j] = sum_{k, l} T[i, j, k, l] u_a[m, i R + k] u_b[m, i R + l]
 * T [G, R, R, R]; u_a, u_b, out [M, G R] (the reference's u_left / u_right rows flattened
 * over walkers and nodes). R must be 32 (the model's d_r, config.py:21); G >= 1, M >= 1.
 */
int hz_quadrilinear_merge(hipStream_t stream, const float* T, const float* u_a, const float* u_b, float* out,
                          int64_t M, int64_t G, int64_t R);

/*
 * Factorized apply with the conditioner product. Replaces _factorized_apply
 * (src/hamiltonzero/compiled/execute.py:24-31), ((x V) * h) U, and with `residual` the
 * merge level's raw + _factorized_apply(raw) (execute.py:104):
 *     y[m, :] = ((x[m, :] V) o h[m mod h_rows, :]) U  (+ residual[m, :])
 * x [M, d_in], V [d_in, R], h [h_rows, R] (one conditioner row per tree node, broadcast over
 * the walkers: rows are walkers x nodes with nodes innermost, h_rows = nodes; h_rows = 1 for
 * the readout), U [R, d_out], residual [M, d_out] or NULL, y [M, d_out].
 * workspace: M * R floats, caller-owned (holds the conditioned product (x V) o h).
 * Any d_in, R, d_out >= 1 (multiples of 4 take the 16-byte staging path; the readout's
 * d_out = 2, re and im, the per-element one).
 */
int hz_factorized_apply(hipStream_t stream, const float* x, const float* V, const float* h, const float* U,
                        const float* residual, float* y, float* workspace, int64_t M, int64_t d_in, int64_t R,
                        int64_t d_out, int64_t h_rows);

/*
 * Bytes of workspace hz_compiled_wavefunction needs for these sizes (d_m = G * d_r), or -1
 * for a size below 1. No counterpart in the reference (JAX allocates its intermediates).
 */
int64_t hz_compiled_wavefunction_workspace(int64_t B, int64_t n_sites, int64_t d_z, int64_t R_leaf, int64_t d_m,
                                           int64_t R_merge, int64_t R_out);

/*
 * The whole compiled per-walker wavefunction. Replaces
 * CompiledFinetuneWaveFunction._forward_plain (src/hamiltonzero/compiled/model.py:143-175)
 * and execute_wavefunction (compiled/execute.py:79-125) for a batch of B walkers:
 *     z      = q W_q                                         (q_to_odd, model.py:210)
 *     u      = ((z V_leaf) o leaf_h[site]) U_leaf,  u /= rms(u),  s = log rms(u)
 *              (normalize_leaf_carriers, model/model.py:31-37: rms = sqrt(mean(u^2) + 1e-30))
 *     per level (widths n/2, n/4, ..., 1; node p merges nodes 2p, 2p + 1):
 *              raw   = quadrilinear_merge(T, u[2p], u[2p + 1])
 *              out   = raw + ((raw V_merge) o merge_h[level][p]) U_merge
 *              scale = sqrt(mean(out^2) + merge_eps)
 *              u[p]  = both * out / scale + left * u[2p] + right * u[2p + 1]
 *              s[p]  = both * (s[2p] + s[2p + 1] + log scale) + left * s[2p] + right * s[2p + 1]
 *              (both / left / right: opcode MERGE / CARRY_LEFT / CARRY_RIGHT; EMPTY gives 0)
 *     psi     = ((u_root V_out) o readout_h) U_out            (2 values: re, im)
 *     log_abs = 0.5 log(re^2 + im^2) + s_root,  phase = atan2(im, re)   (model.py:177-180)
 * Operands (device, row-major, float32 unless noted, 16-byte aligned):
 *   q [B, n_sites, d_q] (routed site features), q_weight [d_q, d_z], leaf_V [d_z, R_leaf],
 *   leaf_U [R_leaf, d_m], leaf_h [n_sites, R_leaf], merge_T [G, d_r, d_r, d_r],
 *   merge_V [d_m, R_merge], merge_U [R_merge, d_m],
 *   merge_h [L, n_sites / 2, R_merge] and opcodes [L, n_sites / 2] uint8 — the reference's
 *   packed per-level storage (model.py:58-90: level l uses its first n_sites >> (l + 1) rows;
 *   L = log2 n_sites), readout_V [d_m, R_out], readout_U [R_out, 2], readout_h [R_out];
 *   outputs log_abs [B], phase [B]; workspace of hz_compiled_wavefunction_workspace() bytes.
 *   With n_sites == 1 there is no merge level: merge_T, merge_V, merge_U, merge_h and
 *   opcodes are not read and may be NULL.
 * n_sites a power of two (level_widths, compiled/types.py:166-169), d_r = 32, d_m = G d_r <=
 * 2048. Fine-tune sizes: d_q 4, d_z 32, R_leaf 1536, G 48, R_merge 1024, R_out 64
 * (config.py:21-29,189-190; tree.py:2360-2361).
 */
int hz_compiled_wavefunction(hipStream_t stream, const float* q, const float* q_weight, const float* leaf_V,
                             const float* leaf_U, const float* leaf_h, const float* merge_T, const float* merge_V,
                             const float* merge_U, const float* merge_h, const uint8_t* opcodes, const float* readout_V,
                             const float* readout_U, const float* readout_h, float* log_abs, float* phase,
                             void* workspace, int64_t workspace_bytes, int64_t B, int64_t n_sites, int64_t d_q,
                             int64_t d_z, int64_t R_leaf, int64_t G, int64_t d_r, int64_t R_merge, int64_t R_out,
                             float merge_eps);

/*
 * Factorized apply that allocates nothing. No counterpart in the reference: it is for callers
 * that cannot allocate device memory or pass a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same operands and result as
 * hz_factorized_apply (bit-identical: the same kernels per row), without `workspace`: the
 * conditioned product lives in a static device array of 8 Mi floats (32 MiB) that every GPU
 * the library runs on holds from its first call there until the process ends. Rows are
 * processed in chunks of floor(8 Mi / R / 128) * 128 rows, so M is limited only by the grid
 * (as in hz_factorized_apply); R <= 65536 (HZ_EINVAL beyond). The array needs no clearing:
 * each chunk writes every entry it reads. All calls on one GPU share its array: calls that
 * overlap on one GPU (concurrent streams or threads) race and must be serialised by the
 * caller. The array is resolved for the device of `stream` on the first call there.
 */
int hz_factorized_apply_noalloc(hipStream_t stream, const float* x, const float* V, const float* h, const float* U,
                                const float* residual, float* y, int64_t M, int64_t d_in, int64_t R, int64_t d_out,
                                int64_t h_rows);

#ifdef __cplusplus
}
#endif

#endif /* HZ_EXECUTOR_H */
