// Host-side launch interface between the C ABI (mhsea_abi.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hz {

// Everything the forward / tangent kernel family reads. Tensors follow include/hz_mhsea.h.
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* e;  // may be null
  const uint8_t* mask;
  const void* qt;  // [T, B, N, H, D]; may be null (zero tangent)
  const void* kt;
  const void* vt;
  const void* et;      // [T, <e layout>]; may be null
  const void* out_in;  // primal out, read by the tangent-only variant
  const float* lse_in;
  void* out;   // written by the forward variants
  float* lse;  // may be null
  void* tout;  // [T, B, N, H, D]
  int B, N, H;
  int64_t t_stride;   // elements between tangent directions of qt/kt/vt/tout
  int64_t et_stride;  // elements between tangent directions of et
  int64_t e_sq, e_sh, e_sk;  // element strides of e inside one walker (walker stride N*N*H)
  float scale;
  int key_mask;  // 1: reference_edge_attention masking (keys only)
  float masked_lse;
  int force_generic;  // 1: always use the LDS-streaming kernel
  // 1: gated head collapse (producer/consumer and LDS-streaming fp32 kernels): out is y [B, N, H/2, D] =
  // sigmoid(O[:, :, h]) * O[:, :, h + H/2], tout its tangents [T, B, N, H/2, D] with
  // y_tstride elements between directions; lse is not written
  int gated;
  int64_t y_tstride;
  // 1: e / et in the compacted physical-pair layout ([B, H, N, ceil4(N)] blocks of n rows of
  // stride ceil4(n), the kernel's own query and key order); producer/consumer kernel only
  int e_compact;
};

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* e;  // may be null
  const uint8_t* mask;
  const float* lse;
  const void* out;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  void* de;  // may be null
  int B, N, H;
  int64_t e_sq, e_sh, e_sk;
  float scale;
  int key_mask;
  int force_generic;  // 1: always use the two-kernel path
};

// T = tangents in this launch (0 = forward only). given_lse selects the tangent-only
// variant that reads out_in / lse_in instead of recomputing the softmax normaliser.
hipError_t launch_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                      hipStream_t stream);

hipError_t launch_bwd(const BwdParams& p, int D, int dtype, hipStream_t stream);

// Register-resident kernel for N <= 64: a wave keeps every key operand of its
// (walker, head) in registers, K/Kt as D/4 and V/Vt as 4 ceil(D/16) floats per key tile
// and tensor; the budget of 128 such floats bounds the number of 16-key tiles.
constexpr int small_max_key_tiles(int D, int T) {
  return (128 / ((D / 4 + 4 * ((D + 15) / 16)) * (1 + T))) > 4
             ? 4
             : (128 / ((D / 4 + 4 * ((D + 15) / 16)) * (1 + T)));
}
template <int D, int T>
struct SmallFits {
  static constexpr int kMaxKeyTiles = small_max_key_tiles(D, T);
};
bool small_fwd_supported(int N, int D, int T);
bool stream_fwd_supported(int N, int D, int T, int dtype);
hipError_t launch_fwd_stream(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                             hipStream_t stream);
bool stream_bwd_supported(int N);
hipError_t launch_bwd_stream(const BwdParams& p, int D, int dtype, hipStream_t stream);
bool bf16_fwd_supported(int D);
// Large-N bfloat16 kernel (N > 128): 128-query workgroups, double-buffered LDS key chunks.
bool bf16_large_fwd_supported(int N, int D);
hipError_t launch_fwd_bf16_large(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream);
// Large-N bfloat16 kernel at D = 64 without a bias (N > 128): 32-query tiles on the 32x32x16
// matrix instruction, each served by a score wave and a value wave (two waves per SIMD);
// forward variants only, scale > 0.
bool bf16_ws_fwd_supported(const FwdParams& p, int D, bool given_lse);
hipError_t launch_fwd_bf16_ws(const FwdParams& p, int T, hipStream_t stream);
bool bf16_bwd_supported(int N, int H, int D);
hipError_t launch_bwd_bf16(const BwdParams& p, int D, hipStream_t stream);
hipError_t launch_fwd_bf16(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream);
// Producer/consumer kernel (float32, N <= 64): key tiles gathered into LDS.
bool pc_fwd_supported(int N, int H, int D, int T, int dtype);
hipError_t launch_fwd_pc(const FwdParams& p, int D, int T, bool given_lse, hipStream_t stream);
// The gated collapse on the LDS-streaming fp32 kernel (any N, D): p.gated layout as above,
// T <= 2 in one launch.
hipError_t launch_fwd_gated_generic(const FwdParams& p, int D, int T, hipStream_t stream);
// dout [B, N, H, D] of the attention from the collapse's cotangent dy [B, N, H/2, D] and the
// attention output out [B, N, H, D] (gate_bwd.hip), fp32, D a multiple of 4.
hipError_t launch_gate_collapse_bwd(const float* out, const float* dy, float* dout, int64_t sites, int H, int D,
                                    hipStream_t stream);
// Compute units of the current device (cached per device).
hipError_t device_cu_count(int* cus);
hipError_t launch_fwd_small(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                            hipStream_t stream);

// Walkers with no physical site under the additive key mask (mhsea_keymask_empty.hip):
// rewrites their results with the reference's float32-rounded penalised logits. Launched
// after the main kernels of every HZ_FLAG_KEY_MASK call; tangent pointers are the bases of
// all T directions. With p.gated it writes the collapse y / ty (float32).
hipError_t launch_keymask_empty_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                                    hipStream_t stream);
hipError_t launch_keymask_empty_bwd(const BwdParams& p, int D, int dtype, hipStream_t stream);

// The compiled executor's products (executor.hip), float32. Quadrilinear merge with rank 32:
// out[m, 32 i + j] = sum_{k,l} T[i, j, k, l] ua[m, 32 i + k] ub[m, 32 i + l] for G groups.
hipError_t launch_quadrilinear_merge(const float* T, const float* ua, const float* ub, float* out, int64_t M, int G,
                                     int64_t ld_in, hipStream_t stream);
// y = ((x V) o h[m mod h_rows]) U (+ residual); work holds the M x R conditioned product.
hipError_t launch_factorized_apply(const float* x, const float* V, const float* h, const float* U,
                                   const float* residual, float* y, float* work, int64_t M, int d_in, int R, int d_out,
                                   int h_rows, hipStream_t stream);
// The same apply with its workspace in a static device array of kApplyScratchFloats floats
// (executor.hip), rows processed in chunks of whole 128-row tiles; R <= kApplyScratchMaxRank.
// Allocates nothing.
// delta = (y W_o) o (mask[row] != 0) over M rows (mask may be null): the attention block's
// output projection after the gate collapse.
hipError_t launch_out_proj(const float* y, const float* w_o, const uint8_t* mask, float* delta, int64_t M, int d_in,
                           int d_out, hipStream_t stream);
// The whole per-walker wavefunction of the compiled executor (leaf, every merge level,
// readout) on one stream; workspace of compiled_wavefunction_workspace_bytes().
struct WaveFnParams {
  const float* q;          // [B, n, d_q]
  const float* q_weight;   // [d_q, d_z]
  const float* leaf_V;     // [d_z, r_leaf]
  const float* leaf_U;     // [r_leaf, d_m]
  const float* leaf_h;     // [n, r_leaf]
  const float* merge_T;    // [d_m / 32, 32, 32, 32]
  const float* merge_V;    // [d_m, r_merge]
  const float* merge_U;    // [r_merge, d_m]
  const float* merge_h;    // [levels, n / 2, r_merge]
  const uint8_t* opcodes;  // [levels, n / 2]
  const float* readout_V;  // [d_m, r_out]
  const float* readout_U;  // [r_out, 2]
  const float* readout_h;  // [r_out]
  float* log_abs;          // [B]
  float* phase;            // [B]
  float* workspace;
  int64_t B;
  int n, d_q, d_z, r_leaf, d_m, r_merge, r_out;
  float merge_eps;
};
constexpr int kRowMaxFloats = 2048;  // widest carrier row the row epilogues take
int64_t compiled_wavefunction_workspace_bytes(int64_t B, int64_t n, int64_t d_z, int64_t r_leaf, int64_t d_m,
                                              int64_t r_merge, int64_t r_out);
hipError_t launch_compiled_wavefunction(const WaveFnParams& p, hipStream_t stream);
constexpr int64_t kApplyScratchFloats = int64_t(8) << 20;           // 32 MiB
constexpr int64_t kApplyScratchMaxRank = kApplyScratchFloats / 128;  // 65536
hipError_t launch_factorized_apply_noalloc(const float* x, const float* V, const float* h, const float* U,
                                           const float* residual, float* y, int64_t M, int d_in, int R, int d_out,
                                           int h_rows, hipStream_t stream);

// Coupling-bias producer of the trunk attention (pair_bias.hip): RMS + one-block MLP +
// 1/div per site pair, written with strides (e_sq, e_sh, e_sk) inside a walker's
// N x N x H block; T = 1 adds the tangent along edge_t into e_t.
struct PairBiasParams {
  const float* edge;     // [B, N, N, C]
  const float* edge_t;   // [B, N, N, C] or null
  const uint8_t* mask;   // [B, N] or null
  const float* ln_w;
  const float* w_in;
  const float* b_in;
  const float* w_1;
  const float* b_1;
  const float* w_2;
  const float* b_2;
  const float* w_out;
  const float* b_out;
  float* e;
  float* e_t;
  int64_t B;
  int N;
  int64_t e_sq, e_sh, e_sk;
  int64_t e_blk;        // > 0: compacted layout, floats per (walker, head) block (N * ceil4(N))
  float gain, eps, div;
  bool key_mask;        // compute every query row (key-mask attention semantics)
  int parts;            // items per walker (set by the launcher)
  int64_t n_items;      // B * parts (set by the launcher)
};
hipError_t launch_pair_bias(PairBiasParams p, int C, int H, bool tan, hipStream_t stream);

// The MLP-class pair-bias producer with the LCA-ALiBi term (pair_mlp_bias.hip).
struct PairMlpParams {
  const float* edge;        // [B, Nq, Nk, C]
  const float* edge_t;      // [B, Nq, Nk, C] or null
  const float* extra;       // [B, Nq, Nk] or null (one more input channel, w_in row C)
  const float* extra_t;     // [B, Nq, Nk] or null
  const uint8_t* mask;      // [B, Nk] or null
  const float* w_in;        // [C (+1), hidden]
  const float* b_in;        // [hidden]
  const float* norm_w;      // [n_blocks, hidden]
  const float* w_1;         // [n_blocks, hidden, hidden]
  const float* b_1;         // [n_blocks, hidden]
  const float* w_2;
  const float* b_2;
  const float* out_norm_w;  // [hidden]
  const float* w_out;       // [hidden, H]
  const float* b_out;       // [H]
  const float* slopes;      // [H] or null (no LCA-ALiBi term)
  float* e;
  float* e_t;
  int64_t B;
  int Nq, Nk, n_blocks, row_offset;
  int64_t e_sq, e_sh, e_sk;
  float gain, eps, div;
  bool key_mask;            // compute every query row (key-mask attention semantics)
  int parts;                // items per walker (set by the launcher)
  int64_t n_items;          // B * parts (set by the launcher)
};
hipError_t launch_pair_mlp_bias(PairMlpParams p, int C, int hidden, int H, bool tan, hipStream_t stream);
// Blocks whose weights fit the LDS next to the other fragments at this hidden width.
int pair_mlp_max_blocks(int hidden);

// Rectangular attention with a dense [B, Nq, Nk, H] bias (rect_attention.hip).
struct RectParams {
  const float* q;      // [B, Nq, H, D]
  const float* k;      // [B, Nk, H, D]
  const float* v;      // [B, Nk, H, D]
  const float* bias;   // [B, Nq, Nk, H]; may be null (zero bias)
  const uint8_t* key_mask;  // [B, Nk]; may be null (every key physical)
  float* out;          // [B, Nq, H, D]; gated: y [B, Nq, H / 2, D]
  int B, Nq, Nk, H;
  float scale;
  int gated;           // 1: y = sigmoid(out[:, :, :H/2]) * out[:, :, H/2:] instead of out
};
hipError_t launch_rect_fwd(const RectParams& p, int D, hipStream_t stream);
// Dynamic LDS the rectangular kernel needs (largest variant for this D, H).
size_t rect_fwd_lds_bytes(int D, int H, int Nk, bool masked, bool gated);

}  // namespace hz
