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
};

// T = tangents in this launch (0 = forward only). given_lse selects the tangent-only
// variant that reads out_in / lse_in instead of recomputing the softmax normaliser.
hipError_t launch_fwd(const FwdParams& p, int D, int T, bool given_lse, int dtype,
                      hipStream_t stream);

hipError_t launch_bwd(const BwdParams& p, int D, int dtype, hipStream_t stream);

}  // namespace hz
