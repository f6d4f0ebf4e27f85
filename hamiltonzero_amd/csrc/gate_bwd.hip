// Cotangent of the trunk's sigmoid-gate head collapse, y = sigmoid(g) v with gate head
// g = out[:, :, h] and value head v = out[:, :, h + H/2] (h < H/2), for the attention
// backward that follows it:
//     dout[:, :, h]        = dy[:, :, h] v sigmoid(g) (1 - sigmoid(g))
//     dout[:, :, h + H/2]  = dy[:, :, h] sigmoid(g)
// One thread per 4 consecutive elements of a (site, head pair) row, float4 in and out.
#include <hip/hip_runtime.h>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

__global__ void __launch_bounds__(256) gate_collapse_bwd_kernel(const float* __restrict__ out,
                                                                 const float* __restrict__ dy,
                                                                 float* __restrict__ dout, int64_t items, int hh,
                                                                 int D) {
  const int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (it >= items) return;
  const int d4 = D / 4;
  const int64_t row = it / (static_cast<int64_t>(hh) * d4);  // site (walker x N)
  const int rem = static_cast<int>(it - row * hh * d4);
  const int h = rem / d4, c = (rem - h * d4) * 4;
  const int64_t g_off = (row * 2 * hh + h) * D + c, v_off = g_off + static_cast<int64_t>(hh) * D;
  const float4 g = *reinterpret_cast<const float4*>(out + g_off);
  const float4 v = *reinterpret_cast<const float4*>(out + v_off);
  const float4 d = *reinterpret_cast<const float4*>(dy + (row * hh + h) * D + c);
  float4 dg, dv;
  auto one = [](float gi, float vi, float di, float& dgi, float& dvi) {
    const float s = __builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * gi));
    dgi = di * vi * s * (1.f - s);
    dvi = di * s;
  };
  one(g.x, v.x, d.x, dg.x, dv.x);
  one(g.y, v.y, d.y, dg.y, dv.y);
  one(g.z, v.z, d.z, dg.z, dv.z);
  one(g.w, v.w, d.w, dg.w, dv.w);
  *reinterpret_cast<float4*>(dout + g_off) = dg;
  *reinterpret_cast<float4*>(dout + v_off) = dv;
}

}  // namespace

hipError_t launch_gate_collapse_bwd(const float* out, const float* dy, float* dout, int64_t sites, int H, int D,
                                    hipStream_t stream) {
  const int hh = H / 2;
  const int64_t items = sites * hh * (D / 4);
  hipLaunchKernelGGL(gate_collapse_bwd_kernel, dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0, stream,
                     out, dy, dout, items, hh, D);
  return hipGetLastError();
}

}  // namespace hz
