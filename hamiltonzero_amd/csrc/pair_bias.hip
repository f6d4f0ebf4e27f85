// The trunk attention's coupling-bias producer on the float32 matrix cores
// (v_mfma_f32_16x16x4_f32): per site pair (i, j) of a walker,
//     y   = x * (w * rsqrt(mean(x^2) + eps))           x = edge[b, i, j, :] (C channels)
//     h0  = y W_in + b_in                               (64 hidden)
//     h1  = h0 + gain * (silu(h0 W_1 + b_1) W_2 + b_2)
//     e   = (h1 W_out + b_out) / div                    (H heads)
// and, with a tangent edge_t, its forward-mode derivative, written straight into the
// attention kernels' bias layout: [B, N, H, N] / [B, N, N, H], or the compacted layout
// (e_blk > 0), where pair (i, j) of the walker's physical-site list goes to i * ceil4(n) + j
// of head h's block, so the attention reads n * ceil4(n) contiguous floats per (walker, head)
// instead of n rows of N.
//
// Orientation: every layer is computed transposed, features x pairs (features = the 16-row
// M blocks, 16 pairs = one N block), so the pairs are the columns of the B operand and the
// weights (staged once per workgroup in LDS, as ready-made A fragments) the A operand. A
// layer's result C[feature 4g + r][pair c] sits in lane (g, c) register r, which is exactly
// the B operand the next layer needs if that layer's K order is permuted: K step (kb, r) of
// lane group g multiplies feature 16 kb + 4 g + r. The weight fragments are stored in that
// order, so the four layers chain in registers with no LDS round trip.
//
// The RMS scale r is a per-pair (column) scale: layer 1 runs on x * w and scales columns by r
// afterwards, so x streams straight from memory into the products while mean(x^2) (and,
// with a tangent, mean(x xdot)) accumulate alongside; the tangent of layer 1 is
// r (xdot * w) W_in + rdot (x * w) W_in with rdot = -0.5 r / v * 2 mean(x xdot).
//
// A tile is 16 pairs with their tangent (T = 1: N block 0 primal, N block 1 tangent) or 32
// pairs (T = 0). With a mask, only pairs whose key site is physical are computed (and, in
// the square-mask semantics, whose query site is physical too): a wave builds the walker's
// list of physical sites with a ballot, then walks the flattened (query, key) pair list.
// Each wave is persistent over (walker, part) items; a workgroup's four waves share the
// staged weights.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

constexpr int kHid = 64;          // bias_mlp hidden width (trunk_attention_bias_hidden_dim)
constexpr int kPBWaves = 4;       // waves per workgroup
constexpr int kPBListN = 256;     // sites per walker the pair compaction handles

template <int C, int HB>
struct PBLds {
  static constexpr int kF1 = 0;                  // W_in fragments: 4 M blocks x C/4 K steps x 64 lanes
  static constexpr int kF2 = kF1 + 64 * C;       // W_1 fragments: 4 x 16 x 64
  static constexpr int kF3 = kF2 + 4096;         // W_2 fragments
  static constexpr int kF4 = kF3 + 4096;         // W_out fragments: HB x 16 x 64
  static constexpr int kBin = kF4 + 1024 * HB;
  static constexpr int kB1 = kBin + kHid;
  static constexpr int kB2 = kB1 + kHid;
  static constexpr int kBout = kB2 + kHid;
  static constexpr int kLnw = kBout + 16 * HB;
  static constexpr int kFloats = kLnw + C;
};

__device__ __forceinline__ float4 lds4(const float* base, int off) {
  return *reinterpret_cast<const float4*>(base + off);
}

__device__ __forceinline__ float comp(const float4& v, int u) {
  return u == 0 ? v.x : (u == 1 ? v.y : (u == 2 ? v.z : v.w));
}

// sigmoid(u) = 1 / (1 + 2^(-u log2 e)) on the hardware exp2 and reciprocal (about 1 ulp each;
// the exponent's rounding adds |u| 2^-24 relative): a few instructions instead of a
// full-precision expf and an IEEE division. u -> -inf gives 2^+inf = inf and 1/inf = 0.
__device__ __forceinline__ float sigmoid(float u) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * -1.44269504088896341f));
}

// The pairs of lane column c in tile t (N block cb): query site qi, key site qj, valid, and
// the pair's offset in a compacted (walker, head) block, row * ceil4(nk) + key (list order).
template <bool TAN>
__device__ __forceinline__ void tile_pairs(int t, int c, int npairs, int nk, bool rows_listed, bool keys_listed,
                                           const unsigned short* list, int qi[2], int qj[2], bool valid[2],
                                           int cpos[2]) {
  constexpr int TP = TAN ? 16 : 32;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int q = TAN ? TP * t + c : TP * t + 16 * cb + c;
    valid[cb] = q < npairs;
    const int qq = valid[cb] ? q : 0;
    const int ii = qq / nk, jj = qq - ii * nk;
    qi[cb] = rows_listed ? list[ii] : ii;
    qj[cb] = keys_listed ? list[jj] : jj;
    cpos[cb] = ii * ((nk + 3) & ~3) + jj;
  }
}

// This lane's quarter (C / 4 channels) of the edge rows of its pairs (T = 1: the pair's edge
// and edge_t rows; T = 0: the rows of the two pairs).
template <int C, bool TAN>
__device__ __forceinline__ void load_rows(const float* edge_b, const float* edge_tb, int N, int g, const int qi[2],
                                          const int qj[2], const bool valid[2], float4 xin[2][C / 16]) {
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int src = TAN ? 0 : cb;
    const float* row = (TAN && cb == 1 ? edge_tb : edge_b) + (static_cast<int64_t>(qi[src]) * N + qj[src]) * C +
                       g * (C / 4);
#pragma unroll
    for (int v = 0; v < C / 16; ++v)
      xin[cb][v] = valid[src] ? *reinterpret_cast<const float4*>(row + 4 * v) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Workgroups per CU: two while the staged weights and the wave lists fit half of the LDS
// (every instantiation but C = 128 with 64 heads, whose weights take 83.5 KB), else one.
template <int C, int HB>
constexpr int pb_occupancy() {
  return (PBLds<C, HB>::kFloats * 4 + kPBWaves * kPBListN * 2) <= 80 * 1024 ? 2 : 1;
}

template <int C, int HB, bool TAN>
__global__ void __launch_bounds__(256, (pb_occupancy<C, HB>())) pair_bias_kernel(PairBiasParams p) {
  using L = PBLds<C, HB>;
  constexpr int C4 = C / 4;    // channels per lane group = layer-1 K steps
  constexpr int CG = C / 16;   // float4 groups per lane group
  constexpr int H = 16 * HB;
  constexpr int TP = TAN ? 16 : 32;  // pairs per tile
  __shared__ __attribute__((aligned(16))) float lds[L::kFloats];
  __shared__ unsigned short lists[kPBWaves][kPBListN];

  // ---- stage the weights as A fragments (once per workgroup) ----
  for (int f = threadIdx.x; f < 64 * C; f += blockDim.x) {
    const int u = f & 3, lane = (f >> 2) & 63, rest = f >> 8;
    const int sg = rest % CG, m = rest / CG;
    const int k = (lane >> 4) * C4 + 4 * sg + u;
    lds[L::kF1 + f] = p.w_in[k * kHid + 16 * m + (lane & 15)];
  }
  for (int f = threadIdx.x; f < 4096; f += blockDim.x) {
    const int u = f & 3, lane = (f >> 2) & 63, kb = (f >> 8) & 3, m = f >> 10;
    const int k = 16 * kb + 4 * (lane >> 4) + u, o = 16 * m + (lane & 15);
    lds[L::kF2 + f] = p.w_1[k * kHid + o];
    lds[L::kF3 + f] = p.w_2[k * kHid + o];
  }
  for (int f = threadIdx.x; f < 1024 * HB; f += blockDim.x) {
    const int u = f & 3, lane = (f >> 2) & 63, kb = (f >> 8) & 3, m = f >> 10;
    const int k = 16 * kb + 4 * (lane >> 4) + u;
    lds[L::kF4 + f] = p.w_out[k * H + 16 * m + (lane & 15)];
  }
  for (int f = threadIdx.x; f < kHid; f += blockDim.x) {
    lds[L::kBin + f] = p.b_in[f];
    lds[L::kB1 + f] = p.b_1[f];
    lds[L::kB2 + f] = p.b_2[f];
  }
  for (int f = threadIdx.x; f < H; f += blockDim.x) lds[L::kBout + f] = p.b_out[f];
  for (int f = threadIdx.x; f < C; f += blockDim.x) lds[L::kLnw + f] = p.ln_w[f];
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  unsigned short* list = lists[wave];
  const int N = p.N;
  const int64_t pair_stride = static_cast<int64_t>(N) * N;
  const bool use_list = p.mask != nullptr && N <= kPBListN;
  const float inv_c = 1.0f / static_cast<float>(C);
  // 1 / sqrt(d_head): exact for the power-of-two d_head the model uses (16), within 1 ulp of
  // the reference's division otherwise.
  const float inv_div = 1.0f / p.div;
  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * kPBWaves;

  for (int64_t item = static_cast<int64_t>(blockIdx.x) * kPBWaves + wave; item < p.n_items; item += total_waves) {
    const int64_t b = item / p.parts;
    const int part = static_cast<int>(item - b * p.parts);

    // ---- the walker's physical sites ----
    int nk = N;
    bool keys_listed = false, rows_listed = false;
    if (use_list) {
      int n = 0;
      for (int s0 = 0; s0 < N; s0 += 64) {
        const int site = s0 + lane;
        const bool phys = site < N && p.mask[b * N + site] != 0;
        const uint64_t bal = __ballot(phys);
        if (phys) list[n + __popcll(bal & ((1ull << lane) - 1ull))] = static_cast<unsigned short>(site);
        n += __popcll(bal);
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (n > 0) {
        nk = n;
        keys_listed = true;
        rows_listed = !p.key_mask;
      } else if (!p.key_mask) {
        continue;  // square mask, no physical site: the attention never reads this walker's bias
      }
    }
    const int nrows = rows_listed ? nk : N;
    const int npairs = nrows * nk;
    const int ntiles = (npairs + TP - 1) / TP;
    const int t0 = static_cast<int>(static_cast<int64_t>(ntiles) * part / p.parts);
    const int t1 = static_cast<int>(static_cast<int64_t>(ntiles) * (part + 1) / p.parts);

    const float* edge_b = p.edge + b * pair_stride * C;
    const float* edge_tb = TAN ? p.edge_t + b * pair_stride * C : nullptr;
    const bool cmp = p.e_blk > 0;
    const int64_t wstride = cmp ? p.e_blk * H : pair_stride * H;
    float* e_b = p.e + b * wstride;
    float* et_b = TAN ? p.e_t + b * wstride : nullptr;

    // The edge rows of the item's first tile; each tile then loads the next tile's rows as
    // soon as its first layer has consumed its own, so the loads fly under layers 2-4.
    int qi[2], qj[2], cpos[2];
    bool valid[2];
    float4 xin[2][CG];
    if (t0 < t1) {
      tile_pairs<TAN>(t0, c, npairs, nk, rows_listed, keys_listed, list, qi, qj, valid, cpos);
      load_rows<C, TAN>(edge_b, edge_tb, N, g, qi, qj, valid, xin);
    }
    for (int t = t0; t < t1; ++t) {
      // The weight fragments are the same for every tile; an offset the compiler cannot see
      // through keeps their LDS reads inside the loop (hoisted, they would need 256 registers).
      int lz = 0;
      asm volatile("" : "+s"(lz));
      const float* W = lds + lz;

      // ---- layer 1: P = (x * w) W_in, with sum(x^2) and sum(x xdot) alongside ----
      v4f acc[4][2];
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = zero4();
      float s0 = 0.f, s1 = 0.f;  // sum x0^2; T = 1: sum x0 xdot, T = 0: sum x1^2
#pragma unroll
      for (int sg = 0; sg < CG; ++sg) {
        const float4 w4 = lds4(W, L::kLnw + g * C4 + 4 * sg);
        float4 a4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) a4[m] = lds4(W, L::kF1 + ((m * CG + sg) * 64 + lane) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float x0 = comp(xin[0][sg], u), x1 = comp(xin[1][sg], u), w = comp(w4, u);
          s0 += x0 * x0;
          s1 += TAN ? x0 * x1 : x1 * x1;
          const float b0 = x0 * w, b1 = x1 * w;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            acc[m][0] = mfma16x4(comp(a4[m], u), b0, acc[m][0]);
            acc[m][1] = mfma16x4(comp(a4[m], u), b1, acc[m][1]);
          }
        }
      }
      s0 += __shfl_xor(s0, 16);
      s0 += __shfl_xor(s0, 32);
      s1 += __shfl_xor(s1, 16);
      s1 += __shfl_xor(s1, 32);
      const float v0 = s0 * inv_c + p.eps;
      const float r0 = 1.0f / sqrtf(v0);
      // T = 1: the tangent's column scale rdot; T = 0: the second pair block's scale
      const float r1 = TAN ? (2.0f * s1 * inv_c) * (-0.5f * r0 / v0) : 1.0f / sqrtf(s1 * inv_c + p.eps);
      int nqi[2] = {qi[0], qi[1]}, nqj[2] = {qj[0], qj[1]}, ncpos[2] = {cpos[0], cpos[1]};
      bool nvalid[2] = {false, false};
      if (t + 1 < t1) {
        tile_pairs<TAN>(t + 1, c, npairs, nk, rows_listed, keys_listed, list, nqi, nqj, nvalid, ncpos);
        load_rows<C, TAN>(edge_b, edge_tb, N, g, nqi, nqj, nvalid, xin);
      }
      v4f h0[4][2];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float4 bi = lds4(W, L::kBin + 16 * m + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float P0 = acc[m][0][r], P1 = acc[m][1][r];
          h0[m][0][r] = r0 * P0 + comp(bi, r);
          h0[m][1][r] = TAN ? r0 * P1 + r1 * P0 : r1 * P1 + comp(bi, r);
        }
      }

      // ---- layer 2: a = silu(h0 W_1 + b_1) (and its tangent) ----
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = zero4();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float4 a4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) a4[m] = lds4(W, L::kF2 + ((m * 4 + kb) * 64 + lane) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            acc[m][0] = mfma16x4(comp(a4[m], u), h0[kb][0][u], acc[m][0]);
            acc[m][1] = mfma16x4(comp(a4[m], u), h0[kb][1][u], acc[m][1]);
          }
      }
      v4f act[4][2];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float4 b1 = lds4(W, L::kB1 + 16 * m + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float u0 = acc[m][0][r] + comp(b1, r);
          const float s = sigmoid(u0);
          act[m][0][r] = u0 * s;
          if (TAN) {
            act[m][1][r] = acc[m][1][r] * (s + u0 * s * (1.0f - s));
          } else {
            const float u1 = acc[m][1][r] + comp(b1, r);
            act[m][1][r] = u1 * sigmoid(u1);
          }
        }
      }

      // ---- layer 3: h1 = h0 + gain * (a W_2 + b_2) ----
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[m][0] = acc[m][1] = zero4();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float4 a4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) a4[m] = lds4(W, L::kF3 + ((m * 4 + kb) * 64 + lane) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            acc[m][0] = mfma16x4(comp(a4[m], u), act[kb][0][u], acc[m][0]);
            acc[m][1] = mfma16x4(comp(a4[m], u), act[kb][1][u], acc[m][1]);
          }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float4 b2 = lds4(W, L::kB2 + 16 * m + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          h0[m][0][r] = h0[m][0][r] + p.gain * (acc[m][0][r] + comp(b2, r));
          h0[m][1][r] = TAN ? h0[m][1][r] + p.gain * acc[m][1][r]
                            : h0[m][1][r] + p.gain * (acc[m][1][r] + comp(b2, r));
        }
      }

      // ---- layer 4: e = (h1 W_out + b_out) / div ----
      v4f o[HB][2];
#pragma unroll
      for (int m = 0; m < HB; ++m) o[m][0] = o[m][1] = zero4();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float4 a4[HB];
#pragma unroll
        for (int m = 0; m < HB; ++m) a4[m] = lds4(W, L::kF4 + ((m * 4 + kb) * 64 + lane) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int m = 0; m < HB; ++m) {
            o[m][0] = mfma16x4(comp(a4[m], u), h0[kb][0][u], o[m][0]);
            o[m][1] = mfma16x4(comp(a4[m], u), h0[kb][1][u], o[m][1]);
          }
      }

      // ---- store: lane (g, c) holds heads 16 m + 4 g + r of its pair ----
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int src = TAN ? 0 : cb;
        if (!valid[src]) continue;
        float* const base = TAN && cb == 1 ? et_b : e_b;
        float* dst = base + static_cast<int64_t>(qi[src]) * p.e_sq + static_cast<int64_t>(qj[src]) * p.e_sk;
        const bool with_bias = !(TAN && cb == 1);
#pragma unroll
        for (int m = 0; m < HB; ++m) {
          const float4 bo = lds4(W, L::kBout + 16 * m + 4 * g);
          float val[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) val[r] = (o[m][cb][r] + (with_bias ? comp(bo, r) : 0.0f)) * inv_div;
          const int h = 16 * m + 4 * g;
          if (cmp) {  // head h's block, the pair's compacted position
#pragma unroll
            for (int r = 0; r < 4; ++r) base[static_cast<int64_t>(h + r) * p.e_blk + cpos[src]] = val[r];
          } else if (p.e_sh == 1) {
            *reinterpret_cast<float4*>(dst + h) = make_float4(val[0], val[1], val[2], val[3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[static_cast<int64_t>(h + r) * p.e_sh] = val[r];
          }
        }
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        qi[cb] = nqi[cb];
        qj[cb] = nqj[cb];
        cpos[cb] = ncpos[cb];
        valid[cb] = nvalid[cb];
      }
    }
  }
}

template <int C, int HB>
hipError_t launch_pb(const PairBiasParams& p, bool tan, int64_t blocks, int cus, hipStream_t stream) {
  const int64_t slots = static_cast<int64_t>(cus) * pb_occupancy<C, HB>();
  const int grid = static_cast<int>(blocks < slots ? blocks : slots);
  if (tan)
    hipLaunchKernelGGL((pair_bias_kernel<C, HB, true>), dim3(grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((pair_bias_kernel<C, HB, false>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int C>
hipError_t launch_pb_c(const PairBiasParams& p, int H, bool tan, int64_t blocks, int cus, hipStream_t stream) {
  switch (H) {
    case 16: return launch_pb<C, 1>(p, tan, blocks, cus, stream);
    case 32: return launch_pb<C, 2>(p, tan, blocks, cus, stream);
    case 64: return launch_pb<C, 4>(p, tan, blocks, cus, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_pair_bias(PairBiasParams p, int C, int H, bool tan, hipStream_t stream) {
  int cus = 0;
  if (hipError_t err = device_cu_count(&cus); err != hipSuccess) return err;
  const int64_t waves = static_cast<int64_t>(cus) * 2 * kPBWaves;
  // Parts per walker: about four items per wave, each part at least four tiles.
  const int64_t tp = tan ? 16 : 32;
  const int64_t tiles = (static_cast<int64_t>(p.N) * p.N + tp - 1) / tp;
  int64_t parts = (4 * waves + p.B - 1) / p.B;
  parts = parts > tiles / 4 ? tiles / 4 : parts;
  parts = parts < 1 ? 1 : (parts > 4096 ? 4096 : parts);
  p.parts = static_cast<int>(parts);
  p.n_items = p.B * parts;
  const int64_t blocks = (p.n_items + kPBWaves - 1) / kPBWaves;
  switch (C) {
    case 32: return launch_pb_c<32>(p, H, tan, blocks, cus, stream);
    case 64: return launch_pb_c<64>(p, H, tan, blocks, cus, stream);
    case 96: return launch_pb_c<96>(p, H, tan, blocks, cus, stream);
    case 128: return launch_pb_c<128>(p, H, tan, blocks, cus, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hz
