// The MLP-class pair-bias producer on the float32 matrix cores (v_mfma_f32_16x16x4_f32): the
// coupling bias of the tree's LevelEdgeAttn (src/hamiltonzero/model/tree.py:1392-1456), of the
// readout context (model/readout_leaf_context.py:694-712) and of the large-N sequence trunk
// (evaluation/sequence_trunk.py:962-972, the tiled pair MLP). Per pair (i, j) of a walker, with
// x = edge[b, i, j, :] (and, for the readout, one more input channel xe = extra[b, i, j]):
//     h   = x W_in + xe w_e + b_in                                   (in_proj)
//     per block:  h += gain * (silu(rms(h) W_1 + b_1) W_2 + b_2)     rms(h) = h * w_n * rsqrt(mean(h^2) + eps)
//     e   = (rms_out(h) W_out + b_out) / div - slope_h * lca(pos_i, pos_j)
// (MLP, model/odd_ops.py:218-276; _RMS, odd_ops.py:183-215 / tree.py:339-375; the LCA-ALiBi
// term lca_alibi_bias, readout_leaf_context.py:140-170, optional), and with a tangent its
// forward-mode derivative, written straight into the attention's bias layout.
//
// Same orientation as the trunk's producer (pair_bias.hip): features x pairs, weights as the A
// operand (staged in LDS as ready-made fragments), 16 pairs as the B operand, every layer's
// result lane (g, c) register r = feature 4g + r of pair c of M block m, which is the next
// layer's B operand when its K order is permuted accordingly. The RMS norms are per-pair
// (column) scales: the norm weight w_n is folded into the next layer's fragments (W_1' =
// diag(w_n) W_1), the layer runs on h itself and its columns are scaled by r = rsqrt(mean(h^2)
// + eps) afterwards (tangent: r (hdot W_1') + rdot (h W_1'), rdot = -r mean(h hdot) / (mean(h^2)
// + eps)); mean(h^2) is a sum over the lane's registers and the four lane groups of its column.
// The residual gain is folded into W_2 and b_2, so the second product of a block accumulates
// straight into h.
//
// At hidden width 128 the fp32 weights (W_in 96 x 128, W_1, W_2 128 x 128) exceed the LDS: W_1
// and W_2 stay in LDS (128 KB) and W_in's fragments are read from memory (an L2-resident 48 KB
// shared by every workgroup), one channel group ahead of the products. One such workgroup fits
// a CU, and its four waves run one per SIMD with the whole register file (about 470 registers:
// at two waves per SIMD the tile's h, activations and fragments spill 350-580 bytes per lane).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

constexpr int kPMListN = 256;   // sites per walker the pair compaction handles
constexpr int kLcaLevels = 13;  // _LCA_MAX_LEVELS (readout_leaf_context.py:131)

template <int C, int KB, int HB>
struct PMShape {
  static constexpr int HID = 16 * KB;
  static constexpr int H = 16 * HB;
  static constexpr int CG = C / 16;                 // float4 groups per lane group
  static constexpr int C4 = C / 4;                  // channels per lane group
  static constexpr bool kWinGlobal = KB == 8;
  static constexpr int NW = 4;                      // waves per workgroup
  static constexpr int kMaxBlocks = KB == 8 ? 1 : 2;
  // LDS floats: W_in fragments (unless global), per block W_1' and gain W_2 fragments, W_out'
  // fragments, then the vectors b_in, w_e, per block b_1 and gain b_2, b_out, slopes
  static constexpr int kWin = kWinGlobal ? 0 : HID * C;
  static constexpr int kBlk = 2 * HID * HID;
  static constexpr int kWout = HID * H;
  static constexpr int kVec = 2 * HID + 2 * HID * kMaxBlocks + 2 * H;
  __host__ __device__ static constexpr int floats(int nb) { return kWin + nb * kBlk + kWout + kVec; }
};

__device__ __forceinline__ float4 ld4(const float* base, int off) {
  return *reinterpret_cast<const float4*>(base + off);
}
__device__ __forceinline__ float cmp(const float4& v, int u) {
  return u == 0 ? v.x : (u == 1 ? v.y : (u == 2 ? v.z : v.w));
}
// sigmoid(u) = 1 / (1 + 2^(-u log2 e)), hardware exp2 and reciprocal (about 1 ulp each).
__device__ __forceinline__ float sigm(float u) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u * -1.44269504088896341f));
}
// lca_level (readout_leaf_context.py:140-148): the number of t in [0, 13) with xor >= 2^t,
// i.e. the bit length of pos_q ^ pos_k, capped at 13.
__device__ __forceinline__ int lca_level(int pq, int pk) {
  const uint32_t x = static_cast<uint32_t>(pq ^ pk);
  const int bits = x == 0 ? 0 : 32 - __clz(x);
  return bits < kLcaLevels ? bits : kLcaLevels;
}

// The pairs of lane column c in tile t (N block cb): query qi, key qj, valid.
template <bool TAN>
__device__ __forceinline__ void pm_tile_pairs(int t, int c, int npairs, int nk, bool rows_listed, bool keys_listed,
                                              const unsigned short* list, int qi[2], int qj[2], bool valid[2]) {
  constexpr int TP = TAN ? 16 : 32;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int q = TAN ? TP * t + c : TP * t + 16 * cb + c;
    valid[cb] = q < npairs;
    const int qq = valid[cb] ? q : 0;
    const int ii = qq / nk, jj = qq - ii * nk;
    qi[cb] = rows_listed ? list[ii] : ii;
    qj[cb] = keys_listed ? list[jj] : jj;
  }
}

// This lane's C/4 channels of its pairs' edge rows (T = 1: the pair's edge and edge_t rows;
// T = 0: the rows of the two pairs) and, with an extra channel, its value(s).
template <int C, bool TAN>
__device__ __forceinline__ void pm_load_rows(const PairMlpParams& p, int64_t b, int g, const int qi[2],
                                             const int qj[2], const bool valid[2], float4 xin[2][C / 16],
                                             float xe[2]) {
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int src = TAN ? 0 : cb;
    const int64_t pair = (b * p.Nq + qi[src]) * static_cast<int64_t>(p.Nk) + qj[src];
    const float* row = (TAN && cb == 1 ? p.edge_t : p.edge) + pair * C + g * (C / 4);
#pragma unroll
    for (int v = 0; v < C / 16; ++v)
      xin[cb][v] = valid[src] ? *reinterpret_cast<const float4*>(row + 4 * v) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float* ex = TAN && cb == 1 ? p.extra_t : p.extra;
    xe[cb] = (ex != nullptr && valid[src]) ? ex[pair] : 0.f;
  }
}

// Per-column RMS statistics of h (both column blocks): r0 = rsqrt(mean(h0^2) + eps) and, with
// a tangent, rd = -r0 mean(h0 h1) / (mean(h0^2) + eps); without, r1 of the second block.
template <int KB, bool TAN>
__device__ __forceinline__ void pm_rms(const v4f (&h)[KB][2], float inv_hid, float eps, float& r0, float& r1) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int m = 0; m < KB; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s0 = fmaf(h[m][0][r], h[m][0][r], s0);
      s1 = fmaf(h[m][1][r], TAN ? h[m][0][r] : h[m][1][r], s1);
    }
  s0 = group_sum(s0);
  s1 = group_sum(s1);
  const float v0 = s0 * inv_hid + eps;
  r0 = 1.0f / sqrtf(v0);
  r1 = TAN ? -r0 * (s1 * inv_hid) / v0 : 1.0f / sqrtf(s1 * inv_hid + eps);
}

template <int C, int KB, int HB, bool TAN>
__global__ void __launch_bounds__((64 * PMShape<C, KB, HB>::NW), (KB == 8 ? 1 : 2))
    pair_mlp_bias_kernel(PairMlpParams p) {
  using S = PMShape<C, KB, HB>;
  constexpr int HID = S::HID, H = S::H, CG = S::CG, C4 = S::C4, NW = S::NW;
  constexpr int TP = TAN ? 16 : 32;  // pairs per tile
  extern __shared__ float4 pm_smem4[];
  float* const lds = reinterpret_cast<float*>(pm_smem4);
  const int nb = p.n_blocks;
  const int oWin = 0, oBlk = S::kWin, oWout = oBlk + nb * S::kBlk, oV = oWout + S::kWout;
  const int oBin = oV, oWe = oBin + HID, oB1 = oWe + HID, oB2 = oB1 + HID * S::kMaxBlocks,
            oBout = oB2 + HID * S::kMaxBlocks, oSl = oBout + H;
  unsigned short* const lists = reinterpret_cast<unsigned short*>(lds + S::floats(nb));

  // ---- stage the weights as A fragments (once per workgroup) ----
  const int nt = blockDim.x;
  if constexpr (!S::kWinGlobal) {
    for (int f = threadIdx.x; f < HID * C; f += nt) {
      const int u = f & 3, lane = (f >> 2) & 63, rest = f >> 8;
      const int sg = rest % CG, m = rest / CG;
      const int k = (lane >> 4) * C4 + 4 * sg + u;
      lds[oWin + f] = p.w_in[k * HID + 16 * m + (lane & 15)];
    }
  }
  for (int blk = 0; blk < nb; ++blk) {
    const float* w1 = p.w_1 + static_cast<int64_t>(blk) * HID * HID;
    const float* w2 = p.w_2 + static_cast<int64_t>(blk) * HID * HID;
    const float* wn = p.norm_w + blk * HID;
    for (int f = threadIdx.x; f < HID * HID; f += nt) {
      const int u = f & 3, lane = (f >> 2) & 63, rest = f >> 8;
      const int kb = rest % KB, m = rest / KB;
      const int k = 16 * kb + 4 * (lane >> 4) + u, o = 16 * m + (lane & 15);
      lds[oBlk + blk * S::kBlk + f] = wn[k] * w1[k * HID + o];
      lds[oBlk + blk * S::kBlk + HID * HID + f] = p.gain * w2[k * HID + o];
    }
    for (int f = threadIdx.x; f < HID; f += nt) {
      lds[oB1 + blk * HID + f] = p.b_1[blk * HID + f];
      lds[oB2 + blk * HID + f] = p.gain * p.b_2[blk * HID + f];
    }
  }
  for (int f = threadIdx.x; f < HID * H; f += nt) {
    const int u = f & 3, lane = (f >> 2) & 63, rest = f >> 8;
    const int kb = rest % KB, m = rest / KB;
    const int k = 16 * kb + 4 * (lane >> 4) + u;
    lds[oWout + f] = p.out_norm_w[k] * p.w_out[k * H + 16 * m + (lane & 15)];
  }
  for (int f = threadIdx.x; f < HID; f += nt) {
    lds[oBin + f] = p.b_in[f];
    lds[oWe + f] = p.extra != nullptr ? p.w_in[C * HID + f] : 0.f;
  }
  for (int f = threadIdx.x; f < H; f += nt) {
    lds[oBout + f] = p.b_out[f];
    lds[oSl + f] = p.slopes != nullptr ? p.slopes[f] : 0.f;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  unsigned short* list = lists + wave * kPMListN;
  const int Nq = p.Nq, Nk = p.Nk;
  const bool use_list = p.mask != nullptr && Nk <= kPMListN;
  const float inv_hid = 1.0f / static_cast<float>(HID);
  const float inv_div = 1.0f / p.div;
  const bool alibi = p.slopes != nullptr;
  const int64_t total_waves = static_cast<int64_t>(gridDim.x) * NW;

  for (int64_t item = static_cast<int64_t>(blockIdx.x) * NW + wave; item < p.n_items; item += total_waves) {
    const int64_t b = item / p.parts;
    const int part = static_cast<int>(item - b * p.parts);

    // ---- the walker's physical sites ----
    int nk = Nk;
    bool keys_listed = false, rows_listed = false;
    if (use_list) {
      int n = 0;
      for (int s0 = 0; s0 < Nk; s0 += 64) {
        const int site = s0 + lane;
        const bool phys = site < Nk && p.mask[b * Nk + site] != 0;
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
    const int nrows = rows_listed ? nk : Nq;
    const int npairs = nrows * nk;
    const int ntiles = (npairs + TP - 1) / TP;
    const int t0 = static_cast<int>(static_cast<int64_t>(ntiles) * part / p.parts);
    const int t1 = static_cast<int>(static_cast<int64_t>(ntiles) * (part + 1) / p.parts);
    float* e_b = p.e + b * static_cast<int64_t>(Nq) * Nk * H;
    float* et_b = TAN ? p.e_t + b * static_cast<int64_t>(Nq) * Nk * H : nullptr;

    int qi[2], qj[2];
    bool valid[2];
    float4 xin[2][CG];
    float xe[2];
    if (t0 < t1) {
      pm_tile_pairs<TAN>(t0, c, npairs, nk, rows_listed, keys_listed, list, qi, qj, valid);
      pm_load_rows<C, TAN>(p, b, g, qi, qj, valid, xin, xe);
    }
    for (int t = t0; t < t1; ++t) {
      // The fragments are the same for every tile; an offset the compiler cannot see through
      // keeps their LDS reads inside the loop (hoisted, they would not fit the registers).
      int lz = 0;
      asm volatile("" : "+s"(lz));
      const float* W = lds + lz;

      // ---- in_proj: h = x W_in (+ xe w_e) + b_in ----
      v4f h[KB][2];
#pragma unroll
      for (int m = 0; m < KB; ++m) h[m][0] = h[m][1] = zero4();
      if constexpr (S::kWinGlobal) {
        // fragments from memory, one channel group ahead of the products
        float4 a4[2][KB];
        auto fetch = [&](int sg, float4 (&dst)[KB]) {
#pragma unroll
          for (int m = 0; m < KB; ++m) {
            const float* col = p.w_in + (g * C4 + 4 * sg) * HID + 16 * m + c;
            dst[m] = make_float4(col[0], col[HID], col[2 * HID], col[3 * HID]);
          }
        };
        fetch(0, a4[0]);
#pragma unroll
        for (int sg = 0; sg < CG; ++sg) {
          if (sg + 1 < CG) fetch(sg + 1, a4[(sg + 1) & 1]);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float x0 = cmp(xin[0][sg], u), x1 = cmp(xin[1][sg], u);
#pragma unroll
            for (int m = 0; m < KB; ++m) {
              h[m][0] = mfma16x4(cmp(a4[sg & 1][m], u), x0, h[m][0]);
              h[m][1] = mfma16x4(cmp(a4[sg & 1][m], u), x1, h[m][1]);
            }
          }
        }
      } else {
#pragma unroll
        for (int sg = 0; sg < CG; ++sg) {
          float4 a4[KB];
#pragma unroll
          for (int m = 0; m < KB; ++m) a4[m] = ld4(W, oWin + ((m * CG + sg) * 64 + lane) * 4);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float x0 = cmp(xin[0][sg], u), x1 = cmp(xin[1][sg], u);
#pragma unroll
            for (int m = 0; m < KB; ++m) {
              h[m][0] = mfma16x4(cmp(a4[m], u), x0, h[m][0]);
              h[m][1] = mfma16x4(cmp(a4[m], u), x1, h[m][1]);
            }
          }
        }
      }
      const float xe0 = xe[0], xe1 = xe[1];
      // the next tile's rows fly under the rest of this tile
      int nqi[2] = {qi[0], qi[1]}, nqj[2] = {qj[0], qj[1]};
      bool nvalid[2] = {false, false};
      if (t + 1 < t1) {
        pm_tile_pairs<TAN>(t + 1, c, npairs, nk, rows_listed, keys_listed, list, nqi, nqj, nvalid);
        pm_load_rows<C, TAN>(p, b, g, nqi, nqj, nvalid, xin, xe);
      }
#pragma unroll
      for (int m = 0; m < KB; ++m) {
        const float4 bi = ld4(W, oBin + 16 * m + 4 * g);
        const float4 we = ld4(W, oWe + 16 * m + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          h[m][0][r] += fmaf(xe0, cmp(we, r), cmp(bi, r));
          h[m][1][r] += TAN ? xe1 * cmp(we, r) : fmaf(xe1, cmp(we, r), cmp(bi, r));
        }
      }

      // ---- blocks: h += gain (silu(rms(h) W_1 + b_1) W_2 + b_2) ----
      for (int blk = 0; blk < nb; ++blk) {
        float r0, r1;
        pm_rms<KB, TAN>(h, inv_hid, p.eps, r0, r1);
        const int f1 = oBlk + blk * S::kBlk, f2 = f1 + HID * HID;
        v4f a[KB][2];
#pragma unroll
        for (int m = 0; m < KB; ++m) a[m][0] = a[m][1] = zero4();
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          float4 a4[KB];
#pragma unroll
          for (int m = 0; m < KB; ++m) a4[m] = ld4(W, f1 + ((m * KB + kb) * 64 + lane) * 4);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < KB; ++m) {
              a[m][0] = mfma16x4(cmp(a4[m], u), h[kb][0][u], a[m][0]);
              a[m][1] = mfma16x4(cmp(a4[m], u), h[kb][1][u], a[m][1]);
            }
        }
#pragma unroll
        for (int m = 0; m < KB; ++m) {
          const float4 b1 = ld4(W, oB1 + blk * HID + 16 * m + 4 * g);
          const float4 b2 = ld4(W, oB2 + blk * HID + 16 * m + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float P0 = a[m][0][r], P1 = a[m][1][r];
            const float u0 = fmaf(r0, P0, cmp(b1, r));
            const float s = sigm(u0);
            a[m][0][r] = u0 * s;
            if (TAN) {
              a[m][1][r] = fmaf(r0, P1, r1 * P0) * (s + u0 * s * (1.0f - s));
            } else {
              const float u1 = fmaf(r1, P1, cmp(b1, r));
              a[m][1][r] = u1 * sigm(u1);
            }
            // the residual's bias (gain b_2, primal columns), then the products accumulate into h
            h[m][0][r] += cmp(b2, r);
            if (!TAN) h[m][1][r] += cmp(b2, r);
          }
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          float4 a4[KB];
#pragma unroll
          for (int m = 0; m < KB; ++m) a4[m] = ld4(W, f2 + ((m * KB + kb) * 64 + lane) * 4);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < KB; ++m) {
              h[m][0] = mfma16x4(cmp(a4[m], u), a[kb][0][u], h[m][0]);
              h[m][1] = mfma16x4(cmp(a4[m], u), a[kb][1][u], h[m][1]);
            }
        }
      }

      // ---- out: e = (rms_out(h) W_out + b_out) / div - slope lca ----
      float ro0, ro1;
      pm_rms<KB, TAN>(h, inv_hid, p.eps, ro0, ro1);
      v4f o[HB][2];
#pragma unroll
      for (int m = 0; m < HB; ++m) o[m][0] = o[m][1] = zero4();
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        float4 a4[HB];
#pragma unroll
        for (int m = 0; m < HB; ++m) a4[m] = ld4(W, oWout + ((m * KB + kb) * 64 + lane) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int m = 0; m < HB; ++m) {
            o[m][0] = mfma16x4(cmp(a4[m], u), h[kb][0][u], o[m][0]);
            o[m][1] = mfma16x4(cmp(a4[m], u), h[kb][1][u], o[m][1]);
          }
      }

      // ---- store: lane (g, c) holds heads 16 m + 4 g + r of its pair ----
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int src = TAN ? 0 : cb;
        if (!valid[src]) continue;
        float* dst = (TAN && cb == 1 ? et_b : e_b) + static_cast<int64_t>(qi[src]) * p.e_sq +
                     static_cast<int64_t>(qj[src]) * p.e_sk;
        const bool tangent = TAN && cb == 1;
        const float lvl = alibi && !tangent ? static_cast<float>(lca_level(p.row_offset + qi[src], qj[src])) : 0.f;
#pragma unroll
        for (int m = 0; m < HB; ++m) {
          const float4 bo = ld4(W, oBout + 16 * m + 4 * g);
          const float4 sl = ld4(W, oSl + 16 * m + 4 * g);
          float val[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (tangent) {
              val[r] = fmaf(ro0, o[m][1][r], ro1 * o[m][0][r]) * inv_div;
            } else {
              const float rr = (TAN || cb == 0) ? ro0 : ro1;
              val[r] = fmaf(rr, o[m][cb][r], cmp(bo, r)) * inv_div - cmp(sl, r) * lvl;
            }
          }
          const int hh = 16 * m + 4 * g;
          if (p.e_sh == 1) {
            *reinterpret_cast<float4*>(dst + hh) = make_float4(val[0], val[1], val[2], val[3]);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[static_cast<int64_t>(hh + r) * p.e_sh] = val[r];
          }
        }
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        qi[cb] = nqi[cb];
        qj[cb] = nqj[cb];
        valid[cb] = nvalid[cb];
      }
    }
  }
}

template <int C, int KB, int HB>
hipError_t launch_pm(const PairMlpParams& p, bool tan, int cus, hipStream_t stream) {
  using S = PMShape<C, KB, HB>;
  const size_t lds = static_cast<size_t>(S::floats(p.n_blocks)) * 4 + S::NW * kPMListN * 2;
  auto kern = tan ? pair_mlp_bias_kernel<C, KB, HB, true> : pair_mlp_bias_kernel<C, KB, HB, false>;
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (err != hipSuccess) return err;
  const int per_cu = KB == 8 ? 1 : (lds <= 80 * 1024 ? 2 : 1);
  const int64_t blocks = (p.n_items + S::NW - 1) / S::NW;
  const int64_t slots = static_cast<int64_t>(cus) * per_cu;
  const int grid = static_cast<int>(blocks < slots ? blocks : slots);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * S::NW), lds, stream, p);
  return hipGetLastError();
}

template <int C, int KB>
hipError_t launch_pm_h(const PairMlpParams& p, int H, bool tan, int cus, hipStream_t stream) {
  switch (H) {
    case 16: return launch_pm<C, KB, 1>(p, tan, cus, stream);
    case 32: return launch_pm<C, KB, 2>(p, tan, cus, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int C>
hipError_t launch_pm_c(const PairMlpParams& p, int hidden, int H, bool tan, int cus, hipStream_t stream) {
  switch (hidden) {
    case 32: return launch_pm_h<C, 2>(p, H, tan, cus, stream);
    case 64: return launch_pm_h<C, 4>(p, H, tan, cus, stream);
    case 128: return launch_pm_h<C, 8>(p, H, tan, cus, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int pair_mlp_max_blocks(int hidden) { return hidden == 128 ? 1 : 2; }

hipError_t launch_pair_mlp_bias(PairMlpParams p, int C, int hidden, int H, bool tan, hipStream_t stream) {
  int cus = 256;
  if (device_cu_count(&cus) != hipSuccess || cus < 1) cus = 256;
  const int64_t waves = static_cast<int64_t>(cus) * 2 * 4;  // two workgroups of four waves per CU at most
  // Parts per walker: about four items per wave, each part at least four tiles.
  const int64_t tp = tan ? 16 : 32;
  const int64_t tiles = (static_cast<int64_t>(p.Nq) * p.Nk + tp - 1) / tp;
  int64_t parts = (4 * waves + p.B - 1) / p.B;
  parts = parts > tiles / 4 ? tiles / 4 : parts;
  parts = parts < 1 ? 1 : (parts > (1 << 20) ? (1 << 20) : parts);
  p.parts = static_cast<int>(parts);
  p.n_items = p.B * parts;
  switch (C) {
    case 32: return launch_pm_c<32>(p, hidden, H, tan, cus, stream);
    case 64: return launch_pm_c<64>(p, hidden, H, tan, cus, stream);
    case 96: return launch_pm_c<96>(p, hidden, H, tan, cus, stream);
    case 128: return launch_pm_c<128>(p, hidden, H, tan, cus, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hz
