// bfloat16 matrix-core reverse-mode (VJP) MHSEA kernel for N <= 64, D in {32, 64}.
//
// Same algebra and work decomposition as the fp32 persistent backward (custom_gradients.py:
// 249-285, :307-347): per (walker, head) item, phase A (query-major) forms S^T, dP^T, P, dS
// and dq^T = K^T dS^T (and de), and leaves P, dS in LDS as bf16; after a barrier phase B
// (key-major) reads them back as B operands of dv^T = dout^T P, dk^T = Q^T dS. Products run on
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation; P, dS are rounded to bf16 only as operands
// of the site contractions.
//
// LDS holds the compacted rows as bf16: row-major q, k, v, dout (A operands of the
// d-contractions, 8 elements per lane) and transposed q, k, dout (A operands of the site
// contractions: lane (g, c) of output row d reads sites kappa(g, i) = 16(2p + i/4) + 4g + i%4
// as two 8-byte runs), plus lse*log2(e) and delta = rowsum(out o dout) in fp32, and P, dS as
// four 16-query tiles of [key][query] rows (phase B's lane (g, c) reads key row c, queries
// kappa(g, i), the same two-run pattern). At D = 64 the tile of query tile w overlays the q
// (P) and dout (dS) rows of those 16 queries, which only wave w reads in phase A, before it
// writes the tile.
#include <atomic>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ uint4 keep4(bool keep, const uint4& u) {
  return make_uint4(keep ? u.x : 0u, keep ? u.y : 0u, keep ? u.z : 0u, keep ? u.w : 0u);
}
__device__ __forceinline__ uint16_t bf16_at(const uint4& u, int e) {
  const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// The value of lane l ^ 1 (DPP quad permutation [1, 0, 3, 2]; every lane active).
__device__ __forceinline__ float swap_lane_pair(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ bf16x8 pack8(v4f a, v4f b) {
  uint4 u;
  u.x = pack2_bf16(a[0], a[1]);
  u.y = pack2_bf16(a[2], a[3]);
  u.z = pack2_bf16(b[0], b[1]);
  u.w = pack2_bf16(b[2], b[3]);
  return as_bf16x8(u);
}
// Two 8-byte runs (sites 16*2p + 4g .. +4 and 16*(2p+1) + 4g .. +4) of a transposed row,
// read as 4-byte words (the runs are 4-byte aligned).
__device__ __forceinline__ bf16x8 tr_operand(const uint16_t* row) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(row);
  return as_bf16x8(make_uint4(w[0], w[1], w[8], w[9]));
}

template <int D>
struct BwdBf16Shape {
  static constexpr int KC = 64;
  static constexpr int LDR = D + 8;   // row-major row, bf16 elements
  // transposed row, bf16 elements (35 words, row starts 4-byte aligned): the pairwise 32-bit
  // transposed writes of one wave hit 64 distinct banks at D = 64 (two lanes per bank at
  // D = 32), and the 32-bit operand reads (lane (g, c) at word 35c + 2g) put at most two
  // lanes on a bank, the least any row stride allows for that read pattern (66 elements,
  // 33 words, put four)
  static constexpr int LDT = KC + 6;
  static constexpr int NS = D / 32;
  static constexpr int DT = D / 16;
  static constexpr int C8 = D / 8;
  static constexpr int kRow = KC * LDR;
  static constexpr int kTr = D * LDT;
  // staging: one thread per (row pair, 8-column chunk); D = 32 leaves waves 2, 3 idle there
  static constexpr int kStageThreads = KC * C8 / 2;
  // P / dS tiles: 16 queries of one key per row, 2 elements of padding (9-word rows)
  static constexpr int kPS = 18;
  static constexpr int kPTile = KC * kPS;
  // D = 64: 16 row-major rows of q (dout) are exactly one P (dS) tile
  static constexpr bool kPAlias = 16 * LDR == kPTile;
  static constexpr size_t kLdsBytes = static_cast<size_t>(4 * kRow + 3 * kTr) * 2 + 2 * KC * 4 +
                                      (kPAlias ? 0 : static_cast<size_t>(2 * 4 * kPTile) * 2);
};

// Row `site` of one (walker, head) slice of a [B, N, H, D] tensor, relative to the slice's
// first row: site * H * D elements. A full-rate 24-bit multiply: bf16_bwd_supported
// guarantees H * D < 2^23 and site < 64, so the product needs no 64-bit arithmetic.
__device__ __forceinline__ uint32_t row_off(int site, uint32_t hd) {
  return __umul24(static_cast<uint32_t>(site), hd);
}

struct Sites {
  uint64_t bal;
  int perm;
  int n_phys;
};

__device__ __forceinline__ Sites make_sites(uint32_t mbyte, int N) {
  const int lane = threadIdx.x & 63;
  const bool on = lane < N && mbyte != 0;
  const uint64_t bal = __ballot(on);
  Sites st;
  st.bal = bal;
  st.n_phys = __popcll(bal);
  const int below = __popcll(bal & ((uint64_t(1) << lane) - 1));
  const int pos = on ? below : (lane < N ? st.n_phys + (lane - below) : lane);
  st.perm = __builtin_amdgcn_ds_permute(pos << 2, lane);
  return st;
}

template <int D, bool HAS_E>
__global__ void __launch_bounds__(256, 2) mhsea_bwd_bf16_kernel(const BwdParams p) {
  using Sh = BwdBf16Shape<D>;
  constexpr int LDR = Sh::LDR, LDT = Sh::LDT, NS = Sh::NS, DT = Sh::DT, C8 = Sh::C8;
  constexpr int NPT = 2;
  constexpr int NT = 4;

  extern __shared__ float4 smem4[];
  uint16_t* const Qr = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* const Kr = Qr + Sh::kRow;
  uint16_t* const Vr = Kr + Sh::kRow;
  uint16_t* const Gr = Vr + Sh::kRow;
  uint16_t* const QT = Gr + Sh::kRow;
  uint16_t* const KT = QT + Sh::kTr;
  uint16_t* const GT = KT + Sh::kTr;
  float* const L2s = reinterpret_cast<float*>(GT + Sh::kTr);
  float* const Dls = L2s + Sh::KC;
  uint16_t* const Pt = Sh::kPAlias ? Qr : reinterpret_cast<uint16_t*>(Dls + Sh::KC);
  uint16_t* const DSt = Sh::kPAlias ? Gr : Pt + 4 * Sh::kPTile;
  constexpr int kPS = Sh::kPS, kPTile = Sh::kPTile;

  const int N = p.N, H = p.H;
  const uint32_t HD = static_cast<uint32_t>(H * D);
  const int64_t nitems = static_cast<int64_t>(p.B) * H;
  const int64_t stride = gridDim.x;
  int64_t item = blockIdx.x;
  if (item >= nitems) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const bool km = p.key_mask != 0;
  auto nq_of = [&](const Sites& s) { return km ? N : s.n_phys; };
  auto nk_of = [&](const Sites& s) { return (km && s.n_phys == 0) ? N : s.n_phys; };
  auto qperm_of = [&](const Sites& s) { return km ? lane : s.perm; };
  auto kperm_of = [&](const Sites& s) { return (km && s.n_phys == 0) ? lane : s.perm; };

  // Staging assignment: thread t < kStageThreads owns rows 2*(t / C8) + {0, 1} (u = 0, 1) of
  // the 8-column chunk t % C8, so the transposed tiles are written as (row r, row r+1) 32-bit
  // pairs. The idle threads (D = 32) are whole waves, so the row-sum shuffles stay wave-uniform.
  static_assert(Sh::kStageThreads == 128 || Sh::kStageThreads == 256, "staging layout");
  uint4 cq[NPT], ck[NPT], cv[NPT], cg[NPT], co[NPT];
  float clse = 0.f;
  const bool st_active = tid < Sh::kStageThreads;
  const int st_c8 = (tid % C8) * 8;
  const int st_r0 = 2 * (tid / C8);
  auto issue_item_loads = [&](int b, int h, const Sites& st) {
    const int qperm = qperm_of(st), kperm = kperm_of(st), nq = nq_of(st), nk = nk_of(st);
    // (walker, head) slice bases are wave-uniform; rows are 32-bit offsets from them
    const int64_t base = bnhd(b, 0, h, N, H, D);
    const uint16_t* const qw = static_cast<const uint16_t*>(p.q) + base;
    const uint16_t* const gw = static_cast<const uint16_t*>(p.dout) + base;
    const uint16_t* const ow = static_cast<const uint16_t*>(p.out) + base;
    const uint16_t* const kw = static_cast<const uint16_t*>(p.k) + base;
    const uint16_t* const vw = static_cast<const uint16_t*>(p.v) + base;
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      if (!st_active) break;
      const int r = st_r0 + u;
      const int sq = __shfl(qperm, r & 63, 64);
      const int sk = __shfl(kperm, r & 63, 64);
      const uint32_t qoff = row_off(r < nq ? sq : 0, HD) + st_c8;
      const uint32_t koff = row_off(r < nk ? sk : 0, HD) + st_c8;
      cq[u] = *reinterpret_cast<const uint4*>(qw + qoff);
      cg[u] = *reinterpret_cast<const uint4*>(gw + qoff);
      co[u] = *reinterpret_cast<const uint4*>(ow + qoff);
      ck[u] = *reinterpret_cast<const uint4*>(kw + koff);
      cv[u] = *reinterpret_cast<const uint4*>(vw + koff);
    }
    const int sl = __shfl(qperm, lane, 64);
    clse = (p.lse + static_cast<int64_t>(b) * N * H + h)[__umul24(static_cast<uint32_t>(lane < nq ? sl : 0), static_cast<uint32_t>(H))];
  };
  auto load_mask_byte = [&](int b) -> uint32_t {
    return lane < N ? static_cast<uint32_t>(p.mask[static_cast<int64_t>(b) * N + lane]) : 0u;
  };

  int b = static_cast<int>(item / H), h = static_cast<int>(item % H);
  Sites cur = make_sites(load_mask_byte(b), N);
  issue_item_loads(b, h, cur);
  int64_t nxt = item + stride;
  uint32_t mnext = 0;
  if (nxt < nitems) mnext = load_mask_byte(static_cast<int>(nxt / H));

  while (true) {
    // ---- stage the current item --------------------------------------------------------
    const int nq = nq_of(cur), nk = nk_of(cur);
    if (st_active) {
      uint4 q8[NPT], g8[NPT], k8[NPT];
#pragma unroll
      for (int u = 0; u < NPT; ++u) {
        const int r = st_r0 + u;
        const bool qok = r < nq, kok = r < nk;
        q8[u] = keep4(qok, cq[u]);
        g8[u] = keep4(qok, cg[u]);
        k8[u] = keep4(kok, ck[u]);
        const uint4 v8 = keep4(kok, cv[u]), o8 = co[u];
        // delta_r over the C8 consecutive lanes that hold row r
        float part = 0.f;
        {
          const uint32_t ow[4] = {o8.x, o8.y, o8.z, o8.w};
          const uint32_t gw[4] = {g8[u].x, g8[u].y, g8[u].z, g8[u].w};
#pragma unroll
          for (int w = 0; w < 4; ++w) part += bf_lo(ow[w]) * bf_lo(gw[w]) + bf_hi(ow[w]) * bf_hi(gw[w]);
        }
#pragma unroll
        for (int w = 1; w < C8; w <<= 1) part += __shfl_xor(part, w, 64);
        *reinterpret_cast<uint4*>(Qr + r * LDR + st_c8) = q8[u];
        *reinterpret_cast<uint4*>(Gr + r * LDR + st_c8) = g8[u];
        *reinterpret_cast<uint4*>(Kr + r * LDR + st_c8) = k8[u];
        *reinterpret_cast<uint4*>(Vr + r * LDR + st_c8) = v8;
        if (st_c8 == 0) Dls[r] = qok ? part : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int o = (st_c8 + e) * LDT + st_r0;  // even: the (r0, r0+1) pair is one word
        *reinterpret_cast<uint32_t*>(QT + o) = bf16_at(q8[0], e) | (static_cast<uint32_t>(bf16_at(q8[1], e)) << 16);
        *reinterpret_cast<uint32_t*>(GT + o) = bf16_at(g8[0], e) | (static_cast<uint32_t>(bf16_at(g8[1], e)) << 16);
        *reinterpret_cast<uint32_t*>(KT + o) = bf16_at(k8[0], e) | (static_cast<uint32_t>(bf16_at(k8[1], e)) << 16);
      }
    }
    if (tid < 64) L2s[tid] = tid < nq ? clse * kLog2e : INFINITY;
    const int bc = b, hc = h;
    const Sites sc_ = cur;
    __syncthreads();

    const bool more = nxt < nitems;
    if (more) {
      b = static_cast<int>(nxt / H);
      h = static_cast<int>(nxt % H);
      cur = make_sites(mnext, N);
      issue_item_loads(b, h, cur);
      const int64_t nn = nxt + stride;
      if (nn < nitems) mnext = load_mask_byte(static_cast<int>(nn / H));
      nxt = nn;
    }

    const int qperm = qperm_of(sc_), kperm = kperm_of(sc_);
    const int nqt = (nq + 15) >> 4, nkt = (nk + 15) >> 4;
    const int64_t e_walker = static_cast<int64_t>(bc) * N * N * H + static_cast<int64_t>(hc) * p.e_sh;
    const int64_t obase_bh = bnhd(bc, 0, hc, N, H, D);  // wave-uniform slice base of the outputs
    const float scale = p.scale;

    // ---- phase A: dq (and de), wave = 16 queries ------------------------------------------
    if (wave < nqt) {
      const int jq = wave * 16 + c;
      const bool qvalid = jq < nq;
      const int qs_ = __shfl(qperm, jq & 63, 64);
      const int qsite = qvalid ? qs_ : -1;
      bf16x8 qf[NS], gf[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(Qr + jq * LDR + 32 * s + 8 * g));
        gf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(Gr + jq * LDR + 32 * s + 8 * g));
      }
      const float lse2 = L2s[jq];
      const float delta = Dls[jq];
      const int64_t e_row = e_walker + static_cast<int64_t>(qsite < 0 ? 0 : qsite) * p.e_sq;
      const bool odd = (c & 1) != 0;
      uint16_t* const ptile = Pt + wave * kPTile + (c & ~1);
      uint16_t* const dstile = DSt + wave * kPTile + (c & ~1);
      v4f dsv[NT];
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) {
        dsv[jt] = zero4();
        if (jt < nkt) {
          v4f sc = zero4(), dp = zero4();
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            sc = mfma_bf16(as_bf16x8(*reinterpret_cast<const uint4*>(Kr + (jt * 16 + c) * LDR + 32 * s + 8 * g)), qf[s], sc);
            dp = mfma_bf16(as_bf16x8(*reinterpret_cast<const uint4*>(Vr + (jt * 16 + c) * LDR + 32 * s + 8 * g)), gf[s], dp);
          }
          float pv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = jt * 16 + 4 * g + r;
            const bool valid = j < nk && qvalid;
            float sv = sc[r] * scale;
            int ks = 0;
            if constexpr (HAS_E) {
              ks = __shfl(kperm, j & 63, 64);
              if (valid) sv += load1<BF16>(p.e, e_row + static_cast<int64_t>(ks) * p.e_sk);
            }
            pv[r] = valid ? lse_weight(sv * kLog2e - lse2) : 0.f;
            dsv[jt][r] = pv[r] * (dp[r] - delta);
            if (p.de != nullptr) {
              if constexpr (!HAS_E) ks = __shfl(kperm, j & 63, 64);
              if (valid) store1<BF16>(p.de, e_row + static_cast<int64_t>(ks) * p.e_sk, dsv[jt][r]);
            }
          }
          // P, dS of keys jt*16 + 4g + r into query tile `wave`: lanes c and c^1 trade one
          // value per key pair, then each writes the (query c&~1, query c|1) word of one key
          // (the even lane key r0, the odd lane key r0 + 1); invalid pairs hold zeros.
#pragma unroll
          for (int r0 = 0; r0 < 4; r0 += 2) {
            const int row = (jt * 16 + 4 * g + r0 + (odd ? 1 : 0)) * kPS;
            const float po = swap_lane_pair(odd ? pv[r0] : pv[r0 + 1]);
            const float dso = swap_lane_pair(odd ? dsv[jt][r0] : dsv[jt][r0 + 1]);
            *reinterpret_cast<uint32_t*>(ptile + row) = odd ? pack2_bf16(po, pv[r0 + 1]) : pack2_bf16(pv[r0], po);
            *reinterpret_cast<uint32_t*>(dstile + row) =
                odd ? pack2_bf16(dso, dsv[jt][r0 + 1]) : pack2_bf16(dsv[jt][r0], dso);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      v4f dqa[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dqa[dt] = zero4();
#pragma unroll
      for (int pp = 0; pp < NT / 2; ++pp) {
        if (2 * pp < nkt) {
          const bf16x8 dw = pack8(dsv[2 * pp], dsv[2 * pp + 1]);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            dqa[dt] = mfma_bf16(tr_operand(KT + (dt * 16 + c) * LDT + 32 * pp + 4 * g), dw, dqa[dt]);
        }
      }
      if (qvalid) {
        void* const dqw = static_cast<uint16_t*>(p.dq) + obase_bh;
        const uint32_t orow = row_off(qsite, HD);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          store4<BF16>(dqw, orow + dt * 16 + 4 * g, dqa[dt][0] * scale, dqa[dt][1] * scale,
                       dqa[dt][2] * scale, dqa[dt][3] * scale);
      }
    }

    __syncthreads();  // the P, dS tiles of every query tile are written

    // ---- phase B: dk and dv, wave = 16 keys ---------------------------------------------
    if (wave < nkt) {
      const int jk = wave * 16 + c;
      const bool kvalid = jk < nk;
      const int ks_ = __shfl(kperm, jk & 63, 64);
      const int ksite = kvalid ? ks_ : -1;
      // B operand of key jk over queries kappa(g, i) of query tiles 2pp, 2pp + 1 (the second
      // is zero when phase A did not write it)
      auto tile_operand = [&](const uint16_t* tiles, int pp) {
        const uint32_t* w0 = reinterpret_cast<const uint32_t*>(tiles + 2 * pp * kPTile + jk * kPS + 4 * g);
        uint4 u = make_uint4(w0[0], w0[1], 0u, 0u);
        if (2 * pp + 1 < nqt) {
          const uint32_t* w1 = w0 + kPTile / 2;
          u.z = w1[0];
          u.w = w1[1];
        }
        return as_bf16x8(u);
      };
      v4f dka[DT], dva[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dka[dt] = dva[dt] = zero4();
#pragma unroll
      for (int pp = 0; pp < NT / 2; ++pp) {
        if (2 * pp < nqt) {
          const bf16x8 pw = tile_operand(Pt, pp);
          const bf16x8 dw = tile_operand(DSt, pp);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            dva[dt] = mfma_bf16(tr_operand(GT + (dt * 16 + c) * LDT + 32 * pp + 4 * g), pw, dva[dt]);
            dka[dt] = mfma_bf16(tr_operand(QT + (dt * 16 + c) * LDT + 32 * pp + 4 * g), dw, dka[dt]);
          }
        }
      }
      if (kvalid) {
        void* const dkw = static_cast<uint16_t*>(p.dk) + obase_bh;
        void* const dvw = static_cast<uint16_t*>(p.dv) + obase_bh;
        const uint32_t orow = row_off(ksite, HD);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          store4<BF16>(dkw, orow + dt * 16 + 4 * g, dka[dt][0] * scale, dka[dt][1] * scale,
                       dka[dt][2] * scale, dka[dt][3] * scale);
          store4<BF16>(dvw, orow + dt * 16 + 4 * g, dva[dt][0], dva[dt][1], dva[dt][2], dva[dt][3]);
        }
      }
    }

    // ---- zeros: dq of masked queries, dk/dv of masked keys, de of invalid pairs -----------
    {
      constexpr int C4 = D / 4;
      const bool key_all = km && sc_.n_phys == 0;
      const int nmask = N - sc_.n_phys;
      if (!key_all) {
        for (int base = 0; base < nmask * C4; base += 256) {
          const int it = base + tid;
          const int site = __shfl(sc_.perm, (sc_.n_phys + it / C4) & 63, 64);
          if (it < nmask * C4) {
            const uint32_t off = row_off(site, HD) + (it % C4) * 4;
            if (!km) store4<BF16>(static_cast<uint16_t*>(p.dq) + obase_bh, off, 0.f, 0.f, 0.f, 0.f);
            store4<BF16>(static_cast<uint16_t*>(p.dk) + obase_bh, off, 0.f, 0.f, 0.f, 0.f);
            store4<BF16>(static_cast<uint16_t*>(p.dv) + obase_bh, off, 0.f, 0.f, 0.f, 0.f);
          }
        }
      }
      if (p.de != nullptr && !key_all) {
        for (int it = tid; it < N * N; it += 256) {
          const int i = it / N, j = it % N;
          const bool mi = (sc_.bal >> i) & 1u, mj = (sc_.bal >> j) & 1u;
          if (!((km || mi) && mj))
            store1<BF16>(p.de, e_walker + static_cast<int64_t>(i) * p.e_sq + static_cast<int64_t>(j) * p.e_sk, 0.f);
        }
      }
    }

    if (!more) break;
    __syncthreads();
  }
}

template <int D, bool HAS_E>
hipError_t launch_t(const BwdParams& p, hipStream_t stream) {
  using Sh = BwdBf16Shape<D>;
  auto kern = mhsea_bwd_bf16_kernel<D, HAS_E>;
  const size_t lds = Sh::kLdsBytes;
  if (lds > 64 * 1024) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         static_cast<int>(lds));
    if (err != hipSuccess) return err;
  }
  // occupancy of this instantiation, computed once; relaxed atomics keep concurrent
  // first calls from several host threads free of data races
  static std::atomic<int> per_cu_cache{0};
  int per_cu = per_cu_cache.load(std::memory_order_relaxed);
  if (per_cu == 0) {
    int n = 0;
    hipError_t err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(kern), 256, lds);
    if (err != hipSuccess) return err;
    per_cu = n > 0 ? n : 1;
    per_cu_cache.store(per_cu, std::memory_order_relaxed);
  }
  int cus = 0;
  hipError_t err = device_cu_count(&cus);
  if (err != hipSuccess) return err;
  const int64_t nitems = static_cast<int64_t>(p.B) * p.H;
  int64_t grid = static_cast<int64_t>(cus) * per_cu;
  if (grid > nitems) grid = nitems;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(256), lds, stream, p);
  return hipGetLastError();
}

}  // namespace

bool bf16_bwd_supported(int N, int H, int D) {
  // row offsets inside a (walker, head) slice use 24-bit multiplies (row_off)
  return N <= 64 && (D == 32 || D == 64) && static_cast<int64_t>(H) * D < (int64_t(1) << 23);
}

hipError_t launch_bwd_bf16(const BwdParams& p, int D, hipStream_t stream) {
  const bool e = p.e != nullptr;
  if (D == 32) return e ? launch_t<32, true>(p, stream) : launch_t<32, false>(p, stream);
  if (D == 64) return e ? launch_t<64, true>(p, stream) : launch_t<64, false>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace hz
