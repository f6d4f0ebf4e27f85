// Persistent, software-pipelined reverse-mode (VJP) MHSEA kernel for N <= 64.
//
// Cotangent algebra (custom_gradients.py:249-285, :307-347) over valid (query i, key j):
//   P = exp(S - lse), dP = dout V^T, delta_i = out_i . dout_i, dS = P o (dP - delta),
//   dq = scale dS K,  dk = scale dS^T Q,  dv = P^T dout,  de = dS.
//
// A fixed grid of workgroups walks the (walker, head) items. Per item the compacted rows of
// q (pre-scaled), k, v and dout are staged in LDS together with lse*log2(e) and delta
// (reduced while staging, so `out` never reaches LDS); the next item's rows are already in
// flight in registers while the current item computes.
//  Phase A (query-major, wave = 16 queries): S^T = K Q^T and dP^T = V dout^T for every key
//    tile, P and dS in registers, dq^T += K^T dS^T; de written from the same registers.
//  Phase B (key-major, wave = 16 keys): S = Q K^T and dP = dout V^T again (cheaper than a
//    transpose of P and dS through LDS at this size), dv^T += dout^T P, dk^T += Q^T dS.
// Every result row is written by exactly one wave: deterministic, no atomics.
//
// Bias rows (ROWS, float32, e in the [B, N, H, N] layout with N a multiple of 4): the item's
// physical query rows of e are loaded whole with 16-byte loads one item ahead and staged in
// LDS (64-float rows, 16-byte chunks XOR-swizzled by row so both phases' gathers are free of
// bank conflicts), instead of one 4-byte load per score in each phase; de is accumulated in
// an LDS tile indexed by site (zero-initialised per item, same swizzle) and written as whole
// rows with 16-byte stores, the zeros of invalid pairs included, instead of one 4-byte store
// per score and a separate pass of zero stores.
#include <atomic>
#include <type_traits>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

// D = 32: the two tiles of dq^T, dk^T, dv^T cover the even and odd features (d = 2 i + dt,
// i = tile row, dt = tile) instead of the low and high halves, so a lane's two values of a
// transposed operand (K in phase A, dout and q in phase B; features 2 c, 2 c + 1) are one
// 8-byte LDS read instead of two 4-byte reads, and a lane's eight results are the contiguous
// features 8 g .. 8 g + 7. While the partner wave's products run, an LDS read instruction
// costs a wave ~80 cycles whatever its width (MI355X): c2vjp 178.0 -> 161.2 us, c2e_vjp
// 245.5 -> 238.0 us. Four features per lane at D = 64 (one 16-byte read) made c3f32 24%
// slower (the one-wave-per-SIMD instantiation) and is not used.
template <int D>
constexpr bool bwd_pack_d() {
  return D == 32;
}
template <int DT>
__device__ __forceinline__ void lds_frag(const float* p, float (&x)[DT]) {
  if constexpr (DT == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  } else {
    const float2 v = *reinterpret_cast<const float2*>(p);
    x[0] = v.x;
    x[1] = v.y;
  }
}

template <int D>
struct BwdStreamShape {
  static constexpr int KC = 64;
  static constexpr int LD = D + 4;
  static constexpr int DG = D / 4;
  static constexpr int DT = (D + 15) / 16;
  static constexpr int C4 = D / 4;
  static constexpr int kTileFloats = KC * LD;
  static constexpr int kItems = KC * C4;
  static constexpr int kPerThread = (kItems + 255) / 256;
  static constexpr size_t kLdsBytes = static_cast<size_t>(4 * kTileFloats + 2 * KC) * 4;
  // ROWS: the staged e rows and the de tile, 64 x 64 floats each
  static constexpr size_t kRowsBytes = static_cast<size_t>(2 * KC * KC) * 4;
  // D = 64: one wave per SIMD, so the next item's prefetched rows (80 registers) and the
  // phase-B accumulators fit without scratch (two waves spilled 180-220 bytes per lane and
  // ran 2.4% slower at [4096, 64, 8, 64] fp32). D = 32 keeps three waves with 44-76 bytes of
  // scratch: two waves without it ran 2.7% slower at [1024, 64, 8, 32].
  static constexpr int kWavesPerEu = D == 64 ? 1 : 3;
};

struct Sites {
  uint64_t bal;  // bit i: site i physical
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

// Float offset of element (row, col) of a 64 x 64 LDS tile whose 16-byte chunks are
// XOR-swizzled by row: 16 rows read at one column hit 16 different chunks.
__device__ __forceinline__ int swz64(int row, int col) {
  return row * 64 + ((((col >> 2) ^ row) & 15) << 2) + (col & 3);
}

template <int D, bool HAS_E, bool ROWS, class S>
// ROWS at D = 32 takes 69 KB of LDS, so two workgroups share a CU: two waves per SIMD, whose
// register budget holds the prefetched e rows without scratch.
__global__ void __launch_bounds__(256, ((ROWS && D == 32) ? 2 : BwdStreamShape<D>::kWavesPerEu))
    mhsea_bwd_stream_kernel(const BwdParams p) {
  using Sh = BwdStreamShape<D>;
  constexpr int LD = Sh::LD, DG = Sh::DG, DT = Sh::DT, C4 = Sh::C4, NPT = Sh::kPerThread;
  constexpr int NT = 4;  // 16-row tiles of the 64-row chunk

  extern __shared__ float4 smem4[];
  float* const Qs = reinterpret_cast<float*>(smem4);  // scale * q rows
  float* const Ks = Qs + Sh::kTileFloats;
  float* const Vs = Ks + Sh::kTileFloats;
  float* const Gs = Vs + Sh::kTileFloats;               // dout rows
  float* const L2s = Gs + Sh::kTileFloats;              // lse * log2(e) per compacted query
  float* const Dls = L2s + Sh::KC;                      // delta per compacted query
  float* const Es = Dls + Sh::KC;                       // ROWS: e rows [compacted query][site]
  float* const Des = Es + Sh::KC * Sh::KC;              // ROWS: de [query site][key site]

  const int N = p.N, H = p.H;
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

  // list helpers: queries are the physical sites (all sites under the key mask); keys are
  // the physical sites (all sites if none is physical under the key mask)
  auto nq_of = [&](const Sites& s) { return km ? N : s.n_phys; };
  auto nk_of = [&](const Sites& s) { return (km && s.n_phys == 0) ? N : s.n_phys; };
  auto qperm_of = [&](const Sites& s) { return km ? lane : s.perm; };
  auto kperm_of = [&](const Sites& s) { return (km && s.n_phys == 0) ? lane : s.perm; };

  Raw4<S> cq[NPT], ck[NPT], cv[NPT], cg[NPT], co[NPT];
  float clse = 0.f;
  constexpr int NE = ROWS && HAS_E ? 4 : 0;  // e float4 per thread: 64 rows x 16 chunks / 256
  v4f ce[NE > 0 ? NE : 1];  // ext-vector type: promoted to registers (float4 arrays went to scratch)
  const int nc4 = N >> 2;                    // 16-byte chunks of one e row (ROWS: N % 4 == 0)

  auto issue_item_loads = [&](int b, int h, const Sites& st) __attribute__((always_inline)) {
    const int qperm = qperm_of(st), kperm = kperm_of(st), nq = nq_of(st), nk = nk_of(st);
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int it = tid + u * 256;
      const int r = it / C4;
      const int sq = __shfl(qperm, r & 63, 64);
      const int sk = __shfl(kperm, r & 63, 64);
      const bool in = Sh::kItems % 256 == 0 || it < Sh::kItems;
      const int64_t qoff = bnhd(b, (in && r < nq) ? sq : 0, h, N, H, D) + (it % C4) * 4;
      const int64_t koff = bnhd(b, (in && r < nk) ? sk : 0, h, N, H, D) + (it % C4) * 4;
      cq[u] = Raw4<S>::load(p.q, qoff);
      cg[u] = Raw4<S>::load(p.dout, qoff);
      co[u] = Raw4<S>::load(p.out, qoff);
      ck[u] = Raw4<S>::load(p.k, koff);
      cv[u] = Raw4<S>::load(p.v, koff);
    }
    const int sl = __shfl(qperm, lane, 64);
    clse = p.lse[(static_cast<int64_t>(b) * N + (lane < nq ? sl : 0)) * H + h];
    if constexpr (NE > 0) {
      const float* ew = static_cast<const float*>(p.e) + static_cast<int64_t>(b) * N * N * H +
                        static_cast<int64_t>(h) * p.e_sh;
#pragma unroll
      for (int u = 0; u < NE; ++u) {
        const int it = tid + u * 256;
        const int r = it >> 4, c4 = it & 15;
        const int sq = __shfl(qperm, r & 63, 64);
        const bool ok = r < nq && c4 < nc4;
        ce[u] = *reinterpret_cast<const v4f*>(ew + static_cast<int64_t>(ok ? sq : 0) * p.e_sq + (ok ? c4 : 0) * 4);
      }
    }
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
    // ---- stage the current item -----------------------------------------------------
    const int nq = nq_of(cur), nk = nk_of(cur);
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int it = tid + u * 256;
      const bool in = Sh::kItems % 256 == 0 || it < Sh::kItems;
      const int r = it / C4;
      const bool qok = in && r < nq, kok = in && r < nk;
      const int so = r * LD + (it % C4) * 4;
      const float4 q4 = cq[u].f(), g4 = cg[u].f(), o4 = co[u].f();
      // delta_r: the C4 threads of row r are consecutive lanes of one wave
      float part = (o4.x * g4.x + o4.y * g4.y) + (o4.z * g4.z + o4.w * g4.w);
#pragma unroll
      for (int w = 1; w < C4; w <<= 1) part += __shfl_xor(part, w, 64);
      if (in) {
        *reinterpret_cast<float4*>(Qs + so) =
            make_float4(qok ? q4.x * p.scale : 0.f, qok ? q4.y * p.scale : 0.f,
                        qok ? q4.z * p.scale : 0.f, qok ? q4.w * p.scale : 0.f);
        *reinterpret_cast<float4*>(Gs + so) =
            make_float4(qok ? g4.x : 0.f, qok ? g4.y : 0.f, qok ? g4.z : 0.f, qok ? g4.w : 0.f);
        const float4 k4 = ck[u].f(), v4 = cv[u].f();
        *reinterpret_cast<float4*>(Ks + so) =
            make_float4(kok ? k4.x : 0.f, kok ? k4.y : 0.f, kok ? k4.z : 0.f, kok ? k4.w : 0.f);
        *reinterpret_cast<float4*>(Vs + so) =
            make_float4(kok ? v4.x : 0.f, kok ? v4.y : 0.f, kok ? v4.z : 0.f, kok ? v4.w : 0.f);
        if (it % C4 == 0) Dls[r] = qok ? part : 0.f;
      }
    }
    if (tid < 64) L2s[tid] = tid < nq ? clse * kLog2e : INFINITY;
    if constexpr (ROWS) {
      // the 64 x 64 tiles: 1024 chunks over 256 threads, chunk u * 256 + tid (written out so
      // the prefetch registers are never indexed at run time)
      const int r0 = tid >> 4, c40 = tid & 15;
      if constexpr (NE > 0) {
        *reinterpret_cast<v4f*>(Es + swz64(r0, 4 * c40)) = ce[0];
        *reinterpret_cast<v4f*>(Es + swz64(r0 + 16, 4 * c40)) = ce[1];
        *reinterpret_cast<v4f*>(Es + swz64(r0 + 32, 4 * c40)) = ce[2];
        *reinterpret_cast<v4f*>(Es + swz64(r0 + 48, 4 * c40)) = ce[3];
      }
      if (p.de != nullptr) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          *reinterpret_cast<float4*>(Des + swz64(r0 + 16 * u, 4 * c40)) = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    const int bc = b, hc = h;
    const Sites sc_ = cur;
    __syncthreads();

    // ---- next item's loads ----------------------------------------------------------
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

    // store u of a lane's [DT][4] results writes features sd0(u) .. sd0(u) + 3, its m-th
    // value being element (sdt(u, m), sr(u, m))
    constexpr bool kPack = bwd_pack_d<D>();
    auto sd0 = [&](int u) { return kPack ? 4 * DT * g + 4 * u : u * 16 + 4 * g; };
    auto sdt = [&](int u, int m) { return kPack ? (4 * u + m) % DT : u; };
    auto sr = [&](int u, int m) { return kPack ? (4 * u + m) / DT : m; };

    // ---- phase A: dq (and de), wave = 16 queries ----------------------------------------
    if (wave < nqt) {
      const int jq = wave * 16 + c;
      const bool qvalid = jq < nq;
      const int qs_ = __shfl(qperm, jq & 63, 64);
      const int qsite = qvalid ? qs_ : -1;
      float qf[DG], gf[DG];
      const float* qrow = Qs + (wave * 16 + c) * LD + g * DG;
      const float* grow = Gs + (wave * 16 + c) * LD + g * DG;
#pragma unroll
      for (int s = 0; s < DG; ++s) {
        qf[s] = qrow[s];
        gf[s] = grow[s];
      }
      const float lse2 = L2s[wave * 16 + c];
      const float delta = Dls[wave * 16 + c];
      const int64_t e_row = e_walker + static_cast<int64_t>(qsite < 0 ? 0 : qsite) * p.e_sq;
      v4f dqa[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dqa[dt] = zero4();
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) {
        if (jt < nkt) {
          const float* krow = Ks + (jt * 16 + c) * LD + g * DG;
          const float* vrow = Vs + (jt * 16 + c) * LD + g * DG;
          v4f sc = zero4(), dp = zero4();
#pragma unroll
          for (int s = 0; s < DG; ++s) {
            sc = mfma16x4(krow[s], qf[s], sc);
            dp = mfma16x4(vrow[s], gf[s], dp);
          }
          float dsv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = jt * 16 + 4 * g + r;
            const bool valid = j < nk && qvalid;
            float sv = sc[r];
            int ks = 0;
            if constexpr (HAS_E) {
              ks = __shfl(kperm, j & 63, 64);
              if constexpr (ROWS) {
                if (valid) sv += Es[swz64(jq, ks)];
              } else {
                if (valid) sv += load1<S>(p.e, e_row + static_cast<int64_t>(ks) * p.e_sk);
              }
            }
            const float pv = valid ? lse_weight(sv * kLog2e - lse2) : 0.f;
            dsv[r] = pv * (dp[r] - delta);
            if (p.de != nullptr) {
              if constexpr (!HAS_E) ks = __shfl(kperm, j & 63, 64);
              if constexpr (ROWS) {
                if (valid) Des[swz64(qsite, ks)] = dsv[r];
              } else {
                if (valid) store1<S>(p.de, e_row + static_cast<int64_t>(ks) * p.e_sk, dsv[r]);
              }
            }
          }
          if constexpr (bwd_pack_d<D>()) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float ka[DT];
              lds_frag<DT>(Ks + (jt * 16 + 4 * g + r) * LD + DT * c, ka);
#pragma unroll
              for (int dt = 0; dt < DT; ++dt) dqa[dt] = mfma16x4(ka[dt], dsv[r], dqa[dt]);
            }
          } else {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = dt * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float ka = (D % 16 == 0 || col < D) ? Ks[(jt * 16 + 4 * g + r) * LD + col] : 0.f;
              dqa[dt] = mfma16x4(ka, dsv[r], dqa[dt]);
            }
          }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (qvalid) {
        const int64_t obase = bnhd(bc, qsite, hc, N, H, D);
#pragma unroll
        for (int u = 0; u < DT; ++u) {
          const int d0 = sd0(u);
          if (D % 16 != 0 && d0 >= D) continue;
          store4<S>(p.dq, obase + d0, dqa[sdt(u, 0)][sr(u, 0)] * p.scale, dqa[sdt(u, 1)][sr(u, 1)] * p.scale,
                    dqa[sdt(u, 2)][sr(u, 2)] * p.scale, dqa[sdt(u, 3)][sr(u, 3)] * p.scale);
        }
      }
    }

    // ---- phase B: dk and dv, wave = 16 keys ------------------------------------------
    if (wave < nkt) {
      const int jk = wave * 16 + c;
      const bool kvalid = jk < nk;
      const int ks_ = __shfl(kperm, jk & 63, 64);
      const int ksite = kvalid ? ks_ : -1;
      float kf[DG], vf[DG];
      const float* krow = Ks + (wave * 16 + c) * LD + g * DG;
      const float* vrow = Vs + (wave * 16 + c) * LD + g * DG;
#pragma unroll
      for (int s = 0; s < DG; ++s) {
        kf[s] = krow[s];
        vf[s] = vrow[s];
      }
      v4f dka[DT], dva[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dka[dt] = dva[dt] = zero4();
#pragma unroll
      for (int it = 0; it < NT; ++it) {
        if (it < nqt) {
          const float* qrow = Qs + (it * 16 + c) * LD + g * DG;
          const float* grow = Gs + (it * 16 + c) * LD + g * DG;
          v4f sc = zero4(), dp = zero4();
#pragma unroll
          for (int s = 0; s < DG; ++s) {
            sc = mfma16x4(qrow[s], kf[s], sc);  // S[query it*16+4g+r][key c]
            dp = mfma16x4(grow[s], vf[s], dp);
          }
          float pv[4], dsv[4];
          // the four rows' lse and delta read ahead of the row loop: one 16-byte read each at
          // D = 32, 4-byte reads at D = 64 (c3f32 1768 -> 1692 us); D <= 16 reads them inside
          // the loop (hoisted, the gated trunk's reverse mode measured 692 -> 737 us)
          float l2r[4], dlr[4];
          if constexpr (D == 32) {
            const float4 l2v = *reinterpret_cast<const float4*>(L2s + it * 16 + 4 * g);
            const float4 dlv = *reinterpret_cast<const float4*>(Dls + it * 16 + 4 * g);
            l2r[0] = l2v.x, l2r[1] = l2v.y, l2r[2] = l2v.z, l2r[3] = l2v.w;
            dlr[0] = dlv.x, dlr[1] = dlv.y, dlr[2] = dlv.z, dlr[3] = dlv.w;
          } else if constexpr (D == 64) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              l2r[r] = L2s[it * 16 + 4 * g + r];
              dlr[r] = Dls[it * 16 + 4 * g + r];
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int il = it * 16 + 4 * g + r;
            const bool valid = il < nq && kvalid;
            float sv = sc[r];
            if constexpr (HAS_E) {
              if constexpr (ROWS) {
                if (valid) sv += Es[swz64(il, ksite)];
              } else {
                const int qs2 = __shfl(qperm, il & 63, 64);
                if (valid)
                  sv += load1<S>(p.e, e_walker + static_cast<int64_t>(qs2) * p.e_sq +
                                          static_cast<int64_t>(ksite) * p.e_sk);
              }
            }
            pv[r] = valid ? lse_weight(sv * kLog2e - (D >= 32 ? l2r[r] : L2s[il])) : 0.f;
            dsv[r] = pv[r] * (dp[r] - (D >= 32 ? dlr[r] : Dls[il]));
          }
          if constexpr (bwd_pack_d<D>()) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = it * 16 + 4 * g + r;
              float ga[DT], qa[DT];
              lds_frag<DT>(Gs + row * LD + DT * c, ga);
              lds_frag<DT>(Qs + row * LD + DT * c, qa);
#pragma unroll
              for (int dt = 0; dt < DT; ++dt) {
                dva[dt] = mfma16x4(ga[dt], pv[r], dva[dt]);
                dka[dt] = mfma16x4(qa[dt], dsv[r], dka[dt]);
              }
            }
          } else {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int col = dt * 16 + c;
            const bool in_d = D % 16 == 0 || col < D;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = it * 16 + 4 * g + r;
              const float ga = in_d ? Gs[row * LD + col] : 0.f;
              const float qa = in_d ? Qs[row * LD + col] : 0.f;
              dva[dt] = mfma16x4(ga, pv[r], dva[dt]);
              dka[dt] = mfma16x4(qa, dsv[r], dka[dt]);
            }
          }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kvalid) {
        const int64_t obase = bnhd(bc, ksite, hc, N, H, D);
#pragma unroll
        for (int u = 0; u < DT; ++u) {
          const int d0 = sd0(u);
          if (D % 16 != 0 && d0 >= D) continue;
          store4<S>(p.dk, obase + d0, dka[sdt(u, 0)][sr(u, 0)], dka[sdt(u, 1)][sr(u, 1)], dka[sdt(u, 2)][sr(u, 2)],
                    dka[sdt(u, 3)][sr(u, 3)]);
          store4<S>(p.dv, obase + d0, dva[sdt(u, 0)][sr(u, 0)], dva[sdt(u, 1)][sr(u, 1)], dva[sdt(u, 2)][sr(u, 2)],
                    dva[sdt(u, 3)][sr(u, 3)]);
        }
      }
    }

    // ---- zeros: dq of masked queries, dk/dv of masked keys, de of invalid pairs ---------
    {
      const bool key_all = km && sc_.n_phys == 0;
      const int nmask = N - sc_.n_phys;
      if (!key_all) {
        // item (b, h) zeroes the masked sites i = h, h + H, ... of its walker for every head,
        // each site's [H, D] rows as one contiguous run (the walker's H items cover every
        // masked site once; per-item 128-byte rows at a stride of H D cost the forward 2.6%)
        const int F = H * C4;
        const int nmine = nmask > hc ? (nmask - hc + H - 1) / H : 0;
        for (int si = static_cast<int>(threadIdx.x >> 6); si < nmine; si += 4) {  // a site per wave
          const int site = __builtin_amdgcn_readlane(sc_.perm, (sc_.n_phys + hc + si * H) & 63);
          const int64_t base = bnhd(bc, site, 0, N, H, D);
          for (int w = static_cast<int>(threadIdx.x & 63); w < F; w += 64) {
            if (!km) store4<S>(p.dq, base + 4 * w, 0.f, 0.f, 0.f, 0.f);
            store4<S>(p.dk, base + 4 * w, 0.f, 0.f, 0.f, 0.f);
            store4<S>(p.dv, base + 4 * w, 0.f, 0.f, 0.f, 0.f);
          }
        }
      }
      if constexpr (ROWS) {
        if (p.de != nullptr) {  // the whole de block of the item from its LDS tile
          __syncthreads();
          float* dw = static_cast<float*>(p.de) + e_walker;
          for (int it = tid; it < N * nc4; it += 256) {
            const int i = it / nc4, c4 = it - i * nc4;
            *reinterpret_cast<float4*>(dw + static_cast<int64_t>(i) * p.e_sq + 4 * c4) =
                *reinterpret_cast<const float4*>(Des + swz64(i, 4 * c4));
          }
        }
      } else if (p.de != nullptr && !key_all) {
        // invalid pairs: every key of a masked query row (square mask), and every masked
        // key of the other rows
        for (int it = tid; it < N * N; it += 256) {
          const int i = it / N, j = it % N;
          const bool mi = (sc_.bal >> i) & 1u, mj = (sc_.bal >> j) & 1u;
          const bool valid = (km || mi) && mj;
          if (!valid)
            store1<S>(p.de, e_walker + static_cast<int64_t>(i) * p.e_sq + static_cast<int64_t>(j) * p.e_sk, 0.f);
        }
      }
    }

    if (!more) break;
    __syncthreads();
  }
}

template <int D, bool HAS_E, bool ROWS, class S>
hipError_t launch_bwd_stream_t(const BwdParams& p, hipStream_t stream) {
  using Sh = BwdStreamShape<D>;
  auto kern = mhsea_bwd_stream_kernel<D, HAS_E, ROWS, S>;
  const size_t lds = Sh::kLdsBytes + (ROWS ? Sh::kRowsBytes : 0);
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

template <int D, class S>
hipError_t dispatch_e(const BwdParams& p, hipStream_t stream) {
  // LDS-staged bias rows and de tile: float32, keys contiguous ([B, N, H, N]), N % 4 == 0,
  // and a bias or a bias cotangent to move
  if constexpr (std::is_same<S, F32>::value) {
    if (p.e_sk == 1 && p.N % 4 == 0 && (p.e != nullptr || p.de != nullptr)) {
      if (p.e != nullptr) return launch_bwd_stream_t<D, true, true, S>(p, stream);
      return launch_bwd_stream_t<D, false, true, S>(p, stream);
    }
  }
  if (p.e != nullptr) return launch_bwd_stream_t<D, true, false, S>(p, stream);
  return launch_bwd_stream_t<D, false, false, S>(p, stream);
}

template <class S>
hipError_t dispatch_d(const BwdParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 8: return dispatch_e<8, S>(p, stream);
    case 16: return dispatch_e<16, S>(p, stream);
    case 32: return dispatch_e<32, S>(p, stream);
    case 64: return dispatch_e<64, S>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool stream_bwd_supported(int N) { return N <= 64; }

hipError_t launch_bwd_stream(const BwdParams& p, int D, int dtype, hipStream_t stream) {
  if (dtype == 1) return dispatch_d<BF16>(p, D, stream);
  return dispatch_d<F32>(p, D, stream);
}

}  // namespace hz
