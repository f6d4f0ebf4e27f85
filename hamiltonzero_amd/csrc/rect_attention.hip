// Rectangular multi-head attention with a dense pair bias (large-N evaluation path).
//
// Replaces the Pallas kernel noncausal_bias_mha (src/hamiltonzero/evaluation/
// pallas_mha.py:43-161) and its wrapper pallas_rectangular_edge_attention
// (evaluation/sequence_parallel.py:59-90):
//   out[b,i,h,:] = sum_j softmax_j( scale q[b,i,h,:].k[b,j,h,:] + bias'[b,i,j,h] ) v[b,j,h,:]
//   bias'        = where(key_mask[b,j], bias[b,i,j,h], -1e30)      (sequence_parallel.py:79-83)
// q, out: [B, Nq, H, D]; k, v: [B, Nk, H, D]; bias: [B, Nq, Nk, H] (heads innermost).
//
// A masked key's score is -1e30 in float32 whatever q.k is (|q.k| is far below half an
// ulp of 1e30), so its weight exp(-1e30 - max) is exactly 0 as soon as one key of the
// system is physical: the kernel compacts the key mask into the list of physical keys and
// never reads a masked key's K, V or bias. If no key is physical every score equals -1e30,
// every weight is 1 and the result is the mean of all Nk value rows; the kernel computes
// exactly that (all keys, scores 0).
//
// Work decomposition. The bias is the largest operand (Nq Nk H floats against
// (2Nq + 2Nk) H D for q, k, v, out) and its heads are innermost, so one head's scores are
// H floats apart in memory. A workgroup therefore owns HG consecutive heads (HG = 4 when H
// is a multiple of 4) of one block of 16 QT queries of one system: it reads the bias as
// HG-float vectors per (query, key), i.e. HG times fewer cache-line visits than one head
// per workgroup, and redistributes the values per head through LDS. Wave w owns head
// h0 + w / QT and query tile w % QT (16 queries) and works in the transposed orientation
//   S^T(16 keys x 16 queries) = K . Q^T,   O^T(d x queries) += V^T . P^T
// with v_mfma_f32_16x16x4_f32, so the online-softmax statistics of a query are lane-local
// and S^T's output layout is directly the B operand of the P.V product. Keys (K and V of
// the HG heads) and the bias block are staged in LDS in chunks of KC = 32 keys; the next
// chunk is loaded into registers while the current one is computed.
//
// Gated mode (the large-N caller's head collapse, sequence_trunk.py:981): head h < H/2 gates
// head h + H/2, y = sigmoid(out_h) * out_{h + H/2}, and only y [B, Nq, H/2, D] is written. A
// workgroup then owns HG/2 consecutive gate heads g0.. and their value heads H/2 + g0..
// (bias read as two HG/2-float vectors per (query, key)); after the key loop the gate waves
// leave their normalised rows in LDS and the value wave of the same query tile combines them.
#include <hip/hip_runtime.h>

#include "mhsea_device.h"
#include "mhsea_launch.h"

namespace hz {
namespace {

template <int D, int HG, int QT>
struct RectShape {
  static constexpr int KC = 32;                // keys per LDS chunk
  static constexpr int NJT = KC / 16;          // 16-key tiles per chunk
  static constexpr int LD = D + 4;             // padded K / V row in LDS, floats
  static constexpr int KCP = KC + 4;           // padded bias row in LDS, floats
  static constexpr int QB = 16 * QT;           // queries per workgroup
  static constexpr int NW = QT * HG;           // waves per workgroup
  static constexpr int NT = 64 * NW;           // threads per workgroup
  static constexpr int DG = D / 4;             // contraction values per lane in K.Q^T
  static constexpr int DT = (D + 15) / 16;     // 16-row tiles of O^T
  static constexpr int C4 = D / 4;             // float4 columns of one head row (D >= 8)
  static constexpr int kRowItems = HG * C4;    // float4 items of one key row (HG heads)
  static constexpr int kKvItems = KC * kRowItems;
  static constexpr int kKvPerThread = (kKvItems + NT - 1) / NT;
  static constexpr int kBiasItems = QB * KC;   // (query, key) pairs per chunk
  static constexpr int kBiasPerThread = kBiasItems / NT;  // = 8 / HG, exact
  static constexpr int kKvFloats = HG * KC * LD;          // one tensor (K or V) in LDS
  static constexpr int kBiasFloats = HG * QB * KCP;
  static_assert(kBiasItems % NT == 0, "bias items must divide evenly over the threads");
  static size_t lds_bytes(int Nk, bool masked) {
    size_t idx = masked ? ((static_cast<size_t>(Nk) * 2 + 15) & ~size_t(15)) : 0;
    return (static_cast<size_t>(2) * kKvFloats + kBiasFloats) * 4 + 16 * 4 /*scratch*/ + idx;
  }
};

// Global head of local head hh of head group gi: HG consecutive heads, or (gated) HG/2 gate
// heads and their HG/2 value heads H/2 further on.
template <int HG, bool GATED>
__device__ __forceinline__ int rect_head(int gi, int hh, int H) {
  if constexpr (GATED) return hh < HG / 2 ? gi * (HG / 2) + hh : H / 2 + gi * (HG / 2) + (hh - HG / 2);
  return gi * HG + hh;
}

// HG consecutive floats (the workgroup's heads of one bias element).
template <int HG>
struct BiasVec;
template <>
struct BiasVec<4> {
  float4 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ float get(int i) const { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
};
template <>
struct BiasVec<2> {
  float2 v;
  __device__ __forceinline__ void load(const float* p) { v = *reinterpret_cast<const float2*>(p); }
  __device__ __forceinline__ float get(int i) const { return i == 0 ? v.x : v.y; }
};
template <>
struct BiasVec<1> {
  float v;
  __device__ __forceinline__ void load(const float* p) { v = *p; }
  __device__ __forceinline__ float get(int) const { return v; }
};

// The workgroup's HG bias values of one (query, key): one HG-float vector, or (gated) the
// HG/2 gate heads' and the HG/2 value heads' vectors.
template <int HG, bool GATED>
struct BiasHeads {
  BiasVec<HG> v;
  __device__ __forceinline__ void load(const float* row, int gi, int H) { v.load(row + gi * HG); }
  __device__ __forceinline__ float get(int i) const { return v.get(i); }
};
template <int HG>
struct BiasHeads<HG, true> {
  BiasVec<HG / 2> gv, vv;
  __device__ __forceinline__ void load(const float* row, int gi, int H) {
    gv.load(row + gi * (HG / 2));
    vv.load(row + H / 2 + gi * (HG / 2));
  }
  __device__ __forceinline__ float get(int i) const { return i < HG / 2 ? gv.get(i) : vv.get(i - HG / 2); }
};

// Compaction of one system's key mask into the ascending list of physical keys, for a
// workgroup of NW waves. Returns the count to every thread. scratch holds NW ints.
template <int NW>
__device__ __forceinline__ int compact_keys(const uint8_t* __restrict__ mask_row, int N,
                                            int16_t* __restrict__ idx, int* __restrict__ scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  int total = 0;
  for (int base = 0; base < N; base += 64 * NW) {
    const int pos = base + tid;
    const bool on = pos < N && mask_row[pos] != 0;
    const uint64_t bal = __ballot(on);
    if (lane == 0) scratch[wave] = __popcll(bal);
    __syncthreads();
    int before = total;
    int all = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      before += w < wave ? scratch[w] : 0;
      all += scratch[w];
    }
    if (on) idx[before + __popcll(bal & ((uint64_t(1) << lane) - 1))] = static_cast<int16_t>(pos);
    total += all;
    __syncthreads();
  }
  return total;
}

// What the staging steps of one workgroup need (fixed for the whole kernel).
struct StageArgs {
  const float* kbase;  // k of this system (head 0)
  const float* vbase;
  const float* ebase;  // bias of this system (head 0); null = no bias
  const int16_t* idx;  // physical keys (LDS), used when gather
  int nk, Nq, Nk, H, q0, gi;
  bool gather;
};

// Issue the global loads of key chunk [kc, kc + KC) into registers: the K and V rows of
// the workgroup's HG heads (one contiguous HG*D run per key, two runs when gated) and the
// bias block [QB queries][KC keys][HG heads]. Every load is in bounds (padding rows read
// key 0 / the last query row); padding is zeroed or ignored when the chunk is written to LDS.
template <int D, int HG, int QT, bool GATED, int KVP, int BP>
__device__ __forceinline__ void rect_load_chunk(float4 (&rk)[KVP], float4 (&rv)[KVP],
                                                BiasHeads<HG, GATED> (&re)[BP], const StageArgs& a, int kc) {
  using Sh = RectShape<D, HG, QT>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < Sh::kKvPerThread; ++u) {
    const int it = tid + u * Sh::NT;
    const int j = kc + it / Sh::kRowItems;
    const bool ok = (Sh::kKvItems % Sh::NT == 0 || it < Sh::kKvItems) && j < a.nk;
    const int n = ok ? (a.gather ? a.idx[j] : j) : 0;
    const int hh = (it % Sh::kRowItems) / Sh::C4;
    const int64_t off = static_cast<int64_t>(n) * a.H * D + rect_head<HG, GATED>(a.gi, hh, a.H) * D +
                        (it % Sh::C4) * 4;
    rk[u] = *reinterpret_cast<const float4*>(a.kbase + off);
    rv[u] = *reinterpret_cast<const float4*>(a.vbase + off);
  }
  if (a.ebase != nullptr) {
#pragma unroll
    for (int u = 0; u < Sh::kBiasPerThread; ++u) {
      const int it = tid + u * Sh::NT;
      const int qi = it / Sh::KC;
      const int j = kc + it % Sh::KC;
      const int qrow = a.q0 + qi < a.Nq ? a.q0 + qi : a.Nq - 1;
      const int n = j < a.nk ? (a.gather ? a.idx[j] : j) : 0;
      re[u].load(a.ebase + (static_cast<int64_t>(qrow) * a.Nk + n) * a.H, a.gi, a.H);
    }
  }
}

// Write the staged chunk to LDS: K and V as [head][key][LD] (rows past the last key
// zeroed), the bias as [head][query][KCP].
template <int D, int HG, int QT, bool GATED, int KVP, int BP>
__device__ __forceinline__ void rect_store_chunk(const float4 (&rk)[KVP], const float4 (&rv)[KVP],
                                                 const BiasHeads<HG, GATED> (&re)[BP], float* Ks, float* Vs,
                                                 float* Es, const StageArgs& a, int kc) {
  using Sh = RectShape<D, HG, QT>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < Sh::kKvPerThread; ++u) {
    const int it = tid + u * Sh::NT;
    if (Sh::kKvItems % Sh::NT == 0 || it < Sh::kKvItems) {
      const int r = it / Sh::kRowItems;
      const int hh = (it % Sh::kRowItems) / Sh::C4;
      const int c4 = it % Sh::C4;
      const bool ok = kc + r < a.nk;
      const int so = (hh * Sh::KC + r) * Sh::LD + c4 * 4;
      // Component-wise selects: a select of whole float4 values is lowered through scratch.
      const float4 x = rk[u], y = rv[u];
      *reinterpret_cast<float4*>(Ks + so) =
          make_float4(ok ? x.x : 0.f, ok ? x.y : 0.f, ok ? x.z : 0.f, ok ? x.w : 0.f);
      *reinterpret_cast<float4*>(Vs + so) =
          make_float4(ok ? y.x : 0.f, ok ? y.y : 0.f, ok ? y.z : 0.f, ok ? y.w : 0.f);
    }
  }
  if (a.ebase != nullptr) {
#pragma unroll
    for (int u = 0; u < Sh::kBiasPerThread; ++u) {
      const int it = tid + u * Sh::NT;
      const int qi = it / Sh::KC;
      const int j = it % Sh::KC;
#pragma unroll
      for (int hh = 0; hh < HG; ++hh) Es[(hh * Sh::QB + qi) * Sh::KCP + j] = re[u].get(hh);
    }
  }
}

template <int D, int HG, int QT, bool GATED>
__global__ void __launch_bounds__(64 * QT * HG) rect_attention_fwd_kernel(const RectParams p) {
  using Sh = RectShape<D, HG, QT>;
  constexpr int KC = Sh::KC, NJT = Sh::NJT, LD = Sh::LD, KCP = Sh::KCP, QB = Sh::QB;
  constexpr int DG = Sh::DG, DT = Sh::DT;
  constexpr int KVP = Sh::kKvPerThread, BP = Sh::kBiasPerThread;

  extern __shared__ float4 smem4[];
  float* const Ks = reinterpret_cast<float*>(smem4);
  float* const Vs = Ks + Sh::kKvFloats;
  float* const Es = Vs + Sh::kKvFloats;
  int* const scratch = reinterpret_cast<int*>(Es + Sh::kBiasFloats);
  int16_t* const idx = reinterpret_cast<int16_t*>(scratch + 16);

  const int Nq = p.Nq, Nk = p.Nk, H = p.H;
  const int nqb = (Nq + QB - 1) / QB;
  const int nhg = H / HG;
  const int64_t nwg = static_cast<int64_t>(p.B) * nqb * nhg;
  // Consecutive logical blocks (the head groups of one query block, then the next query
  // blocks of the same system) share bias cache lines and K / V rows: keep them on one XCD.
  const int64_t lb = xcd_logical_block(blockIdx.x, nwg);
  const int hgi = static_cast<int>(lb % nhg);
  const int qblk = static_cast<int>((lb / nhg) % nqb);
  const int b = static_cast<int>(lb / (static_cast<int64_t>(nhg) * nqb));
  const int q0 = qblk * QB;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int hl = wave / QT;  // local head of this wave
  const int qt = wave % QT;  // query tile of this wave

  // Keys: the physical list (compacted mask), all keys without a mask, or all keys with
  // scores 0 when no key is physical (the -1e30 limit).
  int nk = Nk;
  bool gather = false, uniform = false;
  if (p.key_mask != nullptr) {
    const int n_phys = compact_keys<Sh::NW>(p.key_mask + static_cast<int64_t>(b) * Nk, Nk, idx, scratch);
    if (n_phys > 0) {
      nk = n_phys;
      gather = true;
    } else {
      uniform = true;
    }
  }

  // ---- staging: registers <- global (next chunk), LDS <- registers (this chunk) ---------
  float4 rk[KVP], rv[KVP];
  BiasHeads<HG, GATED> re[BP];
  const float* const kbase = p.k + static_cast<int64_t>(b) * Nk * H * D;
  const float* const vbase = p.v + static_cast<int64_t>(b) * Nk * H * D;
  const float* const ebase = p.bias == nullptr ? nullptr : p.bias + static_cast<int64_t>(b) * Nq * Nk * H;
  const StageArgs sa{kbase, vbase, ebase, idx, nk, Nq, Nk, H, q0, hgi, gather};

  rect_load_chunk<D, HG, QT, GATED>(rk, rv, re, sa, 0);

  // Query fragment in B-operand layout: lane (g, c) holds q[q][h][g*DG .. g*DG + DG), scaled.
  const int qrow = q0 + qt * 16 + c;
  const bool active = q0 + qt * 16 < Nq;  // wave-uniform
  const bool qvalid = qrow < Nq;
  const int h = rect_head<HG, GATED>(hgi, hl, H);
  float qf[DG];
  {
    const int64_t qoff = ((static_cast<int64_t>(b) * Nq + (qvalid ? qrow : 0)) * H + h) * D + g * DG;
    if constexpr (DG >= 4) {
#pragma unroll
      for (int s = 0; s < DG; s += 4) {
        const float4 x = *reinterpret_cast<const float4*>(p.q + qoff + s);
        qf[s] = x.x;
        qf[s + 1] = x.y;
        qf[s + 2] = x.z;
        qf[s + 3] = x.w;
      }
    } else {
      const float2 x = *reinterpret_cast<const float2*>(p.q + qoff);
      qf[0] = x.x;
      qf[1] = x.y;
    }
    const float qs = qvalid && !uniform ? p.scale : 0.f;
#pragma unroll
    for (int s = 0; s < DG; ++s) qf[s] *= qs;
  }
  const bool use_bias = ebase != nullptr && !uniform;

  v4f o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = zero4();
  float m2 = -INFINITY;  // running max of the base-2 scores of this lane's query
  float lsum = 0.f;      // this lane's share of the softmax normaliser

  const float* const Kw = Ks + hl * KC * LD;
  const float* const Vw = Vs + hl * KC * LD;
  const float* const Ew = Es + (hl * QB + qt * 16 + c) * KCP;

  for (int kc = 0; kc < nk; kc += KC) {
    if (kc > 0) __syncthreads();  // every wave is done with the previous chunk
    rect_store_chunk<D, HG, QT, GATED>(rk, rv, re, Ks, Vs, Es, sa, kc);
    __syncthreads();
    if (kc + KC < nk) rect_load_chunk<D, HG, QT, GATED>(rk, rv, re, sa, kc + KC);
    if (!active) continue;

    // Scores of the chunk's key tiles, the tiles' accumulator chains interleaved (one
    // 16-byte K read per tile and four contraction steps).
    v4f sc[NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) sc[jt] = zero4();
    if constexpr (DG >= 4) {
#pragma unroll
      for (int s = 0; s < DG; s += 4) {
        float4 kv[NJT];
#pragma unroll
        for (int jt = 0; jt < NJT; ++jt)
          kv[jt] = *reinterpret_cast<const float4*>(Kw + (jt * 16 + c) * LD + g * DG + s);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jt = 0; jt < NJT; ++jt) sc[jt] = mfma16x4(kv[jt].x, qf[s], sc[jt]);
#pragma unroll
        for (int jt = 0; jt < NJT; ++jt) sc[jt] = mfma16x4(kv[jt].y, qf[s + 1], sc[jt]);
#pragma unroll
        for (int jt = 0; jt < NJT; ++jt) sc[jt] = mfma16x4(kv[jt].z, qf[s + 2], sc[jt]);
#pragma unroll
        for (int jt = 0; jt < NJT; ++jt) sc[jt] = mfma16x4(kv[jt].w, qf[s + 3], sc[jt]);
      }
    } else {
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) {
        const float* krow = Kw + (jt * 16 + c) * LD + g * DG;
#pragma unroll
        for (int s = 0; s < DG; ++s) sc[jt] = mfma16x4(krow[s], qf[s], sc[jt]);
      }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      float4 e4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (use_bias) e4 = *reinterpret_cast<const float4*>(Ew + jt * 16 + 4 * g);
      const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool valid = kc + jt * 16 + 4 * g + r < nk;
        sc[jt][r] = valid ? (sc[jt][r] + ev[r]) * kLog2e : -INFINITY;
        mx = fmaxf(mx, sc[jt][r]);
      }
    }
    // Lazy rescale: the base m2 only moves when the chunk maximum exceeds it by more than 8
    // (base 2), so most chunks skip the rescale (weights stay below 2^8; the first chunk sets
    // m2, which starts at -inf, and alpha is then 0)
    const float cmax = group_max(mx);
    const bool need = cmax > m2 + 8.f;
    if (__any(need)) {  // wave-uniform
      const float mnew = need ? cmax : m2;
      const float alpha = fast_exp2(m2 - mnew);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
      m2 = mnew;
    }
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[jt][r] = fast_exp2(sc[jt][r] - m2);
        lsum += sc[jt][r];
      }

    // O^T += V^T P^T over the chunk's keys.
    // Each key tile's V operands are read into registers before its products, so the
    // LDS latency is paid once per tile rather than once per pair of products.
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      float va[4][DT];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vrow = Vw + (jt * 16 + 4 * g + r) * LD;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int col = dt * 16 + c;
          va[r][dt] = (D % 16 == 0 || col < D) ? vrow[col] : 0.f;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = mfma16x4(va[r][dt], sc[jt][r], o[dt]);
    }
  }

  if constexpr (GATED) {
    // Gate waves (local heads < HG/2) leave sigmoid(out) of their 16 queries in LDS (over
    // the K chunk, free once every wave is past the key loop); the value wave of the same
    // query tile multiplies it into its own rows and writes y.
    constexpr int GLD = D + 4;
    float* const Gs = Ks;  // [HG/2][QB][GLD] floats, within the K chunk region
    static_assert((HG / 2) * QB * GLD <= Sh::kKvFloats, "gate rows must fit the K chunk region");
    __syncthreads();
    const float inv = active ? 1.f / group_sum(lsum) : 0.f;
    float* const grow = Gs + ((hl % (HG / 2)) * QB + qt * 16 + c) * GLD;
    if (hl < HG / 2 && active) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        if (D % 16 != 0 && d0 >= D) continue;
        float sg[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sg[r] = __builtin_amdgcn_rcpf(1.f + fast_exp2(-kLog2e * (o[dt][r] * inv)));
        *reinterpret_cast<float4*>(grow + d0) = make_float4(sg[0], sg[1], sg[2], sg[3]);
      }
    }
    __syncthreads();
    if (hl >= HG / 2 && active && qvalid) {
      float* const yrow = p.out + ((static_cast<int64_t>(b) * Nq + qrow) * (H / 2) + (h - H / 2)) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        if (D % 16 != 0 && d0 >= D) continue;
        const float4 sg = *reinterpret_cast<const float4*>(grow + d0);
        *reinterpret_cast<float4*>(yrow + d0) = make_float4(sg.x * (o[dt][0] * inv), sg.y * (o[dt][1] * inv),
                                                            sg.z * (o[dt][2] * inv), sg.w * (o[dt][3] * inv));
      }
    }
  } else if (active) {
    // The cross-lane reduction runs on the whole wave; only the stores are per lane.
    const float inv = 1.f / group_sum(lsum);
    if (qvalid) {
      float* const orow = p.out + ((static_cast<int64_t>(b) * Nq + qrow) * H + h) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d0 = dt * 16 + 4 * g;
        if (D % 16 != 0 && d0 >= D) continue;
        *reinterpret_cast<float4*>(orow + d0) =
            make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
      }
    }
  }
}

template <int D, int HG, int QT, bool GATED>
hipError_t launch_rect_t(const RectParams& p, hipStream_t stream) {
  using Sh = RectShape<D, HG, QT>;
  const int64_t nwg = static_cast<int64_t>(p.B) * ((p.Nq + Sh::QB - 1) / Sh::QB) * (p.H / HG);
  const size_t lds = Sh::lds_bytes(p.Nk, p.key_mask != nullptr);
  auto kern = rect_attention_fwd_kernel<D, HG, QT, GATED>;
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(nwg)), dim3(Sh::NT), lds, stream, p);
  return hipGetLastError();
}

template <int D, int HG, bool GATED>
hipError_t launch_rect_hg(const RectParams& p, hipStream_t stream) {
  // Four query tiles per workgroup share each staged K / V chunk; fall back to one tile
  // when that would leave CUs idle (fewer than 256 workgroups).
  const int64_t big = static_cast<int64_t>(p.B) * ((p.Nq + 63) / 64) * (p.H / HG);
  if (big >= 256) return launch_rect_t<D, HG, 4, GATED>(p, stream);
  return launch_rect_t<D, HG, 1, GATED>(p, stream);
}

template <int D>
hipError_t launch_rect_d(const RectParams& p, hipStream_t stream) {
  if (p.gated) {
    // head groups of HG/2 gate heads and their value heads: HG/2 must divide H/2
    if (p.H % 2 != 0) return hipErrorInvalidValue;
    if ((p.H / 2) % 2 == 0) return launch_rect_hg<D, 4, true>(p, stream);
    return launch_rect_hg<D, 2, true>(p, stream);
  }
  if (p.H % 4 == 0) return launch_rect_hg<D, 4, false>(p, stream);
  if (p.H % 2 == 0) return launch_rect_hg<D, 2, false>(p, stream);
  return launch_rect_hg<D, 1, false>(p, stream);
}

}  // namespace

hipError_t launch_rect_fwd(const RectParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 8:
      return launch_rect_d<8>(p, stream);
    case 16:
      return launch_rect_d<16>(p, stream);
    case 32:
      return launch_rect_d<32>(p, stream);
    case 64:
      return launch_rect_d<64>(p, stream);
    default:
      return hipErrorInvalidValue;
  }
}

size_t rect_fwd_lds_bytes(int D, int H, int Nk, bool masked, bool gated) {
  const int hg = gated ? ((H / 2) % 2 == 0 ? 4 : 2) : (H % 4 == 0 ? 4 : (H % 2 == 0 ? 2 : 1));
  // The largest variant (four query tiles) bounds the requirement.
  switch (D * 8 + hg) {
#define HZ_RECT_CASE(d, g) \
  case d * 8 + g:          \
    return RectShape<d, g, 4>::lds_bytes(Nk, masked);
    HZ_RECT_CASE(8, 1) HZ_RECT_CASE(8, 2) HZ_RECT_CASE(8, 4)
    HZ_RECT_CASE(16, 1) HZ_RECT_CASE(16, 2) HZ_RECT_CASE(16, 4)
    HZ_RECT_CASE(32, 1) HZ_RECT_CASE(32, 2) HZ_RECT_CASE(32, 4)
    HZ_RECT_CASE(64, 1) HZ_RECT_CASE(64, 2) HZ_RECT_CASE(64, 4)
#undef HZ_RECT_CASE
    default:
      return 0;
  }
}

}  // namespace hz
