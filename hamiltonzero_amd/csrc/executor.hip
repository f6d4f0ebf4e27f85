// The compiled per-walker executor's products on the float32 matrix cores
// (v_mfma_f32_16x16x4_f32): the quadrilinear merge of the tree levels and the factorized
// apply ((x V) o h) U of the leaf, merge and readout factors.
//
// Quadrilinear merge, out[m, iR + j] = sum_{k,l} T[i, j, k, l] a[m, iR + k] b[m, iR + l]:
// for one group i it is one GEMM with a contraction of length R^2 = 1024,
//     out_i[m, j] = sum_kl P_i[m, kl] T_i[kl, j],     P_i[m, kl] = a[m, iR + k] b[m, iR + l],
// whose left operand P_i is never materialised: a lane holds its row's 32 values of a and 8
// values of b and forms each operand value with one multiply right before its product.
// A workgroup owns one group i, one half of the 32 outputs j and 256 rows; T_i's half
// (1024 x 16 floats, 64 KiB) is staged in LDS once and read by every product step (one
// 4-byte read feeds the four 16-row tiles of a wave). Two workgroups per compute unit.
//
// Factorized apply: two launches of one tiled GEMM, C = A B with A [M, K], B [K, N]
// row-major; the first multiplies its result by the conditioner row of each output row
// (h[m mod h_rows], one row per tree node, broadcast over walkers) before storing, the
// second optionally adds a residual (the merge level's raw + apply(raw)). 128 x 128 output
// tiles per 256-thread workgroup, 16-deep K slices double-buffered through LDS.
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "mhsea_device.h"
#include "mhsea_launch.h"

// Workspace of hz_factorized_apply_noalloc: kApplyScratchFloats floats (32 MiB) per device,
// held from the library's first use on that device until the process ends. Every call on a
// device shares that device's array, so calls that overlap on one device race.
static __device__ __align__(256) float scratch[hz::kApplyScratchFloats];

namespace hz {
namespace {

// --------------------------------------------------------------------------------------
// Quadrilinear merge (R = 32)
// --------------------------------------------------------------------------------------
constexpr int kQR = 32;            // rank of the merge tensor
constexpr int kQRows = 256;        // rows per workgroup (4 waves x 4 tiles of 16)
constexpr int kQHalf = 16;         // outputs j per workgroup
constexpr int kQKL = kQR * kQR;    // contraction length

__global__ void __launch_bounds__(256, 2)
quadrilinear_merge_kernel(const float* __restrict__ T, const float* __restrict__ ua, const float* __restrict__ ub,
                          float* __restrict__ out, int64_t M, int G, int64_t ld_in) {
  __shared__ float Ts[kQKL * kQHalf];  // Ts[kl][jj] = T[i][16 jh + jj][k][l], kl = 32 k + l
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int i = blockIdx.y;
  const int jh = blockIdx.z;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kQRows + wave * 64;
  const int64_t ld = static_cast<int64_t>(G) * kQR;  // floats per row of out (ld_in: of a and b)

  // stage T_i's half: thread t takes output jj = t mod 16 and 4 consecutive kl per pass
  const float* Ti = T + (static_cast<int64_t>(i) * kQR + kQHalf * jh) * kQKL;
  for (int base = 0; base < kQKL * kQHalf / 4; base += 256) {
    const int it = base + tid;
    const int jj = it & 15, kl4 = it >> 4;
    const float4 v = *reinterpret_cast<const float4*>(Ti + static_cast<int64_t>(jj) * kQKL + 4 * kl4);
    Ts[(4 * kl4 + 0) * kQHalf + jj] = v.x;
    Ts[(4 * kl4 + 1) * kQHalf + jj] = v.y;
    Ts[(4 * kl4 + 2) * kQHalf + jj] = v.z;
    Ts[(4 * kl4 + 3) * kQHalf + jj] = v.w;
  }

  // this lane's rows (one per 16-row tile): all 32 values of a, and b at l = 4 m + g
  float a[4][kQR], b[4][8];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int64_t row = row0 + 16 * rt + c;
    const bool ok = row < M;
    const float* ar = ua + (ok ? row : 0) * ld_in + i * kQR;
    const float* br = ub + (ok ? row : 0) * ld_in + i * kQR;
#pragma unroll
    for (int q = 0; q < kQR / 4; ++q) {
      const float4 v = ok ? *reinterpret_cast<const float4*>(ar + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
      a[rt][4 * q] = v.x;
      a[rt][4 * q + 1] = v.y;
      a[rt][4 * q + 2] = v.z;
      a[rt][4 * q + 3] = v.w;
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) b[rt][m] = ok ? br[4 * m + g] : 0.f;
  }
  __syncthreads();

  // step t contracts kl = 4 t + g, i.e. k = t / 8, l = 4 (t mod 8) + g
  v4f acc[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) acc[rt] = zero4();
#pragma unroll
  for (int k = 0; k < kQR; ++k) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float tb = Ts[(32 * k + 4 * m + g) * kQHalf + c];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) acc[rt] = mfma16x4(a[rt][k] * b[rt][m], tb, acc[rt]);
    }
  }

  // lane (g, c) holds out[row0 + 16 rt + 4 g + r][i R + 16 jh + c]
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = row0 + 16 * rt + 4 * g + r;
      if (row < M) out[row * ld + i * kQR + kQHalf * jh + c] = acc[rt][r];
    }
}

// --------------------------------------------------------------------------------------
// Tiled GEMM with epilogues
// --------------------------------------------------------------------------------------
constexpr int kBM = 128, kBN = 128, kBK = 16;
// Row lengths of As[k][row] and Bs[k][col] (floats): 16 more than a tile, so the four k rows
// of one operand read (lanes 16 g + c read row g, column c) fall on distinct banks. A's
// transposed stores put column r of k rows 4q .. 4q + 3 at r ^ 16 q, so the four lanes that
// share r (q = 0..3, rows 4 x 144 floats apart, one bank) write four banks; a read's four
// rows share q, so it still covers one aligned 16-column block per row.
constexpr int kAPad = kBM + 16;
constexpr int kBPad = kBN + 16;

enum GemmEpi { kEpiPlain = 0, kEpiCond = 1, kEpiResidual = 2, kEpiRowMask = 3 };

// C[M, N] = A[M, K] B[K, N] (row-major); EPI: kEpiCond multiplies C[m, n] by
// h[((row0 + m) mod h_rows) * N + n] (row0: the first row's index in the caller's full
// row range, nonzero when the rows are processed in chunks); kEpiResidual adds res[m, n];
// kEpiRowMask multiplies row m by (mask[m] != 0), aux then being a uint8 mask.
// C may be the residual itself (each output entry reads its residual entry, then overwrites
// it, in one thread), so neither carries __restrict__. VEC: K and N are multiples of 4
// (16-byte staging loads); otherwise the staging loads are per element.
// Split K (gridDim.z > 1): workgroup z contracts k in [z K, min(z K + K, Ktot)) of A (row
// stride lda) and B and writes its partial product (EPI plain) at C + z cz.
template <int EPI, bool VEC>
__global__ void __launch_bounds__(256, 2)
gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ Bm, float* C, const float* aux, int64_t M, int N,
                int K, int h_rows, int64_t row0, int lda, int Ktot, int64_t cz) {
  {
    const int kbeg = static_cast<int>(blockIdx.z) * K;
    A += kbeg;
    Bm += static_cast<int64_t>(kbeg) * N;
    C += static_cast<int64_t>(blockIdx.z) * cz;
    K = Ktot - kbeg < K ? Ktot - kbeg : K;
  }
  __shared__ float As[2][kBK][kAPad];
  __shared__ float Bs[2][kBK][kBPad];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kBM;
  const int n0 = blockIdx.x * kBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // this wave's 64 x 64 sub-tile

  // global -> register staging: A tile 128 x 16 as 512 float4 (row = it / 4, k4 = it % 4),
  // B tile 16 x 128 as 512 float4 (k = it / 32, n4 = it % 32); two of each per thread
  float4 ra[2], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int it = tid + 256 * u;
      const int64_t row = m0 + (it >> 2);
      const int kk = k0 + 4 * (it & 3);
      if constexpr (VEC) {
        ra[u] = (row < M && kk < K) ? *reinterpret_cast<const float4*>(A + row * lda + kk)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float* ar = A + (row < M ? row : 0) * lda;
        ra[u].x = (row < M && kk < K) ? ar[kk] : 0.f;
        ra[u].y = (row < M && kk + 1 < K) ? ar[kk + 1] : 0.f;
        ra[u].z = (row < M && kk + 2 < K) ? ar[kk + 2] : 0.f;
        ra[u].w = (row < M && kk + 3 < K) ? ar[kk + 3] : 0.f;
      }
      const int kb = k0 + (it >> 5);
      const int nn = n0 + 4 * (it & 31);
      if constexpr (VEC) {
        rb[u] = (kb < K && nn < N) ? *reinterpret_cast<const float4*>(Bm + static_cast<int64_t>(kb) * N + nn)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const float* br = Bm + static_cast<int64_t>(kb < K ? kb : 0) * N;
        rb[u].x = (kb < K && nn < N) ? br[nn] : 0.f;
        rb[u].y = (kb < K && nn + 1 < N) ? br[nn + 1] : 0.f;
        rb[u].z = (kb < K && nn + 2 < N) ? br[nn + 2] : 0.f;
        rb[u].w = (kb < K && nn + 3 < N) ? br[nn + 3] : 0.f;
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int it = tid + 256 * u;
      const int r = it >> 2, k4 = 4 * (it & 3);
      // column r of rows k4 .. k4 + 3 at r ^ 16 ((k4 / 4) mod 4): the four lanes sharing r
      // (k4 = 0, 4, 8, 12) land in four banks instead of one
      const int rs = r ^ (16 * ((k4 >> 2) & 3));
      As[buf][k4 + 0][rs] = ra[u].x;
      As[buf][k4 + 1][rs] = ra[u].y;
      As[buf][k4 + 2][rs] = ra[u].z;
      As[buf][k4 + 3][rs] = ra[u].w;
      *reinterpret_cast<float4*>(&Bs[buf][it >> 5][4 * (it & 31)]) = rb[u];
    }
  };

  v4f acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = zero4();

  const int nk = (K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 4) {
      float af[4], bf[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) af[mt] = As[buf][ks + g][(wm + 16 * mt + c) ^ (16 * ((ks >> 2) & 3))];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) bf[nt] = Bs[buf][ks + g][wn + 16 * nt + c];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma16x4(af[mt], bf[nt], acc[mt][nt]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // lane (g, c) holds C[wm + 16 mt + 4 g + r][wn + 16 nt + c]
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = m0 + wm + 16 * mt + 4 * g + r;
      if (row >= M) continue;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const int col = n0 + wn + 16 * nt + c;
        if (col >= N) continue;
        float v = acc[mt][nt][r];
        if constexpr (EPI == kEpiCond) v *= aux[((row0 + row) % h_rows) * N + col];
        if constexpr (EPI == kEpiResidual) v += aux[row * N + col];
        if constexpr (EPI == kEpiRowMask) v *= reinterpret_cast<const uint8_t*>(aux)[row] != 0 ? 1.f : 0.f;
        C[row * N + col] = v;
      }
    }
}

// Site-masked product C[m, :] = mask[m] != 0 ? A[m, :] B : 0 with the masked rows skipped.
// A workgroup takes kRM rows of A and one 128-column tile of C: its physical rows (in order)
// are compacted into the LDS tile, so only ceil(n / 16) row blocks are multiplied, and its
// masked rows of C are written as zeros. Wave w owns columns [32 w, 32 w + 32) of the tile for
// every row block. Workgroups are numbered so that the column tiles of one row block run on
// one XCD (one L2 holds their A rows). K and N are multiples of 4 (16-byte staging loads).
constexpr int kRM = 256;  // 16 row blocks: the dispatch below instantiates 1..16
constexpr int kRMPad = kRM + 16;

__global__ void __launch_bounds__(256, 2)
gemm_rows_f32_kernel(const float* __restrict__ A, const float* __restrict__ Bm, float* __restrict__ C,
                     const uint8_t* __restrict__ mask, int64_t M, int N, int K, int ncol) {
  __shared__ float As[2][kBK][kRMPad];
  __shared__ float Bs[2][kBK][kBPad];
  __shared__ int16_t prow[kRM], mrow[kRM];
  __shared__ int counts[8];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int64_t L = xcd_logical_block(blockIdx.x, gridDim.x);
  const int64_t m0 = (L / ncol) * kRM;
  const int n0 = static_cast<int>(L % ncol) * kBN;
  const int wn = wave * 32;

  // ---- this workgroup's physical and masked rows, each list in ascending order ---------
  const bool valid = m0 + tid < M;
  const bool phys = valid && mask[m0 + tid] != 0;
  const uint64_t pb = __ballot(phys), mb = __ballot(valid && !phys);
  const uint64_t below = (uint64_t(1) << lane) - 1;
  if (lane == 0) {
    counts[wave] = __popcll(pb);
    counts[4 + wave] = __popcll(mb);
  }
  __syncthreads();
  int pbase = 0, mbase = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    pbase += w < wave ? counts[w] : 0;
    mbase += w < wave ? counts[4 + w] : 0;
  }
  const int n = counts[0] + counts[1] + counts[2] + counts[3];
  const int nm = counts[4] + counts[5] + counts[6] + counts[7];
  if (phys) prow[pbase + __popcll(pb & below)] = static_cast<int16_t>(tid);
  if (valid && !phys) mrow[mbase + __popcll(mb & below)] = static_cast<int16_t>(tid);
  __syncthreads();

  // masked rows: the workgroup of column tile t writes the whole rows (every column) of the
  // masked rows i = t, t + ncol, ... of its row block, each row one contiguous run
  {
    const int t = static_cast<int>(L % ncol);
    const int nmine = nm > t ? (nm - t + ncol - 1) / ncol : 0;
    const int n4 = N / 4;
    for (int i = tid; i < nmine * n4; i += 256) {
      const int mi = t + (i / n4) * ncol;
      *reinterpret_cast<float4*>(C + (m0 + mrow[mi]) * N + 4 * (i % n4)) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  if (n == 0) return;  // workgroup-uniform

  // global -> register staging: A slots 256 x 16 as 1024 float4 (slot = it / 4, k4 = it % 4;
  // slots past n stay zero; each slot's row offset is fixed for the whole K loop), B tile
  // 16 x 128 as 512 float4 (k = it / 32, n4 = it % 32)
  int64_t aoff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int slot = (tid + 256 * u) >> 2;
    aoff[u] = slot < n ? (m0 + prow[slot]) * K : -1;
  }
  float4 ra[4], rb[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int kk = k0 + 4 * ((tid + 256 * u) & 3);
      ra[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (aoff[u] >= 0 && kk < K) ra[u] = *reinterpret_cast<const float4*>(A + aoff[u] + kk);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int it = tid + 256 * u;
      const int kb = k0 + (it >> 5);
      const int nn = n0 + 4 * (it & 31);
      rb[u] = (kb < K && nn < N) ? *reinterpret_cast<const float4*>(Bm + static_cast<int64_t>(kb) * N + nn)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int it = tid + 256 * u;
      const int r = it >> 2, k4 = 4 * (it & 3);
      const int rs = r ^ (16 * ((k4 >> 2) & 3));  // as in gemm_f32_kernel
      As[buf][k4 + 0][rs] = ra[u].x;
      As[buf][k4 + 1][rs] = ra[u].y;
      As[buf][k4 + 2][rs] = ra[u].z;
      As[buf][k4 + 3][rs] = ra[u].w;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int it = tid + 256 * u;
      *reinterpret_cast<float4*>(&Bs[buf][it >> 5][4 * (it & 31)]) = rb[u];
    }
  };

  // the K loop and the stores for NMT = ceil(n / 16) row blocks, a compile-time count so
  // the products run without branches
  auto body = [&](auto nmt_c) {
    constexpr int NMT = decltype(nmt_c)::value;
    v4f acc[NMT][2];
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) acc[mt][0] = acc[mt][1] = zero4();
    const int nk = (K + kBK - 1) / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
      for (int ks = 0; ks < kBK; ks += 4) {
        const float b0 = Bs[buf][ks + g][wn + c];
        const float b1 = Bs[buf][ks + g][wn + 16 + c];
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) {
          const float af = As[buf][ks + g][(16 * mt + c) ^ (16 * ((ks >> 2) & 3))];
          acc[mt][0] = mfma16x4(af, b0, acc[mt][0]);
          acc[mt][1] = mfma16x4(af, b1, acc[mt][1]);
        }
      }
      if (kt + 1 < nk) sstore(buf ^ 1);
      __syncthreads();
    }
    // lane (g, c) holds C[prow[16 mt + 4 g + r]][n0 + wn + 16 nt + c]
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int slot = 16 * mt + 4 * g + r;
        const int64_t row = m0 + prow[slot < n ? slot : 0];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int col = n0 + wn + 16 * nt + c;
          if (slot < n && col < N) C[row * N + col] = acc[mt][nt][r];
        }
      }
  };
  using std::integral_constant;
  switch ((n + 15) >> 4) {
    case 1: body(integral_constant<int, 1>{}); break;
    case 2: body(integral_constant<int, 2>{}); break;
    case 3: body(integral_constant<int, 3>{}); break;
    case 4: body(integral_constant<int, 4>{}); break;
    case 5: body(integral_constant<int, 5>{}); break;
    case 6: body(integral_constant<int, 6>{}); break;
    case 7: body(integral_constant<int, 7>{}); break;
    case 8: body(integral_constant<int, 8>{}); break;
    case 9: body(integral_constant<int, 9>{}); break;
    case 10: body(integral_constant<int, 10>{}); break;
    case 11: body(integral_constant<int, 11>{}); break;
    case 12: body(integral_constant<int, 12>{}); break;
    case 13: body(integral_constant<int, 13>{}); break;
    case 14: body(integral_constant<int, 14>{}); break;
    case 15: body(integral_constant<int, 15>{}); break;
    default: body(integral_constant<int, 16>{}); break;
  }
}

// Sum of the split-K partial products P[z] (z in order) with the GEMM's epilogue; N % 4 == 0.
// C may be the residual (aux): each element reads it, then overwrites it, in one thread.
template <int EPI>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ P, float* C, const float* aux,
                                                            int64_t M, int N, int S, int64_t cz, int h_rows,
                                                            int64_t row0) {
  const int64_t i4 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i4 >= M * N / 4) return;
  float4 v = *reinterpret_cast<const float4*>(P + 4 * i4);
  for (int z = 1; z < S; ++z) {
    const float4 w = *reinterpret_cast<const float4*>(P + z * cz + 4 * i4);
    v.x += w.x;
    v.y += w.y;
    v.z += w.z;
    v.w += w.w;
  }
  const int64_t row = 4 * i4 / N;
  const int col = static_cast<int>(4 * i4 - row * N);
  if constexpr (EPI == kEpiCond) {
    const float4 hv = *reinterpret_cast<const float4*>(aux + ((row0 + row) % h_rows) * N + col);
    v.x *= hv.x;
    v.y *= hv.y;
    v.z *= hv.z;
    v.w *= hv.w;
  }
  if constexpr (EPI == kEpiResidual) {
    const float4 rv = *reinterpret_cast<const float4*>(aux + row * N + col);
    v.x += rv.x;
    v.y += rv.y;
    v.z += rv.z;
    v.w += rv.w;
  }
  if constexpr (EPI == kEpiRowMask) {
    const float mk = reinterpret_cast<const uint8_t*>(aux)[row] != 0 ? 1.f : 0.f;
    v.x *= mk;
    v.y *= mk;
    v.z *= mk;
    v.w *= mk;
  }
  *reinterpret_cast<float4*>(C + 4 * i4) = v;
}

template <int EPI>
hipError_t launch_gemm(const float* A, const float* B, float* C, const float* aux, int64_t M, int N, int K,
                       int h_rows, int64_t row0, hipStream_t stream, float* split_ws = nullptr,
                       int64_t split_cap = 0) {
  const dim3 grid(static_cast<unsigned>((N + kBN - 1) / kBN), static_cast<unsigned>((M + kBM - 1) / kBM));
  // Split K where the tiles leave most CUs idle (the tree's deep levels: 1024-4096 rows,
  // 64-512 tiles of 96-step K chains): S parts of K into split_ws [S, M, N], then one pass
  // that sums the parts in order and applies the epilogue (deterministic).
  if (split_ws != nullptr && N % 4 == 0 && K % 4 == 0 && K >= 256) {
    int cus = 0;
    if (hipError_t err = device_cu_count(&cus); err != hipSuccess) return err;
    const int64_t tiles = static_cast<int64_t>(grid.x) * grid.y;
    const int64_t mn = M * N;
    int64_t S = tiles < cus ? (2 * cus + tiles - 1) / tiles : 1;
    S = S > 8 ? 8 : S;
    S = S > K / 128 ? K / 128 : S;
    S = S > split_cap / mn ? split_cap / mn : S;
    if (S >= 2) {
      const int kp = static_cast<int>(((K + S - 1) / S + kBK - 1) / kBK * kBK);
      const int parts = (K + kp - 1) / kp;
      const dim3 gs(grid.x, grid.y, static_cast<unsigned>(parts));
      hipLaunchKernelGGL((gemm_f32_kernel<kEpiPlain, true>), gs, dim3(256), 0, stream, A, B, split_ws, nullptr, M, N,
                         kp, 1, int64_t(0), K, K, mn);
      if (hipError_t err = hipGetLastError(); err != hipSuccess) return err;
      const int64_t n4 = mn / 4;
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI>), dim3(static_cast<unsigned>((n4 + 255) / 256)), dim3(256), 0,
                         stream, split_ws, C, aux, M, N, parts, mn, h_rows, row0);
      return hipGetLastError();
    }
  }
  if (N % 4 == 0 && K % 4 == 0)
    hipLaunchKernelGGL((gemm_f32_kernel<EPI, true>), grid, dim3(256), 0, stream, A, B, C, aux, M, N, K, h_rows, row0,
                       K, K, int64_t(0));
  else
    hipLaunchKernelGGL((gemm_f32_kernel<EPI, false>), grid, dim3(256), 0, stream, A, B, C, aux, M, N, K, h_rows,
                       row0, K, K, int64_t(0));
  return hipGetLastError();
}

// One factorized apply over rows [row0, row0 + M) of the caller's range: x, residual and y
// point at row row0; work holds M x R floats; split_ws (split_cap floats, may be null) is free
// scratch for split-K partial products.
hipError_t apply_rows(const float* x, const float* V, const float* h, const float* U, const float* residual,
                      float* y, float* work, int64_t M, int d_in, int R, int d_out, int h_rows, int64_t row0,
                      hipStream_t stream, float* split_ws = nullptr, int64_t split_cap = 0) {
  hipError_t err = launch_gemm<kEpiCond>(x, V, work, h, M, R, d_in, h_rows, row0, stream, split_ws, split_cap);
  if (err != hipSuccess) return err;
  if (residual != nullptr)
    return launch_gemm<kEpiResidual>(work, U, y, residual, M, d_out, R, 1, 0, stream, split_ws, split_cap);
  return launch_gemm<kEpiPlain>(work, U, y, nullptr, M, d_out, R, 1, 0, stream, split_ws, split_cap);
}

// Device addresses of the no-alloc workspace, one per device, resolved on first use.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// --------------------------------------------------------------------------------------
// Row epilogues of the executor, one wave per row of d floats (d a multiple of 4,
// d <= 64 * 4 * kRowVec): the leaf carriers' RMS normalisation, a level's rescale and
// opcode gate, and the readout's log|psi| and phase. Each row's sum of squares is reduced
// across the wave in a fixed order (results reproducible run to run).
// --------------------------------------------------------------------------------------
constexpr int kRowVec = 8;  // float4 per lane: rows up to 2048 floats

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float sum_sq(const float4& v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }

// u[m, :] /= rms, s[m] = log(rms), rms = sqrt(mean(u[m]^2) + 1e-30)
__global__ void __launch_bounds__(256) normalize_rows_kernel(float* __restrict__ u, float* __restrict__ s, int64_t M,
                                                              int d) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  float4* ur = reinterpret_cast<float4*>(u + row * d);
  const int d4 = d / 4;
  float4 v[kRowVec];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < kRowVec; ++t) {
    const int c4 = lane + 64 * t;
    v[t] = c4 < d4 ? ur[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    ss += sum_sq(v[t]);
  }
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / static_cast<float>(d) + 1e-30f);
#pragma unroll
  for (int t = 0; t < kRowVec; ++t) {
    const int c4 = lane + 64 * t;
    if (c4 < d4) ur[c4] = make_float4(v[t].x / rms, v[t].y / rms, v[t].z / rms, v[t].w / rms);
  }
  if (lane == 0) s[row] = logf(rms);
}

// One tree level's epilogue for output row m = (walker, node p), M = walkers x width:
//   scale = sqrt(mean(out[m]^2) + eps), candidate = out[m] / scale,
//   u'[m] = both * candidate + left * u[2m] + right * u[2m + 1]   (gates from opcode[p])
//   s'[m] = both * (s[2m] + s[2m + 1] + log(scale)) + left * s[2m] + right * s[2m + 1]
__global__ void __launch_bounds__(256) level_gate_kernel(const float* __restrict__ out, const float* __restrict__ u_in,
                                                          const float* __restrict__ s_in,
                                                          const uint8_t* __restrict__ opcodes, float* __restrict__ u_out,
                                                          float* __restrict__ s_out, int64_t M, int width, int d,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int d4 = d / 4;
  const float4* orow = reinterpret_cast<const float4*>(out + row * d);
  const float4* lrow = reinterpret_cast<const float4*>(u_in + 2 * row * d);
  const float4* rrow = lrow + d4;
  float4 v[kRowVec];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < kRowVec; ++t) {
    const int c4 = lane + 64 * t;
    v[t] = c4 < d4 ? orow[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    ss += sum_sq(v[t]);
  }
  ss = wave_sum(ss);
  const float scale = sqrtf(ss / static_cast<float>(d) + eps);
  const int op = opcodes[row % width];
  const float both = op == 0 ? 1.f : 0.f, left = op == 1 ? 1.f : 0.f, right = op == 2 ? 1.f : 0.f;
  float4* urow = reinterpret_cast<float4*>(u_out + row * d);
#pragma unroll
  for (int t = 0; t < kRowVec; ++t) {
    const int c4 = lane + 64 * t;
    if (c4 < d4) {
      const float4 a = lrow[c4], b = rrow[c4];
      float4 r;
      r.x = both * (v[t].x / scale) + left * a.x + right * b.x;
      r.y = both * (v[t].y / scale) + left * a.y + right * b.y;
      r.z = both * (v[t].z / scale) + left * a.z + right * b.z;
      r.w = both * (v[t].w / scale) + left * a.w + right * b.w;
      urow[c4] = r;
    }
  }
  if (lane == 0) {
    const float sl = s_in[2 * row], sr = s_in[2 * row + 1];
    s_out[row] = both * (sl + sr + logf(scale)) + left * sl + right * sr;
  }
}

// log|psi| = 0.5 log(re^2 + im^2) + s_root, phase = atan2(im, re); psi [B, 2]
__global__ void __launch_bounds__(256) readout_kernel(const float* __restrict__ psi, const float* __restrict__ s_root,
                                                       float* __restrict__ log_abs, float* __restrict__ phase, int64_t B) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b >= B) return;
  const float re = psi[2 * b], im = psi[2 * b + 1];
  log_abs[b] = 0.5f * logf(re * re + im * im) + s_root[b];
  phase[b] = atan2f(im, re);
}

// Workspace sections of the whole-wavefunction executor, in floats, each rounded up to 64
// floats (256 bytes).
struct WaveFnWorkspace {
  int64_t z, work, u0, u1, raw, s0, s1, psi, total;
  WaveFnWorkspace(int64_t B, int64_t n, int64_t d_z, int64_t r_leaf, int64_t d_m, int64_t r_merge, int64_t r_out) {
    auto up = [](int64_t x) { return (x + 63) / 64 * 64; };
    const int64_t half = n > 1 ? n / 2 : 1;
    int64_t wk = B * n * r_leaf;
    if (B * half * r_merge > wk) wk = B * half * r_merge;
    if (B * r_out > wk) wk = B * r_out;
    z = 0;
    work = z + up(B * n * d_z);
    u0 = work + up(wk);
    u1 = u0 + up(B * n * d_m);
    raw = u1 + up(B * half * d_m);
    s0 = raw + up(B * half * d_m);
    s1 = s0 + up(B * n);
    psi = s1 + up(B * half);
    total = psi + up(2 * B);
  }
};

}  // namespace

int64_t compiled_wavefunction_workspace_bytes(int64_t B, int64_t n, int64_t d_z, int64_t r_leaf, int64_t d_m,
                                              int64_t r_merge, int64_t r_out) {
  return WaveFnWorkspace(B, n, d_z, r_leaf, d_m, r_merge, r_out).total * static_cast<int64_t>(sizeof(float));
}

hipError_t launch_compiled_wavefunction(const WaveFnParams& p, hipStream_t stream) {
  const WaveFnWorkspace L(p.B, p.n, p.d_z, p.r_leaf, p.d_m, p.r_merge, p.r_out);
  float* ws = p.workspace;
  float *z = ws + L.z, *work = ws + L.work, *raw = ws + L.raw, *psi = ws + L.psi;
  float* u_buf[2] = {ws + L.u0, ws + L.u1};
  float* s_buf[2] = {ws + L.s0, ws + L.s1};
  // the carrier buffer a step does not use holds its split-K partial products
  const int64_t u_cap[2] = {L.u1 - L.u0, L.raw - L.u1};
  const int64_t rows = p.B * p.n;
  const int G = p.d_m / kQR;
  hipError_t err;
  // leaf: z = q W_q; u = ((z V) o leaf_h[site]) U; carriers RMS-normalised, s = log rms
  if ((err = launch_gemm<kEpiPlain>(p.q, p.q_weight, z, nullptr, rows, p.d_z, p.d_q, 1, 0, stream)) != hipSuccess)
    return err;
  if ((err = apply_rows(z, p.leaf_V, p.leaf_h, p.leaf_U, nullptr, u_buf[0], work, rows, p.d_z, p.r_leaf, p.d_m, p.n, 0,
                        stream, u_buf[1], u_cap[1])) != hipSuccess)
    return err;
  hipLaunchKernelGGL(normalize_rows_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, stream,
                     u_buf[0], s_buf[0], rows, p.d_m);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // levels: node pairs (2p, 2p + 1) merged into node p, widths n/2, n/4, ..., 1
  int cur = 0;
  for (int level = 0, width = p.n / 2; width >= 1; ++level, width /= 2) {
    const int64_t m = p.B * width;
    const float* u_in = u_buf[cur];
    const float* h_level = p.merge_h + static_cast<int64_t>(level) * (p.n / 2) * p.r_merge;
    const uint8_t* ops = p.opcodes + static_cast<int64_t>(level) * (p.n / 2);
    if ((err = launch_quadrilinear_merge(p.merge_T, u_in, u_in + p.d_m, raw, m, G, 2 * static_cast<int64_t>(p.d_m),
                                         stream)) != hipSuccess)
      return err;
    // out = raw + ((raw V) o h_level[node]) U, written over raw
    if ((err = apply_rows(raw, p.merge_V, h_level, p.merge_U, raw, raw, work, m, p.d_m, p.r_merge, p.d_m, width, 0,
                          stream, u_buf[cur ^ 1], u_cap[cur ^ 1])) != hipSuccess)
      return err;
    hipLaunchKernelGGL(level_gate_kernel, dim3(static_cast<unsigned>((m + 3) / 4)), dim3(256), 0, stream, raw, u_in,
                       s_buf[cur], ops, u_buf[cur ^ 1], s_buf[cur ^ 1], m, width, p.d_m, p.merge_eps);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    cur ^= 1;
  }
  // readout: psi = ((u_root V) o readout_h) U, then log|psi| and phase
  if ((err = apply_rows(u_buf[cur], p.readout_V, p.readout_h, p.readout_U, nullptr, psi, work, p.B, p.d_m, p.r_out, 2,
                        1, 0, stream, u_buf[cur ^ 1], u_cap[cur ^ 1])) != hipSuccess)
    return err;
  hipLaunchKernelGGL(readout_kernel, dim3(static_cast<unsigned>((p.B + 255) / 256)), dim3(256), 0, stream, psi,
                     s_buf[cur], p.log_abs, p.phase, p.B);
  return hipGetLastError();
}

hipError_t launch_quadrilinear_merge(const float* T, const float* ua, const float* ub, float* out, int64_t M, int G,
                                     int64_t ld_in, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((M + kQRows - 1) / kQRows), static_cast<unsigned>(G), 2);
  hipLaunchKernelGGL(quadrilinear_merge_kernel, grid, dim3(256), 0, stream, T, ua, ub, out, M, G, ld_in);
  return hipGetLastError();
}

hipError_t launch_factorized_apply(const float* x, const float* V, const float* h, const float* U,
                                   const float* residual, float* y, float* work, int64_t M, int d_in, int R, int d_out,
                                   int h_rows, hipStream_t stream) {
  return apply_rows(x, V, h, U, residual, y, work, M, d_in, R, d_out, h_rows, 0, stream);
}

hipError_t launch_out_proj(const float* y, const float* w_o, const uint8_t* mask, float* delta, int64_t M, int d_in,
                           int d_out, hipStream_t stream) {
  // The row-compacting kernel where its 256-row workgroups fill the chip; below that (few
  // rows, e.g. one large-N system's 4096 query rows: 64 workgroups for 256 CUs) the 128 x 128
  // tiled GEMM with the row mask in its epilogue runs twice the workgroups and multiplies the
  // masked rows too (the large-N tail's W_O on 4096 rows: about 93 -> 53 us).
  int cus = 0;
  if (hipError_t err = device_cu_count(&cus); err != hipSuccess) return err;
  const int64_t ncol = (d_out + kBN - 1) / kBN;
  const int64_t blocks = ncol * ((M + kRM - 1) / kRM);
  if (mask != nullptr && d_out % 4 == 0 && d_in % 4 == 0 && blocks >= cus) {
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_rows_f32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, y, w_o, delta,
                       mask, M, d_out, d_in, static_cast<int>(ncol));
    return hipGetLastError();
  }
  if (mask != nullptr)
    return launch_gemm<kEpiRowMask>(y, w_o, delta, reinterpret_cast<const float*>(mask), M, d_out, d_in, 1, 0, stream);
  return launch_gemm<kEpiPlain>(y, w_o, delta, nullptr, M, d_out, d_in, 1, 0, stream);
}

static hipError_t apply_scratch_address(int device, float** ptr) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    int current = -1;
    hipError_t err = hipGetDevice(&current);
    if (err != hipSuccess) return err;
    if (current != device && (err = hipSetDevice(device)) != hipSuccess) return err;
    // `scratch` names the array only inside kernels; host code uses this device's address.
    void* addr = nullptr;
    err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (current != device) {
      const hipError_t restore = hipSetDevice(current);
      if (err == hipSuccess) err = restore;
    }
    if (err != hipSuccess) return err;
    if (addr == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = static_cast<float*>(addr);
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

hipError_t launch_factorized_apply_noalloc(const float* x, const float* V, const float* h, const float* U,
                                           const float* residual, float* y, int64_t M, int d_in, int R, int d_out,
                                           int h_rows, hipStream_t stream) {
  if (R > kApplyScratchMaxRank) return hipErrorInvalidValue;
  int device = -1;
  hipError_t err = hipStreamGetDevice(stream, &device);
  if (err != hipSuccess) return err;
  float* work = nullptr;
  if ((err = apply_scratch_address(device, &work)) != hipSuccess) return err;
  // Whole 128-row tiles of R floats per chunk; every workspace entry a chunk's second GEMM
  // reads is written by its first, so the array needs no clearing between calls.
  const int64_t chunk = kApplyScratchFloats / R / kBM * kBM;
  for (int64_t r0 = 0; r0 < M; r0 += chunk) {
    const int64_t rows = M - r0 < chunk ? M - r0 : chunk;
    err = apply_rows(x + r0 * d_in, V, h, U, residual == nullptr ? nullptr : residual + r0 * d_out, y + r0 * d_out,
                     work, rows, d_in, R, d_out, h_rows, r0, stream);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace hz
