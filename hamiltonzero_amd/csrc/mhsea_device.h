// Device-side helpers shared by the MHSEA kernels (gfx950 / CDNA4, wave64).
//
// Matrix-core convention used throughout (v_mfma_f32_16x16x4_f32, one 16x16 block):
//   lane l = 16*g + c   (g = l / 16 in 0..3, c = l % 16)
//   A operand (16 x 4):  lane supplies A[row = c][k = g]
//   B operand (4 x 16):  lane supplies B[k = g][col = c]
//   C/D       (16 x 16): lane holds    C[row = 4*g + r][col = c], r = 0..3 (a v4f)
// The contraction index k may be any permutation of the summed dimension as long as the
// A and B operands of one instruction agree, which the kernels use to keep every lane's
// operands contiguous in memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hz {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Score of an invalid (query, key) pair under the square mask (utils.py:51-52).
constexpr float kMaskScore = -10000.0f;

__device__ __forceinline__ v4f mfma16x4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4f zero4() { return v4f{0.f, 0.f, 0.f, 0.f}; }

// 2^x with the hardware transcendental (v_exp_f32, ~1 ulp). Results below the float32
// normal range may flush to zero, which only affects softmax weights < 2^-126 relative to
// the row maximum.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A softmax weight rebuilt from a stored lse, P = 2^(s log2e - lse log2e), clamped to [0, 1]
// (one med3, or the clamp bit of v_exp_f32). P <= 1 by construction, but the two products
// are rounded separately: in a row whose every score is the same huge number (a bias of -1e30
// on every key, as the route decoder passes for queries with no valid key,
// route_pointer.py:2042-2048) lse equals that score up to rounding and the difference is
// +-1 ulp of 1.4e30, whose 2^x overflows. The reference's exp(s - lse) is exactly 1 there
// (custom_gradients.py, mhsea_tuned_jvp.py: both in natural units); clamped, such a row
// gets weight 1 or 0 and stays finite. Elsewhere the clamp changes at most a rounding
// excess above 1.
__device__ __forceinline__ float clamp01(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, 1.f); }
__device__ __forceinline__ float lse_weight(float x) { return clamp01(fast_exp2(x)); }

// bfloat16 <-> float32. Round-to-nearest-even on the way down; NaN stays NaN.
__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
// Hardware conversion (v_cvt_pk_bf16_f32 on gfx950): round to nearest even, NaN stays NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pack2_bf16(f, 0.f) & 0xffffu);
}

// Storage policy: F32 tensors are float, BF16 tensors are uint16_t bit patterns.
struct F32 {
  typedef float T;
  static constexpr int kBytes = 4;
};
struct BF16 {
  typedef uint16_t T;
  static constexpr int kBytes = 2;
};

// Load 4 consecutive elements (16 B aligned for F32, 8 B for BF16) as float.
template <class S>
__device__ __forceinline__ float4 load4(const void* base, int64_t off);
template <>
__device__ __forceinline__ float4 load4<F32>(const void* base, int64_t off) {
  return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
}
template <>
__device__ __forceinline__ float4 load4<BF16>(const void* base, int64_t off) {
  uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                     __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
}

// Four consecutive elements in their storage format, for values that are loaded early and
// used late (prefetch registers): bfloat16 keeps half the registers of float.
template <class S>
struct Raw4;
template <>
struct Raw4<F32> {
  float4 v;
  __device__ __forceinline__ static Raw4 load(const void* base, int64_t off) {
    return Raw4{*reinterpret_cast<const float4*>(static_cast<const float*>(base) + off)};
  }
  __device__ __forceinline__ float4 f() const { return v; }
};
template <>
struct Raw4<BF16> {
  uint2 v;
  __device__ __forceinline__ static Raw4 load(const void* base, int64_t off) {
    return Raw4{*reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off)};
  }
  __device__ __forceinline__ float4 f() const {
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
  }
};

// Load 2 consecutive elements (8 B aligned for F32, 4 B for BF16) as float.
template <class S>
__device__ __forceinline__ float2 load2(const void* base, int64_t off);
template <>
__device__ __forceinline__ float2 load2<F32>(const void* base, int64_t off) {
  return *reinterpret_cast<const float2*>(static_cast<const float*>(base) + off);
}
template <>
__device__ __forceinline__ float2 load2<BF16>(const void* base, int64_t off) {
  uint32_t u = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(base) + off);
  return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
}

template <class S>
__device__ __forceinline__ float load1(const void* base, int64_t off);
template <>
__device__ __forceinline__ float load1<F32>(const void* base, int64_t off) {
  return static_cast<const float*>(base)[off];
}
template <>
__device__ __forceinline__ float load1<BF16>(const void* base, int64_t off) {
  return bf16_to_f32(static_cast<const uint16_t*>(base)[off]);
}

// Output stores. The 16-byte fp32 stores use the non-temporal cache policy (outputs are
// written once and not read back; on MI355X 2-4% faster for the fp32 forward kernels at
// [512, 256, 8, 64] and with a bias at [1024, 64, 8, 32]); the 8-byte bf16 stores stay
// cached: non-temporal 8-byte stores made the bf16 forward + backward at [4096, 64, 8, 64]
// 55% slower.
template <class S>
__device__ __forceinline__ void store4(void* base, int64_t off, float a, float b, float c,
                                       float d);
template <>
__device__ __forceinline__ void store4<F32>(void* base, int64_t off, float a, float b,
                                            float c, float d) {
  typedef float v4nt __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4nt{a, b, c, d}, reinterpret_cast<v4nt*>(static_cast<float*>(base) + off));
}
template <>
__device__ __forceinline__ void store4<BF16>(void* base, int64_t off, float a, float b,
                                             float c, float d) {
  uint2 u;
  u.x = pack2_bf16(a, b);
  u.y = pack2_bf16(c, d);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + off) = u;
}

template <class S>
__device__ __forceinline__ void store1(void* base, int64_t off, float a);
template <>
__device__ __forceinline__ void store1<F32>(void* base, int64_t off, float a) {
  static_cast<float*>(base)[off] = a;
}
template <>
__device__ __forceinline__ void store1<BF16>(void* base, int64_t off, float a) {
  static_cast<uint16_t*>(base)[off] = f32_to_bf16(a);
}

// Sum / max over the four lane groups g that share one column c (lanes c, c+16, c+32, c+48).
// v_permlane16_swap / v_permlane32_swap with both operands x hand each lane the pair
// {x[l], x[l ^ 16]} (resp. x[l ^ 32]) in VALU registers, without a round trip through
// the LDS crossbar; the pair is combined in an order-independent way, so every lane of a
// column ends with the same bits as the xor-shuffle reduction.
__device__ __forceinline__ float xor16_pair_sum(float x) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor32_pair_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float group_sum(float x) { return xor32_pair_sum(xor16_pair_sum(x)); }
__device__ __forceinline__ float group_max(float x) {
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
  s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Offset of element (b, n, h, d) of a [B, N, H, D] tensor.
__device__ __forceinline__ int64_t bnhd(int b, int n, int h, int N, int H, int D) {
  return ((static_cast<int64_t>(b) * N + n) * H + h) * D;
}

// Per-walker compaction of the mask into the list of physical sites (ascending).
// Writes idx[0..count) and returns count to every thread of the workgroup.
// Must be called by all threads of a 256-thread workgroup; `scratch` holds 5 ints.
__device__ __forceinline__ int compact_mask(const uint8_t* __restrict__ mask_row, int N,
                                            int16_t* __restrict__ idx,
                                            int* __restrict__ scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  int total = 0;
  for (int base = 0; base < N; base += 256) {
    const int pos = base + tid;
    const bool on = (pos < N) && (mask_row[pos] != 0);
    const uint64_t bal = __ballot(on);
    if (lane == 0) scratch[wave] = __popcll(bal);
    __syncthreads();
    int before = total;
    for (int w = 0; w < wave; ++w) before += scratch[w];
    const int mine = __popcll(bal & ((uint64_t(1) << lane) - 1));
    if (on) idx[before + mine] = static_cast<int16_t>(pos);
    total += scratch[0] + scratch[1] + scratch[2] + scratch[3];
    __syncthreads();
  }
  return total;
}

// Per-walker compaction of the mask, one global round trip per 4096 sites: each thread
// reads 16 consecutive mask bytes, a workgroup-wide scan of the per-thread counts places
// the physical sites in idx[0..count) (ascending), and the raw bytes are kept in mask_s
// for later tests without touching global memory again. Returns count to every thread.
// Must be called by all threads of a 256-thread workgroup; `scratch` holds 4 ints;
// mask_s must be 16-byte aligned.
__device__ __forceinline__ int compact_mask_lds(const uint8_t* __restrict__ mask_row, int N,
                                                int16_t* __restrict__ idx,
                                                uint8_t* __restrict__ mask_s,
                                                int* __restrict__ scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const bool vec = (reinterpret_cast<uintptr_t>(mask_row) & 15u) == 0;
  int total = 0;
  for (int base = 0; base < N; base += 4096) {
    const int s0 = base + tid * 16;
    uint32_t bits = 0;
    if (vec && s0 + 16 <= N) {
      const uint4 w = *reinterpret_cast<const uint4*>(mask_row + s0);
      *reinterpret_cast<uint4*>(mask_s + s0) = w;
      const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          bits |= (((words[q] >> (8 * i)) & 0xffu) != 0u ? 1u : 0u) << (4 * q + i);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (s0 + i < N) {
          const uint8_t m = mask_row[s0 + i];
          mask_s[s0 + i] = m;
          bits |= (m != 0 ? 1u : 0u) << i;
        }
      }
    }
    const int cnt = __popc(bits);
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    int pos = total + incl - cnt;
    for (int w = 0; w < wave; ++w) pos += scratch[w];
    while (bits != 0u) {
      const int i = __ffs(bits) - 1;
      idx[pos++] = static_cast<int16_t>(s0 + i);
      bits &= bits - 1u;
    }
    total += scratch[0] + scratch[1] + scratch[2] + scratch[3];
    __syncthreads();
  }
  return total;
}

// Byte loads of one walker's mask row through a raw buffer resource (gfx9 descriptor,
// dword3 = 0x00020000: 32-bit data format, no swizzle). The walker offset b*N goes into
// the scalar offset, the lane into the vector offset. Lanes past the row (lane >= N) get
// the vector offset num_records, which is out of range whether or not the hardware adds
// the scalar offset before its range check, so they read 0 and never touch memory. The
// host guarantees B*N <= 2^31 - 1, so offsets never wrap.
struct MaskReader {
  __amdgpu_buffer_rsrc_t rsrc;
  int nrec;
  __device__ __forceinline__ MaskReader(const uint8_t* mask, int64_t bytes)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(mask), static_cast<short>(0),
                                               static_cast<int>(bytes), 0x00020000)),
        nrec(static_cast<int>(bytes)) {}
  __device__ __forceinline__ uint32_t byte(int b, int N, int lane) const {
    const int voff = lane < N ? lane : nrec;
    return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(rsrc, voff, b * N, 0));
  }
};

// Map blockIdx.x to a logical workgroup id so that consecutive logical ids (which share
// K/V rows of one walker and head) land on the same XCD. Workgroups are dispatched to
// the 8 XCDs round-robin by hardware id.
__device__ __forceinline__ int64_t xcd_logical_block(int64_t hw, int64_t nblocks) {
  constexpr int kXcd = 8;
  if (nblocks % kXcd != 0) return hw;
  const int64_t per = nblocks / kXcd;
  return (hw % kXcd) * per + hw / kXcd;
}

// Mask compaction for a workgroup of W waves (64 W threads): idx[0..count) = physical sites
// (ascending), mask_s = the raw mask bytes. Returns count to every thread.
template <int W>
__device__ __forceinline__ int compact_mask_wg(const uint8_t* __restrict__ mask_row, int N, int16_t* __restrict__ idx,
                                               uint8_t* __restrict__ mask_s, int* __restrict__ scratch) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  int total = 0;
  for (int base = 0; base < N; base += (64 * W)) {
    const int pos = base + tid;
    const uint8_t m = pos < N ? mask_row[pos] : 0;
    if (pos < N) mask_s[pos] = m;
    const bool on = m != 0;
    const uint64_t bal = __ballot(on);
    if (lane == 0) scratch[wave] = __popcll(bal);
    __syncthreads();
    int before = total;
    for (int w = 0; w < wave; ++w) before += scratch[w];
    if (on) idx[before + __popcll(bal & ((uint64_t(1) << lane) - 1))] = static_cast<int16_t>(pos);
    for (int w = 0; w < W; ++w) total += scratch[w];
    __syncthreads();
  }
  return total;
}

}  // namespace hz
