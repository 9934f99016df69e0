// Device-side helpers shared by the gfx950 kernels of libdflash_gfx950.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dflash {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 -> fp32 is exact: the bf16 bits are the high half of the fp32 bits.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xffff0000u);
}

// fp32 -> bf16, round to nearest, ties to even; NaN stays a quiet NaN.
// This is the rounding torch's Tensor.to(torch.bfloat16) applies.
// Branch-free (a select, not a jump), so it does not split the caller's basic
// blocks around memory operations.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = (u >> 16) | 0x0040u;
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? quiet_nan : rounded);
}

// fp16 -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// DPP controls of gfx9 (CDNA): quad permutations and 16-lane row mirrors.
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of one DPP row (lanes 16r .. 16r+15).  Every lane of
// the row ends with the same bits: each step adds a value to its mirror
// partner, and fp32 addition is commutative.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<kDppQuadSwap1>(x);
  x += dpp_mov<kDppQuadSwap2>(x);
  x += dpp_mov<kDppRowHalfMirror>(x);
  x += dpp_mov<kDppRowMirror>(x);
  return x;
}

// Order-preserving map of fp32 onto uint32 for argmax keys: -0 and +0 map to
// the same key, every NaN maps above +inf.
__device__ __forceinline__ uint32_t f32_order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// 64-bit argmax key: larger value wins, then the lower index wins.
__device__ __forceinline__ uint64_t argmax_key(float f, int idx) {
  return ((uint64_t)f32_order_key(f) << 32) |
         (uint64_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int argmax_key_index(uint64_t key) {
  return (int)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
}

__device__ __forceinline__ uint64_t u64_max(uint64_t a, uint64_t b) {
  return a > b ? a : b;
}

// Max over the 64 lanes of a wavefront; every lane gets the result.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    uint32_t lo = __shfl_xor((unsigned)(x & 0xffffffffu), off, 64);
    uint32_t hi = __shfl_xor((unsigned)(x >> 32), off, 64);
    x = u64_max(x, ((uint64_t)hi << 32) | lo);
  }
  return x;
}

}  // namespace dflash
