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

// Last-arriver merges across workgroups (the accept finish of the
// single-launch verify step, the tiled GEMMs' tail split, the argmax keys
// those read).  Producers store their partial results with relaxed
// agent-scope atomic stores, wait for them (s_waitcnt 0), then count
// themselves with a relaxed agent-scope fetch_add; the workgroup whose add
// returns the last count merges the partials with relaxed agent-scope atomic
// loads.  No workgroup waits on another.
//
// Relaxed atomics create no happens-before edge in the HIP (C++) memory
// model: the language does not promise that the last arriver sees the other
// producers' stores.  The protocol rests on what gfx950 does with these
// instructions instead:
//   1. an agent-scope atomic store is performed at the point where every XCD
//      of the device sees the same memory (not held in the issuing XCD's
//      L2), and s_waitcnt vmcnt(0) returns only once it is acknowledged
//      there; the count is issued after that wait;
//   2. the count is an atomic at the same point, so the add that returns the
//      last count comes after every producer's add, hence after every
//      producer's acknowledged stores;
//   3. the last arriver's loads are issued only after its add has returned
//      (they sit behind a branch on the returned value), and agent-scope
//      atomic loads read that point, not a stale L1/L2 line.
// The formal alternative, a release on every producer's count and an acquire
// on the last arriver's, makes every producer write back its XCD's whole L2
// (buffer_wbl2 at agent scope): next to the scan's tape stores that measured
// 31.9 us against 8.5 us for the accept, so the kernels keep the protocol
// above, and the tests that compare each merged result with the same work
// done in separate launches, bit for bit, are its check.

}  // namespace dflash
