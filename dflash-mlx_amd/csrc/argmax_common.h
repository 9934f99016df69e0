// Argmax phase of the greedy accept, shared by the accept entry points and
// the verify scan that runs it in the same launch: one workgroup reduces one
// contiguous slice of one logits row to a 64-bit key (order-preserving value
// bits << 32 | ~index, argmax_key in device_common.h), so an integer max
// gives the largest value and, among equal values, the lowest index.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

constexpr int kArgmaxThreads = 256;

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p) {
  return bf16_bits_to_f32(*p);
}
struct F16Tag { uint16_t bits; };
template <>
__device__ __forceinline__ float load_logit<F16Tag>(const F16Tag* p) {
  return f16_bits_to_f32(p->bits);
}

// Keys of 16 bytes holding 16/sizeof(T) consecutive logits starting at idx.
template <typename T>
__device__ __forceinline__ uint64_t key16(u32x4 raw, int idx, uint64_t best);
template <>
__device__ __forceinline__ uint64_t key16<float>(u32x4 raw, int idx, uint64_t best) {
  best = u64_max(best, argmax_key(__uint_as_float(raw.x), idx + 0));
  best = u64_max(best, argmax_key(__uint_as_float(raw.y), idx + 1));
  best = u64_max(best, argmax_key(__uint_as_float(raw.z), idx + 2));
  best = u64_max(best, argmax_key(__uint_as_float(raw.w), idx + 3));
  return best;
}
template <>
__device__ __forceinline__ uint64_t key16<uint16_t>(u32x4 raw, int idx, uint64_t best) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    best = u64_max(best, argmax_key(bf16_lo(w[j]), idx + 2 * j));
    best = u64_max(best, argmax_key(bf16_hi(w[j]), idx + 2 * j + 1));
  }
  return best;
}
template <>
__device__ __forceinline__ uint64_t key16<F16Tag>(u32x4 raw, int idx, uint64_t best) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    best = u64_max(best, argmax_key(f16_bits_to_f32((uint16_t)(w[j] & 0xffffu)), idx + 2 * j));
    best = u64_max(best, argmax_key(f16_bits_to_f32((uint16_t)(w[j] >> 16)), idx + 2 * j + 1));
  }
  return best;
}

// One workgroup of kArgmaxThreads threads: the key of slice `split` of logits
// row `row` (sequence row / N, position row % N) to keys[row * splits + split],
// stored by thread 0 (agent_store: with an agent-scope store, for a reader in
// another workgroup of the same launch).
template <typename T, bool VECTOR>
__device__ __forceinline__ void argmax_partial_block(
    const T* __restrict__ logits, int64_t bstride, int64_t rstride, int N, int V, int chunk,
    int splits, uint64_t* __restrict__ keys, int row, int split, bool agent_store = false) {
  const int b = row / N;
  const int i = row - b * N;
  const T* base = logits + (int64_t)b * bstride + (int64_t)i * rstride;
  const int start = split * chunk;
  const int end = min(V, start + chunk);
  uint64_t best = 0;
  if (VECTOR) {
    constexpr int PER = 16 / sizeof(T);
    const int nvec = (end - start) / PER;
    const u32x4* vbase = reinterpret_cast<const u32x4*>(base + start);
    int j = threadIdx.x;
    // Four independent 16-byte loads in flight per lane.
    for (; j + 3 * kArgmaxThreads < nvec; j += 4 * kArgmaxThreads) {
      const u32x4 r0 = __builtin_nontemporal_load(vbase + j);
      const u32x4 r1 = __builtin_nontemporal_load(vbase + j + kArgmaxThreads);
      const u32x4 r2 = __builtin_nontemporal_load(vbase + j + 2 * kArgmaxThreads);
      const u32x4 r3 = __builtin_nontemporal_load(vbase + j + 3 * kArgmaxThreads);
      best = key16<T>(r0, start + j * PER, best);
      best = key16<T>(r1, start + (j + kArgmaxThreads) * PER, best);
      best = key16<T>(r2, start + (j + 2 * kArgmaxThreads) * PER, best);
      best = key16<T>(r3, start + (j + 3 * kArgmaxThreads) * PER, best);
    }
    for (; j < nvec; j += kArgmaxThreads) best = key16<T>(vbase[j], start + j * PER, best);
    for (int idx = start + nvec * PER + threadIdx.x; idx < end; idx += kArgmaxThreads)
      best = u64_max(best, argmax_key(load_logit<T>(base + idx), idx));
  } else {
    for (int idx = start + threadIdx.x; idx < end; idx += kArgmaxThreads)
      best = u64_max(best, argmax_key(load_logit<T>(base + idx), idx));
  }
  best = wave_max_u64(best);
  __shared__ uint64_t wbest[kArgmaxThreads / 64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  if (lane == 0) wbest[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t m = wbest[0];
#pragma unroll
    for (int w = 1; w < kArgmaxThreads / 64; ++w) m = u64_max(m, wbest[w]);
    if (agent_store)  // read by a last arriver: the protocol of device_common.h
      __hip_atomic_store(keys + (int64_t)row * splits + split, m, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    else
      keys[(int64_t)row * splits + split] = m;
  }
}

struct Split {
  int splits;
  int chunk;
};

// Deterministic split of one vocabulary row; the workspace size depends on it.
Split plan_split(int B, int N, int V) {
  const int64_t rows = (int64_t)B * N;
  int64_t splits = ceil_div(2048, rows > 0 ? rows : 1);
  const int64_t max_by_len = ceil_div(V, 2048);
  if (splits > max_by_len) splits = max_by_len;
  if (splits < 1) splits = 1;
  if (splits > 1024) splits = 1024;
  int64_t chunk = ceil_div(V, splits);
  chunk = ceil_div(chunk, 16) * 16;  // keeps 16-byte alignment of each slice
  splits = ceil_div(V, chunk);
  return Split{(int)splits, (int)chunk};
}

}  // namespace
}  // namespace dflash
