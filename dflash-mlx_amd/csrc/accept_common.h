// Finalize phase shared by the greedy accept and the fused LM-head accept:
// merge per-slice argmax keys, write the posterior tokens, prefix-compare the
// draft, write matched/bonus.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"

namespace dflash {
namespace {

constexpr int kFinalizeWaves = 16;

// keys: [B*N rows, splits] 64-bit argmax keys (argmax_key in device_common.h).
// grid: B workgroups of kFinalizeWaves wavefronts; wave w merges rows w,
// w + kFinalizeWaves, ... of its sequence; dynamic LDS = N int32.
// The reference's accept: matched = leading positions where
// draft == posterior, bonus = posterior[matched] (dflash_mlx/runtime.py:41-47,
// :145-147, :163).
__global__ __launch_bounds__(64 * kFinalizeWaves) void accept_finalize_kernel(
    const uint64_t* __restrict__ keys, int splits, int N, const int32_t* __restrict__ draft,
    int64_t dstride, int n_draft, int32_t* __restrict__ posterior,
    int32_t* __restrict__ matched, int32_t* __restrict__ bonus) {
  extern __shared__ int32_t post[];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int mlen = min(n_draft, N);
  int draft0 = 0;  // draft token `lane` of the first 64, loaded with the keys (wavefront 0)
  if (wave == 0 && lane < mlen && (matched != nullptr || bonus != nullptr))
    draft0 = draft[(int64_t)b * dstride + lane];
  for (int r = wave; r < N; r += kFinalizeWaves) {
    const uint64_t* kr = keys + ((int64_t)b * N + r) * splits;
    uint64_t m = 0;
    // Batches of 16 loads per lane issued together (the fused LM head leaves
    // ~1 200 keys per row: two batches); indices past the row repeat its
    // last key, which leaves the max as is.
    for (int s0 = lane; s0 < splits; s0 += 64 * 16) {
      uint64_t v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = kr[min(s0 + 64 * i, splits - 1)];
#pragma unroll
      for (int i = 0; i < 16; ++i) m = u64_max(m, v[i]);
    }
    m = wave_max_u64(m);
    if (lane == 0) {
      const int tok = argmax_key_index(m);
      post[r] = tok;
      if (posterior != nullptr) posterior[(int64_t)b * N + r] = tok;
    }
  }
  __syncthreads();
  if (wave != 0 || (matched == nullptr && bonus == nullptr)) return;
  int first = mlen;
  for (int base0 = 0; base0 < mlen; base0 += 64) {
    const int j = base0 + lane;
    const int dj = base0 == 0 ? draft0 : (j < mlen ? draft[(int64_t)b * dstride + j] : 0);
    const bool mismatch = (j < mlen) && (dj != post[j]);
    const unsigned long long mask = __ballot(mismatch);
    if (mask != 0ull) {
      first = base0 + __ffsll(mask) - 1;
      break;
    }
  }
  if (lane == 0) {
    if (matched != nullptr) matched[b] = first;
    if (bonus != nullptr) bonus[b] = first < N ? post[first] : -1;
  }
}

inline hipError_t launch_accept_finalize(const uint64_t* keys, int splits, int B, int N,
                                         const int32_t* draft, int64_t dstride, int n_draft,
                                         int32_t* posterior, int32_t* matched, int32_t* bonus,
                                         hipStream_t s) {
  hipLaunchKernelGGL(accept_finalize_kernel, dim3(B), dim3(64 * kFinalizeWaves),
                     sizeof(int32_t) * (size_t)N, s, keys, splits, N, draft, dstride, n_draft,
                     posterior, matched, bonus);
  return hipGetLastError();
}

}  // namespace
}  // namespace dflash
