// Conv-window rollback shared by dflash_conv_rollback and the fused accept +
// conv rollback: the new window of (layer l, sequence b) after accepting a
// block tokens is rows a .. a+K1-1 of concat(conv_in[b] (K1 rows), qkv[b])
// (dflash_mlx/custom_qwen35_model.py:1044-1051).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash_gdn.h"
#include "host_common.h"

namespace dflash {
namespace {

constexpr int kConvThreads = 256;
constexpr int kMaxConvRows = 8;
// Candidate rows the speculative window copy holds (used when T + K1 <= this).
constexpr int kConvCandidates = 20;

struct ConvTable {
  const char* cin[kMaxLayersPerLaunch];
  const char* qkv[kMaxLayersPerLaunch];
  char* cout[kMaxLayersPerLaunch];
};

// Column units c = blockIdx.x * kConvThreads + threadIdx.x, grid-strided: one
// lane owns one column unit for all K1 rows and reads every source row before
// it writes, so conv_out may alias conv_in.
template <typename U>
__device__ __forceinline__ void conv_window_copy(const ConvTable& tab, int l, int b, int a, int K1,
                                                 int64_t Cu, int64_t qkv_bs, int64_t qkv_rs,
                                                 int64_t c_begin = -1) {
  const U* cin = reinterpret_cast<const U*>(tab.cin[l]) + (int64_t)b * K1 * Cu;
  const U* qkv = reinterpret_cast<const U*>(tab.qkv[l]) + (int64_t)b * qkv_bs;
  U* cout = reinterpret_cast<U*>(tab.cout[l]) + (int64_t)b * K1 * Cu;
  for (int64_t c = c_begin >= 0 ? c_begin : (int64_t)blockIdx.x * kConvThreads + threadIdx.x; c < Cu;
       c += (int64_t)gridDim.x * kConvThreads) {
    U vals[kMaxConvRows];
#pragma unroll
    for (int r = 0; r < kMaxConvRows; ++r) {
      if (r < K1) {
        const int j = a + r;
        vals[r] = j < K1 ? cin[(int64_t)j * Cu + c] : qkv[(int64_t)(j - K1) * qkv_rs + c];
      }
    }
#pragma unroll
    for (int r = 0; r < kMaxConvRows; ++r)
      if (r < K1) cout[(int64_t)r * Cu + c] = vals[r];
  }
}

// The same copy with the accepted count not yet known: the lane's first column
// unit's rows 0 .. T+K1-1 of concat(conv_in, qkv) (every row a window can
// start at, T + K1 <= CAND) are loaded by prefetch() before a is computed;
// store() then writes the K1 rows at a and copies any further column units as
// conv_window_copy does.  All loads precede the stores, so conv_out may alias
// conv_in.
template <typename U, int CAND>
struct ConvWindowPrefetch {
  U rows[CAND];

  // Lanes past the last column unit load unit Cu - 1 and rows past T + K1 - 1
  // repeat that row (valid addresses, no branch around the loads; never stored).
  __device__ __forceinline__ void prefetch(const ConvTable& tab, int l, int b, int T, int K1,
                                           int64_t Cu, int64_t qkv_bs, int64_t qkv_rs) {
    const int64_t c = min((int64_t)blockIdx.x * kConvThreads + threadIdx.x, Cu - 1);
    const U* cin = reinterpret_cast<const U*>(tab.cin[l]) + (int64_t)b * K1 * Cu + c;
    const U* qkv = reinterpret_cast<const U*>(tab.qkv[l]) + (int64_t)b * qkv_bs + c;
#pragma unroll
    for (int r = 0; r < CAND; ++r) {
      const int j = min(r, T + K1 - 1);
      rows[r] = j < K1 ? cin[(int64_t)j * Cu] : qkv[(int64_t)(j - K1) * qkv_rs];
    }
  }

  __device__ __forceinline__ void store(const ConvTable& tab, int l, int b, int a, int K1,
                                        int64_t Cu, int64_t qkv_bs, int64_t qkv_rs) {
    const int64_t c = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
    if (c < Cu) {
      U* cout = reinterpret_cast<U*>(tab.cout[l]) + (int64_t)b * K1 * Cu + c;
      // every row under a compile-time index (the array stays in registers);
      // a is uniform, so the tests branch the whole wavefront together
#pragma unroll
      for (int j = 0; j < CAND; ++j) {
        const int r = j - a;
        if (r >= 0 && r < K1) cout[(int64_t)r * Cu] = rows[j];
      }
    }
    conv_window_copy<U>(tab, l, b, a, K1, Cu, qkv_bs, qkv_rs, c + (int64_t)gridDim.x * kConvThreads);
  }
};

// Workgroups along x of a (chunks, B, L) copy grid over `units` units:
// ~2048 workgroups in total, at least one per (sequence, layer).
inline int copy_grid_chunks(int64_t units, int per_block, int B, int L) {
  int64_t want = ceil_div(2048, (int64_t)B * L);
  const int64_t most = ceil_div(units, per_block);
  if (want > most) want = most;
  if (want < 1) want = 1;
  if (want > 65535) want = 65535;
  return (int)want;
}

// Host-side checks shared by both entry points; fills the launch geometry.
struct ConvPlan {
  int unit;  // bytes per column unit: 16, 4 or 2
  int64_t Cu, qbs, qrs;
};

inline int conv_plan(const void* const* conv_in, const void* const* qkv, void* const* conv_out,
                     int L, int T, int K1, int64_t C, int64_t qkv_batch_stride,
                     int64_t qkv_row_stride, int elem_bytes, ConvPlan* plan) {
  if (L < 0 || T < 0 || K1 < 0 || C < 0) return DFLASH_ERR_SHAPE;
  if (K1 > kMaxConvRows) return DFLASH_ERR_UNSUPPORTED;
  if (elem_bytes != 2 && elem_bytes != 4) return DFLASH_ERR_UNSUPPORTED;
  if (conv_in == nullptr || qkv == nullptr || conv_out == nullptr) return DFLASH_ERR_NULL;
  const int64_t row_bytes = C * elem_bytes;
  bool vec = (row_bytes % 16 == 0) && ((qkv_batch_stride * elem_bytes) % 16 == 0) &&
             ((qkv_row_stride * elem_bytes) % 16 == 0);
  for (int l = 0; l < L; ++l) {
    if (conv_in[l] == nullptr || (T > 0 && qkv[l] == nullptr) || conv_out[l] == nullptr)
      return DFLASH_ERR_NULL;
    const uintptr_t any = (uintptr_t)conv_in[l] | (uintptr_t)qkv[l] | (uintptr_t)conv_out[l];
    if (any & 15) vec = false;
    if (any & (uintptr_t)(elem_bytes - 1)) return DFLASH_ERR_ALIGN;
  }
  plan->unit = vec ? 16 : elem_bytes;
  plan->Cu = row_bytes / plan->unit;
  plan->qbs = qkv_batch_stride * elem_bytes / plan->unit;
  plan->qrs = qkv_row_stride * elem_bytes / plan->unit;
  return DFLASH_OK;
}

inline ConvTable conv_table(const void* const* conv_in, const void* const* qkv,
                            void* const* conv_out, int l0, int nl) {
  ConvTable tab{};
  for (int j = 0; j < nl; ++j) {
    tab.cin[j] = static_cast<const char*>(conv_in[l0 + j]);
    tab.qkv[j] = static_cast<const char*>(qkv[l0 + j]);
    tab.cout[j] = static_cast<char*>(conv_out[l0 + j]);
  }
  return tab;
}

}  // namespace
}  // namespace dflash
