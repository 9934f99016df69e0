// Cache rollback to the accepted length, for all linear-attention layers of
// a verify step in one launch each.
//
// The reference rebuilds the recurrent state by replaying the accepted
// prefix and slides the conv window by concatenation
// (dflash_mlx/custom_qwen35_model.py:1029-1074).  With the state tape the
// recurrent state is a gather of tape[a-1]; the conv window is a gather of
// K-1 rows from [conv_in; qkv].  Both are HBM copies.  The accepted count is
// read on the device, so no host synchronisation is needed between the
// accept and the rollback.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "conv_window.h"
#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

struct TapeTable {
  const float* tape[kMaxLayersPerLaunch];
  const float* sin[kMaxLayersPerLaunch];
  float* sout[kMaxLayersPerLaunch];
};

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;

// grid: (chunks, B, layers).  Each lane copies kCopyUnroll units of VEC
// floats, all loads issued before the stores.
template <int VEC>
__global__ __launch_bounds__(kCopyThreads) void tape_select_kernel(
    const TapeTable tab, const int32_t* __restrict__ accepted, int T,
    int64_t S, int64_t tape_tstride) {
  const int l = blockIdx.z;
  const int b = blockIdx.y;
  const int a = min(max(accepted[b], 0), T);
  const float* src = a >= 1 ? tab.tape[l] + (int64_t)(a - 1) * tape_tstride + (int64_t)b * S
                            : tab.sin[l] + (int64_t)b * S;
  float* dst = tab.sout[l] + (int64_t)b * S;
  if (src == dst) return;
  const int64_t units = S / VEC;
  const int64_t step = (int64_t)gridDim.x * kCopyThreads;
  for (int64_t u0 = (int64_t)blockIdx.x * kCopyThreads * kCopyUnroll + threadIdx.x; u0 < units;
       u0 += step * kCopyUnroll) {
    if constexpr (VEC == 4) {
      f32x4 x[kCopyUnroll];
#pragma unroll
      for (int j = 0; j < kCopyUnroll; ++j) {
        const int64_t u = u0 + (int64_t)j * kCopyThreads;
        if (u < units) x[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src) + u);
      }
#pragma unroll
      for (int j = 0; j < kCopyUnroll; ++j) {
        const int64_t u = u0 + (int64_t)j * kCopyThreads;
        if (u < units) reinterpret_cast<f32x4*>(dst)[u] = x[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < kCopyUnroll; ++j) {
        const int64_t u = u0 + (int64_t)j * kCopyThreads;
        if (u < units) dst[u] = src[u];
      }
    }
  }
}

// grid: (column chunks, B, layers).  CAND > 0 (T + K1 <= CAND): the window
// rows are loaded with the accepted count instead of after it.
template <typename U, int CAND>
__global__ __launch_bounds__(kConvThreads) void conv_rollback_kernel(
    const ConvTable tab, const int32_t* __restrict__ accepted, int T, int K1,
    int64_t Cu, int64_t qkv_bs, int64_t qkv_rs) {
  const int b = blockIdx.y;
  if constexpr (CAND > 0) {
    const int a = accepted[b];
    ConvWindowPrefetch<U, CAND> win;
    win.prefetch(tab, blockIdx.z, b, T, K1, Cu, qkv_bs, qkv_rs);
    win.store(tab, blockIdx.z, b, min(max(a, 0), T), K1, Cu, qkv_bs, qkv_rs);
  } else {
    conv_window_copy<U>(tab, blockIdx.z, b, min(max(accepted[b], 0), T), K1, Cu, qkv_bs, qkv_rs);
  }
}


}  // namespace
}  // namespace dflash

extern "C" int dflash_tape_select(const float* const* tapes,
                                  const float* const* states_in,
                                  float* const* states_out,
                                  const int32_t* accepted, int L, int B, int T,
                                  int64_t state_elems, int64_t tape_token_stride,
                                  void* stream) {
  using namespace dflash;
  if (L < 0 || B < 0 || T < 0 || state_elems < 0 || tape_token_stride < 0)
    return DFLASH_ERR_SHAPE;
  if (L == 0 || B == 0 || state_elems == 0) return DFLASH_OK;
  if (B > 65535) return DFLASH_ERR_SHAPE;
  if (tapes == nullptr || states_in == nullptr || states_out == nullptr || accepted == nullptr)
    return DFLASH_ERR_NULL;
  bool vec = state_elems % 4 == 0;
  for (int l = 0; l < L; ++l) {
    if ((T > 0 && tapes[l] == nullptr) || states_in[l] == nullptr || states_out[l] == nullptr)
      return DFLASH_ERR_NULL;
    if (((uintptr_t)tapes[l] | (uintptr_t)states_in[l] | (uintptr_t)states_out[l]) & 15) vec = false;
    if (((uintptr_t)tapes[l] | (uintptr_t)states_in[l] | (uintptr_t)states_out[l]) & 3)
      return DFLASH_ERR_ALIGN;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t units = vec ? state_elems / 4 : state_elems;
  const int64_t tstride = tape_token_stride > 0 ? tape_token_stride : (int64_t)B * state_elems;
  if (vec && tstride % 4 != 0) vec = false;
  for (int l0 = 0; l0 < L; l0 += kMaxLayersPerLaunch) {
    const int nl = L - l0 < kMaxLayersPerLaunch ? L - l0 : kMaxLayersPerLaunch;
    TapeTable tab{};
    for (int j = 0; j < nl; ++j) {
      tab.tape[j] = tapes[l0 + j];
      tab.sin[j] = states_in[l0 + j];
      tab.sout[j] = states_out[l0 + j];
    }
    dim3 grid(copy_grid_chunks(units, kCopyThreads * kCopyUnroll, B, nl), B, nl);
    if (vec)
      hipLaunchKernelGGL(tape_select_kernel<4>, grid, dim3(kCopyThreads), 0, s, tab, accepted, T,
                         state_elems, tstride);
    else
      hipLaunchKernelGGL(tape_select_kernel<1>, grid, dim3(kCopyThreads), 0, s, tab, accepted, T,
                         state_elems, tstride);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return DFLASH_OK;
}

extern "C" int dflash_conv_rollback(const void* const* conv_in, const void* const* qkv,
                                    void* const* conv_out, const int32_t* accepted, int L,
                                    int B, int T, int K1, int64_t C,
                                    int64_t qkv_batch_stride, int64_t qkv_row_stride,
                                    int elem_bytes, void* stream) {
  using namespace dflash;
  if (L < 0 || B < 0 || T < 0 || K1 < 0 || C < 0) return DFLASH_ERR_SHAPE;
  if (K1 > kMaxConvRows) return DFLASH_ERR_UNSUPPORTED;
  if (elem_bytes != 2 && elem_bytes != 4) return DFLASH_ERR_UNSUPPORTED;
  if (L == 0 || B == 0 || K1 == 0 || C == 0) return DFLASH_OK;
  if (B > 65535) return DFLASH_ERR_SHAPE;
  if (accepted == nullptr) return DFLASH_ERR_NULL;
  ConvPlan pl;
  const int st = conv_plan(conv_in, qkv, conv_out, L, T, K1, C, qkv_batch_stride, qkv_row_stride,
                           elem_bytes, &pl);
  if (st != DFLASH_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int l0 = 0; l0 < L; l0 += kMaxLayersPerLaunch) {
    const int nl = L - l0 < kMaxLayersPerLaunch ? L - l0 : kMaxLayersPerLaunch;
    const ConvTable tab = conv_table(conv_in, qkv, conv_out, l0, nl);
    dim3 grid(copy_grid_chunks(pl.Cu, kConvThreads, B, nl), B, nl);
    const bool spec = T + K1 <= kConvCandidates;
#define DFLASH_CR(U, C)                                                                            \
  hipLaunchKernelGGL((conv_rollback_kernel<U, C>), grid, dim3(kConvThreads), 0, s, tab, accepted, T, \
                     K1, pl.Cu, pl.qbs, pl.qrs)
    if (pl.unit == 16) {
      if (spec) DFLASH_CR(u32x4, kConvCandidates); else DFLASH_CR(u32x4, 0);
    } else if (pl.unit == 4) {
      if (spec) DFLASH_CR(uint32_t, kConvCandidates); else DFLASH_CR(uint32_t, 0);
    } else {
      if (spec) DFLASH_CR(uint16_t, kConvCandidates); else DFLASH_CR(uint16_t, 0);
    }
#undef DFLASH_CR
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return DFLASH_OK;
}
