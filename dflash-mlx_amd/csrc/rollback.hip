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

struct ConvTable {
  const char* cin[kMaxLayersPerLaunch];
  const char* qkv[kMaxLayersPerLaunch];
  char* cout[kMaxLayersPerLaunch];
};

constexpr int kMaxConvRows = 8;

// grid: (column chunks, B, layers).  One lane owns one column unit of one
// (layer, sequence) for all K1 rows: it reads every source row before it
// writes, so conv_out may alias conv_in.
template <typename U>
__global__ __launch_bounds__(kCopyThreads) void conv_rollback_kernel(
    const ConvTable tab, const int32_t* __restrict__ accepted, int T, int K1,
    int64_t Cu, int64_t qkv_bs, int64_t qkv_rs) {
  const int l = blockIdx.z;
  const int b = blockIdx.y;
  const int a = min(max(accepted[b], 0), T);
  const U* cin = reinterpret_cast<const U*>(tab.cin[l]) + (int64_t)b * K1 * Cu;
  const U* qkv = reinterpret_cast<const U*>(tab.qkv[l]) + (int64_t)b * qkv_bs;
  U* cout = reinterpret_cast<U*>(tab.cout[l]) + (int64_t)b * K1 * Cu;
  for (int64_t c = (int64_t)blockIdx.x * kCopyThreads + threadIdx.x; c < Cu;
       c += (int64_t)gridDim.x * kCopyThreads) {
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

int grid_chunks(int64_t units, int per_block, int B, int L) {
  // Aim for ~2048 workgroups in total; at least one per (sequence, layer).
  int64_t want = ceil_div(2048, (int64_t)B * L);
  const int64_t most = ceil_div(units, per_block);
  if (want > most) want = most;
  if (want < 1) want = 1;
  if (want > 65535) want = 65535;
  return (int)want;
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
    dim3 grid(grid_chunks(units, kCopyThreads * kCopyUnroll, B, nl), B, nl);
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
  if (conv_in == nullptr || qkv == nullptr || conv_out == nullptr || accepted == nullptr)
    return DFLASH_ERR_NULL;
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int unit = vec ? 16 : elem_bytes;
  const int64_t Cu = row_bytes / unit;
  const int64_t qbs = qkv_batch_stride * elem_bytes / unit;
  const int64_t qrs = qkv_row_stride * elem_bytes / unit;
  for (int l0 = 0; l0 < L; l0 += kMaxLayersPerLaunch) {
    const int nl = L - l0 < kMaxLayersPerLaunch ? L - l0 : kMaxLayersPerLaunch;
    ConvTable tab{};
    for (int j = 0; j < nl; ++j) {
      tab.cin[j] = static_cast<const char*>(conv_in[l0 + j]);
      tab.qkv[j] = static_cast<const char*>(qkv[l0 + j]);
      tab.cout[j] = static_cast<char*>(conv_out[l0 + j]);
    }
    dim3 grid(grid_chunks(Cu, kCopyThreads, B, nl), B, nl);
    if (unit == 16)
      hipLaunchKernelGGL(conv_rollback_kernel<u32x4>, grid, dim3(kCopyThreads), 0, s, tab,
                         accepted, T, K1, Cu, qbs, qrs);
    else if (unit == 4)
      hipLaunchKernelGGL(conv_rollback_kernel<uint32_t>, grid, dim3(kCopyThreads), 0, s, tab,
                         accepted, T, K1, Cu, qbs, qrs);
    else
      hipLaunchKernelGGL(conv_rollback_kernel<uint16_t>, grid, dim3(kCopyThreads), 0, s, tab,
                         accepted, T, K1, Cu, qbs, qrs);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return DFLASH_OK;
}
