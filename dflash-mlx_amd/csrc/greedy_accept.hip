// Greedy verify accept: vocabulary argmax + longest agreeing draft prefix.
//
// Reference semantics: sample_tokens with temperature 0 is mx.argmax over the
// last axis (dflash_mlx/runtime.py:22-29); the accept is
// longest_prefix_match(block[1:], posterior[:-1]) with the bonus token
// posterior[matched] (runtime.py:41-47, :145-147, :163).
//
// Two launches, HBM-bound on the logits read:
//   1. argmax_partial: grid (B*N rows, splits).  Each workgroup reduces one
//      contiguous slice of one logits row to a 64-bit key (argmax_common.h).
//   2. accept_finalize: one workgroup per sequence, one wavefront per logits
//      row, merges the split keys of all rows at once, writes the posterior
//      tokens, then finds the first draft mismatch with a 64-lane ballot.
// The kernel boundary orders the two phases; no cross-workgroup atomics or
// cache write-backs are needed.  Only the small matched/bonus/posterior arrays
// leave the device.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "accept_common.h"
#include "argmax_common.h"
#include "conv_window.h"
#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

constexpr int kMaxAcceptRows = 16384;

template <typename T, bool VECTOR>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(
    const T* __restrict__ logits, int64_t bstride, int64_t rstride, int N, int V, int chunk,
    int splits, uint64_t* __restrict__ keys) {
  argmax_partial_block<T, VECTOR>(logits, bstride, rstride, N, V, chunk, splits, keys, blockIdx.x,
                                  blockIdx.y);
}

template <typename T>
hipError_t launch_partial(const void* logits, int64_t bs, int64_t rs, int B, int N, int V,
                          const Split& sp, uint64_t* keys, hipStream_t s) {
  const T* lp = static_cast<const T*>(logits);
  const int per = 16 / (int)sizeof(T);
  const bool vec = ((uintptr_t)logits % 16 == 0) && (bs % per == 0) && (rs % per == 0);
  const dim3 grid(B * N, sp.splits);
  if (vec)
    hipLaunchKernelGGL((argmax_partial_kernel<T, true>), grid, dim3(kArgmaxThreads), 0, s, lp, bs,
                       rs, N, V, sp.chunk, sp.splits, keys);
  else
    hipLaunchKernelGGL((argmax_partial_kernel<T, false>), grid, dim3(kArgmaxThreads), 0, s, lp, bs,
                       rs, N, V, sp.chunk, sp.splits, keys);
  return hipGetLastError();
}

// The accept's finalize and the conv-window rollback in one launch, grid
// (column chunks, B, layers): every workgroup merges its sequence's argmax
// keys (N rows x splits), prefix-compares
// the draft as accept_finalize_kernel does, then copies its columns of the
// window for a = matched + accepted_offset.  The workgroup (0, b, 0) of the
// first launch (write_accept) also writes posterior / matched / bonus of b
// and, when accepted_out is given, the clamped a (the keep count the next
// step's rolled-back state load reads).
// CAND > 0 (T + K1 <= CAND): the lane's window rows are loaded with the keys
// and the first 64 draft tokens, before the accepted count is known, so the
// kernel waits on memory once instead of three times.
// Dynamic LDS: N int32.
template <typename U, int CAND>
__global__ __launch_bounds__(kConvThreads) void accept_conv_rollback_kernel(
    const uint64_t* __restrict__ keys, int splits, int N, const int32_t* __restrict__ draft,
    int64_t dstride, int n_draft, int32_t* __restrict__ posterior, int32_t* __restrict__ matched,
    int32_t* __restrict__ bonus, int write_accept, int accepted_offset,
    int32_t* __restrict__ accepted_out, const ConvTable tab, int T,
    int K1, int64_t Cu, int64_t qkv_bs, int64_t qkv_rs) {
  extern __shared__ int32_t post[];
  __shared__ int s_first;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int mlen = min(n_draft, N);
  int draft0 = 0;  // draft token `lane` of the first 64 (wavefront 0)
  if (wave == 0 && lane < mlen) draft0 = draft[(int64_t)b * dstride + lane];
  ConvWindowPrefetch<U, (CAND > 0 ? CAND : 1)> win;
  if (CAND > 0) win.prefetch(tab, blockIdx.z, b, T, K1, Cu, qkv_bs, qkv_rs);
  // 16 lanes per row, 16 rows per pass: every lane's key loads are issued
  // together, then a max over its 16 lanes (exact, so order-free).
  const int sub = threadIdx.x & 15;
  for (int r0 = 0; r0 < N; r0 += kConvThreads / 16) {
    const int r = r0 + (threadIdx.x >> 4);
    uint64_t m = 0;
    if (r < N) {
      const uint64_t* kr = keys + ((int64_t)b * N + r) * splits;
      // batches of 8 loads issued together (one batch up to 128 splits);
      // indices past the row repeat its last key, which leaves the max as is
      for (int s0 = sub; s0 < splits; s0 += 16 * 8) {
        uint64_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = kr[min(s0 + 16 * i, splits - 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i) m = u64_max(m, v[i]);
      }
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
      const uint32_t lo = __shfl_xor((unsigned)(m & 0xffffffffu), off, 16);
      const uint32_t hi = __shfl_xor((unsigned)(m >> 32), off, 16);
      m = u64_max(m, ((uint64_t)hi << 32) | lo);
    }
    if (sub == 0 && r < N) post[r] = argmax_key_index(m);
  }
  __syncthreads();
  if (wave == 0) {
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
    if (lane == 0) s_first = first;
  }
  __syncthreads();
  const int first = s_first;
  if (write_accept && blockIdx.x == 0 && blockIdx.z == 0) {
    if (posterior != nullptr)
      for (int r = threadIdx.x; r < N; r += kConvThreads) posterior[(int64_t)b * N + r] = post[r];
    if (threadIdx.x == 0) {
      if (matched != nullptr) matched[b] = first;
      if (bonus != nullptr) bonus[b] = first < N ? post[first] : -1;
      if (accepted_out != nullptr) accepted_out[b] = min(max(first + accepted_offset, 0), T);
    }
  }
  const int a = min(max(first + accepted_offset, 0), T);
  if (CAND > 0)
    win.store(tab, blockIdx.z, b, a, K1, Cu, qkv_bs, qkv_rs);
  else
    conv_window_copy<U>(tab, blockIdx.z, b, a, K1, Cu, qkv_bs, qkv_rs);
}


}  // namespace
}  // namespace dflash

extern "C" size_t dflash_greedy_accept_workspace_bytes(int B, int N, int V) {
  if (B <= 0 || N <= 0 || V <= 0) return 0;
  const dflash::Split sp = dflash::plan_split(B, N, V);
  return sizeof(uint64_t) * (size_t)B * N * sp.splits;
}

extern "C" int dflash_greedy_accept(const void* logits, int logits_dtype,
                                    int64_t logits_batch_stride,
                                    int64_t logits_row_stride,
                                    const int32_t* draft, int64_t draft_stride,
                                    int n_draft, int32_t* posterior,
                                    int32_t* matched, int32_t* bonus, int B,
                                    int N, int V, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  using namespace dflash;
  if (B < 0 || N <= 0 || V <= 0 || n_draft < 0) return DFLASH_ERR_SHAPE;
  if (N > kMaxAcceptRows || (int64_t)B * N > INT32_MAX) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  if (logits == nullptr || workspace == nullptr) return DFLASH_ERR_NULL;
  if (n_draft > 0 && draft == nullptr) return DFLASH_ERR_NULL;
  if (posterior == nullptr && matched == nullptr && bonus == nullptr) return DFLASH_ERR_NULL;
  if (logits_dtype != DFLASH_DTYPE_F32 && logits_dtype != DFLASH_DTYPE_BF16 &&
      logits_dtype != DFLASH_DTYPE_F16)
    return DFLASH_ERR_UNSUPPORTED;
  if (workspace_bytes < dflash_greedy_accept_workspace_bytes(B, N, V)) return DFLASH_ERR_WORKSPACE;
  if ((uintptr_t)workspace % 8 != 0) return DFLASH_ERR_ALIGN;
  const Split sp = plan_split(B, N, V);
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (logits_dtype == DFLASH_DTYPE_F32)
    e = launch_partial<float>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  else if (logits_dtype == DFLASH_DTYPE_BF16)
    e = launch_partial<uint16_t>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  else
    e = launch_partial<F16Tag>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  if (e != hipSuccess) return (int)e;
  return to_status(launch_accept_finalize(keys, sp.splits, B, N, draft, draft_stride, n_draft,
                                          posterior, matched, bonus, s));
}

namespace dflash {
namespace {
// dflash_greedy_accept_conv_rollback; with logits == nullptr the argmax keys
// are already in the workspace (dflash_accept_keys_conv_rollback).
int accept_conv_rollback(
    const void* logits, int logits_dtype, int64_t logits_batch_stride,
    int64_t logits_row_stride, const int32_t* draft, int64_t draft_stride, int n_draft,
    int32_t* posterior, int32_t* matched, int32_t* bonus, int B, int N, int V, void* workspace,
    size_t workspace_bytes, const void* const* conv_in, const void* const* qkv,
    void* const* conv_out, int accepted_offset, int32_t* accepted_out, int L, int T, int K1,
    int64_t C, int64_t qkv_batch_stride, int64_t qkv_row_stride, int elem_bytes, void* stream,
    bool run_argmax) {
  if (B < 0 || N <= 0 || V <= 0 || n_draft < 0) return DFLASH_ERR_SHAPE;
  if (N > kMaxAcceptRows || (int64_t)B * N > INT32_MAX) return DFLASH_ERR_SHAPE;
  if (L < 0 || T < 0 || K1 < 0 || C < 0 || B > 65535) return DFLASH_ERR_SHAPE;
  if (K1 > kMaxConvRows) return DFLASH_ERR_UNSUPPORTED;
  if (elem_bytes != 2 && elem_bytes != 4) return DFLASH_ERR_UNSUPPORTED;
  if (B == 0) return DFLASH_OK;
  if ((run_argmax && logits == nullptr) || workspace == nullptr) return DFLASH_ERR_NULL;
  if (n_draft > 0 && draft == nullptr) return DFLASH_ERR_NULL;
  if (run_argmax && logits_dtype != DFLASH_DTYPE_F32 && logits_dtype != DFLASH_DTYPE_BF16 &&
      logits_dtype != DFLASH_DTYPE_F16)
    return DFLASH_ERR_UNSUPPORTED;
  if (workspace_bytes < dflash_greedy_accept_workspace_bytes(B, N, V)) return DFLASH_ERR_WORKSPACE;
  if ((uintptr_t)workspace % 8 != 0) return DFLASH_ERR_ALIGN;
  const bool conv = L > 0 && K1 > 0 && C > 0;
  if (!conv && accepted_out != nullptr) return DFLASH_ERR_UNSUPPORTED;  // written by the copy
  ConvPlan pl{2, 0, 0, 0};
  if (conv) {
    const int st = conv_plan(conv_in, qkv, conv_out, L, T, K1, C, qkv_batch_stride,
                             qkv_row_stride, elem_bytes, &pl);
    if (st != DFLASH_OK) return st;
  }
  const Split sp = plan_split(B, N, V);
  uint64_t* keys = static_cast<uint64_t*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (!run_argmax)
    ;
  else if (logits_dtype == DFLASH_DTYPE_F32)
    e = launch_partial<float>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  else if (logits_dtype == DFLASH_DTYPE_BF16)
    e = launch_partial<uint16_t>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  else
    e = launch_partial<F16Tag>(logits, logits_batch_stride, logits_row_stride, B, N, V, sp, keys, s);
  if (e != hipSuccess) return (int)e;
  if (!conv) {
    if (posterior == nullptr && matched == nullptr && bonus == nullptr) return DFLASH_OK;
    return to_status(launch_accept_finalize(keys, sp.splits, B, N, draft, draft_stride, n_draft,
                                            posterior, matched, bonus, s));
  }
  const size_t lds = sizeof(int32_t) * (size_t)N;
  for (int l0 = 0; l0 < L; l0 += kMaxLayersPerLaunch) {
    const int nl = L - l0 < kMaxLayersPerLaunch ? L - l0 : kMaxLayersPerLaunch;
    const ConvTable tab = conv_table(conv_in, qkv, conv_out, l0, nl);
    const dim3 grid(copy_grid_chunks(pl.Cu, kConvThreads, B, nl), B, nl);
    const int first = l0 == 0;
    const bool spec = T + K1 <= kConvCandidates;
#define DFLASH_ACR(U, C)                                                                          \
  hipLaunchKernelGGL((accept_conv_rollback_kernel<U, C>), grid, dim3(kConvThreads), lds, s, keys, \
                     sp.splits, N, draft, draft_stride, n_draft, posterior, matched, bonus, first,  \
                     accepted_offset, accepted_out, tab, T, K1, pl.Cu, pl.qbs, pl.qrs)
    if (pl.unit == 16) {
      if (spec) DFLASH_ACR(u32x4, kConvCandidates); else DFLASH_ACR(u32x4, 0);
    } else if (pl.unit == 4) {
      if (spec) DFLASH_ACR(uint32_t, kConvCandidates); else DFLASH_ACR(uint32_t, 0);
    } else {
      if (spec) DFLASH_ACR(uint16_t, kConvCandidates); else DFLASH_ACR(uint16_t, 0);
    }
#undef DFLASH_ACR
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return DFLASH_OK;
}
}  // namespace
}  // namespace dflash

extern "C" int dflash_greedy_accept_conv_rollback(
    const void* logits, int logits_dtype, int64_t logits_batch_stride,
    int64_t logits_row_stride, const int32_t* draft, int64_t draft_stride, int n_draft,
    int32_t* posterior, int32_t* matched, int32_t* bonus, int B, int N, int V, void* workspace,
    size_t workspace_bytes, const void* const* conv_in, const void* const* qkv,
    void* const* conv_out, int accepted_offset, int32_t* accepted_out, int L, int T, int K1,
    int64_t C, int64_t qkv_batch_stride, int64_t qkv_row_stride, int elem_bytes, void* stream) {
  return dflash::accept_conv_rollback(
      logits, logits_dtype, logits_batch_stride, logits_row_stride, draft, draft_stride, n_draft,
      posterior, matched, bonus, B, N, V, workspace, workspace_bytes, conv_in, qkv, conv_out,
      accepted_offset, accepted_out, L, T, K1, C, qkv_batch_stride, qkv_row_stride, elem_bytes,
      stream, true);
}

extern "C" int dflash_accept_keys_conv_rollback(
    const int32_t* draft, int64_t draft_stride, int n_draft, int32_t* posterior, int32_t* matched,
    int32_t* bonus, int B, int N, int V, const void* workspace, size_t workspace_bytes,
    const void* const* conv_in, const void* const* qkv, void* const* conv_out,
    int accepted_offset, int32_t* accepted_out, int L, int T, int K1, int64_t C,
    int64_t qkv_batch_stride, int64_t qkv_row_stride, int elem_bytes, void* stream) {
  return dflash::accept_conv_rollback(
      nullptr, DFLASH_DTYPE_F32, 0, 0, draft, draft_stride, n_draft, posterior, matched, bonus, B,
      N, V, const_cast<void*>(workspace), workspace_bytes, conv_in, qkv, conv_out,
      accepted_offset, accepted_out, L, T, K1, C, qkv_batch_stride, qkv_row_stride, elem_bytes,
      stream, false);
}

// ------------------------------------------------ allocation-free variant
// The argmax keys of dflash_greedy_accept_noalloc live in this file-scope
// device array instead of a caller workspace.  Every device the library runs
// on holds one copy for the life of the process; its device address comes
// from hipGetSymbolAddress once per device (the array's name in host code is
// only a host-side stand-in, never a device address).  Every key slot a call
// uses is written by its argmax launch before the finalize reads it, so
// nothing needs clearing; calls that overlap on one device share the array
// and race.
namespace dflash {
namespace {
constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
constexpr int kMaxDevices = 64;
}  // namespace
}  // namespace dflash

static __device__ __align__(256) uint64_t scratch[dflash::kNoAllocScratchBytes / sizeof(uint64_t)];

namespace dflash {
namespace {
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// Device address of `scratch` on the current device (resolved on the first
// call made with that device current); nullptr with *status set on failure.
uint64_t* scratch_for_current_device(int* status) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *status = (int)e;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *status = DFLASH_ERR_UNSUPPORTED;
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return static_cast<uint64_t*>(p);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      *status = e != hipSuccess ? (int)e : DFLASH_ERR_NULL;
      return nullptr;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return static_cast<uint64_t*>(p);
}
}  // namespace
}  // namespace dflash

extern "C" size_t dflash_greedy_accept_noalloc_max_bytes(void) {
  return dflash::kNoAllocScratchBytes;
}

extern "C" int dflash_greedy_accept_noalloc(const void* logits, int logits_dtype,
                                            int64_t logits_batch_stride,
                                            int64_t logits_row_stride, const int32_t* draft,
                                            int64_t draft_stride, int n_draft,
                                            int32_t* posterior, int32_t* matched,
                                            int32_t* bonus, int B, int N, int V, void* stream) {
  using namespace dflash;
  if (B < 0 || N <= 0 || V <= 0 || n_draft < 0) return DFLASH_ERR_SHAPE;
  if (N > kMaxAcceptRows || (int64_t)B * N > INT32_MAX) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  const size_t need = dflash_greedy_accept_workspace_bytes(B, N, V);
  if (need > kNoAllocScratchBytes) return DFLASH_ERR_WORKSPACE;
  int status = DFLASH_OK;
  uint64_t* keys = scratch_for_current_device(&status);
  if (keys == nullptr) return status;
  return dflash_greedy_accept(logits, logits_dtype, logits_batch_stride, logits_row_stride, draft,
                              draft_stride, n_draft, posterior, matched, bonus, B, N, V, keys,
                              kNoAllocScratchBytes, stream);
}
