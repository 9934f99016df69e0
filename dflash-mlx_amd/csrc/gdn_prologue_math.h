// Per-element arithmetic of the gated-delta layer prologue, shared by the
// standalone prologue kernel and the verify scan that runs the prologue on
// the fly, so that both round the same fp32 expressions to the same bf16.
//
// Reference layer body (dflash_mlx/custom_qwen35_model.py:431-450):
//   conv_out = silu(depthwise conv1d(concat(conv_state, qkv)))   (:431-435)
//   q = Dk^-1 * rms_norm(q); k = Dk^-0.5 * rms_norm(k)            (:446-448)
//   beta = sigmoid(b); g = compute_g(A_log, a, dt_bias)           (:449-450)
// compute_g is mlx-lm 0.31.2's published Qwen3-Next form
// g = exp(-exp(A_log) * softplus(a + dt_bias)).
#pragma once

#include <hip/hip_runtime.h>

namespace dflash {

constexpr int kMaxConvTaps = 8;

__device__ __forceinline__ float pro_silu(float x) { return x / (1.f + __expf(-x)); }
__device__ __forceinline__ float pro_sigmoid(float x) { return 1.f / (1.f + __expf(-x)); }
// softplus(x) = log(1 + exp(x)), evaluated without overflow.
__device__ __forceinline__ float pro_softplus(float x) {
  return x > 20.f ? x : log1pf(__expf(x));
}

// Sum over the 64 lanes of a wavefront by an xor butterfly (offsets 32 .. 1):
// every lane ends with the same value, summed in a fixed tree order.
__device__ __forceinline__ float pro_wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Depthwise causal conv tap sum then silu: x[j] is row t + j of
// concat(conv_state, qkv), w[j] the channel's tap j.
__device__ __forceinline__ float pro_conv_silu(const float* w, const float* x, int K) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxConvTaps; ++j)
    if (j < K) acc = fmaf(w[j], x[j], acc);
  return pro_silu(acc);
}

// The same sum with NT taps held in registers: NT == kMaxConvTaps takes the
// run-time K (<= NT), any other NT is the tap count itself.
template <int NT>
__device__ __forceinline__ float pro_conv_silu_n(const float* w, const float* x, int K) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NT; ++j)
    if (NT != kMaxConvTaps || j < K) acc = fmaf(w[j], x[j], acc);
  return pro_silu(acc);
}

// Scale of a q/k head from the sum of squares of its Dk conv outputs.
__device__ __forceinline__ float pro_head_scale(float ss, int Dk, float eps, float scale) {
  return rsqrtf(ss / (float)Dk + eps) * scale;
}

// Per-token decay of a value head.
__device__ __forceinline__ float pro_decay(float A_log, float a, float dt_bias) {
  return __expf(-__expf(A_log) * pro_softplus(a + dt_bias));
}

}  // namespace dflash
