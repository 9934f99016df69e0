// Prologue and epilogue of a gated-delta layer around the verify scan.
//
// Reference layer body (dflash_mlx/custom_qwen35_model.py:409-484):
//   conv_input = concat(conv_state, qkv)              (:431-433)
//   new_conv_state = conv_input[:, -(K-1):]            (:434)
//   conv_out = silu(depthwise conv1d(conv_input))      (:435; weight [C, K, 1], :718-725)
//   q, k, v = split(conv_out) per head                 (:437-444)
//   q = Dk^-1 * rms_norm(q, eps=1e-6); k = Dk^-0.5 * rms_norm(k)   (:446-448)
//   beta = sigmoid(b); g = compute_g(A_log, a, dt_bias)            (:449-450)
//   ... scan ...
//   out = RMSNormGated(out, z)                         (:478)
// compute_g and RMSNormGated live in the un-vendored mlx-lm 0.31.2; they are
// the published Qwen3-Next forms: g = exp(-exp(A_log) * softplus(a + dt_bias))
// and y = weight * rms_norm(x) * silu(z).
//
// Both kernels are small and HBM/launch-bound; all arithmetic is fp32 and
// only the outputs are rounded (q/k/v to bf16, the scan's input type).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash_gdn.h"
#include "device_common.h"
#include "gdn_prologue_math.h"
#include "host_common.h"

namespace dflash {
namespace {

struct ProParams {
  const uint16_t* qkv;  // [B, T, C] bf16, C contiguous
  int64_t qkv_sb, qkv_st;
  const uint16_t* conv_state;  // [B, K1, C] bf16 contiguous
  const uint16_t* conv_w;      // [C, K] bf16 (the MLX [C, K, 1] layout)
  const uint16_t* a;           // [B, T, Hv] bf16
  const uint16_t* b;           // [B, T, Hv] bf16
  int64_t a_sb, a_st, b_sb, b_st;
  const float* A_log;       // [Hv] fp32
  const uint16_t* dt_bias;  // [Hv] bf16
  uint16_t* act;            // [B, T, C] bf16: q | k (normalised, scaled) | v
  float* g;                 // [B, T, Hv]
  float* beta;              // [B, T, Hv]
  uint16_t* new_conv_state; // [B, K1, C]
  int T, C, K, Hk, Hv, Dk;
  float eps, q_scale, k_scale;
};

__device__ __forceinline__ float ldbf(const uint16_t* p) { return bf16_bits_to_f32(*p); }

// silu(conv1d) of NC consecutive channels c0 .. c0+NC-1 at token t of
// sequence b.  All K taps of every channel are loaded before any is used.
template <int NC>
__device__ __forceinline__ void conv_silu(const ProParams& p, int b, int t, int c0, float* out) {
  const int K1 = p.K - 1;
  float x[kMaxConvTaps][NC];
  float w[NC][kMaxConvTaps];
#pragma unroll
  for (int j = 0; j < kMaxConvTaps; ++j) {
    if (j < p.K) {
      const int s = t + j;  // row of concat(conv_state, qkv)
      const uint16_t* src = s < K1 ? p.conv_state + ((int64_t)b * K1 + s) * p.C + c0
                                   : p.qkv + b * p.qkv_sb + (int64_t)(s - K1) * p.qkv_st + c0;
#pragma unroll
      for (int i = 0; i < NC; ++i) x[j][i] = ldbf(src + i);
    }
  }
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int j = 0; j < kMaxConvTaps; ++j)
      if (j < p.K) w[i][j] = ldbf(p.conv_w + (int64_t)(c0 + i) * p.K + j);
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float xi[kMaxConvTaps];
#pragma unroll
    for (int j = 0; j < kMaxConvTaps; ++j) xi[j] = x[j][i];
    out[i] = pro_conv_silu(w[i], xi, p.K);
  }
}

// Work units of one (sequence, token): 2*Hk q/k heads (one wavefront each,
// with the head's rms-norm), then value chunks of 256 channels (one
// wavefront each, 4 channels per lane), then one unit for g / beta and the
// new conv window.  grid: (B*T, ceil(units / 4)), 256 threads.
template <int PER>  // Dk / 64 channels per lane
__global__ __launch_bounds__(256) void gdn_prologue_kernel(const ProParams p) {
  const int bt = blockIdx.x;
  const int b = bt / p.T;
  const int t = bt - b * p.T;
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int n_qk = 2 * p.Hk;
  const int v0 = 2 * p.Hk * p.Dk;
  const int n_v = (p.C - v0 + 255) / 256;
  uint16_t* act = p.act + (int64_t)bt * p.C;

  if (unit < n_qk) {
    // q heads first, then k heads (the split order); lane owns PER channels.
    const int c0 = unit * p.Dk + lane * PER;
    float vals[PER];
    conv_silu<PER>(p, b, t, c0, vals);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) ss = fmaf(vals[i], vals[i], ss);
    ss = pro_wave_sum(ss);
    const float r = pro_head_scale(ss, p.Dk, p.eps, unit < p.Hk ? p.q_scale : p.k_scale);
#pragma unroll
    for (int i = 0; i < PER; ++i) act[c0 + i] = f32_to_bf16_rne(vals[i] * r);
  } else if (unit < n_qk + n_v) {
    const int c0 = v0 + (unit - n_qk) * 256 + lane * 4;
    if (c0 + 4 <= p.C) {
      float vals[4];
      conv_silu<4>(p, b, t, c0, vals);
#pragma unroll
      for (int i = 0; i < 4; ++i) act[c0 + i] = f32_to_bf16_rne(vals[i]);
    } else {
      for (int c = c0; c < p.C; ++c) {
        float v1[1];
        conv_silu<1>(p, b, t, c, v1);
        act[c] = f32_to_bf16_rne(v1[0]);
      }
    }
  } else if (unit == n_qk + n_v) {
    // Per-head decay and write strength.
    for (int h = lane; h < p.Hv; h += 64) {
      const float av = ldbf(p.a + b * p.a_sb + (int64_t)t * p.a_st + h);
      const float bv = ldbf(p.b + b * p.b_sb + (int64_t)t * p.b_st + h);
      p.g[(int64_t)bt * p.Hv + h] = pro_decay(p.A_log[h], av, ldbf(p.dt_bias + h));
      p.beta[(int64_t)bt * p.Hv + h] = pro_sigmoid(bv);
    }
  } else {
    // New conv window = the last K-1 rows of concat(conv_state, qkv): row r
    // is stream row T + r.  Token t writes the rows that are qkv[t]; token 0
    // also writes rows still coming from the old state (when T < K-1).  This
    // unit copies channels [c0, c0 + 512) of those rows, 8 per lane.
    const int c0 = (unit - n_qk - n_v - 1) * 512 + lane * 8;
    const int K1 = p.K - 1;
    for (int r = 0; r < K1; ++r) {
      const int s = p.T + r;
      const bool mine = (s >= K1) ? (s - K1 == t) : (t == 0);
      if (!mine) continue;
      uint16_t* dst = p.new_conv_state + ((int64_t)b * K1 + r) * p.C;
      const uint16_t* src = s >= K1 ? p.qkv + b * p.qkv_sb + (int64_t)(s - K1) * p.qkv_st
                                    : p.conv_state + ((int64_t)b * K1 + s) * p.C;
      uint16_t tmp[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < p.C) tmp[i] = src[c0 + i];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < p.C) dst[c0 + i] = tmp[i];
    }
  }
}

// The same prologue for long inputs (a prompt pass): a workgroup covers a
// tile of kPTile consecutive tokens of one sequence, and a wavefront owns a
// unit's channels for the whole tile.  Its lanes load the tile's kPTile + K-1
// stream rows of their channels once (every load issued before any use), so
// the conv window slides in registers instead of every token re-reading its
// K taps; the per-token arithmetic (tap order, silu, the head's butterfly sum
// and scale) is the per-token kernel's, so the outputs are the same bits.
// Units as there: 2*Hk q/k heads, value chunks of 256 channels, one unit for
// g / beta of the tile's tokens, then 512-channel units of the new conv
// window (written by the tiles that hold its rows).
constexpr int kPTile = 16;
// Inputs longer than this many tokens take the tiled kernel.
constexpr int kPromptTokens = 32;

// x[r] = stream row t0 + r of concat(conv_state, qkv) for r < kPTile + NT - 1
// (rows past the input's last one are clamped to it and never used).
template <int NC, int NT>
__device__ __forceinline__ void load_tile_rows(const ProParams& p, int b, int t0, int c0,
                                               float (&x)[kPTile + NT - 1][NC]) {
  const int K1 = p.K - 1;
#pragma unroll
  for (int r = 0; r < kPTile + NT - 1; ++r) {
    const int s = min(t0 + r, p.T + K1 - 1);
    const uint16_t* src = s < K1 ? p.conv_state + ((int64_t)b * K1 + s) * p.C + c0
                                 : p.qkv + b * p.qkv_sb + (int64_t)(s - K1) * p.qkv_st + c0;
    if constexpr (NC == 2) {  // one 4-byte load (c0 even; rows 4-byte aligned)
      const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
      x[r][0] = bf16_lo(w);
      x[r][1] = bf16_hi(w);
    } else if constexpr (NC == 4) {  // one 8-byte load (c0 % 4 == 0; rows 8-byte aligned)
      const uint2 w = *reinterpret_cast<const uint2*>(src);
      x[r][0] = bf16_lo(w.x);
      x[r][1] = bf16_hi(w.x);
      x[r][2] = bf16_lo(w.y);
      x[r][3] = bf16_hi(w.y);
    } else {
#pragma unroll
      for (int i = 0; i < NC; ++i) x[r][i] = ldbf(src + i);
    }
  }
}

// NC consecutive bf16 outputs of one token in one store.
template <int NC>
__device__ __forceinline__ void store_run(uint16_t* dst, const float* v) {
  if constexpr (NC == 2) {
    *reinterpret_cast<uint32_t*>(dst) =
        (uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16);
  } else if constexpr (NC == 4) {
    *reinterpret_cast<uint2*>(dst) =
        uint2{(uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
              (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16)};
  } else {
#pragma unroll
    for (int i = 0; i < NC; ++i) dst[i] = f32_to_bf16_rne(v[i]);
  }
}

// silu(conv1d) of NC channels at tile token t from the tile's rows; taps in
// the order of pro_conv_silu (the per-token kernel's).
template <int NC, int NT>
__device__ __forceinline__ void tile_conv_silu(const ProParams& p, int t,
                                               const float (&x)[kPTile + NT - 1][NC],
                                               const float (&w)[NC][NT], float* out) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    float xi[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) xi[j] = x[t + j][i];
    out[i] = pro_conv_silu_n<NT>(w[i], xi, p.K);
  }
}

template <int NC, int NT>
__device__ __forceinline__ void load_taps(const ProParams& p, int c0, float (&w)[NC][NT]) {
#pragma unroll
  for (int i = 0; i < NC; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
      w[i][j] = (NT != kMaxConvTaps || j < p.K) ? ldbf(p.conv_w + (int64_t)(c0 + i) * p.K + j) : 0.f;
}

// NT: the tap count held in registers (K itself, or kMaxConvTaps for any K).
template <int PER, int NT>
__global__ __launch_bounds__(256) void gdn_prologue_tile_kernel(const ProParams p) {
  const int tiles = (p.T + kPTile - 1) / kPTile;
  const int b = blockIdx.x / tiles;
  const int t0 = (blockIdx.x - b * tiles) * kPTile;
  const int nt = min(kPTile, p.T - t0);
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int n_qk = 2 * p.Hk;
  const int v0 = 2 * p.Hk * p.Dk;
  const int n_v = (p.C - v0 + 255) / 256;
  uint16_t* act = p.act + ((int64_t)b * p.T + t0) * p.C;

  if (unit < n_qk) {
    const int c0 = unit * p.Dk + lane * PER;
    float x[kPTile + NT - 1][PER];
    load_tile_rows<PER, NT>(p, b, t0, c0, x);
    float w[PER][NT];
    load_taps<PER, NT>(p, c0, w);
    const float scale = unit < p.Hk ? p.q_scale : p.k_scale;
    // Every token of the tile is computed (the rows past the input are
    // clamped copies) and only the stores are guarded: a loop that stops at
    // the run-time tile length would not unroll, and the row array would be
    // indexed at run time, out of registers.
#pragma unroll
    for (int t = 0; t < kPTile; ++t) {
      float vals[PER];
      tile_conv_silu<PER, NT>(p, t, x, w, vals);
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < PER; ++i) ss = fmaf(vals[i], vals[i], ss);
      ss = pro_wave_sum(ss);
      const float r = pro_head_scale(ss, p.Dk, p.eps, scale);
      float o[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i) o[i] = vals[i] * r;
      if (t < nt) store_run<PER>(act + (int64_t)t * p.C + c0, o);
    }
  } else if (unit < n_qk + n_v) {
    const int c0 = v0 + (unit - n_qk) * 256 + lane * 4;
    if (c0 + 4 <= p.C) {
      float x[kPTile + NT - 1][4];
      load_tile_rows<4, NT>(p, b, t0, c0, x);
      float w[4][NT];
      load_taps<4, NT>(p, c0, w);
#pragma unroll
      for (int t = 0; t < kPTile; ++t) {
        float vals[4];
        tile_conv_silu<4, NT>(p, t, x, w, vals);
        if (t < nt) store_run<4>(act + (int64_t)t * p.C + c0, vals);
      }
    } else {
      for (int t = 0; t < nt; ++t)
        for (int c = c0; c < p.C; ++c) {
          float v1[1];
          conv_silu<1>(p, b, t0 + t, c, v1);
          act[(int64_t)t * p.C + c] = f32_to_bf16_rne(v1[0]);
        }
    }
  } else if (unit == n_qk + n_v) {
    for (int e = lane; e < nt * p.Hv; e += 64) {
      const int t = t0 + e / p.Hv, h = e % p.Hv;
      const float av = ldbf(p.a + b * p.a_sb + (int64_t)t * p.a_st + h);
      const float bv = ldbf(p.b + b * p.b_sb + (int64_t)t * p.b_st + h);
      const int64_t bt = (int64_t)b * p.T + t;
      p.g[bt * p.Hv + h] = pro_decay(p.A_log[h], av, ldbf(p.dt_bias + h));
      p.beta[bt * p.Hv + h] = pro_sigmoid(bv);
    }
  } else {
    // New conv window row r is stream row T + r, i.e. qkv[T - K1 + r] (the
    // tile path runs only when T >= K - 1): the tile holding that token
    // copies it.
    const int c0 = (unit - n_qk - n_v - 1) * 512 + lane * 8;
    const int K1 = p.K - 1;
    for (int r = 0; r < K1; ++r) {
      const int t = p.T - K1 + r;
      if (t < t0 || t >= t0 + nt) continue;
      uint16_t* dst = p.new_conv_state + ((int64_t)b * K1 + r) * p.C;
      const uint16_t* src = p.qkv + b * p.qkv_sb + (int64_t)t * p.qkv_st;
      uint16_t tmp[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < p.C) tmp[i] = src[c0 + i];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (c0 + i < p.C) dst[c0 + i] = tmp[i];
    }
  }
}

struct NormParams {
  const uint16_t* x;  // [rows, D] bf16 contiguous (scan out [B,T,Hv,Dv])
  const uint16_t* z;  // gate, [B, T, Hv, D] with strides
  int64_t z_sb, z_st, z_sh;
  const uint16_t* w;  // [D] bf16
  uint16_t* y;        // [rows, D] bf16
  int T, H, D, rows;
  float eps;
};

// One wavefront per (b, t, h) row of D = 64 * PER channels; 4 rows per
// workgroup.  Lane l holds channels l, l + 64, ...; its x, z and weight loads
// all go out before the row's sum of squares (one round of memory latency in
// a kernel that is nothing but latency at verify sizes).
template <int PER>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const NormParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int h = row % p.H;
  const int bt = row / p.H;
  const int t = bt % p.T;
  const int b = bt / p.T;
  const uint16_t* x = p.x + (int64_t)row * p.D;
  const uint16_t* z = p.z + b * p.z_sb + (int64_t)t * p.z_st + (int64_t)h * p.z_sh;
  float xv[PER], zv[PER], wv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    xv[i] = ldbf(x + i * 64 + lane);
    zv[i] = ldbf(z + i * 64 + lane);
    wv[i] = ldbf(p.w + i * 64 + lane);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) ss = fmaf(xv[i], xv[i], ss);
  ss = pro_wave_sum(ss);
  const float r = rsqrtf(ss / (float)p.D + p.eps);
#pragma unroll
  for (int i = 0; i < PER; ++i)
    p.y[(int64_t)row * p.D + i * 64 + lane] = f32_to_bf16_rne(xv[i] * r * wv[i] * pro_silu(zv[i]));
}

// The same norm with 16-byte accesses, for prompt-sized launches whose rows
// and gates start 16-byte aligned: L = D / 8 lanes a row (lane j of a row holds channels
// 8j .. 8j+7 of x, z and the weight), 64 / L rows a wavefront, 4 wavefronts
// a workgroup.  One load instruction moves 1 KB instead of 128 B, which is
// what bounds the norm over a prompt's thousands of rows.
template <int L>
__global__ __launch_bounds__(256) void gated_rmsnorm_vec_kernel(const NormParams p) {
  constexpr int RW = 64 / L;
  const int lane = threadIdx.x & 63;
  const int j = lane % L;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RW + lane / L;
  const bool live = row0 < p.rows;
  const int row = live ? row0 : p.rows - 1;  // idle row slots redo the last row, unstored
  const int h = row % p.H;
  const int bt = row / p.H;
  const int t = bt % p.T;
  const int b = bt / p.T;
  const uint16_t* x = p.x + (int64_t)row * p.D + 8 * j;
  const uint16_t* z = p.z + b * p.z_sb + (int64_t)t * p.z_st + (int64_t)h * p.z_sh + 8 * j;
  const u32x4 xr = *reinterpret_cast<const u32x4*>(x);
  const u32x4 zr = *reinterpret_cast<const u32x4*>(z);
  const u32x4 wr = *reinterpret_cast<const u32x4*>(p.w + 8 * j);
  float xv[8], zv[8], wv[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xv[2 * i] = bf16_bits_to_f32(xr[i] & 0xffffu);
    xv[2 * i + 1] = bf16_bits_to_f32(xr[i] >> 16);
    zv[2 * i] = bf16_bits_to_f32(zr[i] & 0xffffu);
    zv[2 * i + 1] = bf16_bits_to_f32(zr[i] >> 16);
    wv[2 * i] = bf16_bits_to_f32(wr[i] & 0xffffu);
    wv[2 * i + 1] = bf16_bits_to_f32(wr[i] >> 16);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(xv[i], xv[i], ss);
#pragma unroll
  for (int o = L / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);  // the row's L lanes
  const float r = rsqrtf(ss / (float)p.D + p.eps);
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    out[i] = (uint32_t)f32_to_bf16_rne(xv[2 * i] * r * wv[2 * i] * pro_silu(zv[2 * i])) |
             ((uint32_t)f32_to_bf16_rne(xv[2 * i + 1] * r * wv[2 * i + 1] *
                                        pro_silu(zv[2 * i + 1])) << 16);
  if (live) *reinterpret_cast<u32x4*>(p.y + (int64_t)row * p.D + 8 * j) = out;
}

}  // namespace
}  // namespace dflash

extern "C" int dflash_gdn_prologue(const void* qkv, int64_t qkv_batch_stride,
                                   int64_t qkv_row_stride, const void* conv_state,
                                   const void* conv_weight, const void* a, const void* b,
                                   const int64_t* ab_strides, const float* A_log,
                                   const void* dt_bias, void* act, float* g, float* beta,
                                   void* new_conv_state, int B, int T, int K, int Hk, int Hv,
                                   int Dk, int Dv, float eps, void* stream) {
  using namespace dflash;
  if (B < 0 || T < 0 || K < 1 || K > kMaxConvTaps || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0)
    return DFLASH_ERR_SHAPE;
  if (Hv % Hk != 0) return DFLASH_ERR_SHAPE;
  if (Dk % 64 != 0 || Dk > 256) return DFLASH_ERR_UNSUPPORTED;
  // grid.x = B * T; channel indices are int
  if ((int64_t)B * T > INT32_MAX || 2LL * Hk * Dk + (int64_t)Hv * Dv > INT32_MAX)
    return DFLASH_ERR_SHAPE;
  if (B == 0 || T == 0) return DFLASH_OK;
  if (qkv == nullptr || (K > 1 && conv_state == nullptr) || conv_weight == nullptr ||
      a == nullptr || b == nullptr || A_log == nullptr || dt_bias == nullptr || act == nullptr ||
      g == nullptr || beta == nullptr || (K > 1 && new_conv_state == nullptr))
    return DFLASH_ERR_NULL;
  if (K > 1 && new_conv_state == conv_state) return DFLASH_ERR_SHAPE;  // see the header
  if (((uintptr_t)qkv | (uintptr_t)conv_state | (uintptr_t)conv_weight | (uintptr_t)a |
       (uintptr_t)b | (uintptr_t)dt_bias | (uintptr_t)act | (uintptr_t)new_conv_state) & 1)
    return DFLASH_ERR_ALIGN;
  ProParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_sb = qkv_batch_stride;
  p.qkv_st = qkv_row_stride;
  p.conv_state = static_cast<const uint16_t*>(conv_state);
  p.conv_w = static_cast<const uint16_t*>(conv_weight);
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  const int64_t C = 2LL * Hk * Dk + (int64_t)Hv * Dv;
  if (ab_strides != nullptr) {
    p.a_sb = ab_strides[0]; p.a_st = ab_strides[1]; p.b_sb = ab_strides[2]; p.b_st = ab_strides[3];
  } else {
    p.a_st = p.b_st = Hv;
    p.a_sb = p.b_sb = (int64_t)T * Hv;
  }
  p.A_log = A_log;
  p.dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.act = static_cast<uint16_t*>(act);
  p.g = g;
  p.beta = beta;
  p.new_conv_state = static_cast<uint16_t*>(new_conv_state);
  p.T = T;
  p.C = (int)C;
  p.K = K;
  p.Hk = Hk;
  p.Hv = Hv;
  p.Dk = Dk;
  p.eps = eps;
  p.k_scale = 1.0f / sqrtf((float)Dk);
  p.q_scale = p.k_scale * p.k_scale;
  const int64_t units = 2LL * Hk + ceil_div(C - 2LL * Hk * Dk, 256) + 1 + ceil_div(C, 512);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the tiled kernel's 4- and 8-byte row accesses: qkv, the conv window and
  // act 8-byte aligned, row and batch strides and C multiples of 4 elements
  const bool vec_ok =
      !(((uintptr_t)qkv | (uintptr_t)conv_state | (uintptr_t)act) & 7) &&
      qkv_row_stride % 4 == 0 && qkv_batch_stride % 4 == 0 && C % 4 == 0;
  if (T > kPromptTokens && Dk == 128 && vec_ok) {
    // a prompt: token tiles, each stream row read once (same bits)
    const dim3 tgrid((unsigned)(B * ceil_div(T, kPTile)), (unsigned)ceil_div(units, 4));
    if (K == 4)
      hipLaunchKernelGGL((gdn_prologue_tile_kernel<2, 4>), tgrid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((gdn_prologue_tile_kernel<2, kMaxConvTaps>), tgrid, dim3(256), 0, s, p);
    return to_status(hipGetLastError());
  }
  const dim3 grid(B * T, (unsigned)ceil_div(units, 4));
  switch (Dk / 64) {
    case 1: hipLaunchKernelGGL(gdn_prologue_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(gdn_prologue_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 3: hipLaunchKernelGGL(gdn_prologue_kernel<3>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(gdn_prologue_kernel<4>, grid, dim3(256), 0, s, p); break;
  }
  return to_status(hipGetLastError());
}

extern "C" int dflash_gdn_gated_rmsnorm(const void* x, const void* z, const int64_t* z_strides,
                                        const void* weight, void* y, int B, int T, int H, int D,
                                        float eps, void* stream) {
  using namespace dflash;
  if (B < 0 || T < 0 || H <= 0 || D <= 0) return DFLASH_ERR_SHAPE;
  if (D % 64 != 0 || D > 256) return DFLASH_ERR_UNSUPPORTED;
  if ((int64_t)B * T * H > INT32_MAX) return DFLASH_ERR_SHAPE;  // rows are int
  if (B == 0 || T == 0) return DFLASH_OK;
  if (x == nullptr || z == nullptr || weight == nullptr || y == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x | (uintptr_t)z | (uintptr_t)weight | (uintptr_t)y) & 1) return DFLASH_ERR_ALIGN;
  NormParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.z = static_cast<const uint16_t*>(z);
  if (z_strides != nullptr) {
    p.z_sb = z_strides[0]; p.z_st = z_strides[1]; p.z_sh = z_strides[2];
  } else {
    p.z_sh = D; p.z_st = (int64_t)H * D; p.z_sb = (int64_t)T * H * D;
  }
  p.w = static_cast<const uint16_t*>(weight);
  p.y = static_cast<uint16_t*>(y);
  p.T = T;
  p.H = H;
  p.D = D;
  p.rows = B * T * H;
  p.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 16-byte accesses over a prompt's rows when every row and gate start
  // allows them (D % 64 == 0 already makes the row a multiple of 8
  // channels).  At verify sizes (hundreds of rows) the one-wave-a-row form
  // is faster: it spreads the same rows over 4x-8x the workgroups, and
  // latency, not instructions, bounds it there.
  const bool vec = p.rows >= 4096 &&
                   ((((uintptr_t)x | (uintptr_t)z | (uintptr_t)weight | (uintptr_t)y) & 15) == 0) &&
                   p.z_sb % 8 == 0 && p.z_st % 8 == 0 && p.z_sh % 8 == 0;
  if (vec) {
    const int L = D / 8;  // 8, 16, 24 or 32 lanes a row
    if (L == 8 || L == 16 || L == 32) {
      const dim3 vgrid((unsigned)ceil_div(p.rows, 4 * (64 / L)));
      if (L == 8) hipLaunchKernelGGL(gated_rmsnorm_vec_kernel<8>, vgrid, dim3(256), 0, s, p);
      else if (L == 16) hipLaunchKernelGGL(gated_rmsnorm_vec_kernel<16>, vgrid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL(gated_rmsnorm_vec_kernel<32>, vgrid, dim3(256), 0, s, p);
      return to_status(hipGetLastError());
    }
  }
  const dim3 grid((unsigned)ceil_div(p.rows, 4));
  switch (D / 64) {
    case 1: hipLaunchKernelGGL(gated_rmsnorm_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL(gated_rmsnorm_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 3: hipLaunchKernelGGL(gated_rmsnorm_kernel<3>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(gated_rmsnorm_kernel<4>, grid, dim3(256), 0, s, p); break;
  }
  return to_status(hipGetLastError());
}
