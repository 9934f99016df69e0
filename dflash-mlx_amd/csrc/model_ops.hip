// The non-GEMM operators of the Qwen3.5 hybrid target's verify step on gfx950.
//
// Around the gated-delta layers (gdn_layer_ops.hip, gdn_scan.hip) the
// reference's target model (DecoderLayer, dflash_mlx/custom_qwen35_model.py:
// 815-846; Qwen3_5TextModel.__call__ :860-881) runs, per decoder layer:
//   residual add + RMSNorm (nn.RMSNorm input/post-attention layernorms,
//   :824-827, applied :841-845; final norm :881), the MLP silu(gate) * up
//   (mlx-lm Qwen3NextMLP, :845),
//   and on every 4th layer the gated full attention of
//   forward_full_attention_layer_explicit (:487-540): q/k RMSNorm, partial
//   rotary embedding at the cache offset, KV-cache append, causal SDPA over the
//   cache, output * sigmoid(gate).
// The projections are this package's GEMMs (skinny_gemm.hip at verify
// sizes, prefill_gemm.hip over a prompt) and stay with the caller.  Cache
// lengths live in device memory, so a whole verify step (append, attend,
// accept, commit) runs without a host round trip.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <stdint.h>

#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

__device__ __forceinline__ void unpack8(u32x4 w, float* f) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  return u32x4{pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7])};
}

__device__ __forceinline__ float bf16_round(float x) { return bf16_bits_to_f32(f32_to_bf16_rne(x)); }

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Max over the 16 lanes of one DPP row; every lane of the row gets it.
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_mov<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp_mov<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp_mov<kDppRowHalfMirror>(x));
  x = fmaxf(x, dpp_mov<kDppRowMirror>(x));
  return x;
}

__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }

// ------------------------------------------------------------ add + RMSNorm
// h = bf16(x + r) (the residual stream, stored to h_out), y = bf16(h *
// rsqrt(mean(h^2) + eps) * w), fp32 arithmetic.  The branch r is either bf16
// [M, H] or (PART) the fp32 split-K partial sums of the projection that
// produced it, rp[nsplit][M][H], rounded to bf16 after the sum (where the
// projection's own output would be rounded).  One workgroup per row (verify
// steps have only B*T rows) of one thread per 8-element chunk (H / 8 threads,
// up to 1024): every thread issues all of its loads (x, and every split of
// r: NS of them, a compile-time count for the common split factors) before
// using any, so a row costs one memory round trip.  With tok != nullptr, x
// is the embedding table and row m reads table row tok[m] (clamped to
// [0, vocab)), stored to h_out as the residual stream's start.  With hc !=
// nullptr, h is also stored to row m of hc (row stride hc_stride elements):
// the target hidden state a drafter reads at selected layers.
template <bool PART, int NS>
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(const uint16_t* x, const int32_t* tok,
                                                           int vocab, const uint16_t* r,
                                                           const float* rp, int nsplit,
                                                           const uint16_t* w, uint16_t* h_out,
                                                           uint16_t* hc, int64_t hc_stride,
                                                           uint16_t* y, int M, int H, float eps) {
  __shared__ float wsum[16];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int ch = tid;
  const bool live = ch < (H >> 3);
  const int chc = live ? ch : 0;  // idle threads load chunk 0 and drop it
  const int64_t xrow = tok != nullptr ? (int64_t)min(max(tok[row], 0), vocab - 1) : row;
  const u32x4 wraw = ld16(w + chc * 8);  // the norm weight, up front with the row's loads
  float v[8];
  unpack8(ld16(x + xrow * H + chc * 8), v);
  if (PART) {
    const float* src = rp + (int64_t)row * H + chc * 8;
    const int64_t sstride = (int64_t)M * H;
    f32x4 p0[NS > 0 ? NS : 1], p1[NS > 0 ? NS : 1];
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    if (NS > 0) {
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        p0[k] = *reinterpret_cast<const f32x4*>(src + k * sstride);
        p1[k] = *reinterpret_cast<const f32x4*>(src + k * sstride + 4);
      }
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        s0 += p0[k];
        s1 += p1[k];
      }
    } else {
#pragma unroll 8
      for (int k = 0; k < nsplit; ++k) {
        s0 += *reinterpret_cast<const f32x4*>(src + k * sstride);
        s1 += *reinterpret_cast<const f32x4*>(src + k * sstride + 4);
      }
    }
    const float rv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bf16_round(v[e] + bf16_round(rv[e]));
  } else if (r != nullptr) {
    float rv[8];
    unpack8(ld16(r + (int64_t)row * H + chc * 8), rv);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bf16_round(v[e] + rv[e]);
  }
  float ss = 0.f;
  if (live) {
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) wsum[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += wsum[i];
  const float inv = 1.f / sqrtf(tot / (float)H + eps);
  if (live) {
    if ((PART || r != nullptr || tok != nullptr) && h_out != nullptr)
      *reinterpret_cast<u32x4*>(h_out + (int64_t)row * H + ch * 8) = pack8(v);
    if (hc != nullptr) *reinterpret_cast<u32x4*>(hc + (int64_t)row * hc_stride + ch * 8) = pack8(v);
    float wv[8], o[8];
    unpack8(wraw, wv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = v[e] * inv * wv[e];
    *reinterpret_cast<u32x4*>(y + (int64_t)row * H + ch * 8) = pack8(o);
  }
}

// ------------------------------------------------------------------ SwiGLU
// out[m][i] = bf16(silu(gu[m][i]) * gu[m][I + i]).
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* gu, uint16_t* out, int M,
                                                     int I) {
  const int per_row = I >> 3;
  const int64_t n = (int64_t)M * per_row;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int m = (int)(e / per_row);
    const int c = (int)(e - (int64_t)m * per_row);
    const uint16_t* row = gu + (int64_t)m * 2 * I;
    float g[8], u[8], o[8];
    unpack8(ld16(row + c * 8), g);
    unpack8(ld16(row + I + c * 8), u);
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = silu(g[k]) * u[k];
    *reinterpret_cast<u32x4*>(out + (int64_t)m * I + c * 8) = pack8(o);
  }
}

// ------------------------------------------------------- attention: prepare
// One wave per (token, head slot); D = 128, lane l holds features 2l, 2l+1.
// Slots [0, Hq): query heads (RMSNorm with q_norm_w, rotary, -> q_out);
// [Hq, Hq+Hkv): key heads (RMSNorm with k_norm_w, rotary, -> K cache row);
// [Hq+Hkv, Hq+2Hkv): value heads (-> V^T cache column).  Position of token t
// of sequence b: lens[b] + t.  Rotary (non-interleaved, first `rot` features):
// feature i < rot/2 pairs with i + rot/2 at angle pos * base^(-2i/rot).
struct AttnPrepParams {
  const uint16_t* proj;  // [B*T, row_stride]: Hq x (q | gate) of D each, then Hkv x k, Hkv x v
  int64_t row_stride;
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  const int32_t* lens;
  uint16_t* k_cache;   // [B, Hkv, Smax, D]
  uint16_t* vt_cache;  // [B, Hkv, D, Smax]
  uint16_t* q_out;     // [B, T, Hq, D]
  int32_t* overflow;   // [B] or null: set to 1 when a block position falls outside [0, Smax)
  int B, T, Hq, Hkv, Smax, rot;
  int skip_v;          // value heads left to attn_prep_vt_kernel
  double log2_base;
  float eps;
};

constexpr int kHD = 128;  // attention head dim supported by these kernels

// pos * base^(-2i/rot) reduced to [0, 2*pi), computed in fp64.
__device__ __forceinline__ float rope_angle(int pos, int i, int rot, double log2_base) {
  const double inv_freq = exp2(-(double)(2 * i) / (double)rot * log2_base);
  const double a = (double)pos * inv_freq;
  const double two_pi = 6.283185307179586476925286766559;
  return (float)(a - two_pi * floor(a / two_pi));
}

__global__ __launch_bounds__(256) void attn_prep_kernel(const AttnPrepParams p) {
  const int bt = blockIdx.x;
  const int slot = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (slot >= p.Hq + 2 * p.Hkv) return;
  const int b = bt / p.T;
  const int t = bt - b * p.T;
  const int pos = p.lens[b] + t;
  // A position outside the cache is never written; the sequence's overflow
  // word records it so the host can refuse the step's output.
  const bool in_cache = pos >= 0 && pos < p.Smax;
  if (!in_cache && slot == 0 && lane == 0 && p.overflow != nullptr) p.overflow[b] = 1;
  const uint16_t* row = p.proj + (int64_t)bt * p.row_stride;
  const int d0 = 2 * lane;
  if (slot >= p.Hq + p.Hkv) {  // value head: V^T cache column
    if (p.skip_v) return;
    const int h = slot - p.Hq - p.Hkv;
    const uint32_t vv = *reinterpret_cast<const uint32_t*>(row + p.Hq * 2 * kHD + p.Hkv * kHD + h * kHD + d0);
    if (in_cache) {
      uint16_t* col = p.vt_cache + (((int64_t)b * p.Hkv + h) * kHD + d0) * p.Smax + pos;
      col[0] = (uint16_t)vv;
      col[p.Smax] = (uint16_t)(vv >> 16);
    }
    return;
  }
  const bool is_q = slot < p.Hq;
  const int h = is_q ? slot : slot - p.Hq;
  const uint16_t* src = is_q ? row + h * 2 * kHD : row + p.Hq * 2 * kHD + h * kHD;
  const uint32_t xv = *reinterpret_cast<const uint32_t*>(src + d0);
  const uint32_t wv = *reinterpret_cast<const uint32_t*>((is_q ? p.q_norm_w : p.k_norm_w) + d0);
  float x0 = bf16_lo(xv), x1 = bf16_hi(xv);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float inv = 1.f / sqrtf(ss / (float)kHD + p.eps);
  x0 = x0 * inv * bf16_lo(wv);
  x1 = x1 * inv * bf16_hi(wv);
  if (p.rot > 0) {
    const int half = p.rot >> 1;
    const float p0 = __shfl_xor(x0, p.rot >> 2, 64);
    const float p1 = __shfl_xor(x1, p.rot >> 2, 64);
    if (d0 < p.rot) {
      const bool lo_half = d0 < half;
      const int i0 = lo_half ? d0 : d0 - half;
      // Angles in fp64, reduced modulo 2*pi before the fp32 sincos: at
      // positions of several thousand an fp32 angle would carry ~1e-4 rad of
      // rounding.
      float s0, c0, s1, c1;
      sincosf(rope_angle(pos, i0, p.rot, p.log2_base), &s0, &c0);
      sincosf(rope_angle(pos, i0 + 1, p.rot, p.log2_base), &s1, &c1);
      if (lo_half) {
        x0 = x0 * c0 - p0 * s0;
        x1 = x1 * c1 - p1 * s1;
      } else {
        x0 = x0 * c0 + p0 * s0;
        x1 = x1 * c1 + p1 * s1;
      }
    }
  }
  const uint32_t packed = pack2(x0, x1);
  if (is_q) {
    *reinterpret_cast<uint32_t*>(p.q_out + ((int64_t)bt * p.Hq + h) * kHD + d0) = packed;
  } else if (in_cache) {
    *reinterpret_cast<uint32_t*>(p.k_cache + (((int64_t)b * p.Hkv + h) * p.Smax + pos) * kHD + d0) =
        packed;
  }
}

// The value heads of a long input (a prompt pass) into the transposed cache:
// workgroup (block of kVtTile tokens, value head h, sequence b).  Per token
// the value row is one 256-byte run of proj, but in vt_cache each of its 128
// features lands in another row (Smax positions apart), so one wave a token
// scatters 2-byte stores.  Here the block's rows go to LDS (16 bytes a
// thread) and each feature's kVtTile positions are then stored by
// consecutive lanes: one 128-byte run a store.  Positions outside
// [0, Smax) are not written (attn_prep_kernel's query head 0 records them
// in the overflow word).  The values are copied bit for bit.
constexpr int kVtTile = 64;

__global__ __launch_bounds__(256) void attn_prep_vt_kernel(const AttnPrepParams p) {
  __shared__ uint32_t sv[kVtTile][kHD / 2 + 1];  // a row of 128 bf16, 4 bytes of pad
  const int t0 = blockIdx.x * kVtTile, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int nt = min(kVtTile, p.T - t0);
  // piece e: token e / 16, features 8 (e % 16) .. +7
#pragma unroll
  for (int i = 0; i < kVtTile * kHD / 8 / 256; ++i) {
    const int e = tid + 256 * i;
    const int tk = e >> 4, c = e & 15;
    if (tk < nt) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(
          p.proj + ((int64_t)b * p.T + t0 + tk) * p.row_stride + p.Hq * 2 * kHD + p.Hkv * kHD +
          h * kHD + 8 * c);
#pragma unroll
      for (int w = 0; w < 4; ++w) sv[tk][4 * c + w] = v[w];
    }
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  const int pos = p.lens[b] + t0 + lane;
  if (lane >= nt || pos < 0 || pos >= p.Smax) return;
  uint16_t* col = p.vt_cache + ((int64_t)b * p.Hkv + h) * kHD * p.Smax + pos;
  for (int d = wave; d < kHD; d += 4) {
    const uint32_t pair = sv[lane][d >> 1];
    col[(int64_t)d * p.Smax] = (uint16_t)((d & 1) ? (pair >> 16) : pair);
  }
}

// ------------------------------------------------ attention: split-K partials
// Workgroup per (key split s, kv head h, sequence b), one wave per query head
// of the group (REP = Hq / Hkv waves).  Wave rows are the T <= 16 block
// tokens; keys are the split's KC = 64 cache positions.  The split's K rows
// (64 x 256 B) and V^T rows (128 x 128 B) are read once per workgroup, every
// thread loading its share of 16-byte pieces, into LDS (rows padded by 16 B
// against bank conflicts); each wave then reads its MFMA fragments from LDS.
// (With one global read per wave, the REP waves fetched the same 32 KB REP
// times: 12.9 us per call at the Qwen3.5-4B shape against 7.4 us staged.)
// S = Q K^T and O = P V on v_mfma_f32_16x16x32_bf16 (A lane = (row l%16,
// k 8(l/16)..+7), B lane = (col l%16, same k), D lane = (col l%16, rows
// 4(l/16)+e)).  Keys at or past lens[b] + T, and keys past lens[b] + t for
// row t (causal), get no weight.  Writes per (row, split): the running max
// m, the sum l of exp(S - m) and the unnormalised O.
constexpr int KC = 64;

struct AttnParams {
  const uint16_t* q;         // [B, T, Hq, D]
  const uint16_t* k_cache;   // [B, Hkv, Smax, D]
  const uint16_t* vt_cache;  // [B, Hkv, D, Smax]
  const int32_t* lens;
  const uint16_t* gate_src;  // proj rows: gate of head qh at qh*2D + D
  int64_t gate_row_stride;
  uint16_t* out;             // [B, T, Hq*D]
  float* part_o;             // [B, Hkv, nsplit, rep, 16, D]
  float* part_ml;            // [B, Hkv, nsplit, rep, 16, 2]
  int B, T, Hq, Hkv, Smax, nsplit;
  float scale;
};

template <int REP>
__global__ __launch_bounds__(256) void attn_partial_kernel(const AttnParams p) {
  constexpr int NT = 64 * REP;                      // threads
  constexpr int PIECES = KC * kHD * 2 / 16;         // 16-byte pieces of K (and of V^T)
  constexpr int PER = (PIECES + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t sK[KC][kHD + 8];
  __shared__ __attribute__((aligned(16))) uint16_t sV[kHD][KC + 8];
  __shared__ __attribute__((aligned(16))) uint16_t sP[REP][16][KC + 8];
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int qh = h * REP + wave;
  const int base_len = p.lens[b];
  const int L = base_len + p.T;
  const int k0 = s * KC;
  const int64_t prow = (((int64_t)b * p.Hkv + h) * p.nsplit + s) * REP + wave;  // x 16 rows
  if (k0 >= L) {  // split past the keys: no weight
    if (r16 == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p.part_ml[(prow * 16 + 4 * g4 + e) * 2] = -INFINITY;
        p.part_ml[(prow * 16 + 4 * g4 + e) * 2 + 1] = 0.f;
      }
    }
    return;
  }
  // The split's K and V^T, every piece's load issued before any is stored.
  const uint16_t* kbase = p.k_cache + (((int64_t)b * p.Hkv + h) * p.Smax + k0) * kHD;
  const uint16_t* vbase = p.vt_cache + ((int64_t)b * p.Hkv + h) * kHD * p.Smax + k0;
  u32x4 kv[PER], vv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = min(tid + NT * i, PIECES - 1);
    kv[i] = ld16(kbase + (int64_t)(e >> 4) * kHD + (e & 15) * 8);
    vv[i] = ld16(vbase + (int64_t)(e >> 3) * p.Smax + (e & 7) * 8);
  }
  // Q rows (block tokens), 4 k-steps of 32 features.
  const int tq = r16 < p.T ? r16 : p.T - 1;
  const uint16_t* qr = p.q + (((int64_t)b * p.T + tq) * p.Hq + qh) * kHD + g4 * 8;
  u32x4 qa[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 v = ld16(qr + 32 * k);
    qa[k] = r16 < p.T ? v : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid + NT * i;
    if (e < PIECES) {
      *reinterpret_cast<u32x4*>(&sK[e >> 4][(e & 15) * 8]) = kv[i];
      *reinterpret_cast<u32x4*>(&sV[e >> 3][(e & 7) * 8]) = vv[i];
    }
  }
  __syncthreads();
  // S tiles for the 4 groups of 16 keys.
  f32x4 sacc[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, qa[k]),
          __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&sK[16 * n + r16][32 * k + 8 * g4])),
          acc, 0, 0, 0);
    sacc[n] = acc;
  }
  // Masked, scaled scores; row max and sum over the split (row = 4 g4 + e,
  // spread over the 16 lanes of DPP row g4 and the 4 key groups).
  float sv[4][4];
  float m[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 4 * g4 + e;
    float mx = -INFINITY;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int key = k0 + 16 * n + r16;
      const bool ok = (t < p.T) && (key < L) && (key <= base_len + t);
      sv[n][e] = ok ? sacc[n][e] * p.scale : -INFINITY;
      mx = fmaxf(mx, sv[n][e]);
    }
    m[e] = row16_max(mx);
    const float ms = m[e] == -INFINITY ? 0.f : m[e];
    float sum = 0.f;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const float pe = __expf(sv[n][e] - ms);
      sv[n][e] = pe;
      sum += pe;
    }
    l[e] = row16_sum(sum);
  }
  // P (bf16) through LDS into A-operand order: rows t, keys contiguous.
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int n = 0; n < 4; ++n) sP[wave][4 * g4 + e][16 * n + r16] = f32_to_bf16_rne(sv[n][e]);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's P writes are visible to it
  u32x4 pa[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) pa[k] = *reinterpret_cast<const u32x4*>(&sP[wave][r16][32 * k + 8 * g4]);
  // O = P V over 8 tiles of 16 features; V^T rows hold the keys contiguously.
  float* po = p.part_o + prow * 16 * kHD;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 2; ++k)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
          __builtin_bit_cast(bf16x8, pa[k]),
          __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&sV[16 * dt + r16][32 * k + 8 * g4])),
          acc, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) po[(4 * g4 + e) * kHD + 16 * dt + r16] = acc[e];
  }
  if (r16 == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p.part_ml[(prow * 16 + 4 * g4 + e) * 2] = m[e];
      p.part_ml[(prow * 16 + 4 * g4 + e) * 2 + 1] = l[e];
    }
  }
}

// ------------------------------------------------- attention: combine + gate
// One workgroup per (token, query head): wave w merges the live splits
// s = w, w+4, ... (lane l holds features 2l, 2l+1), then the four partial
// (max, sum, O) merge through LDS; normalise, multiply by sigmoid(gate),
// write bf16.  Splits past lens[b] + T are never read.
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnParams p) {
  __shared__ float sm[4], sl[4];
  __shared__ f32x2 so[4][64];
  const int bt = blockIdx.x;
  const int qh = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int b = bt / p.T;
  const int t = bt - b * p.T;
  const int rep = p.Hq / p.Hkv;
  const int h = qh / rep, w = qh - h * rep;
  const int live = min(p.nsplit, (p.lens[b] + p.T + KC - 1) / KC);
  const int64_t prow0 = (((int64_t)b * p.Hkv + h) * p.nsplit) * rep + w;  // split 0
  // running merge over this wave's splits, 4 loads in flight per step
  float m = -INFINITY, l = 0.f, a0 = 0.f, a1 = 0.f;
  for (int s0 = wave; s0 < live; s0 += 16) {
    float ms[4], ls[4];
    f32x2 os[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = min(s0 + 4 * u, live - 1);
      const int64_t r = (prow0 + (int64_t)s * rep) * 16 + t;
      ms[u] = (s0 + 4 * u < live) ? p.part_ml[r * 2] : -INFINITY;
      ls[u] = p.part_ml[r * 2 + 1];
      os[u] = *reinterpret_cast<const f32x2*>(p.part_o + r * kHD + 2 * lane);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (ms[u] == -INFINITY) continue;  // no visible key in that split (wave-uniform)
      const float mn = fmaxf(m, ms[u]);
      const float ca = (m == -INFINITY) ? 0.f : __expf(m - mn);
      const float cb = __expf(ms[u] - mn);
      l = l * ca + ls[u] * cb;
      a0 = a0 * ca + os[u].x * cb;
      a1 = a1 * ca + os[u].y * cb;
      m = mn;
    }
  }
  if (lane == 0) {
    sm[wave] = m;
    sl[wave] = l;
  }
  so[wave][lane] = f32x2{a0, a1};
  __syncthreads();
  if (wave != 0) return;
  float mm = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; ++k) mm = fmaxf(mm, sm[k]);
  float lsum = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (sm[k] == -INFINITY) continue;
    const float c = __expf(sm[k] - mm);
    lsum = fmaf(sl[k], c, lsum);
    o0 = fmaf(so[k][lane].x, c, o0);
    o1 = fmaf(so[k][lane].y, c, o1);
  }
  const float inv = 1.f / lsum;
  const uint32_t gv = *reinterpret_cast<const uint32_t*>(
      p.gate_src + (int64_t)bt * p.gate_row_stride + qh * 2 * kHD + kHD + 2 * lane);
  const float g0 = 1.f / (1.f + __expf(-bf16_lo(gv)));
  const float g1 = 1.f / (1.f + __expf(-bf16_hi(gv)));
  *reinterpret_cast<uint32_t*>(p.out + ((int64_t)bt * p.Hq + qh) * kHD + 2 * lane) =
      pack2(o0 * inv * g0, o1 * inv * g1);
}

// ------------------------------------------------ attention over a prompt
// The same causal SDPA + gate for the P rows of a prompt pass (one sequence,
// cache length lens[0] before the prompt; prompt row i sees keys 0 ..
// lens[0] + i).  One workgroup per (16-row query block, kv head), one wave
// per query head of the group, as the verify kernel; instead of one key
// split per workgroup, the workgroup walks every 64-key tile its block can
// see, keeping a running max m, sum l and unnormalised O per row in
// registers (rescaled by exp(m_old - m_new) when the max grows), so nothing
// goes through a workspace.  Each tile's K and V^T are loaded once per
// workgroup into LDS (the next tile's loads issued before this tile's
// products), shared by the REP waves.  Query blocks are launched last block
// first: later blocks see more keys and set the launch's end.
struct AttnPrefillParams {
  const uint16_t* q;         // [P, Hq, D]
  const uint16_t* k_cache;   // [Hkv, Smax, D]
  const uint16_t* vt_cache;  // [Hkv, D, Smax]
  const int32_t* lens;       // [1]
  const uint16_t* gate_src;  // prompt row i's gate of head qh at i*gate_row_stride + qh*2D + D
  int64_t gate_row_stride;
  uint16_t* out;             // [P, Hq*D]
  int P, Hq, Hkv, Smax, nblk;
  float scale;
};

template <int REP>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const AttnPrefillParams p) {
  constexpr int NT = 64 * REP;
  constexpr int PIECES = KC * kHD * 2 / 16;
  constexpr int PER = (PIECES + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t sK[KC][kHD + 8];
  __shared__ __attribute__((aligned(16))) uint16_t sV[kHD][KC + 8];
  __shared__ __attribute__((aligned(16))) uint16_t sP[REP][16][KC + 8];
  const int blk = p.nblk - 1 - (int)blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int r16 = lane & 15, g4 = lane >> 4;
  const int qh = h * REP + wave;
  const int base = min(max(p.lens[0], 0), p.Smax);
  const int t0 = blk * 16;
  const int Tb = min(16, p.P - t0);  // live rows of this block
  const int L = min(base + t0 + Tb, p.Smax);  // keys the block's last row sees
  const int ntiles = (L + KC - 1) / KC;
  const uint16_t* kbase = p.k_cache + (int64_t)h * p.Smax * kHD;
  const uint16_t* vbase = p.vt_cache + (int64_t)h * kHD * p.Smax;
  u32x4 kv[PER], vv[PER];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = min(tid + NT * i, PIECES - 1);
      kv[i] = ld16(kbase + (int64_t)(k0 + (e >> 4)) * kHD + (e & 15) * 8);
      vv[i] = ld16(vbase + (int64_t)(e >> 3) * p.Smax + k0 + (e & 7) * 8);
    }
  };
  load_tile(0);
  const int tq = r16 < Tb ? r16 : Tb - 1;
  const uint16_t* qr = p.q + ((int64_t)(t0 + tq) * p.Hq + qh) * kHD + g4 * 8;
  u32x4 qa[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const u32x4 v = ld16(qr + 32 * k);
    qa[k] = r16 < Tb ? v : u32x4{0u, 0u, 0u, 0u};
  }
  float m[4], l[4];
  f32x4 o[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m[e] = -INFINITY;
    l[e] = 0.f;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < ntiles; ++j) {
    const int k0 = j * KC;
    __syncthreads();  // every wave is done with the previous tile's K and V^T
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + NT * i;
      if (e < PIECES) {
        *reinterpret_cast<u32x4*>(&sK[e >> 4][(e & 15) * 8]) = kv[i];
        *reinterpret_cast<u32x4*>(&sV[e >> 3][(e & 7) * 8]) = vv[i];
      }
    }
    __syncthreads();
    if (j + 1 < ntiles) load_tile(k0 + KC);  // in flight during this tile's products
    f32x4 sacc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, qa[k]),
            __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&sK[16 * n + r16][32 * k + 8 * g4])),
            acc, 0, 0, 0);
      sacc[n] = acc;
    }
    float sv[4][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 4 * g4 + e;
      const int last = base + t0 + t;  // the last key row t sees
      float mx = -INFINITY;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int key = k0 + 16 * n + r16;
        const bool ok = (t < Tb) && (key <= last) && (key < L);
        sv[n][e] = ok ? sacc[n][e] * p.scale : -INFINITY;
        mx = fmaxf(mx, sv[n][e]);
      }
      const float mn = fmaxf(m[e], row16_max(mx));
      const float alpha = (m[e] == -INFINITY) ? 0.f : __expf(m[e] - mn);
      const float ms = mn == -INFINITY ? 0.f : mn;
      float sum = 0.f;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const float pe = __expf(sv[n][e] - ms);
        sv[n][e] = pe;
        sum += pe;
      }
      l[e] = l[e] * alpha + row16_sum(sum);
      m[e] = mn;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt][e] *= alpha;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int n = 0; n < 4; ++n) sP[wave][4 * g4 + e][16 * n + r16] = f32_to_bf16_rne(sv[n][e]);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's P writes are visible to it
    u32x4 pa[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) pa[k] = *reinterpret_cast<const u32x4*>(&sP[wave][r16][32 * k + 8 * g4]);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int k = 0; k < 2; ++k)
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, pa[k]),
            __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&sV[16 * dt + r16][32 * k + 8 * g4])),
            o[dt], 0, 0, 0);
  }
  // out = O / l * sigmoid(gate); lane (r16, g4) holds row 4 g4 + e, feature 16 dt + r16.
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 4 * g4 + e;
    if (t >= Tb) continue;
    const int64_t row = t0 + t;
    const float inv = 1.f / l[e];
    const uint16_t* gr = p.gate_src + row * p.gate_row_stride + qh * 2 * kHD + kHD;
    uint16_t* orow = p.out + (row * p.Hq + qh) * kHD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const float gt = bf16_bits_to_f32(gr[16 * dt + r16]);
      orow[16 * dt + r16] = f32_to_bf16_rne(o[dt][e] * inv * (1.f / (1.f + __expf(-gt))));
    }
  }
}

// --------------------------------------------------------- commit an accept
// keep[b] = matched[b] + 1 (the block's first token plus the accepted drafts,
// runtime.py:146), lens[b] += keep[b] (the KV trim of adapters.py:505-508
// seen from the other side: the cache keeps lens + keep positions).
__global__ void commit_accept_kernel(const int32_t* matched, int32_t* keep, int32_t* lens, int B,
                                     int T) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int k = min(max(matched[b], 0), T - 1) + 1;
  keep[b] = k;
  if (lens != nullptr) lens[b] += k;
}

}  // namespace
}  // namespace dflash

using namespace dflash;

namespace dflash {
namespace {
int launch_add_rmsnorm(const void* x, const int32_t* tok, int vocab, const void* r, const float* rp,
                       int nsplit, const void* weight, void* h_out, void* h_copy,
                       int64_t h_copy_stride, void* y, int M, int H, float eps, void* stream) {
  if (M < 0 || H <= 0 || H % 8 != 0 || H > 1024 * 8 || nsplit < 0) return DFLASH_ERR_SHAPE;
  if (h_copy != nullptr && h_copy_stride < H) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || weight == nullptr || y == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)r & 15) || ((uintptr_t)rp & 15) ||
      ((uintptr_t)weight & 15) || ((uintptr_t)h_out & 15) || ((uintptr_t)y & 15) ||
      ((uintptr_t)h_copy & 15) || (h_copy != nullptr && (h_copy_stride % 8)))
    return DFLASH_ERR_ALIGN;
  auto* hcp = static_cast<uint16_t*>(h_copy);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)M);
  const dim3 block((unsigned)ceil_div(H / 8, 64) * 64);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* rpb = static_cast<const uint16_t*>(r);
  const auto* wp = static_cast<const uint16_t*>(weight);
  auto* hp = static_cast<uint16_t*>(h_out);
  auto* yp = static_cast<uint16_t*>(y);
  if (rp != nullptr) {
    switch (nsplit) {
#define DFLASH_ARN(ns)                                                                           \
  case ns:                                                                                       \
    hipLaunchKernelGGL((add_rmsnorm_kernel<true, ns>), grid, block, 0, s, xp, tok, vocab, nullptr, \
                       rp, nsplit, wp, hp, hcp, h_copy_stride, yp, M, H, eps);                   \
    break;
      DFLASH_ARN(1) DFLASH_ARN(2) DFLASH_ARN(3) DFLASH_ARN(4) DFLASH_ARN(5) DFLASH_ARN(6)
      DFLASH_ARN(7) DFLASH_ARN(8)
#undef DFLASH_ARN
      default:
        hipLaunchKernelGGL((add_rmsnorm_kernel<true, 0>), grid, block, 0, s, xp, tok, vocab, nullptr,
                           rp, nsplit, wp, hp, hcp, h_copy_stride, yp, M, H, eps);
    }
  } else {
    hipLaunchKernelGGL((add_rmsnorm_kernel<false, 0>), grid, block, 0, s, xp, tok, vocab, rpb,
                       nullptr, 0, wp, hp, hcp, h_copy_stride, yp, M, H, eps);
  }
  return to_status(hipGetLastError());
}
}  // namespace
}  // namespace dflash

extern "C" int dflash_add_rmsnorm(const void* x, const void* r, const void* weight, void* h_out,
                                  void* y, int M, int H, float eps, void* stream) {
  return launch_add_rmsnorm(x, nullptr, 0, r, nullptr, 0, weight, h_out, nullptr, 0, y, M, H, eps,
                            stream);
}

extern "C" int dflash_add_rmsnorm_splitk(const void* x, const float* r_partials, int nsplit,
                                         const void* weight, void* h_out, void* y, int M, int H,
                                         float eps, void* stream) {
  if (r_partials == nullptr || nsplit < 1) return DFLASH_ERR_NULL;
  return launch_add_rmsnorm(x, nullptr, 0, nullptr, r_partials, nsplit, weight, h_out, nullptr, 0,
                            y, M, H, eps, stream);
}

extern "C" int dflash_add_rmsnorm_capture(const void* x, const void* r, const float* r_partials,
                                          int nsplit, const void* weight, void* h_out,
                                          void* h_copy, int64_t h_copy_row_stride, void* y, int M,
                                          int H, float eps, void* stream) {
  if (r_partials != nullptr && (r != nullptr || nsplit < 1)) return DFLASH_ERR_SHAPE;
  if (h_copy == nullptr) return DFLASH_ERR_NULL;
  return launch_add_rmsnorm(x, nullptr, 0, r, r_partials, r_partials ? nsplit : 0, weight, h_out,
                            h_copy, h_copy_row_stride, y, M, H, eps, stream);
}

extern "C" int dflash_embed_rmsnorm(const void* table, const int32_t* tokens, int vocab,
                                    const void* weight, void* h_out, void* y, int M, int H,
                                    float eps, void* stream) {
  if (vocab <= 0) return DFLASH_ERR_SHAPE;
  if (tokens == nullptr || h_out == nullptr) return DFLASH_ERR_NULL;
  return launch_add_rmsnorm(table, tokens, vocab, nullptr, nullptr, 0, weight, h_out, nullptr, 0, y,
                            M, H, eps, stream);
}

extern "C" int dflash_swiglu(const void* gate_up, void* out, int M, int I, void* stream) {
  if (M < 0 || I <= 0 || I % 8 != 0) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (gate_up == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)gate_up & 15) || ((uintptr_t)out & 15)) return DFLASH_ERR_ALIGN;
  const int64_t n = (int64_t)M * (I / 8);
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(n, 256), 2048);
  hipLaunchKernelGGL(swiglu_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), M, I);
  return to_status(hipGetLastError());
}

extern "C" int dflash_attn_prep(const void* proj, int64_t proj_row_stride, const void* q_norm_w,
                                const void* k_norm_w, const int32_t* lens, void* k_cache,
                                void* vt_cache, void* q_out, int32_t* overflow, int B, int T,
                                int Hq, int Hkv, int D, int Smax, int rot_dims, float rope_base,
                                float eps, void* stream) {
  if (B < 0 || T < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Smax <= 0) return DFLASH_ERR_SHAPE;
  if (D != kHD) return DFLASH_ERR_UNSUPPORTED;
  if (!(rot_dims == 0 || rot_dims == 16 || rot_dims == 32 || rot_dims == 64 || rot_dims == 128))
    return DFLASH_ERR_UNSUPPORTED;
  if (proj_row_stride < (int64_t)(2 * Hq + 2 * Hkv) * D) return DFLASH_ERR_SHAPE;
  if ((int64_t)B * T > INT32_MAX) return DFLASH_ERR_SHAPE;  // grid.x = B * T
  if (B == 0 || T == 0) return DFLASH_OK;
  if (proj == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || lens == nullptr ||
      k_cache == nullptr || vt_cache == nullptr || q_out == nullptr)
    return DFLASH_ERR_NULL;
  if (((uintptr_t)proj & 3) || (proj_row_stride % 2) || ((uintptr_t)q_norm_w & 3) ||
      ((uintptr_t)k_norm_w & 3) || ((uintptr_t)k_cache & 3) || ((uintptr_t)q_out & 3))
    return DFLASH_ERR_ALIGN;
  AttnPrepParams p{};
  p.proj = static_cast<const uint16_t*>(proj);
  p.row_stride = proj_row_stride;
  p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  p.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
  p.lens = lens;
  p.k_cache = static_cast<uint16_t*>(k_cache);
  p.vt_cache = static_cast<uint16_t*>(vt_cache);
  p.q_out = static_cast<uint16_t*>(q_out);
  p.overflow = overflow;
  p.B = B; p.T = T; p.Hq = Hq; p.Hkv = Hkv; p.Smax = Smax; p.rot = rot_dims;
  p.log2_base = log2((double)rope_base);
  p.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Long inputs with 16-byte aligned value rows: the value heads through
  // attn_prep_vt_kernel's tiles instead of a wave a token.
  p.skip_v = T >= kVtTile && ((uintptr_t)proj & 15) == 0 && proj_row_stride % 8 == 0;
  const int slots = p.skip_v ? Hq + Hkv : Hq + 2 * Hkv;
  const dim3 grid((unsigned)(B * T), (unsigned)ceil_div(slots, 4));
  hipLaunchKernelGGL(attn_prep_kernel, grid, dim3(256), 0, s, p);
  if (p.skip_v) {
    const dim3 vgrid((unsigned)ceil_div(T, kVtTile), (unsigned)Hkv, (unsigned)B);
    hipLaunchKernelGGL(attn_prep_vt_kernel, vgrid, dim3(256), 0, s, p);
  }
  return to_status(hipGetLastError());
}

extern "C" size_t dflash_attn_verify_workspace_bytes(int B, int Hq, int Hkv, int max_len) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || max_len <= 0) return 0;
  const int64_t nsplit = ceil_div(max_len, KC);
  const int64_t rows = (int64_t)B * Hq * nsplit * 16;  // Hkv * rep = Hq
  return (size_t)(rows * (kHD + 2) * sizeof(float));
}

extern "C" int dflash_attn_verify(const void* q, const void* k_cache, const void* vt_cache,
                                  const int32_t* lens, const void* gate_src,
                                  int64_t gate_row_stride, void* out, int B, int T, int Hq,
                                  int Hkv, int D, int Smax, int max_len, float scale,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (B < 0 || T < 0 || T > 16 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Hq / Hkv > 4)
    return DFLASH_ERR_SHAPE;
  if (D != kHD) return DFLASH_ERR_UNSUPPORTED;
  if (Smax <= 0 || Smax % KC != 0 || max_len <= 0 || max_len > Smax) return DFLASH_ERR_SHAPE;
  if (B > 65535) return DFLASH_ERR_SHAPE;  // grid.z of the partials = B
  if (B == 0 || T == 0) return DFLASH_OK;
  if (q == nullptr || k_cache == nullptr || vt_cache == nullptr || lens == nullptr ||
      gate_src == nullptr || out == nullptr || workspace == nullptr)
    return DFLASH_ERR_NULL;
  if (workspace_bytes < dflash_attn_verify_workspace_bytes(B, Hq, Hkv, max_len))
    return DFLASH_ERR_WORKSPACE;
  if (((uintptr_t)q & 15) || ((uintptr_t)k_cache & 15) || ((uintptr_t)vt_cache & 15) ||
      ((uintptr_t)gate_src & 3) || (gate_row_stride % 2) || ((uintptr_t)out & 3) ||
      ((uintptr_t)workspace & 15))
    return DFLASH_ERR_ALIGN;
  AttnParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k_cache = static_cast<const uint16_t*>(k_cache);
  p.vt_cache = static_cast<const uint16_t*>(vt_cache);
  p.lens = lens;
  p.gate_src = static_cast<const uint16_t*>(gate_src);
  p.gate_row_stride = gate_row_stride;
  p.out = static_cast<uint16_t*>(out);
  p.B = B; p.T = T; p.Hq = Hq; p.Hkv = Hkv; p.Smax = Smax;
  p.nsplit = (int)ceil_div(max_len, KC);
  p.scale = scale;
  const int64_t rows = (int64_t)B * Hq * p.nsplit * 16;
  p.part_o = static_cast<float*>(workspace);
  p.part_ml = p.part_o + rows * kHD;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rep = Hq / Hkv;
  const dim3 pgrid(p.nsplit, Hkv, B);
  switch (rep) {
    case 1: hipLaunchKernelGGL(attn_partial_kernel<1>, pgrid, dim3(64), 0, s, p); break;
    case 2: hipLaunchKernelGGL(attn_partial_kernel<2>, pgrid, dim3(128), 0, s, p); break;
    case 3: hipLaunchKernelGGL(attn_partial_kernel<3>, pgrid, dim3(192), 0, s, p); break;
    default: hipLaunchKernelGGL(attn_partial_kernel<4>, pgrid, dim3(256), 0, s, p); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(B * T, Hq), dim3(256), 0, s, p);
  return to_status(hipGetLastError());
}

extern "C" int dflash_attn_prefill(const void* q, const void* k_cache, const void* vt_cache,
                                   const int32_t* lens, const void* gate_src,
                                   int64_t gate_row_stride, void* out, int P, int Hq, int Hkv,
                                   int D, int Smax, float scale, void* stream) {
  if (P < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Hq / Hkv > 4) return DFLASH_ERR_SHAPE;
  if (D != kHD) return DFLASH_ERR_UNSUPPORTED;
  if (Smax <= 0 || Smax % KC != 0 || Hkv > 65535) return DFLASH_ERR_SHAPE;
  if (gate_row_stride < (int64_t)2 * Hq * D) return DFLASH_ERR_SHAPE;
  if (P == 0) return DFLASH_OK;
  if (q == nullptr || k_cache == nullptr || vt_cache == nullptr || lens == nullptr ||
      gate_src == nullptr || out == nullptr)
    return DFLASH_ERR_NULL;
  if (((uintptr_t)q & 15) || ((uintptr_t)k_cache & 15) || ((uintptr_t)vt_cache & 15) ||
      ((uintptr_t)gate_src & 1) || ((uintptr_t)out & 1))
    return DFLASH_ERR_ALIGN;
  AttnPrefillParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k_cache = static_cast<const uint16_t*>(k_cache);
  p.vt_cache = static_cast<const uint16_t*>(vt_cache);
  p.lens = lens;
  p.gate_src = static_cast<const uint16_t*>(gate_src);
  p.gate_row_stride = gate_row_stride;
  p.out = static_cast<uint16_t*>(out);
  p.P = P; p.Hq = Hq; p.Hkv = Hkv; p.Smax = Smax;
  p.nblk = (int)ceil_div(P, 16);
  p.scale = scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)p.nblk, (unsigned)Hkv);
  switch (Hq / Hkv) {
    case 1: hipLaunchKernelGGL(attn_prefill_kernel<1>, grid, dim3(64), 0, s, p); break;
    case 2: hipLaunchKernelGGL(attn_prefill_kernel<2>, grid, dim3(128), 0, s, p); break;
    case 3: hipLaunchKernelGGL(attn_prefill_kernel<3>, grid, dim3(192), 0, s, p); break;
    default: hipLaunchKernelGGL(attn_prefill_kernel<4>, grid, dim3(256), 0, s, p); break;
  }
  return to_status(hipGetLastError());
}

extern "C" int dflash_commit_accept(const int32_t* matched, int32_t* keep, int32_t* lens, int B,
                                    int T, void* stream) {
  if (B < 0 || T <= 0) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  if (matched == nullptr || keep == nullptr) return DFLASH_ERR_NULL;
  hipLaunchKernelGGL(commit_accept_kernel, dim3((unsigned)ceil_div(B, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), matched, keep, lens, B, T);
  return to_status(hipGetLastError());
}
