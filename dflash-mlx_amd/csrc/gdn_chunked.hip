// Chunked (WY / UT-transform) gated-delta prefill on MFMA.
//
// The reference prefills with the sequential scan (mlx-lm gated_delta_update,
// dflash_mlx/custom_qwen35_model.py:790-801, called from the prompt pass at
// runtime.py:384-388).  Over a chunk of C = 64 tokens starting from state S0
// ([Dv, Dk]) the same recurrence unrolls to (G = cumulative log-decay in the
// chunk, gamma = exp(G)):
//   A[i][j] = beta_i exp(G_i - G_j) k_i.k_j  (j < i),   T = (I + A)^-1
//   W  = T diag(beta gamma) K,   U~ = T diag(beta) V     [C, Dk], [C, Dv]
//   U  = U~ - W S0^T                                     (the per-token deltas)
//   O  = diag(gamma) Q S0^T + P U,  P[i][j] = exp(G_i - G_j) q_i.k_j (j <= i)
//   S_C = gamma_C S0 + (diag(exp(G_C - G)) U)^T K
//
// Phase 1 (chunk_prep_kernel, parallel over (head, chunk)): K K^T and Q K^T
// on bf16 MFMA (exact products of bf16 inputs), T by forward substitution in
// fp32, then W^T = K^T (T diag(beta gamma))^T and U~ = (T diag(beta)) V on
// bf16 MFMA with T split into hi + lo bf16 halves.  Everything phase 2 reads
// is written pre-arranged in the operand order of its MFMAs.
// Phase 2 (chunk_state_kernel, sequential over chunks, parallel over (head,
// 16 state rows)): the state stays in registers in fp32; every product with
// an fp32 operand splits it into hi + lo bf16 halves (x = hi + lo to about
// 2^-16 relative) and accumulates hi*hi + hi*lo + lo*hi in fp32, so the state
// keeps fp32-level accuracy over all chunks while running on the bf16 matrix
// cores.  The next chunk's operands are prefetched into registers, and the two
// barriers per chunk wait on LDS traffic only, not on those loads.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int CH = 64;   // chunk length
constexpr int D = 128;   // Dk = Dv supported by these kernels
constexpr int RB = 16;   // state rows per phase-2 workgroup
constexpr int KTP = 72;  // bf16 row pitch of the K^T / V^T tiles in LDS
constexpr int TPF = 68;  // fp32 row pitch of A / T in LDS

// Workspace of one (head, chunk), in bytes.  Layouts:
//   W_HI / W_LO: bf16 [64 i][4 s][4 g][8]: slot t*4+e holds W[i][32s+16t+4g+e]
//   KT:          bf16 [128 dk][64 j]        (K transposed)
//   P_HI / P_LO: bf16 [64 i][64 j]          (row-major)
//   UT:          fp32 [8 rb][4 w][64 lane][4]: U~[16w + 4(lane/16) + e][16rb + lane%16]
//   EG:          fp32 [64] exp(G_i);  ED: fp32 [64] exp(G_63 - G_i)  (decays)
constexpr size_t kWHi = 0;
constexpr size_t kWLo = kWHi + CH * D * 2;
constexpr size_t kKT = kWLo + CH * D * 2;
constexpr size_t kPHi = kKT + D * CH * 2;
constexpr size_t kPLo = kPHi + CH * CH * 2;
constexpr size_t kUT = kPLo + CH * CH * 2;
constexpr size_t kEG = kUT + CH * D * 4;
constexpr size_t kED = kEG + CH * 4;
constexpr size_t kWsChunk = kED + CH * 4;
static_assert(kWsChunk % 16 == 0, "per-chunk workspace must keep 16-byte alignment");

struct ChunkParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g;
  const float* beta;
  const float* state_in;
  uint16_t* out;
  float* final_state;
  int64_t q_sb, q_st, q_sh, k_sb, k_st, k_sh, v_sb, v_st, v_sh, g_sb, g_st, b_sb, b_st;
  int B, T, Hv, rep, NC;
  uint8_t* ws;  // [B*Hv][NC][kWsChunk]
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 x) { return __builtin_bit_cast(bf16x8, x); }

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// x = hi + lo: hi = x truncated to bf16 (the remainder is exact in fp32),
// lo = bf16(x - hi).  Two values packed per 32-bit word, element 0 low.
__device__ __forceinline__ uint32_t pack_hi(float x0, float x1) {
  return (__float_as_uint(x0) >> 16) | (__float_as_uint(x1) & 0xFFFF0000u);
}
// Two fp32 to packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));
}
__device__ __forceinline__ uint32_t pack_lo(float x0, float x1) {
  const float r0 = x0 - __uint_as_float(__float_as_uint(x0) & 0xFFFF0000u);
  const float r1 = x1 - __uint_as_float(__float_as_uint(x1) & 0xFFFF0000u);
  return cvt_pk_bf16(r0, r1);
}

__device__ __forceinline__ void split8(const float* x, u32x4& hi, u32x4& lo) {
  hi = u32x4{pack_hi(x[0], x[1]), pack_hi(x[2], x[3]), pack_hi(x[4], x[5]), pack_hi(x[6], x[7])};
  lo = u32x4{pack_lo(x[0], x[1]), pack_lo(x[2], x[3]), pack_lo(x[4], x[5]), pack_lo(x[6], x[7])};
}

__device__ __forceinline__ void split4(f32x4 x, u32x2& hi, u32x2& lo) {
  hi = u32x2{pack_hi(x.x, x.y), pack_hi(x.z, x.w)};
  lo = u32x2{pack_lo(x.x, x.y), pack_lo(x.z, x.w)};
}

// Workgroup barrier that waits for this wave's LDS traffic only: global loads
// in flight (the next chunk's prefetch) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ const uint16_t* krow(const ChunkParams& p, int b, int hk, int t) {
  return p.k + b * p.k_sb + (int64_t)t * p.k_st + hk * p.k_sh;
}
__device__ __forceinline__ const uint16_t* qrow(const ChunkParams& p, int b, int hk, int t) {
  return p.q + b * p.q_sb + (int64_t)t * p.q_st + hk * p.q_sh;
}
__device__ __forceinline__ const uint16_t* vrow(const ChunkParams& p, int b, int hv, int t) {
  return p.v + b * p.v_sb + (int64_t)t * p.v_st + hv * p.v_sh;
}

__device__ __forceinline__ u32x4 ld16(const void* ptr) { return *reinterpret_cast<const u32x4*>(ptr); }
__device__ __forceinline__ u32x2 ld8(const void* ptr) { return *reinterpret_cast<const u32x2*>(ptr); }

// ------------------------------------------------------------------ phase 1
// grid (NC, B*Hv), 256 threads.
__global__ __launch_bounds__(256) void chunk_prep_kernel(const ChunkParams p) {
  __shared__ float sA[CH][TPF];
  __shared__ float sT[CH][TPF];
  __shared__ __attribute__((aligned(16))) uint16_t sKT[D][KTP];
  __shared__ __attribute__((aligned(16))) uint16_t sVT[D][KTP];
  __shared__ float sG[CH];
  __shared__ float sBeta[CH];
  const int c = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.Hv;
  const int hv = bh - b * p.Hv;
  const int hk = hv / p.rep;
  const int t0 = c * CH;
  const int n = min(CH, p.T - t0);  // valid tokens in this chunk
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  uint8_t* ws = p.ws + ((int64_t)bh * p.NC + c) * kWsChunk;

  // K^T and V^T tiles (padded tokens are zero).  Rows past the chunk's valid
  // tokens read row n-1 and are zeroed by a select, so all eight 16-byte
  // loads of a thread are in flight together.
  {
    u32x4 kk[4], vv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = tid + 256 * m;
      const int j = e >> 4, piece = e & 15;
      const int jr = j < n ? j : n - 1;
      kk[m] = ld16(krow(p, b, hk, t0 + jr) + piece * 8);
      vv[m] = ld16(vrow(p, b, hv, t0 + jr) + piece * 8);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = tid + 256 * m;
      const int j = e >> 4, piece = e & 15;
      const bool valid = j < n;
      const uint32_t kw[4] = {kk[m].x, kk[m].y, kk[m].z, kk[m].w};
      const uint32_t vw[4] = {vv[m].x, vv[m].y, vv[m].z, vv[m].w};
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const uint32_t kx = valid ? kw[x] : 0u, vx = valid ? vw[x] : 0u;
        sKT[piece * 8 + 2 * x][j] = (uint16_t)kx;
        sKT[piece * 8 + 2 * x + 1][j] = (uint16_t)(kx >> 16);
        sVT[piece * 8 + 2 * x][j] = (uint16_t)vx;
        sVT[piece * 8 + 2 * x + 1][j] = (uint16_t)(vx >> 16);
      }
    }
  }
  // Cumulative log-decay and beta (padded tokens: g = 1, beta = 0).
  if (wave == 0) {
    float lg = 0.f, bt = 0.f;
    if (lane < n) {
      lg = logf(fmaxf(p.g[b * p.g_sb + (int64_t)(t0 + lane) * p.g_st + hv], 1e-38f));
      bt = p.beta[b * p.b_sb + (int64_t)(t0 + lane) * p.b_st + hv];
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(lg, off, 64);
      if (lane >= off) lg += o;
    }
    sG[lane] = lg;
    sBeta[lane] = bt;
    const float lg_end = __shfl(lg, CH - 1, 64);
    reinterpret_cast<float*>(ws + kEG)[lane] = __expf(lg);
    reinterpret_cast<float*>(ws + kED)[lane] = __expf(lg_end - lg);
  }
  __syncthreads();

  // K K^T -> A (strictly lower, scaled), Q K^T -> P (lower, decay-masked).
  // Wave w computes the 16-row tile w; tiles above the diagonal are zero.
  {
    const int i0 = wave * 16;
    uint16_t* phi = reinterpret_cast<uint16_t*>(ws + kPHi);
    uint16_t* plo = reinterpret_cast<uint16_t*>(ws + kPLo);
    // A-operand rows (this wave's 16 tokens) once, for all column tiles.
    const int ti = i0 + r16;
    const bool vi = ti < n;
    const uint16_t* kri = krow(p, b, hk, t0 + (vi ? ti : n - 1)) + g4 * 8;
    const uint16_t* qri = qrow(p, b, hk, t0 + (vi ? ti : n - 1)) + g4 * 8;
    u32x4 ka[D / 32], qa[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      const u32x4 kv = ld16(kri + ks * 32), qv = ld16(qri + ks * 32);
      ka[ks] = vi ? kv : u32x4{0u, 0u, 0u, 0u};
      qa[ks] = vi ? qv : u32x4{0u, 0u, 0u, 0u};
    }
    for (int jt = 0; jt < 4; ++jt) {
      const int j0 = jt * 16;
      f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
      if (jt <= wave) {
        const int tj = j0 + r16;
        const bool vj = tj < n;
        const uint16_t* krj = krow(p, b, hk, t0 + (vj ? tj : n - 1)) + g4 * 8;
        u32x4 kb[D / 32];
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
          const u32x4 kv = ld16(krj + ks * 32);
          kb[ks] = vj ? kv : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
          kk = mfma(ka[ks], kb[ks], kk);
          qk = mfma(qa[ks], kb[ks], qk);
        }
      }
      // Tile element (i, j): lane holds j = j0 + r16, i = i0 + 4*g4 + e.
      const float vkk[4] = {kk.x, kk.y, kk.z, kk.w};
      const float vqk[4] = {qk.x, qk.y, qk.z, qk.w};
      const int j = j0 + r16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = i0 + g4 * 4 + e;
        const float dec = (j <= i) ? __expf(sG[i] - sG[j]) : 0.f;
        sA[i][j] = (j < i) ? sBeta[i] * dec * vkk[e] : 0.f;
        const float pv = (j <= i) ? dec * vqk[e] : 0.f;
        const uint32_t hb = __float_as_uint(pv) & 0xFFFF0000u;
        phi[i * CH + j] = (uint16_t)(hb >> 16);
        plo[i * CH + j] = f32_to_bf16_rne(pv - __uint_as_float(hb));
      }
    }
  }
  // K^T to the workspace (rows of 64 tokens, 16-byte pieces).
  {
    uint16_t* kt = reinterpret_cast<uint16_t*>(ws + kKT);
    for (int e = tid; e < D * (CH / 8); e += 256) {
      const int dk = e >> 3, piece = e & 7;
      *reinterpret_cast<u32x4*>(kt + dk * CH + piece * 8) =
          *reinterpret_cast<const u32x4*>(&sKT[dk][piece * 8]);
    }
  }
  __syncthreads();

  // T = (I + A)^-1 in 16x16 blocks (A is strictly lower-triangular).
  // Step 1: wave w inverts diagonal block w by forward substitution (lane
  // c < 16 owns column c) and zeroes the blocks right of it.
  {
    const int base = wave * 16;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) {
        if (j & 1) s1 = fmaf(sA[base + i][base + j], t[j], s1);
        else s0 = fmaf(sA[base + i][base + j], t[j], s0);
      }
      t[i] = (i == lane) ? 1.f : ((i < lane) ? 0.f : -(s0 + s1));
    }
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sT[base + i][base + lane] = t[i];
    }
    const int wide = CH - base - 16;
    for (int e = lane; e < 16 * wide; e += 64) sT[base + e / wide][base + 16 + e % wide] = 0.f;
  }
  __syncthreads();
  // Step 2: wave w fills its block column below the diagonal, top to bottom:
  //   T[bi][w] = -T[bi][bi] * sum_{bk=w}^{bi-1} A[bi][bk] T[bk][w]
  // on fp32 MFMA (16x16x4: A lane = (row l%16, k l/16), B lane = (k l/16,
  // column l%16), D lane = (rows 4(l/16)+e, column l%16)).
  for (int bi = wave + 1; bi < 4; ++bi) {
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    for (int bk = wave; bk < bi; ++bk) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        x = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[16 * bi + r16][16 * bk + 4 * s4 + g4],
                                                 sT[16 * bk + 4 * s4 + g4][16 * wave + r16], x,
                                                 0, 0, 0);
    }
    const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) sT[16 * bi + 4 * g4 + e][16 * wave + r16] = xv[e];
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      y = __builtin_amdgcn_mfma_f32_16x16x4f32(sT[16 * bi + r16][16 * bi + 4 * s4 + g4],
                                               sT[16 * bi + 4 * s4 + g4][16 * wave + r16], y,
                                               0, 0, 0);
    const float yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) sT[16 * bi + 4 * g4 + e][16 * wave + r16] = -yv[e];
  }
  __syncthreads();

  // W^T[dk][i] = sum_j K^T[dk][j] T'[i][j],  T' = T diag(beta gamma)   (wave w: dk tiles 2w, 2w+1)
  // U~[i][dv]  = sum_j T_b[i][j] V^T[dv][j], T_b = T diag(beta)       (wave w: dv tiles 2w, 2w+1)
  {
    uint16_t* whi = reinterpret_cast<uint16_t*>(ws + kWHi);
    uint16_t* wlo = reinterpret_cast<uint16_t*>(ws + kWLo);
    float* ut = reinterpret_cast<float*>(ws + kUT);
    for (int it = 0; it < 4; ++it) {
      f32x4 aw[2], au[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        aw[x] = f32x4{0.f, 0.f, 0.f, 0.f};
        au[x] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      const int i = it * 16 + r16;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int j0 = s * 32 + g4 * 8;
        float tw[8], tb[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          tb[x] = sT[i][j0 + x] * sBeta[j0 + x];
          tw[x] = tb[x] * __expf(sG[j0 + x]);
        }
        u32x4 twh, twl, tbh, tbl;
        split8(tw, twh, twl);
        split8(tb, tbh, tbl);
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int tile = 2 * wave + x;
          const u32x4 ka = *reinterpret_cast<const u32x4*>(&sKT[tile * 16 + r16][j0]);
          aw[x] = mfma(ka, twh, aw[x]);
          aw[x] = mfma(ka, twl, aw[x]);
          const u32x4 vb = *reinterpret_cast<const u32x4*>(&sVT[tile * 16 + r16][j0]);
          au[x] = mfma(tbh, vb, au[x]);
          au[x] = mfma(tbl, vb, au[x]);
        }
      }
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int tile = 2 * wave + x;
        // aw: lane holds W[i][dk], dk = 16 tile + 4 g4 + e -> s = tile/2, t = tile%2.
        u32x2 hi, lo;
        split4(aw[x], hi, lo);
        const int off = i * D + (tile >> 1) * 32 + g4 * 8 + (tile & 1) * 4;
        *reinterpret_cast<u32x2*>(whi + off) = hi;
        *reinterpret_cast<u32x2*>(wlo + off) = lo;
        // au: lane holds U~[16 it + 4 g4 + e][16 tile + r16] -> UT[tile][it][lane].
        *reinterpret_cast<f32x4*>(ut + ((tile * 4 + it) * 64 + lane) * 4) = au[x];
      }
    }
  }
}

// ------------------------------------------------------------------ phase 2
// Per-wave operands of one chunk (wave w owns token rows 16w .. 16w+15 for the
// W / Q / P products and state columns 32w .. 32w+31 for the state update).
struct ChunkOps {
  u32x4 whi[4], wlo[4];  // W rows, k-steps s = 0..3
  u32x2 q[8];            // Q rows: [2s + t] = dk 32s + 16t + 4g .. +3
  u32x4 phi[2], plo[2];  // P rows, j-steps 0..1
  u32x4 kt[4];           // K^T rows 32w + 16t + r16, j-step s: [2t + s]
  f32x4 ut;              // U~ for this lane's 4 token rows
  f32x4 eg;              // exp(G) of this lane's 4 token rows
  f32x4 ed;              // exp(G_end - G) of the same rows
  float egC;             // exp(G_end)
};

__device__ __forceinline__ void load_ops(const ChunkParams& p, int bh, int b, int hk, int c, int rb,
                                         int wave, int lane, ChunkOps& o) {
  const int r16 = lane & 15, g4 = lane >> 4;
  const uint8_t* ws = p.ws + ((int64_t)bh * p.NC + c) * kWsChunk;
  const int i = wave * 16 + r16;
  const uint16_t* whi = reinterpret_cast<const uint16_t*>(ws + kWHi) + i * D + g4 * 8;
  const uint16_t* wlo = reinterpret_cast<const uint16_t*>(ws + kWLo) + i * D + g4 * 8;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    o.whi[s] = ld16(whi + s * 32);
    o.wlo[s] = ld16(wlo + s * 32);
  }
  // Rows past T (partial last chunk) read row T-1 and are zeroed by a select:
  // no branch around the loads.
  const int t = c * CH + i;
  const bool valid = t < p.T;
  const uint16_t* qr = qrow(p, b, hk, valid ? t : p.T - 1) + 4 * g4;
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const u32x2 qv = ld8(qr + (x >> 1) * 32 + (x & 1) * 16);
    o.q[x] = u32x2{valid ? qv.x : 0u, valid ? qv.y : 0u};
  }
  const uint16_t* phi = reinterpret_cast<const uint16_t*>(ws + kPHi) + i * CH + g4 * 8;
  const uint16_t* plo = reinterpret_cast<const uint16_t*>(ws + kPLo) + i * CH + g4 * 8;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    o.phi[s] = ld16(phi + s * 32);
    o.plo[s] = ld16(plo + s * 32);
  }
  const uint16_t* kt = reinterpret_cast<const uint16_t*>(ws + kKT) + (wave * 32 + r16) * CH + g4 * 8;
#pragma unroll
  for (int x = 0; x < 4; ++x) o.kt[x] = ld16(kt + (x >> 1) * 16 * CH + (x & 1) * 32);
  o.ut = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(ws + kUT) +
                                         ((rb * 4 + wave) * 64 + lane) * 4);
  const float* eg = reinterpret_cast<const float*>(ws + kEG);
  const float* ed = reinterpret_cast<const float*>(ws + kED);
  o.eg = *reinterpret_cast<const f32x4*>(eg + wave * 16 + 4 * g4);
  o.ed = *reinterpret_cast<const f32x4*>(ed + wave * 16 + 4 * g4);
  o.egC = eg[CH - 1];
}

// The wave's own 8 state values (slot t*4+e = sown[t][e]) as hi / lo bf16
// halves, published for the other waves; fetch_state gathers all 32 columns of
// k-steps 0..3 (k-step s = the columns owned by wave s).
__device__ __forceinline__ void publish_state(const f32x4 (&sown)[2], u32x4 (*sS)[4][64], int wave,
                                              int lane) {
  sS[0][wave][lane] = u32x4{pack_hi(sown[0].x, sown[0].y), pack_hi(sown[0].z, sown[0].w),
                            pack_hi(sown[1].x, sown[1].y), pack_hi(sown[1].z, sown[1].w)};
  sS[1][wave][lane] = u32x4{pack_lo(sown[0].x, sown[0].y), pack_lo(sown[0].z, sown[0].w),
                            pack_lo(sown[1].x, sown[1].y), pack_lo(sown[1].z, sown[1].w)};
}

__device__ __forceinline__ void fetch_state(u32x4 (*sS)[4][64], int lane, u32x4 (&shi)[4],
                                            u32x4 (&slo)[4]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    shi[s] = sS[0][s][lane];
    slo[s] = sS[1][s][lane];
  }
}

// One chunk of phase 2 for this wave: U, the output rows, the state update.
__device__ __forceinline__ void chunk_step(const ChunkParams& p, const ChunkOps& ops, int c, int b,
                                           int hv, int rb, int wave, int lane, f32x4 (&sown)[2],
                                           u32x4 (&shi)[4], u32x4 (&slo)[4], u32x4 (*sS)[4][64],
                                           uint16_t (*sU)[RB][CH + 8]) {
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  const int t0 = c * CH;

  // (a) U = U~ - W S^T for this wave's 16 token rows x 16 state rows.
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a0 = mfma(ops.whi[s], shi[s], a0);
    a1 = mfma(ops.whi[s], slo[s], a1);
    a2 = mfma(ops.wlo[s], shi[s], a2);
  }
  const f32x4 u = ops.ut - (a0 + a1 + a2);
  const f32x4 ud = ops.ed * u;
  {
    u32x2 hi, lo;
    const int j = wave * 16 + 4 * g4;
    split4(u, hi, lo);
    *reinterpret_cast<u32x2*>(&sU[0][r16][j]) = hi;
    *reinterpret_cast<u32x2*>(&sU[1][r16][j]) = lo;
    split4(ud, hi, lo);
    *reinterpret_cast<u32x2*>(&sU[2][r16][j]) = hi;
    *reinterpret_cast<u32x2*>(&sU[3][r16][j]) = lo;
  }
  lds_barrier();

  // (b) O = diag(gamma) Q S^T + P U.
  f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x4 qa = {ops.q[2 * s].x, ops.q[2 * s].y, ops.q[2 * s + 1].x, ops.q[2 * s + 1].y};
    o0 = mfma(qa, shi[s], o0);
    o1 = mfma(qa, slo[s], o1);
  }
  f32x4 o = ops.eg * (o0 + o1);
  {
    f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = {0.f, 0.f, 0.f, 0.f}, p2 = {0.f, 0.f, 0.f, 0.f};
    // Both j-steps for every wave (P is exactly zero above the diagonal), so
    // the loop has no wave-dependent branch.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 uh = *reinterpret_cast<const u32x4*>(&sU[0][r16][s * 32 + g4 * 8]);
      const u32x4 ul = *reinterpret_cast<const u32x4*>(&sU[1][r16][s * 32 + g4 * 8]);
      p0 = mfma(ops.phi[s], uh, p0);
      p1 = mfma(ops.phi[s], ul, p1);
      p2 = mfma(ops.plo[s], uh, p2);
    }
    o += p0 + p1 + p2;
  }
  {
    const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + wave * 16 + 4 * g4 + e;
      if (t < p.T)
        p.out[(((int64_t)b * p.T + t) * p.Hv + hv) * D + rb * RB + r16] = f32_to_bf16_rne(ov[e]);
    }
  }

  // (c) own state columns: S^T[dk][r] = gamma_C S^T + sum_j K^T[dk][j] Ud[j][r].
  const float gam = ops.egC;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x4 acc = gam * sown[t];
    f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 dh = *reinterpret_cast<const u32x4*>(&sU[2][r16][s * 32 + g4 * 8]);
      const u32x4 dl = *reinterpret_cast<const u32x4*>(&sU[3][r16][s * 32 + g4 * 8]);
      acc = mfma(ops.kt[2 * t + s], dh, acc);
      acc2 = mfma(ops.kt[2 * t + s], dl, acc2);
    }
    sown[t] = acc + acc2;
  }
  publish_state(sown, sS, wave, lane);
  lds_barrier();
  fetch_state(sS, lane, shi, slo);
}

// grid (B*Hv, D / RB), 256 threads.
__global__ __launch_bounds__(256) void chunk_state_kernel(const ChunkParams p) {
  __shared__ u32x4 sS[2][4][64];  // state exchange: hi / lo halves, [owner wave][lane]
  __shared__ __attribute__((aligned(16))) uint16_t sU[4][RB][CH + 8];  // U hi/lo, Ud hi/lo, [r][j]
  const int bh = blockIdx.x;
  const int rb = blockIdx.y;
  const int b = bh / p.Hv;
  const int hv = bh - b * p.Hv;
  const int hk = hv / p.rep;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;

  // Own state columns: sown[t] = S[16rb + r16][32 wave + 16 t + 4 g4 + (0..3)].
  f32x4 sown[2];
  {
    const float* s0 = p.state_in + ((int64_t)bh * D + rb * RB + r16) * D + wave * 32 + 4 * g4;
    sown[0] = *reinterpret_cast<const f32x4*>(s0);
    sown[1] = *reinterpret_cast<const f32x4*>(s0 + 16);
  }
  publish_state(sown, sS, wave, lane);
  ChunkOps opsA;
  load_ops(p, bh, b, hk, 0, rb, wave, lane, opsA);
  lds_barrier();
  // Full state as the B operand of the W / Q products: k-step s holds the
  // columns owned by wave s, in the slot order of the W workspace layout.
  u32x4 shi[4], slo[4];
  fetch_state(sS, lane, shi, slo);

  // Two operand sets in turn: the loads of chunk c + 1 are in flight while
  // chunk c computes, with no register copies between iterations.
  // The prefetch past the last chunk re-reads the last chunk (unconditional
  // loads keep the wait counts exact: no branch merges around them).
  const int last = p.NC - 1;
  ChunkOps opsB;
  for (int c = 0; c < p.NC; c += 2) {
    load_ops(p, bh, b, hk, min(c + 1, last), rb, wave, lane, opsB);
    chunk_step(p, opsA, c, b, hv, rb, wave, lane, sown, shi, slo, sS, sU);
    if (c + 1 >= p.NC) break;
    load_ops(p, bh, b, hk, min(c + 2, last), rb, wave, lane, opsA);
    chunk_step(p, opsB, c + 1, b, hv, rb, wave, lane, sown, shi, slo, sS, sU);
  }
  if (p.final_state != nullptr) {
    float* s1 = p.final_state + ((int64_t)bh * D + rb * RB + r16) * D + wave * 32 + 4 * g4;
    *reinterpret_cast<f32x4*>(s1) = sown[0];
    *reinterpret_cast<f32x4*>(s1 + 16) = sown[1];
  }
}

}  // namespace
}  // namespace dflash

extern "C" size_t dflash_gdn_chunked_prefill_workspace_bytes(int B, int T, int Hv, int Dk, int Dv) {
  using namespace dflash;
  if (B <= 0 || T <= 0 || Hv <= 0 || Dk != D || Dv != D) return 0;
  return (size_t)B * Hv * (size_t)ceil_div(T, CH) * kWsChunk;
}

extern "C" int dflash_gdn_chunked_prefill(const void* q, const void* k, const void* v,
                                          const float* g, const float* beta,
                                          const float* state_in, void* out, float* final_state,
                                          int B, int T, int Hk, int Hv, int Dk, int Dv,
                                          const int64_t* strides, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  using namespace dflash;
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk != 0) return DFLASH_ERR_SHAPE;
  if (Dk != D || Dv != D) return DFLASH_ERR_UNSUPPORTED;
  if (B == 0 || T == 0) return DFLASH_OK;
  if ((int64_t)B * Hv > 65535) return DFLASH_ERR_SHAPE;  // grid.y of phase 1
  if (q == nullptr || k == nullptr || v == nullptr || g == nullptr || beta == nullptr ||
      state_in == nullptr || out == nullptr || workspace == nullptr)
    return DFLASH_ERR_NULL;
  if (workspace_bytes < dflash_gdn_chunked_prefill_workspace_bytes(B, T, Hv, Dk, Dv))
    return DFLASH_ERR_WORKSPACE;
  ChunkParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.g = g;
  p.beta = beta;
  p.state_in = state_in;
  p.out = static_cast<uint16_t*>(out);
  p.final_state = final_state;
  if (strides != nullptr) {
    p.q_sb = strides[0]; p.q_st = strides[1]; p.q_sh = strides[2];
    p.k_sb = strides[3]; p.k_st = strides[4]; p.k_sh = strides[5];
    p.v_sb = strides[6]; p.v_st = strides[7]; p.v_sh = strides[8];
    p.g_sb = strides[9]; p.g_st = strides[10];
    p.b_sb = strides[11]; p.b_st = strides[12];
  } else {
    p.q_sh = D; p.q_st = (int64_t)Hk * D; p.q_sb = (int64_t)T * Hk * D;
    p.k_sh = p.q_sh; p.k_st = p.q_st; p.k_sb = p.q_sb;
    p.v_sh = D; p.v_st = (int64_t)Hv * D; p.v_sb = (int64_t)T * Hv * D;
    p.g_st = Hv; p.g_sb = (int64_t)T * Hv;
    p.b_st = Hv; p.b_sb = (int64_t)T * Hv;
  }
  // 16-byte row loads of q, k, v; float4 state loads and stores.
  if (((uintptr_t)q & 15) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) || (p.q_sb % 8) ||
      (p.q_st % 8) || (p.q_sh % 8) || (p.k_sb % 8) || (p.k_st % 8) || (p.k_sh % 8) ||
      (p.v_sb % 8) || (p.v_st % 8) || (p.v_sh % 8) || ((uintptr_t)g & 3) ||
      ((uintptr_t)beta & 3) || ((uintptr_t)state_in & 15) || ((uintptr_t)final_state & 15) ||
      ((uintptr_t)out & 1) || ((uintptr_t)workspace & 15))
    return DFLASH_ERR_ALIGN;
  p.B = B;
  p.T = T;
  p.Hv = Hv;
  p.rep = Hv / Hk;
  p.NC = (int)ceil_div(T, CH);
  p.ws = static_cast<uint8_t*>(workspace);
  const unsigned nbh = (unsigned)((int64_t)B * Hv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(chunk_prep_kernel, dim3(p.NC, nbh), dim3(256), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(chunk_state_kernel, dim3(nbh, D / RB), dim3(256), 0, s, p);
  return to_status(hipGetLastError());
}
