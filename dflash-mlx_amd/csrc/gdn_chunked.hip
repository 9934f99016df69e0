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
// Phase 2 (chunk_state_kernel, sequential over chunks, one workgroup per
// (head, 16 state rows)): the state stays in registers in fp32; every
// product with an fp32 operand splits it into hi + lo bf16 halves (x = hi +
// lo to about 2^-16 relative) and accumulates hi*hi + hi*lo + lo*hi in fp32,
// so the state keeps fp32-level accuracy over all chunks while running on
// the bf16 matrix cores.  Four state waves each own 32 of the 128 state
// columns: per chunk each forms its partial of W S^T over its columns, the
// partials meet in LDS, each wave reduces one 16-token tile of U and
// publishes U and diag(ED) U as bf16 halves, and each updates its own
// columns of S (two barriers per chunk).  Two output waves compute
// O = diag(EG) Q S^T + P U from the same LDS exchange, off the chain.
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
// Phase-2 state waves per workgroup; each owns 128 / kStateWaves state
// columns of the workgroup's 16 rows (1, 2 or 4), and output waves, each of
// which computes 64 / kOutputWaves of a chunk's output rows (1 or 2).
constexpr int kStateWaves = 4;
constexpr int kOutputWaves = 2;
constexpr int KTP = 72;  // bf16 row pitch of the K^T / V^T tiles in LDS
constexpr int TPF = 68;  // fp32 row pitch of A / T in LDS

// Workspace of one (head, chunk), in bytes.  Every matrix is stored as the
// MFMA operand fragments phase 2 loads: fragment f is 64 lanes x 16 bytes,
// lane l = r + 16g holding row r of the fragment's 16-row tile and, in slot
// t*4+e, column 32s + 16t + 4g + e of k-step s.  That slot order is also the
// order in which a pair of 16x16 result tiles holds its rows, so results feed
// the next product without a shuffle; and each fragment is one 1 KB load of
// eight whole cache lines.
//   W_HI / W_LO: bf16 fragments [4 it][4 s]: W[16it + r][32s+16t+4g+e]
//   Q:           bf16 fragments [4 it][4 s]: Q[16it + r][32s+16t+4g+e] (padded rows zero)
//   KT:          bf16 fragments [8 dt][2 s]: K[32s+16t+4g+e][16dt + r]
//   P_HI / P_LO: bf16 fragments [4 it][2 s]: P[16it + r][32s+16t+4g+e]
//   UT:          fp32 [8 rb][4 it][64 lane][4]: U~[16it + 4(lane/16) + e][16rb + lane%16]
//   EG:          fp32 [64] exp(G_i);  ED: fp32 [64] exp(G_63 - G_i)  (decays)
// Q and KT depend on the key head only: they are stored in the slots of the
// first value head of each key head (hv % rep == 0) and read from there by
// every value head of the group; the other heads' Q / KT slots stay unused.
constexpr size_t kWHi = 0;
constexpr size_t kWLo = kWHi + CH * D * 2;
constexpr size_t kQ = kWLo + CH * D * 2;
constexpr size_t kKT = kQ + CH * D * 2;
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

__device__ __forceinline__ const uint16_t* krow(const ChunkParams& p, int b, int hk, int t) {
  return p.k + b * p.k_sb + (int64_t)t * p.k_st + hk * p.k_sh;
}
__device__ __forceinline__ const uint16_t* qrow(const ChunkParams& p, int b, int hk, int t) {
  return p.q + b * p.q_sb + (int64_t)t * p.q_st + hk * p.q_sh;
}
__device__ __forceinline__ const uint16_t* vrow(const ChunkParams& p, int b, int hv, int t) {
  return p.v + b * p.v_sb + (int64_t)t * p.v_st + hv * p.v_sh;
}

// Column of token `col` (< CH) in row `row` of the K^T / V^T tiles: the
// 16-byte column chunks are XOR-swizzled by bits 3..5 of the row, so the
// transposed writes (one lane per 8-row group, rows 8 apart) spread over the
// LDS banks instead of meeting in one; readers use the same map, so the tile
// holds the same values.  Padding columns (>= CH) are not swizzled.
__device__ __forceinline__ int tcol(int row, int col) { return col ^ (((row >> 3) & 7) << 3); }

__device__ __forceinline__ u32x4 ld16(const void* ptr) { return *reinterpret_cast<const u32x4*>(ptr); }
__device__ __forceinline__ u32x2 ld8(const void* ptr) { return *reinterpret_cast<const u32x2*>(ptr); }
__device__ __forceinline__ f32x4 ldf4(const void* ptr) { return *reinterpret_cast<const f32x4*>(ptr); }

// ------------------------------------------------------------------ phase 1
// grid (NC, B*Hv), 256 threads.
// LDS is held to 53 KB so that three workgroups fit on a CU (the registers
// allow three as well): A (read until T is formed) and V^T (read from the
// U~ products on) share one buffer, V^T staying in registers until the
// inverse is done, and g / beta live in the padding columns of the K^T tile
// (64 .. 67, never read as K^T).
static_assert(sizeof(float) * CH * TPF <= sizeof(uint16_t) * D * KTP, "A fits the V^T buffer");
static_assert(KTP >= CH + 4 && CH <= D, "g and beta fit the K^T padding");
__global__ __launch_bounds__(256) void chunk_prep_kernel(const ChunkParams p) {
  __shared__ __attribute__((aligned(16))) float sT[CH][TPF];
  __shared__ __attribute__((aligned(16))) uint16_t sKT[D][KTP];
  __shared__ __attribute__((aligned(16))) uint16_t sAV[D][KTP];
  float(*sA)[TPF] = reinterpret_cast<float(*)[TPF]>(&sAV[0][0]);
  uint16_t(*sVT)[KTP] = sAV;
  auto sG = [&](int j) -> float& { return *reinterpret_cast<float*>(&sKT[j][CH]); };
  auto sBeta = [&](int j) -> float& { return *reinterpret_cast<float*>(&sKT[j][CH + 2]); };
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

  // All global loads first, so their latencies overlap.  Rows past the
  // chunk's valid tokens read row n-1 and are zeroed by a select (no branch
  // around the loads).
  //  kk / vv: rows 4jq..4jq+3 of K and V, bf16 columns 8 piece .. +7, for
  //           the transposed tiles K^T / V^T;
  //  kf / qf: this wave's 16 token rows of K and Q as MFMA fragments in slot
  //           order (k-step s: columns 32s+4g..+3 and 32s+16+4g..+3).
  const int piece = tid & 15, jq = tid >> 4;
  u32x4 kk[4], vv[4], kf[4], qf[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int jr = min(4 * jq + r, n - 1);
    kk[r] = ld16(krow(p, b, hk, t0 + jr) + piece * 8);
    vv[r] = ld16(vrow(p, b, hv, t0 + jr) + piece * 8);
  }
  const int ti = wave * 16 + r16;
  const bool vi = ti < n;
  {
    const uint16_t* kr = krow(p, b, hk, t0 + min(ti, n - 1)) + 4 * g4;
    const uint16_t* qr = qrow(p, b, hk, t0 + min(ti, n - 1)) + 4 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x2 k0 = ld8(kr + 32 * s), k1 = ld8(kr + 32 * s + 16);
      const u32x2 q0 = ld8(qr + 32 * s), q1 = ld8(qr + 32 * s + 16);
      kf[s] = vi ? u32x4{k0.x, k0.y, k1.x, k1.y} : u32x4{0u, 0u, 0u, 0u};
      qf[s] = vi ? u32x4{q0.x, q0.y, q1.x, q1.y} : u32x4{0u, 0u, 0u, 0u};
    }
  }
  float lg = 0.f, bt = 0.f;
  if (wave == 0 && lane < n) {
    lg = logf(fmaxf(p.g[b * p.g_sb + (int64_t)(t0 + lane) * p.g_st + hv], 1e-38f));
    bt = p.beta[b * p.b_sb + (int64_t)(t0 + lane) * p.b_st + hv];
  }

  // K^T tile (padded tokens zero; V's rows are zeroed here and written as
  // V^T after the inverse): a 4-token x 8-column block per thread,
  // transposed in registers and written as 8-byte rows of 4 tokens.
  {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (4 * jq + r >= n) {
        kk[r] = u32x4{0u, 0u, 0u, 0u};
        vv[r] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const uint32_t k0 = kk[0][x], k1 = kk[1][x], k2 = kk[2][x], k3 = kk[3][x];
      // column 2x: low halves of tokens 0..3; column 2x+1: high halves.
      *reinterpret_cast<u32x2*>(&sKT[piece * 8 + 2 * x][tcol(piece * 8 + 2 * x, 4 * jq)]) =
          u32x2{__builtin_amdgcn_perm(k1, k0, 0x05040100u), __builtin_amdgcn_perm(k3, k2, 0x05040100u)};
      *reinterpret_cast<u32x2*>(&sKT[piece * 8 + 2 * x + 1][tcol(piece * 8 + 2 * x + 1, 4 * jq)]) =
          u32x2{__builtin_amdgcn_perm(k1, k0, 0x07060302u), __builtin_amdgcn_perm(k3, k2, 0x07060302u)};
    }
  }
  // This wave's K fragments, shared (the A operand of the other waves' K K^T
  // and Q K^T tiles); they live in sT's space until T is formed.
  u32x4(*sKf)[64] = reinterpret_cast<u32x4(*)[64]>(&sT[0][0]);
#pragma unroll
  for (int s = 0; s < 4; ++s) sKf[wave * 4 + s][lane] = kf[s];
  // Q and K^T depend on the key head only: the first value head of each key
  // head stores them, the others read that head's (phase 2, qk_base).
  const bool own_qk = hv % p.rep == 0;
  // Q fragments go to the workspace as loaded.
  if (own_qk) {
    u32x4* qw = reinterpret_cast<u32x4*>(ws + kQ);
#pragma unroll
    for (int s = 0; s < 4; ++s) qw[(wave * 4 + s) * 64 + lane] = qf[s];
  }
  // Cumulative log-decay and beta (padded tokens: g = 1, beta = 0).
  if (wave == 0) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(lg, off, 64);
      if (lane >= off) lg += o;
    }
    sG(lane) = lg;
    sBeta(lane) = bt;
    const float lg_end = __shfl(lg, CH - 1, 64);
    reinterpret_cast<float*>(ws + kEG)[lane] = __expf(lg);
    reinterpret_cast<float*>(ws + kED)[lane] = __expf(lg_end - lg);
  }
  __syncthreads();

  // K K^T -> A (strictly lower, scaled) and Q K^T -> P (lower, decay-masked)
  // for this wave's token rows i = 16 wave + r16, computed transposed
  // (A operand = K rows j, B operand = this wave's K / Q rows), so lane
  // (r16, g4) holds columns j = 16 jt + 4 g4 + e: four consecutive entries
  // of row i, written to A as one 16-byte row piece, and tile pair
  // (2s, 2s+1) is exactly P fragment (wave, s).  Tiles above the diagonal
  // are zero (A's are never read).
  {
    const int i = wave * 16 + r16;
    const float gi = sG(i), bi = sBeta(i);
    uint32_t phw[4], plw[4];  // one fragment (8 slots) as hi / lo words
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      if (jt <= wave) {
        f32x4 kq = {0.f, 0.f, 0.f, 0.f}, qq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4 ka = sKf[jt * 4 + s][lane];
          kq = mfma(ka, kf[s], kq);
          qq = mfma(ka, qf[s], qq);
        }
        float av[4], pv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = jt * 16 + 4 * g4 + e;
          const float dec = (j <= i) ? __expf(gi - sG(j)) : 0.f;
          av[e] = (j < i) ? bi * dec * kq[e] : 0.f;
          pv[e] = dec * qq[e];
        }
        *reinterpret_cast<f32x4*>(&sA[i][jt * 16 + 4 * g4]) = f32x4{av[0], av[1], av[2], av[3]};
        phw[(jt & 1) * 2] = pack_hi(pv[0], pv[1]);
        phw[(jt & 1) * 2 + 1] = pack_hi(pv[2], pv[3]);
        plw[(jt & 1) * 2] = pack_lo(pv[0], pv[1]);
        plw[(jt & 1) * 2 + 1] = pack_lo(pv[2], pv[3]);
      } else {
        phw[(jt & 1) * 2] = phw[(jt & 1) * 2 + 1] = 0u;
        plw[(jt & 1) * 2] = plw[(jt & 1) * 2 + 1] = 0u;
      }
      // Phase 2 reads P fragments (it, s) with s < (it < 2 ? 1 : 2).
      if ((jt & 1) && (jt >> 1) < (wave < 2 ? 1 : 2)) {
        const int f = wave * 2 + (jt >> 1);
        reinterpret_cast<u32x4*>(ws + kPHi)[f * 64 + lane] = u32x4{phw[0], phw[1], phw[2], phw[3]};
        reinterpret_cast<u32x4*>(ws + kPLo)[f * 64 + lane] = u32x4{plw[0], plw[1], plw[2], plw[3]};
      }
    }
  }
  // K^T fragments [8 dt][2 s]: 16 bytes per (dk, s, g).
  if (own_qk) {
    uint16_t* kt = reinterpret_cast<uint16_t*>(ws + kKT);
    for (int e = tid; e < D * 8; e += 256) {
      const int dk = e >> 3, s = (e >> 2) & 1, g = e & 3;
      const u32x2 a = *reinterpret_cast<const u32x2*>(&sKT[dk][tcol(dk, 32 * s + 4 * g)]);
      const u32x2 z = *reinterpret_cast<const u32x2*>(&sKT[dk][tcol(dk, 32 * s + 16 + 4 * g)]);
      *reinterpret_cast<u32x4*>(kt + (((dk >> 4) * 2 + s) * 64 + (dk & 15) + 16 * g) * 8) =
          u32x4{a.x, a.y, z.x, z.y};
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
  // V^T tile into the buffer A used (every wave is past its last read of A),
  // transposed in registers as K^T was.
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const uint32_t v0 = vv[0][x], v1 = vv[1][x], v2 = vv[2][x], v3 = vv[3][x];
    *reinterpret_cast<u32x2*>(&sVT[piece * 8 + 2 * x][tcol(piece * 8 + 2 * x, 4 * jq)]) =
        u32x2{__builtin_amdgcn_perm(v1, v0, 0x05040100u), __builtin_amdgcn_perm(v3, v2, 0x05040100u)};
    *reinterpret_cast<u32x2*>(&sVT[piece * 8 + 2 * x + 1][tcol(piece * 8 + 2 * x + 1, 4 * jq)]) =
        u32x2{__builtin_amdgcn_perm(v1, v0, 0x07060302u), __builtin_amdgcn_perm(v3, v2, 0x07060302u)};
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
        const f32x4 ta = *reinterpret_cast<const f32x4*>(&sT[i][j0]);      // two 16-byte reads
        const f32x4 tc = *reinterpret_cast<const f32x4*>(&sT[i][j0 + 4]);  // of T's row piece
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          tb[x] = (x < 4 ? ta[x & 3] : tc[x & 3]) * sBeta(j0 + x);
          tw[x] = tb[x] * __expf(sG(j0 + x));
        }
        u32x4 twh, twl, tbh, tbl;
        split8(tw, twh, twl);
        split8(tb, tbh, tbl);
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int tile = 2 * wave + x;
          const u32x4 ka = *reinterpret_cast<const u32x4*>(&sKT[tile * 16 + r16][tcol(tile * 16 + r16, j0)]);
          aw[x] = mfma(ka, twh, aw[x]);
          aw[x] = mfma(ka, twl, aw[x]);
          const u32x4 vb = *reinterpret_cast<const u32x4*>(&sVT[tile * 16 + r16][tcol(tile * 16 + r16, j0)]);
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
        const int off = ((it * 4 + (tile >> 1)) * 64 + lane) * 8 + (tile & 1) * 4;
        *reinterpret_cast<u32x2*>(whi + off) = hi;
        *reinterpret_cast<u32x2*>(wlo + off) = lo;
        // au: lane holds U~[16 it + 4 g4 + e][16 tile + r16] -> UT[tile][it][lane].
        *reinterpret_cast<f32x4*>(ut + ((tile * 4 + it) * 64 + lane) * 4) = au[x];
      }
    }
  }
}

// ------------------------------------------------------------------ phase 2
// A workgroup owns state rows r = 16rb + (lane % 16) of one head.  The
// state is held as the 8 result tiles of the state update S^T[dk][r] (tile
// dt: lane holds columns 16dt + 4g + e, g = lane / 16), split over the state
// waves by column.  Read pairwise, tiles 2s and 2s+1 are exactly the B
// operand of k-step s of the products with S (slot t*4+e = column
// 32s+16t+4g+e), and the U tiles of the W product are the B operand of P U
// and of the state update in the same way, so the state chain
//   U = U~ - W S^T,  S^T <- gamma_C S^T + K^T diag(ED) U
// is MFMAs, register arithmetic and LDS exchanges.  S and U (as bf16 hi / lo
// operand halves) are double-buffered in LDS for the output waves, which
// compute O = diag(EG) Q S^T + P U between the same two barriers per chunk.

struct UOps {                // state wave, per chunk (loaded at the chunk's start)
  f32x4 ut[4];               // U~[16it + 4g + e][16rb + lane%16]
  f32x4 ed[4];               // exp(G_63 - G) of the same token rows
  float egC;                 // exp(G_63)
};
struct Exchange {            // one chunk's S, U and diag(ED) U operand halves, [k-step][lane]
  u32x4 shi[4][64], slo[4][64];
  u32x4 uh[2][64], ul[2][64];
  u32x4 dh[2][64], dl[2][64];
};

__device__ __forceinline__ void load_u(const uint8_t* wsc, uint32_t lu, uint32_t ld, UOps& o) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    o.ut[it] = ldf4(wsc + kUT + lu + it * 1024);
    o.ed[it] = ldf4(wsc + kED + ld + it * 64);
  }
  o.egC = *reinterpret_cast<const float*>(wsc + kEG + (CH - 1) * 4);
}

// Tiles x0 (slots 0..3) and x1 (slots 4..7) as one B operand, hi and lo halves.
__device__ __forceinline__ void split_pair(f32x4 x0, f32x4 x1, u32x4& hi, u32x4& lo) {
  hi = u32x4{pack_hi(x0.x, x0.y), pack_hi(x0.z, x0.w), pack_hi(x1.x, x1.y), pack_hi(x1.z, x1.w)};
  lo = u32x4{pack_lo(x0.x, x0.y), pack_lo(x0.z, x0.w), pack_lo(x1.x, x1.y), pack_lo(x1.z, x1.w)};
}

// Workgroup barrier that waits for this wave's LDS traffic only: global loads
// in flight stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Output rows 16it + 4g + e (e = 0..3) of column r: bf16, rounded to nearest even.
template <bool GUARD>
__device__ __forceinline__ void store_out(uint16_t* obase, int64_t row_stride, f32x4 o, int row0,
                                          int nvalid) {
  const uint32_t p01 = cvt_pk_bf16(o.x, o.y), p23 = cvt_pk_bf16(o.z, o.w);
  const uint16_t v[4] = {(uint16_t)p01, (uint16_t)(p01 >> 16), (uint16_t)p23, (uint16_t)(p23 >> 16)};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (!GUARD || row0 + e < nvalid) obase[(row0 + e) * row_stride] = v[e];
}

// Workspace of the first value head sharing bh's key head: its slots hold
// the Q and K^T fragments of every value head of the group.
__device__ __forceinline__ const uint8_t* qk_base(const ChunkParams& p, int bh) {
  const int hv = bh % p.Hv;
  return p.ws + (int64_t)(bh - hv % p.rep) * p.NC * kWsChunk;
}

// State wave h of NSW owns state columns [128h/NSW, 128(h+1)/NSW): result
// tiles dt in [8h/NSW, 8(h+1)/NSW) and k-steps s in [4h/NSW, 4(h+1)/NSW) of
// the products with S, and token tiles [4h/NSW, 4(h+1)/NSW) of U.  Per chunk
// it forms its partial W[:, its k] S[:, its k]^T for every token tile and
// hands the other waves theirs through LDS (first barrier); it sums the
// partials of its own token tiles in wave order and publishes U and
// diag(ED) U as bf16 halves (second barrier); then every wave updates its
// own columns of S from the whole diag(ED) U.  The output waves read S after
// the first barrier and U after the second.
template <int NSW>
struct Partials {            // the state waves' W S^T partials, [wave][token tile][lane]
  f32x4 p[NSW][4][64];
};

// The wave index H is a template argument, so which tiles are the wave's own
// is known at compile time (no exec-masked selects around the LDS traffic).
template <int NSW, int H>
__device__ __forceinline__ void state_wave(const ChunkParams& p, int bh, int rb, int lane,
                                           Exchange* xb, Partials<NSW>* xp) {
  constexpr int NT = 8 / NSW;   // own result tiles (state columns / 16)
  constexpr int NS = 4 / NSW;   // own k-steps (state columns / 32)
  constexpr int TPW = 4 / NSW;  // own token tiles of U (reduced by this wave)
  constexpr int dt0 = NT * H, s0 = NS * H, it0 = TPW * H;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  const uint32_t lf = lane * 16;              // operand fragments
  const uint32_t lu = rb * 4096 + lane * 16;  // U~
  const uint32_t ld = g4 * 16;                // ED
  const uint8_t* ws0 = p.ws + (int64_t)bh * p.NC * kWsChunk;
  const uint8_t* wk0 = qk_base(p, bh);
  const int last = p.NC - 1;

  f32x4 sT[NT];
  {
    const float* sp = p.state_in + ((int64_t)bh * D + rb * RB + r16) * D + 4 * g4;
#pragma unroll
    for (int j = 0; j < NT; ++j) sT[j] = ldf4(sp + 16 * (dt0 + j));
  }
  u32x4 whi[4][NS], wlo[4][NS];  // this chunk's W rows, own k-steps
  u32x4 kt[NT][2];               // this chunk's K^T, own tiles
  auto load_w_own = [&](const uint8_t* wsc) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        whi[it][j] = ld16(wsc + kWHi + lf + (it * 4 + s0 + j) * 1024);
        wlo[it][j] = ld16(wsc + kWLo + lf + (it * 4 + s0 + j) * 1024);
      }
    }
  };
  auto load_kt_own = [&](const uint8_t* wsc) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
#pragma unroll
      for (int s = 0; s < 2; ++s) kt[j][s] = ld16(wsc + kKT + lf + ((dt0 + j) * 2 + s) * 1024);
    }
  };
  auto load_u_own = [&](const uint8_t* wsc, UOps& o) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      o.ut[i] = ldf4(wsc + kUT + lu + (it0 + i) * 1024);
      o.ed[i] = ldf4(wsc + kED + ld + (it0 + i) * 64);
    }
    o.egC = *reinterpret_cast<const float*>(wsc + kEG + (CH - 1) * 4);
  };
  // One chunk of the chain.  uo holds this chunk's U~ / decays for the
  // wave's own token tiles (loaded a chunk ahead); un receives the next
  // chunk's.  The loop below runs it twice per trip with the two register
  // sets swapped, so the prefetched values never need a register copy (a
  // copy would wait for the load).
  auto chunk = [&](int c, const UOps& uo, UOps& un) {
    const uint8_t* wsn = ws0 + (int64_t)min(c + 1, last) * kWsChunk;
    Exchange& x = xb[c & 1];
    __builtin_amdgcn_sched_barrier(0);
    load_u_own(ws0 + (int64_t)min(c + 1, last) * kWsChunk, un);
    __builtin_amdgcn_sched_barrier(0);

    // Own columns of S as the B operand (k = state column), hi / lo halves.
    u32x4 shi[NS], slo[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      split_pair(sT[2 * j], sT[2 * j + 1], shi[j], slo[j]);
      x.shi[s0 + j][lane] = shi[j];
      x.slo[s0 + j][lane] = slo[j];
    }
    // Own partial of W S^T for every token tile, the four tiles' accumulation
    // chains interleaved (each tile still sums its terms in the same order):
    // the wave's own tiles stay in registers, the others go to the waves that
    // own them.
    f32x4 acc[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) acc[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int it = 0; it < 4; ++it) acc[it] = mfma(whi[it][j], shi[j], acc[it]);
#pragma unroll
      for (int it = 0; it < 4; ++it) acc[it] = mfma(whi[it][j], slo[j], acc[it]);
#pragma unroll
      for (int it = 0; it < 4; ++it) acc[it] = mfma(wlo[it][j], shi[j], acc[it]);
    }
#pragma unroll
    for (int it = 0; it < 4; ++it)
      if (it / TPW != H) xp->p[H][it][lane] = acc[it];
    __builtin_amdgcn_sched_barrier(0);
    load_w_own(wsn);  // this chunk's W is consumed
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // partials (and S) published

    // Own token tiles: U = U~ - the partials summed in wave order,
    // Ud = diag(ED) U; their hi / lo operand halves go to LDS (U for the
    // output waves, Ud for the state update of every state wave).  Tile it
    // fills words 2(it % 2), +1 of k-step it / 2.
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int it = it0 + i;
      f32x4 sum = H == 0 ? acc[it] : xp->p[0][it][lane];
#pragma unroll
      for (int w = 1; w < NSW; ++w) sum = sum + (w == H ? acc[it] : xp->p[w][it][lane]);
      const f32x4 u = uo.ut[i] - sum;
      const f32x4 ud = uo.ed[i] * u;
      u32x2 hi, lo;
      split4(u, hi, lo);
      const int sk = it >> 1, wd = (it & 1) * 8;  // byte offset of the two words
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(&x.uh[sk][lane]) + wd) = hi;
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(&x.ul[sk][lane]) + wd) = lo;
      split4(ud, hi, lo);
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(&x.dh[sk][lane]) + wd) = hi;
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(&x.dl[sk][lane]) + wd) = lo;
    }
    const float egC = uo.egC;
    lds_barrier();  // chunk c's U and Ud are complete; the partials are read

    // Own columns: S^T = gamma_C S^T + K^T Ud  (K^T exact in bf16: two terms).
    u32x4 dh[2], dl[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      dh[s] = x.dh[s][lane];
      dl[s] = x.dl[s][lane];
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      f32x4 a = egC * sT[j];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        a = mfma(kt[j][s], dh[s], a);
        a = mfma(kt[j][s], dl[s], a);
      }
      sT[j] = a;
    }
    __builtin_amdgcn_sched_barrier(0);
    load_kt_own(wk0 + (int64_t)min(c + 1, last) * kWsChunk);
    __builtin_amdgcn_sched_barrier(0);
  };

  UOps ua, ub;
  load_u_own(ws0, ua);
  load_w_own(ws0);
  load_kt_own(wk0);
  // Chunks past the last re-read the last one: the loads stay unconditional.
  for (int c = 0; c < p.NC; c += 2) {
    chunk(c, ua, ub);
    if (c + 1 < p.NC) chunk(c + 1, ub, ua);  // uniform: NC is the same for every wave
  }
  if (p.final_state != nullptr) {
    float* s1 = p.final_state + ((int64_t)bh * D + rb * RB + r16) * D + 4 * g4;
#pragma unroll
    for (int j = 0; j < NT; ++j) *reinterpret_cast<f32x4*>(s1 + 16 * (dt0 + j)) = sT[j];
  }
}

// Output wave j of NOW computes O = diag(EG) Q S^T + P U for token tiles
// it in [4j/NOW, 4(j+1)/NOW) of each chunk: Q S^T between the state waves'
// two barriers (S is published at the first), P U and the stores after the
// second, so neither half holds the chain up at a barrier.
template <int NOW>
__device__ __forceinline__ void output_wave(const ChunkParams& p, int bh, int rb, int j, int lane,
                                            const Exchange* xb) {
  constexpr int NIT = 4 / NOW;  // own token tiles
  const int it0 = NIT * j;
  const int r16 = lane & 15;
  const int g4 = lane >> 4;
  const uint32_t lf = lane * 16;
  const uint32_t ld = g4 * 16;  // EG
  const int b = bh / p.Hv;
  const int hv = bh - b * p.Hv;
  const uint8_t* ws0 = p.ws + (int64_t)bh * p.NC * kWsChunk;
  const uint8_t* wk0 = qk_base(p, bh);
  const int last = p.NC - 1;
  const int64_t orow = (int64_t)p.Hv * D;  // out row stride (elements)

  // L2 prefetch (output wave 0): the output wave has slack on the chain, so
  // it touches one dword per 128-byte line of chunk c + 3 of this head (its
  // eighth of the lines), for the state waves' W and K^T loads two chunks
  // later.  Each touch is consumed (waited for) one chunk after it is
  // issued, and after that chunk's own loads, so in-order completion never
  // holds them up.
  const uint32_t t0o = min((uint32_t)((rb * 113 + lane) * 128), (uint32_t)(kWsChunk - 4));
  const uint32_t t1o = min((uint32_t)((rb * 113 + min(lane + 64, 112)) * 128), (uint32_t)(kWsChunk - 4));
  // Lines of the Q / K^T range are touched in the key head's slot.
  const uint8_t* t0b = (t0o >= kQ && t0o < kPHi) ? wk0 : ws0;
  const uint8_t* t1b = (t1o >= kQ && t1o < kPHi) ? wk0 : ws0;
  u32x4 q[NIT][4], ph[NIT][2], pl[NIT][2];
  f32x4 eg[NIT];
  auto load_q_own = [&](const uint8_t* wsq, const uint8_t* wsc) {
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int it = it0 + i;
#pragma unroll
      for (int s = 0; s < 4; ++s) q[i][s] = ld16(wsq + kQ + lf + (it * 4 + s) * 1024);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 0 || it >= 2) {  // P tiles 0, 1 hold only k-step 0 (causal)
          ph[i][s] = ld16(wsc + kPHi + lf + (it * 2 + s) * 1024);
          pl[i][s] = ld16(wsc + kPLo + lf + (it * 2 + s) * 1024);
        }
      }
      eg[i] = ldf4(wsc + kEG + ld + it * 64);
    }
  };
  load_q_own(wk0, ws0);
  // The first touches (chunk 2) go after chunk 0's Q / P loads, as in the
  // loop, so the wait for Q / P at the loop head counts the same on entry.
  __builtin_amdgcn_sched_barrier(0);
  uint32_t ta = 0, tb = 0;
  if (j == 0) {
    const int64_t co = (int64_t)min(2, last) * kWsChunk;
    ta = *reinterpret_cast<const uint32_t*>(t0b + co + t0o);
    tb = *reinterpret_cast<const uint32_t*>(t1b + co + t1o);
  }
  __builtin_amdgcn_sched_barrier(0);
  for (int c = 0; c < p.NC; ++c) {
    lds_barrier();  // the state waves have published chunk c's S
    const Exchange& x = xb[c & 1];
    f32x4 o[NIT];
    {
      u32x4 shi[4], slo[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        shi[s] = x.shi[s][lane];
        slo[s] = x.slo[s][lane];
      }
#pragma unroll
      for (int i = 0; i < NIT; ++i) {
        o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          o[i] = mfma(q[i][s], shi[s], o[i]);
          o[i] = mfma(q[i][s], slo[s], o[i]);
        }
        o[i] = eg[i] * o[i];
      }
    }
    lds_barrier();  // ... and U
    u32x4 uh[2], ul[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uh[s] = x.uh[s][lane];
      ul[s] = x.ul[s][lane];
    }
    const int nvalid = p.T - c * CH;
    uint16_t* obase = p.out + ((int64_t)b * p.T + (int64_t)c * CH) * orow + hv * D + rb * RB + r16;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int it = it0 + i;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (s == 0 || it >= 2) {
          o[i] = mfma(ph[i][s], uh[s], o[i]);
          o[i] = mfma(ph[i][s], ul[s], o[i]);
          o[i] = mfma(pl[i][s], uh[s], o[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int it = it0 + i;
      if (nvalid >= CH)
        store_out<false>(obase, orow, o[i], 16 * it + 4 * g4, nvalid);
      else
        store_out<true>(obase, orow, o[i], 16 * it + 4 * g4, nvalid);
    }
    // Loads after the stores: waiting for them next chunk never depends on
    // how many stores the guarded path issued.
    __builtin_amdgcn_sched_barrier(0);
    {  // this chunk's Q, P consumed
      const int64_t cn = (int64_t)min(c + 1, last) * kWsChunk;
      load_q_own(wk0 + cn, ws0 + cn);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j == 0) {
      asm volatile("" ::"v"(ta), "v"(tb));
      const int64_t co = (int64_t)min(c + 3, last) * kWsChunk;
      ta = *reinterpret_cast<const uint32_t*>(t0b + co + t0o);
      tb = *reinterpret_cast<const uint32_t*>(t1b + co + t1o);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("" ::"v"(ta), "v"(tb));
}

// Runs state wave `wave` (uniform) with its index as a template argument.
template <int NSW, int H = 0>
__device__ __forceinline__ void state_dispatch(int wave, const ChunkParams& p, int bh, int rb,
                                               int lane, Exchange* xb, Partials<NSW>* xp) {
  if constexpr (H < NSW) {
    if (wave == H)
      state_wave<NSW, H>(p, bh, rb, lane, xb, xp);
    else
      state_dispatch<NSW, H + 1>(wave, p, bh, rb, lane, xb, xp);
  }
}

// grid 64 * ceil(B*Hv / 8) workgroups of NSW state waves + NOW output waves.
// Workgroup id x -> head
// bh = 8 (x / 64) + x % 8, rows 16 ((x / 8) % 8): the 8 workgroups of a head
// share x % 8, which places them on one XCD (workgroups go round-robin over
// the 8 XCDs), so a chunk's operands come from HBM once and from that XCD's
// L2 for the other 7.  Every wave passes the same number of barriers (two
// per chunk) and they leave together.
template <int NSW, int NOW>
__global__ __launch_bounds__(64 * (NSW + NOW)) void chunk_state_kernel(const ChunkParams p) {
  __shared__ Exchange xb[2];
  __shared__ Partials<NSW> xp;
  const int id = blockIdx.x;
  const int rb = (id >> 3) & 7;
  const int bh = (id >> 6) * 8 + (id & 7);
  if (bh >= p.B * p.Hv) return;  // uniform over the workgroup
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave < NSW)
    state_dispatch<NSW>(wave, p, bh, rb, lane, xb, &xp);
  else
    output_wave<NOW>(p, bh, rb, wave - NSW, lane, xb);
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
  const dim3 sgrid((unsigned)(64 * ceil_div(nbh, 8)));
  hipLaunchKernelGGL((chunk_state_kernel<kStateWaves, kOutputWaves>), sgrid,
                     dim3(64 * (kStateWaves + kOutputWaves)), 0, s, p);
  return to_status(hipGetLastError());
}
