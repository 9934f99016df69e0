// Verify-sized GEMMs: out[M, N] = x[M, K] . W[N, K]^T with M = B*T <= 64.
//
// Every projection of the hybrid target's verify step (the stacked
// gated-delta in_proj, out_proj, the attention q/k/v and o projections, the
// MLP gate/up and down; dflash_mlx/custom_qwen35_model.py:726-736 and the
// Linear layers of mlx-lm Qwen3NextAttention / Qwen3NextMLP) is this shape: a
// stream of the bf16 weight against 16 activation rows.  The kernel is built
// for the stream:
//   - A workgroup (4 waves) owns 64 * VT consecutive weight rows and a range
//     of k-steps (split-K grid dimension); each wave owns 16 * VT rows.
//   - Weight loads are coalesced (8 lanes read one row's 128-byte k-step line,
//     8 rows per load instruction) and run D k-steps ahead in a register
//     ring; each step goes through the wave's private LDS tile into MFMA
//     fragment order (no barrier: a wave's LDS operations complete in order).
//   - v_mfma_f32_16x16x32_bf16 with A = 16 weight rows, B = 16 activation
//     rows (L2-resident); fp32 accumulation; lane (r16 = l % 16, g = l / 16)
//     holds elements 16g .. 16g+15 of the 64-wide step for both operands, so
//     the contraction is exact whatever order the hardware gives the k-slots.
//   - Tiled weights (dflash_weight_tile_bf16, once at load time): the weight
//     stored as those A fragments, [K/64 k-steps][N/16 row tiles][2 halves]
//     [64 lanes][8], so every fragment is one contiguous 1 KB load straight
//     into MFMA registers (no LDS step; nontemporal loads, measured 2-7 %
//     faster per projection than ordinary ones), and the workgroups in flight, which
//     walk their k-ranges in step, read within a narrow window of memory (a
//     few pages) rather than each in its own region.  Same k-slots, so the
//     same sums, bit for bit, as the row-major path.
//   - Epilogue, nsplit == 1 requested: bf16 (round to nearest even) into
//     out, or (dflash_gemm_bf16_swiglu) the MLP gating silu(gate) * up of a
//     weight whose 32-row blocks are 16 gate rows then the 16 matching up
//     rows: a wave's two row tiles are then the gate and up of the same
//     output columns, and the gate|up product never leaves registers.  nsplit > 1 requested: fp32 partial sums into
//     out_f32[split][M][N] for the splits actually used (see
//     dflash_gemm_splits); the consumer sums them (dflash_add_rmsnorm_splitk,
//     dflash_splitk_reduce).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kGThreads = 256;
constexpr int kGKStep = 64;
constexpr int kGTileRowBytes = 128 + 16;

struct GemmParams {
  const uint16_t* x;
  int64_t xs;  // activation row stride (elements)
  const uint16_t* w;
  int64_t ws;  // weight row stride (elements)
  uint16_t* out;
  int64_t os;  // output row stride (elements)
  float* part;  // [nsplit][M][N] when f32_out
  int M, N, K, nsplit, ks_per_split, f32_out;
  int swiglu;  // bf16 epilogue silu(tile 0) * tile 1 into column block N/2 (VT == 2)
  // fin (KW == 16, one 16-column tile per workgroup): the projection's output
  // r = bf16(x . w^T) is added to the residual stream, h = bf16(resid + r)
  // to h_out (and hc), and the tile's per-row sum of h^2 goes to
  // row_sumsq[tile][m]; nothing else is stored.
  int fin;
  const uint16_t* resid;  // [M][N], may alias h_out
  uint16_t* h_out;        // [M][N]
  uint16_t* hc;           // [M] rows of stride hc_stride, or null
  int64_t hc_stride;
  float* row_sumsq;       // [N / 16][M]
  // NRM kernels: x holds h, and the B operand is the RMSNorm output
  // bf16((h * inv[m]) * nw[k]) with inv[m] = 1 / sqrt(sum_t norm_sumsq[t][m]
  // / K + eps), the sum over the norm_tiles row sums of the producing call.
  const uint16_t* nw;          // [K]
  const float* norm_sumsq;     // [norm_tiles][M]
  int norm_tiles;
  float eps;
  float* row_inv_out;          // [M] or null: inv, stored by workgroup (0, 0)
  // Tail split (KW == 4, one k-split, bf16 epilogue).  U row groups on C CUs
  // make R = U / C whole rounds and a last round of T = U - R*C row groups
  // that would leave most CUs idle while the slowest CUs run a round more.
  // Those T run instead as 4T one-wave units (row group tail_first + u % T,
  // k-quarter u / T), launched first, one per CU.  A unit stores its fp32
  // sums in tail_part and counts itself in tail_count[tile]; the last of a
  // row group's four to arrive adds the quarters in k order, as the
  // workgroup's LDS merge does (same bits), resets the count to zero and
  // runs the epilogue.
  int tail_units, tail_tiles, tail_first;
  float* tail_part;  // [tail_tiles][4 quarters][VT * MT tiles][4 elements][64 lanes]
  int* tail_count;   // [tail_tiles], zero between calls
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <int MT, int VT>
struct GStage {
  u32x4 a[2 * VT];
  u32x4 b[MT][2];
};

// Largest K of an NRM launch: the norm weight of the workgroup's k-range is
// staged in LDS (2 bytes per k).
constexpr int kMaxNormK = 16384;


typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// bf16((h * inv) * w) for 8 packed bf16 h and w: the RMSNorm output, with the
// arithmetic of the standalone add + RMSNorm kernel (the packing is the
// hardware round to nearest even, v_cvt_pk_bf16_f32: the same bits for every
// finite value).
__device__ __forceinline__ u32x4 norm8(u32x4 h, u32x4 w, float inv) {
  const uint32_t hv[4] = {h.x, h.y, h.z, h.w}, wv[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = bf16_lo(hv[i]) * inv * bf16_lo(wv[i]);
    const float b = bf16_hi(hv[i]) * inv * bf16_hi(wv[i]);
    o[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ float bf16r(float x) { return bf16_bits_to_f32(f32_to_bf16_rne(x)); }

// The fin epilogue's residual values, lane (r16, g) of tile (vt, mt):
// resid[m = mt*16 + r16][n = nwave + vt*16 + 4g .. +3] (rows past M and
// tiles past N read clamped addresses; those lanes store nothing).  Loaded
// by wave 0 ahead of its weight ring, so the epilogue does not wait on a
// memory round trip of its own.
template <int MT, int VT>
__device__ __forceinline__ void residual_load(const GemmParams& p, u32x2 (&rr)[MT][VT], int nwave,
                                              int lane) {
  const int r16 = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mc = min(mt * 16 + r16, p.M - 1);
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int n = min(nwave + vt * 16, p.N - 16) + 4 * g;
      rr[mt][vt] = *reinterpret_cast<const u32x2*>(p.resid + (int64_t)mc * p.N + n);
    }
  }
}

// The fin epilogue (KW 8 or 16): wave 0 holds the workgroup's whole tile.
// Lane (r16, g) of tile (vt, mt) holds out[m = mt*16 + r16][n = nwave +
// vt*16 + 4g .. +3].
template <int MT, int VT>
__device__ __forceinline__ void residual_tile(const GemmParams& p, const f32x4 (&acc)[VT][MT],
                                              const u32x2 (&rres)[MT][VT], int nwave, int lane) {
  const int r16 = lane & 15;
  const int g = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r16;
    const bool mv = m < p.M;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int n = nwave + vt * 16 + 4 * g;
      if (n >= p.N) continue;  // N % 16 == 0: whole 16-column tiles
      float ss = 0.f;
      const u32x2 rr = rres[mt][vt];
      float v[4] = {bf16_lo(rr.x), bf16_hi(rr.x), bf16_lo(rr.y), bf16_hi(rr.y)};
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = bf16r(v[i] + bf16r(acc[vt][mt][i]));
      const u32x2 hv = u32x2{(uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16),
                             (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16)};
      if (mv) {
        *reinterpret_cast<u32x2*>(p.h_out + (int64_t)m * p.N + n) = hv;
        if (p.hc != nullptr) *reinterpret_cast<u32x2*>(p.hc + (int64_t)m * p.hc_stride + n) = hv;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = fmaf(v[i], v[i], ss);
      ss += __shfl_xor(ss, 16, 64);  // the row's four column groups, in a fixed tree
      ss += __shfl_xor(ss, 32, 64);
      if (g == 0 && mv) p.row_sumsq[(int64_t)(nwave / 16 + vt) * p.M + m] = ss;
    }
  }
}

// NRM prologue: inv[m] for every row from the producer's per-tile row sums.
// Fixed order whatever M and the launch shape: row m's sums are split over
// 16 groups (group j takes tiles j, j + 16, ...; in order), the 16 group
// sums added in order.  Uses the first 256 threads; ends with a barrier.
__device__ __forceinline__ void norm_inv(const GemmParams& p, float* invp, float* invs) {
  const int t = threadIdx.x;
  for (int m0 = 0; m0 < p.M; m0 += 16) {
    if (t < 256) {
      const int m = m0 + (t & 15), j = t >> 4;
      const int mc = min(m, p.M - 1);
      float part = 0.f;
      for (int t0 = j; t0 < p.norm_tiles; t0 += 16 * 16) {  // 16 loads in flight
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[i] = p.norm_sumsq[(int64_t)min(t0 + 16 * i, p.norm_tiles - 1) * p.M + mc];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (t0 + 16 * i < p.norm_tiles) part += v[i];
      }
      invp[j * 16 + (t & 15)] = part;
    }
    __syncthreads();
    if (t < 16 && m0 + t < p.M) {
      float tot = 0.f;
      for (int j = 0; j < 16; ++j) tot += invp[j * 16 + t];
      const float iv = 1.f / sqrtf(tot / (float)p.K + p.eps);
      invs[m0 + t] = iv;
      if (p.row_inv_out != nullptr && blockIdx.x == 0 && blockIdx.y == 0) p.row_inv_out[m0 + t] = iv;
    }
    __syncthreads();
  }
}

template <int MT, int VT, int D, int KW, bool TILED, bool NRM = false>
__global__ __launch_bounds__(KW >= 8 ? 64 * KW : kGThreads) void skinny_gemm_kernel(const GemmParams p) {
  constexpr int kThreads = KW >= 8 ? 64 * KW : kGThreads;  // KW 8 / 16: one row group
  // the row-major path's per-wave staging tile (tiled weights load straight
  // into registers)
  __shared__ __attribute__((aligned(16))) unsigned char atile[kThreads / 64][TILED ? 16 : VT * 16 * kGTileRowBytes];
  __shared__ f32x4 red[KW > 1 ? KW - 1 : 1][VT * MT][64];
  __shared__ __attribute__((aligned(16))) uint16_t nwl[NRM ? kMaxNormK : 8];
  __shared__ float invp[NRM ? 256 : 1], invs[NRM ? 64 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  constexpr int kRowGroups = (kThreads / 64) / KW;  // row groups per workgroup
  static_assert(KW == 1 || kRowGroups == 1, "red[] holds the k-parts of one row group");
  int kpart = wave % KW;  // this wave's quarter of the k-range
  int rgroup = blockIdx.x;
  bool tail = false;  // a tail unit: wave 0 alone runs k-quarter kpart of row group rgroup
  if (KW == 4 && p.tail_units > 0) {
    if ((int)blockIdx.x < p.tail_units) {
      tail = true;
      rgroup = p.tail_first + (int)blockIdx.x % p.tail_tiles;
      kpart = (int)blockIdx.x / p.tail_tiles;
    } else {
      rgroup = (int)blockIdx.x - p.tail_units;
    }
  }
  const bool idle = tail && wave != 0;  // NRM: still needed for the shared prologue
  if (idle && !NRM) return;
  const int nwave = (rgroup * kRowGroups + wave / KW) * VT * 16;
  const int split = blockIdx.y;
  const int nks_all = p.K / kGKStep;
  const int split_begin = split * p.ks_per_split;
  const int split_len = min(p.ks_per_split, nks_all - split_begin);
  const int part_len = (split_len + KW - 1) / KW;
  const int ks_begin = split_begin + min(kpart * part_len, split_len);
  const int nks = idle ? 0 : min(part_len, split_begin + split_len - ks_begin);

  const uint16_t* wrow[2 * VT];
  if (TILED) {  // fragment (k-step, row tile, half): 1 KB at ((ks * N/16 + rt) * 2 + h) KB
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int rt = min(nwave / 16 + vt, p.N / 16 - 1);  // tail tiles re-read the last
      wrow[2 * vt] = p.w + ((int64_t)ks_begin * (p.N / 16) + rt) * (2 * 512) + lane * 8;
      wrow[2 * vt + 1] = wrow[2 * vt] + 512;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2 * VT; ++i) {
      const int n = min(nwave + i * 8 + (lane >> 3), p.N - 1);  // tail rows re-read row N-1
      wrow[i] = p.w + (int64_t)n * p.ws + (int64_t)ks_begin * kGKStep + (lane & 7) * 8;
    }
  }
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = p.x + (int64_t)min(mt * 16 + r16, p.M - 1) * p.xs + (int64_t)ks_begin * kGKStep + g * 16;
  // this wave's norm-weight pieces: k-step ks at nwb + ks * kGKStep
  const uint16_t* nwb = nwl + (ks_begin - split_begin) * kGKStep + g * 16;

  auto load = [&](GStage<MT, VT>& st, int ks) {
    const int off = ks * kGKStep;
    const int64_t woff = TILED ? (int64_t)ks * (p.N / 16) * 1024 : off;
#pragma unroll
    for (int i = 0; i < 2 * VT; ++i) {
      const u32x4* src = reinterpret_cast<const u32x4*>(wrow[i] + woff);
      st.a[i] = TILED ? __builtin_nontemporal_load(src) : *src;
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      st.b[mt][0] = *reinterpret_cast<const u32x4*>(xrow[mt] + off);
      st.b[mt][1] = *reinterpret_cast<const u32x4*>(xrow[mt] + off + 8);
    }
  };

  f32x4 acc[VT][MT];
#pragma unroll
  for (int vt = 0; vt < VT; ++vt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[vt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  unsigned char* tile = atile[wave];

  u32x2 rres[MT][VT] = {};
  if (KW >= 8 && p.fin && wave == 0) residual_load<MT, VT>(p, rres, nwave, lane);

  GStage<MT, VT> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nks) load(ring[d], d);

  // NRM: with the first weight loads in flight, the norm weight of the
  // split's k-range goes to LDS and inv[m] is formed (every wave is here).
  float inv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) inv[mt] = 1.f;
  if (NRM) {
    const int k0 = split_begin * kGKStep, n8 = split_len * (kGKStep / 8);
    for (int i = threadIdx.x; i < n8; i += kThreads)
      *reinterpret_cast<u32x4*>(nwl + 8 * i) = *reinterpret_cast<const u32x4*>(p.nw + k0 + 8 * i);
    norm_inv(p, invp, invs);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) inv[mt] = invs[min(mt * 16 + r16, p.M - 1)];
  }
  if (idle) return;

  for (int ks0 = 0; ks0 < nks; ks0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int ks = ks0 + d;
      if (ks < nks) {
        u32x4 a[VT][2];
        if (TILED) {
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            a[vt][0] = ring[d].a[2 * vt];
            a[vt][1] = ring[d].a[2 * vt + 1];
          }
        } else {
#pragma unroll
          for (int i = 0; i < 2 * VT; ++i)
            *reinterpret_cast<u32x4*>(tile + (i * 8 + (lane >> 3)) * kGTileRowBytes + (lane & 7) * 16) =
                ring[d].a[i];
#pragma unroll
          for (int vt = 0; vt < VT; ++vt)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              a[vt][h] = *reinterpret_cast<const u32x4*>(tile + (vt * 16 + r16) * kGTileRowBytes + (2 * g + h) * 16);
        }
        u32x4 b[MT][2];
        u32x4 nwv[2] = {};
        if (NRM) {
          nwv[0] = *reinterpret_cast<const u32x4*>(nwb + ks * kGKStep);
          nwv[1] = *reinterpret_cast<const u32x4*>(nwb + ks * kGKStep + 8);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            b[mt][h] = NRM ? norm8(ring[d].b[mt][h], nwv[h], inv[mt]) : ring[d].b[mt][h];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(a[vt][0]), as_bf16x8(b[mt][0]), acc[vt][mt], 0, 0, 0);
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(a[vt][1]), as_bf16x8(b[mt][1]), acc[vt][mt], 0, 0, 0);
          }
        if (ks + D < nks) load(ring[d], ks + D);
      }
    }
  }

  if (KW == 4 && tail) {
    // Cross-workgroup merge by the last arriver (the protocol and the
    // hardware ordering it relies on, which relaxed atomics do not give in
    // the HIP memory model: device_common.h).  The quarters travel as
    // agent-scope atomic stores and loads; the wave waits for its stores to
    // complete before it counts itself, and the last arriver issues its
    // loads only once its count has returned.  No wave waits on another.
    constexpr int kUnit = VT * MT * 4 * 64;  // floats per quarter
    const int tile = rgroup - p.tail_first;
    float* tp = p.tail_part + (int64_t)tile * 4 * kUnit;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          __hip_atomic_store(tp + kpart * kUnit + ((vt * MT + mt) * 4 + i) * 64 + lane, acc[vt][mt][i],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    int arrived = 0;
    if (lane == 0)
      arrived = __hip_atomic_fetch_add(p.tail_count + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    arrived = __shfl(arrived, 0, 64);
    if (arrived != 3) return;
    if (lane == 0) __hip_atomic_store(p.tail_count + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    f32x4 sum[VT][MT];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f32x4 v = acc[vt][mt];
          if (q != kpart) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              v[i] = __hip_atomic_load(tp + q * kUnit + ((vt * MT + mt) * 4 + i) * 64 + lane,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          sum[vt][mt] = q == 0 ? v : sum[vt][mt] + v;
        }
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[vt][mt] = sum[vt][mt];
  } else if (KW > 1) {  // merge the k-quarters: waves 1..KW-1 hand their sums to wave 0
    if (kpart > 0) {
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) red[kpart - 1][vt * MT + mt][lane] = acc[vt][mt];
    }
    __syncthreads();
    if (kpart > 0) return;
#pragma unroll
    for (int q = 0; q < KW - 1; ++q)
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[vt][mt] += red[q][vt * MT + mt][lane];
  }
  if (KW >= 8 && p.fin) {
    residual_tile<MT, VT>(p, acc, rres, nwave, lane);
    return;
  }
  // Lane (r16, g) of tile (vt, mt) holds out[m = mt*16 + r16][n = nwave + vt*16 + 4g .. +3].
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r16;
    if (m >= p.M) continue;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int n = nwave + vt * 16 + 4 * g;
      if (n >= p.N) continue;
      const f32x4 v = acc[vt][mt];
      if (VT == 2 && p.swiglu) {  // rows nwave.. are gate, nwave+16.. the matching up rows
        if (vt == 1) continue;
        const f32x4 u = acc[1][mt];
        const int j = (nwave >> 1) + 4 * g;  // output column
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = v[i] / (1.f + __expf(-v[i])) * u[i];
        *reinterpret_cast<u32x2*>(p.out + (int64_t)m * p.os + j) =
            u32x2{(uint32_t)f32_to_bf16_rne(o[0]) | ((uint32_t)f32_to_bf16_rne(o[1]) << 16),
                  (uint32_t)f32_to_bf16_rne(o[2]) | ((uint32_t)f32_to_bf16_rne(o[3]) << 16)};
        continue;
      }
      if (p.f32_out) {
        float* dst = p.part + ((int64_t)split * p.M + m) * p.N + n;
        if (n + 4 <= p.N && (p.N & 3) == 0) {  // rows 16-byte aligned only when N % 4 == 0
          *reinterpret_cast<f32x4*>(dst) = v;
        } else {
          for (int i = 0; i < min(4, p.N - n); ++i) dst[i] = v[i];
        }
      } else {
        uint16_t* dst = p.out + (int64_t)m * p.os + n;
        if (n + 4 <= p.N) {
          *reinterpret_cast<u32x2*>(dst) =
              u32x2{(uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16),
                    (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16)};
        } else {
          for (int i = 0; i < min(4, p.N - n); ++i) dst[i] = f32_to_bf16_rne(v[i]);
        }
      }
    }
  }
}

// out[m][n] = bf16(sum_s part[s][m][n]).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int nsplit, int M,
                                                            int N, uint16_t* out, int64_t os) {
  const int64_t nv = (int64_t)M * (N / 4);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < nv; e += (int64_t)gridDim.x * 256) {
    const int m = (int)(e / (N / 4));
    const int n = (int)(e - (int64_t)m * (N / 4)) * 4;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nsplit; ++k)
      s += *reinterpret_cast<const f32x4*>(part + ((int64_t)k * M + m) * N + n);
    *reinterpret_cast<u32x2*>(out + (int64_t)m * os + n) =
        u32x2{(uint32_t)f32_to_bf16_rne(s.x) | ((uint32_t)f32_to_bf16_rne(s.y) << 16),
              (uint32_t)f32_to_bf16_rne(s.z) | ((uint32_t)f32_to_bf16_rne(s.w) << 16)};
  }
}

// The gated form over partials in the w_pairs column order (32-column
// blocks: 16 gate columns, then the 16 matching up columns): out[m][j] =
// bf16(silu(g) * u) with g, u the split sums of column 32 (j / 16) + j % 16
// and that column + 16.  Four outputs a thread.
__global__ __launch_bounds__(256) void splitk_swiglu_reduce_kernel(const float* part, int nsplit,
                                                                   int M, int N, uint16_t* out,
                                                                   int64_t os) {
  const int I = N / 2;
  const int64_t nv = (int64_t)M * (I / 4);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < nv; e += (int64_t)gridDim.x * 256) {
    const int m = (int)(e / (I / 4));
    const int j = (int)(e - (int64_t)m * (I / 4)) * 4;
    const int gc = 32 * (j >> 4) + (j & 15);
    f32x4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nsplit; ++k) {
      const float* row = part + ((int64_t)k * M + m) * N;
      g += *reinterpret_cast<const f32x4*>(row + gc);
      u += *reinterpret_cast<const f32x4*>(row + gc + 16);
    }
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = g[i] / (1.f + __expf(-g[i])) * u[i];
    *reinterpret_cast<u32x2*>(out + (int64_t)m * os + j) =
        u32x2{(uint32_t)f32_to_bf16_rne(o[0]) | ((uint32_t)f32_to_bf16_rne(o[1]) << 16),
              (uint32_t)f32_to_bf16_rne(o[2]) | ((uint32_t)f32_to_bf16_rne(o[3]) << 16)};
  }
}

template <int MT, int VT, int KW, bool TILED, bool NRM = false>
hipError_t launch_gemm(const GemmParams& p, hipStream_t s) {
  constexpr int D = MT == 1 ? 4 : (MT == 2 ? 4 : 2);
  constexpr int kThreads = KW >= 8 ? 64 * KW : kGThreads;
  const int rows_per_wg = (kThreads / 64 / KW) * VT * 16;
  dim3 grid((unsigned)ceil_div(p.N, rows_per_wg), (unsigned)p.nsplit);
  if (p.tail_units > 0) grid.x = (unsigned)(p.tail_first + p.tail_units);
  hipLaunchKernelGGL((skinny_gemm_kernel<MT, VT, D, KW, TILED, NRM>), grid, dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

// Workspace of the tail split: the tile counters, then the quarters' fp32
// sums (VT * MT <= 16 tiles of 4 x 64 floats per quarter).
constexpr int kTailMaxTiles = 64;
constexpr size_t kTailCountBytes = 1024;
constexpr size_t kTailWorkspaceBytes = kTailCountBytes + (size_t)kTailMaxTiles * 4 * 16 * 4 * 64 * 4;

// Plans the tail split (GemmParams::tail_*) of a one-split KW == 4 launch of
// rows_per_wg weight rows per workgroup.  A CU streams about the same bytes
// per microsecond however many workgroups share it, so the launch lasts
// about as long as the busiest CU's share: R whole rounds plus a last round
// of T row groups cost R + 1 groups on that CU, while the 4T quarters, one
// per CU, cost R + 1/4.  Used when the quarters fit one per CU (4T <= CUs):
// on MI355X the split was slower wherever they did not (T = 130 and 160 of
// 256 CUs).  No workspace: no tail split.
int plan_tail(GemmParams& p, int rows_per_wg, void* ws, size_t ws_bytes) {
  if (ws == nullptr) return DFLASH_OK;
  if (ws_bytes < kTailWorkspaceBytes) return DFLASH_ERR_WORKSPACE;
  if ((uintptr_t)ws & 255) return DFLASH_ERR_ALIGN;
  const int cus = device_cus();
  if (cus <= 0 || p.nsplit != 1) return DFLASH_OK;
  const int U = (int)ceil_div(p.N, rows_per_wg);
  const int R = U / cus, T = U - R * cus;
  if (T == 0 || 4 * T > cus || T > kTailMaxTiles) return DFLASH_OK;
  p.tail_units = 4 * T;
  p.tail_tiles = T;
  p.tail_first = R * cus;
  p.tail_count = static_cast<int*>(ws);
  p.tail_part = reinterpret_cast<float*>(static_cast<char*>(ws) + kTailCountBytes);
  return DFLASH_OK;
}

template <int VT, int KW, bool TILED = false, bool NRM = false>
hipError_t launch_m(const GemmParams& p, hipStream_t s) {
  const int mt = (int)ceil_div(p.M, 16);
  return mt == 1 ? launch_gemm<1, VT, KW, TILED, NRM>(p, s)
       : mt == 2 ? launch_gemm<2, VT, KW, TILED, NRM>(p, s)
       : mt == 3 ? launch_gemm<3, VT, KW, TILED, NRM>(p, s)
                 : launch_gemm<4, VT, KW, TILED, NRM>(p, s);
}


// dst = src stored as A fragments: dst[((ks * (N/16) + rt) * 2 + h) * 512 + lane * 8 + e]
//   = src[16 rt + lane % 16][64 ks + 16 (lane / 16) + 8 h + e].
__global__ __launch_bounds__(256) void weight_tile_kernel(const uint16_t* src, int64_t ss,
                                                          uint16_t* dst, int N, int K) {
  const int nks = K / kGKStep;
  const int64_t nfrag = (int64_t)(N / 16) * nks * 2 * 64;  // 16-byte pieces
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < nfrag; e += (int64_t)gridDim.x * 256) {
    const int lane = (int)(e & 63);
    const int64_t f = e >> 6;  // (ks * N/16 + rt) * 2 + h
    const int h = (int)(f & 1);
    const int64_t tk = f >> 1;
    const int rt = (int)(tk % (N / 16));
    const int ks = (int)(tk / (N / 16));
    const uint16_t* s = src + (int64_t)(16 * rt + (lane & 15)) * ss + 64 * ks + 16 * (lane >> 4) + 8 * h;
    *reinterpret_cast<u32x4*>(dst + e * 8) = *reinterpret_cast<const u32x4*>(s);
  }
}

}  // namespace
}  // namespace dflash

using namespace dflash;

extern "C" int dflash_gemm_bf16(const void* x, int64_t x_row_stride, const void* w,
                                int64_t w_row_stride, void* out, int64_t out_row_stride, int M,
                                int N, int K, int nsplit, int rows_per_wave, int k_waves,
                                void* stream) {
  if (M < 0 || M > 64 || N <= 0 || K <= 0 || K % kGKStep != 0 || nsplit < 1) return DFLASH_ERR_SHAPE;
  if ((rows_per_wave != 16 && rows_per_wave != 32) || (k_waves != 1 && k_waves != 4))
    return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || (x_row_stride % 8) || (w_row_stride % 8) ||
      x_row_stride < K || w_row_stride < K)
    return DFLASH_ERR_ALIGN;
  GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w);
  p.ws = w_row_stride;
  p.M = M;
  p.N = N;
  p.K = K;
  const int nks = K / kGKStep;
  const int want = std::min(nsplit, nks);
  p.ks_per_split = (int)ceil_div(nks, want);
  p.nsplit = (int)ceil_div(nks, p.ks_per_split);  // no empty split
  p.f32_out = nsplit > 1;  // as requested: the consumer reads fp32 partials
  if (p.f32_out) {
    if ((uintptr_t)out & 15) return DFLASH_ERR_ALIGN;
    p.part = static_cast<float*>(out);
  } else {
    if (((uintptr_t)out & 7) || (out_row_stride % 4) || out_row_stride < N) return DFLASH_ERR_ALIGN;
    p.out = static_cast<uint16_t*>(out);
    p.os = out_row_stride;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (rows_per_wave == 16)
    e = k_waves == 1 ? launch_m<1, 1>(p, s) : launch_m<1, 4>(p, s);
  else
    e = k_waves == 1 ? launch_m<2, 1>(p, s) : launch_m<2, 4>(p, s);
  return to_status(e);
}

extern "C" int dflash_gemm_bf16_swiglu(const void* x, int64_t x_row_stride, const void* w_pairs,
                                       int64_t w_row_stride, void* out, int64_t out_row_stride,
                                       int M, int N, int K, int k_waves, void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 32 != 0 || K <= 0 || K % kGKStep != 0)
    return DFLASH_ERR_SHAPE;
  if (k_waves != 1 && k_waves != 4) return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_pairs == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_pairs & 15) || (x_row_stride % 8) ||
      (w_row_stride % 8) || x_row_stride < K || w_row_stride < K || ((uintptr_t)out & 7) ||
      (out_row_stride % 4) || out_row_stride < N / 2)
    return DFLASH_ERR_ALIGN;
  GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w_pairs);
  p.ws = w_row_stride;
  p.out = static_cast<uint16_t*>(out);
  p.os = out_row_stride;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ks_per_split = K / kGKStep;
  p.nsplit = 1;
  p.swiglu = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return to_status(k_waves == 1 ? launch_m<2, 1>(p, s) : launch_m<2, 4>(p, s));
}

extern "C" int dflash_gemm_splits(int K, int nsplit) {
  if (K <= 0 || K % kGKStep != 0 || nsplit < 1) return DFLASH_ERR_SHAPE;
  const int nks = K / kGKStep;
  nsplit = std::min(nsplit, nks);
  const int per = (int)ceil_div(nks, nsplit);
  return (int)ceil_div(nks, per);
}

extern "C" int dflash_splitk_reduce(const float* partials, int nsplit, int M, int N, void* out,
                                    int64_t out_row_stride, void* stream) {
  if (M < 0 || N <= 0 || N % 4 != 0 || nsplit < 1) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (partials == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)partials & 15) || ((uintptr_t)out & 7) || (out_row_stride % 4)) return DFLASH_ERR_ALIGN;
  const int64_t nv = (int64_t)M * (N / 4);
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(nv, 256), 1024);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     partials, nsplit, M, N, static_cast<uint16_t*>(out), out_row_stride);
  return to_status(hipGetLastError());
}

extern "C" int dflash_splitk_swiglu_reduce(const float* partials, int nsplit, int M, int N,
                                           void* out, int64_t out_row_stride, void* stream) {
  if (M < 0 || N <= 0 || N % 32 != 0 || nsplit < 1) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (partials == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)partials & 15) || ((uintptr_t)out & 7) || (out_row_stride % 4) ||
      out_row_stride < N / 2)
    return DFLASH_ERR_ALIGN;
  const int64_t nv = (int64_t)M * (N / 8);
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(nv, 256), 1024);
  hipLaunchKernelGGL(splitk_swiglu_reduce_kernel, dim3(grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), partials, nsplit, M, N,
                     static_cast<uint16_t*>(out), out_row_stride);
  return to_status(hipGetLastError());
}

extern "C" size_t dflash_weight_tile_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % kGKStep != 0) return 0;
  return (size_t)N * K * 2;
}

extern "C" int dflash_weight_tile_bf16(const void* w, int64_t w_row_stride, void* w_tiled, int N,
                                       int K, void* stream) {
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % kGKStep != 0) return DFLASH_ERR_SHAPE;
  if (w == nullptr || w_tiled == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)w & 15) || ((uintptr_t)w_tiled & 15) || (w_row_stride % 8) || w_row_stride < K)
    return DFLASH_ERR_ALIGN;
  const int64_t nfrag = (int64_t)N * K / 8;
  const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(nfrag, 256), 4096);
  hipLaunchKernelGGL(weight_tile_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(w), w_row_stride, static_cast<uint16_t*>(w_tiled),
                     N, K);
  return to_status(hipGetLastError());
}

extern "C" int dflash_gemm_bf16_tiled(const void* x, int64_t x_row_stride, const void* w_tiled,
                                      void* out, int64_t out_row_stride, int M, int N, int K,
                                      int nsplit, int rows_per_wave, int k_waves, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 16 != 0 || K <= 0 || K % kGKStep != 0 || nsplit < 1)
    return DFLASH_ERR_SHAPE;
  if ((rows_per_wave != 16 && rows_per_wave != 32 && rows_per_wave != 64) ||
      (k_waves != 1 && k_waves != 4))
    return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_tiled == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_tiled & 15) || (x_row_stride % 8) || x_row_stride < K)
    return DFLASH_ERR_ALIGN;
  GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w_tiled);
  p.M = M;
  p.N = N;
  p.K = K;
  const int nks = K / kGKStep;
  const int want = std::min(nsplit, nks);
  p.ks_per_split = (int)ceil_div(nks, want);
  p.nsplit = (int)ceil_div(nks, p.ks_per_split);
  p.f32_out = nsplit > 1;
  if (p.f32_out) {
    if ((uintptr_t)out & 15) return DFLASH_ERR_ALIGN;
    p.part = static_cast<float*>(out);
  } else {
    if (((uintptr_t)out & 7) || (out_row_stride % 4) || out_row_stride < N) return DFLASH_ERR_ALIGN;
    p.out = static_cast<uint16_t*>(out);
    p.os = out_row_stride;
  }
  if (k_waves == 4) {
    const int st = plan_tail(p, rows_per_wave, workspace, workspace_bytes);
    if (st != DFLASH_OK) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (rows_per_wave == 16)
    e = k_waves == 1 ? launch_m<1, 1, true>(p, s) : launch_m<1, 4, true>(p, s);
  else if (rows_per_wave == 32)
    e = k_waves == 1 ? launch_m<2, 1, true>(p, s) : launch_m<2, 4, true>(p, s);
  else
    e = k_waves == 1 ? launch_m<4, 1, true>(p, s) : launch_m<4, 4, true>(p, s);
  return to_status(e);
}

extern "C" size_t dflash_gemm_tail_workspace_bytes(void) { return kTailWorkspaceBytes; }

extern "C" int dflash_gemm_bf16_swiglu_tiled(const void* x, int64_t x_row_stride,
                                             const void* w_pairs_tiled, void* out,
                                             int64_t out_row_stride, int M, int N, int K,
                                             int k_waves, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 32 != 0 || K <= 0 || K % kGKStep != 0)
    return DFLASH_ERR_SHAPE;
  if (k_waves != 1 && k_waves != 4) return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_pairs_tiled == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_pairs_tiled & 15) || (x_row_stride % 8) ||
      x_row_stride < K || ((uintptr_t)out & 7) || (out_row_stride % 4) || out_row_stride < N / 2)
    return DFLASH_ERR_ALIGN;
  GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w_pairs_tiled);
  p.out = static_cast<uint16_t*>(out);
  p.os = out_row_stride;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ks_per_split = K / kGKStep;
  p.nsplit = 1;
  p.swiglu = 1;
  if (k_waves == 4) {
    const int st = plan_tail(p, 32, workspace, workspace_bytes);
    if (st != DFLASH_OK) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  return to_status(k_waves == 1 ? launch_m<2, 1, true>(p, s) : launch_m<2, 4, true>(p, s));
}

// ----------------------------------------------- residual + RMSNorm folded in
// The decoder's `h = h + proj(...)` then `x = rms_norm(h, w)` (the residual
// adds and norms around every projection pair) without a launch of their
// own: the projection that produces the branch adds it to h and stores h's
// per-tile row sums of squares (fin: 16 waves per workgroup split K, so a
// workgroup owns whole output columns and needs nothing from another), and
// the next projection forms the norm's row scale from them and normalizes
// its activation rows on load (NRM).

extern "C" int dflash_gemm_bf16_tiled_residual_norm(const void* x, int64_t x_row_stride,
                                                    const void* w_tiled, int M, int N, int K,
                                                    const void* resid, void* h_out, void* h_copy,
                                                    int64_t h_copy_row_stride, float* row_sumsq,
                                                    void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 16 != 0 || K <= 0 || K % kGKStep != 0) return DFLASH_ERR_SHAPE;
  if (h_copy != nullptr && h_copy_row_stride < N) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_tiled == nullptr || resid == nullptr || h_out == nullptr ||
      row_sumsq == nullptr)
    return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || ((uintptr_t)w_tiled & 15) || (x_row_stride % 8) || x_row_stride < K ||
      ((uintptr_t)resid & 7) || ((uintptr_t)h_out & 7) || ((uintptr_t)h_copy & 7) ||
      (h_copy != nullptr && (h_copy_row_stride % 4)) || ((uintptr_t)row_sumsq & 3))
    return DFLASH_ERR_ALIGN;
  GemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w_tiled);
  p.M = M;
  p.N = N;
  p.K = K;
  p.ks_per_split = K / kGKStep;
  p.nsplit = 1;
  p.fin = 1;
  p.resid = static_cast<const uint16_t*>(resid);
  p.h_out = static_cast<uint16_t*>(h_out);
  p.hc = static_cast<uint16_t*>(h_copy);
  p.hc_stride = h_copy_row_stride;
  p.row_sumsq = row_sumsq;
  return to_status(launch_m<1, 16, true>(p, static_cast<hipStream_t>(stream)));
}

namespace dflash {
namespace {
int set_norm_input(GemmParams& p, const void* h, int64_t h_row_stride, const void* norm_weight,
                   const float* row_sumsq, int norm_tiles, float eps, float* row_inv_out, int K) {
  if (K > kMaxNormK || norm_tiles < 1) return DFLASH_ERR_SHAPE;
  if (h == nullptr || norm_weight == nullptr || row_sumsq == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)h & 15) || ((uintptr_t)norm_weight & 15) || (h_row_stride % 8) ||
      h_row_stride < K || ((uintptr_t)row_sumsq & 3) || ((uintptr_t)row_inv_out & 3))
    return DFLASH_ERR_ALIGN;
  p.x = static_cast<const uint16_t*>(h);
  p.xs = h_row_stride;
  p.nw = static_cast<const uint16_t*>(norm_weight);
  p.norm_sumsq = row_sumsq;
  p.norm_tiles = norm_tiles;
  p.eps = eps;
  p.row_inv_out = row_inv_out;
  return DFLASH_OK;
}
}  // namespace
}  // namespace dflash

extern "C" int dflash_gemm_bf16_tiled_normed(const void* h, int64_t h_row_stride,
                                             const void* norm_weight, const float* row_sumsq,
                                             int norm_tiles, float eps, float* row_inv_out,
                                             const void* w_tiled, void* out, int64_t out_row_stride,
                                             int M, int N, int K, int nsplit, int rows_per_wave,
                                             int k_waves, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 16 != 0 || K <= 0 || K % kGKStep != 0 || nsplit < 1)
    return DFLASH_ERR_SHAPE;
  if ((rows_per_wave != 16 && rows_per_wave != 32 && rows_per_wave != 64) || k_waves != 4)
    return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  GemmParams p{};
  int st = set_norm_input(p, h, h_row_stride, norm_weight, row_sumsq, norm_tiles, eps, row_inv_out, K);
  if (st != DFLASH_OK) return st;
  if (w_tiled == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if ((uintptr_t)w_tiled & 15) return DFLASH_ERR_ALIGN;
  p.w = static_cast<const uint16_t*>(w_tiled);
  p.M = M;
  p.N = N;
  p.K = K;
  const int nks = K / kGKStep;
  p.ks_per_split = (int)ceil_div(nks, std::min(nsplit, nks));
  p.nsplit = (int)ceil_div(nks, p.ks_per_split);
  p.f32_out = nsplit > 1;
  if (p.f32_out) {
    if ((uintptr_t)out & 15) return DFLASH_ERR_ALIGN;
    p.part = static_cast<float*>(out);
  } else {
    if (((uintptr_t)out & 7) || (out_row_stride % 4) || out_row_stride < N) return DFLASH_ERR_ALIGN;
    p.out = static_cast<uint16_t*>(out);
    p.os = out_row_stride;
  }
  st = plan_tail(p, rows_per_wave, workspace, workspace_bytes);
  if (st != DFLASH_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (rows_per_wave == 16) e = launch_m<1, 4, true, true>(p, s);
  else if (rows_per_wave == 32) e = launch_m<2, 4, true, true>(p, s);
  else e = launch_m<4, 4, true, true>(p, s);
  return to_status(e);
}

extern "C" int dflash_gemm_bf16_swiglu_tiled_normed(const void* h, int64_t h_row_stride,
                                                    const void* norm_weight, const float* row_sumsq,
                                                    int norm_tiles, float eps, float* row_inv_out,
                                                    const void* w_pairs_tiled, void* out,
                                                    int64_t out_row_stride, int M, int N, int K,
                                                    int k_waves, void* workspace,
                                                    size_t workspace_bytes, void* stream) {
  if (M < 0 || M > 64 || N <= 0 || N % 32 != 0 || K <= 0 || K % kGKStep != 0)
    return DFLASH_ERR_SHAPE;
  if (k_waves != 4) return DFLASH_ERR_UNSUPPORTED;
  if (M == 0) return DFLASH_OK;
  GemmParams p{};
  int st = set_norm_input(p, h, h_row_stride, norm_weight, row_sumsq, norm_tiles, eps, row_inv_out, K);
  if (st != DFLASH_OK) return st;
  if (w_pairs_tiled == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)w_pairs_tiled & 15) || ((uintptr_t)out & 7) || (out_row_stride % 4) ||
      out_row_stride < N / 2)
    return DFLASH_ERR_ALIGN;
  p.w = static_cast<const uint16_t*>(w_pairs_tiled);
  p.out = static_cast<uint16_t*>(out);
  p.os = out_row_stride;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ks_per_split = K / kGKStep;
  p.nsplit = 1;
  p.swiglu = 1;
  st = plan_tail(p, 32, workspace, workspace_bytes);
  if (st != DFLASH_OK) return st;
  return to_status(launch_m<2, 4, true, true>(p, static_cast<hipStream_t>(stream)));
}
