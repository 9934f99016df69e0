// Fused greedy LM head: argmax_v (hidden . W[v]) without materialising the
// logits, feeding the verify accept.
//
// Reference: MLXTargetAdapter.lm_head_argmax(model, hidden_states)
// (dflash_mlx/adapters.py:267-271, "can replace this with a fused top-1
// LM-head kernel"; caller verify_block_parallel_greedy_argmax,
// runtime.py:246-292), followed by longest_prefix_match and the bonus pick
// (runtime.py:41-47, :281-289).
//
// Verify-sized M (= B*T <= 64 hidden rows) makes this a weight stream: W is
// [V, H] bf16 (778 MB at V=151936, H=2560) against 16..64 rows.  Mapping:
//   - MFMA v_mfma_f32_16x16x32_bf16: A = 16 vocab rows, B = 16 hidden rows
//     (L2-resident), fp32 accumulators, one 64-wide k-step = two MFMAs.  A
//     wavefront owns VT 16-row vocab tiles; a 256-thread workgroup 4*VT.
//   - Weight loads are coalesced (8 lanes read a row's full 128-byte k-step
//     line, 8 rows per instruction) and kept D steps ahead in a register
//     ring; the wave bounces each step through a private LDS tile into MFMA
//     fragment layout.  A wave's LDS operations complete in order, so the
//     loop has no barrier (a HIP __syncthreads also waits for every
//     outstanding global load, which drained the prefetch of an earlier
//     LDS-staged version).  Plain loads: with the non-temporal hint each
//     half-line request went to DRAM on its own.
//   - Fragment layout: lane (r16 = l % 16, g = l / 16) holds row r16 and
//     elements 16g .. 16g+15 of the step for both A and B, so the contraction
//     is exact whatever order the hardware gives the k-slots.
//   - Epilogue: the accumulators of tile (vt, mt) (lane l: hidden row
//     mt*16 + l % 16, vocab rows 4*(l/16) .. +3) become 64-bit argmax keys
//     (order-preserving value bits << 32 | ~index); the workgroup's best per
//     hidden row goes to keys[row, workgroup], and the accept's finalize
//     kernel merges them, compares the draft and picks the bonus.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "accept_common.h"
#include "dflash_gdn.h"
#include "device_common.h"
#include "host_common.h"

namespace dflash {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kLmThreads = 256;   // 4 wavefronts
constexpr int kKStep = 64;        // k per step: two 16x16x32 MFMAs
constexpr int kMaxLmRows = 64;    // hidden rows (B*N) per call
constexpr int kVT = 2;            // 16-row vocab tiles per wavefront
constexpr int kVocabRowsPerBlock = (kLmThreads / 64) * kVT * 16;
// Bytes per row of a wave's LDS transpose tile: one k-step (128 B) plus 16 B
// so the 16 rows of one fragment read spread over the LDS banks.
constexpr int kTileRowBytes = 128 + 16;

struct LmParams {
  const uint16_t* hidden;
  int64_t hs;  // hidden row stride (elements)
  const uint16_t* weight;
  int64_t ws;  // weight row stride (elements)
  int M, H, V;
  int nwg;         // workgroups (= gridDim.x)
  uint64_t* keys;  // [M, nwg]
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 x) { return __builtin_bit_cast(bf16x8, x); }

// One k-step of operands for one lane.
template <int MT, int VT>
struct LmStage {
  u32x4 a[2 * VT];  // coalesced weight loads: instruction i reads tile rows 8i .. 8i+7
  u32x4 b[MT][2];   // hidden fragments, two 8-element halves per M tile
};

template <int MT, int VT, int D>
__global__ __launch_bounds__(kLmThreads) void lm_head_argmax_kernel(const LmParams p) {
  __shared__ uint64_t wkeys[kLmThreads / 64][MT * 16];
  __shared__ __attribute__((aligned(16))) unsigned char
      atile[kLmThreads / 64][VT * 16 * kTileRowBytes];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int vwave = blockIdx.x * kVocabRowsPerBlock + wave * VT * 16;

  // Coalesced layout: instruction i reads rows vwave + 8i + lane/8, elements
  // 8*(lane%8) .. +7 of the step.  Tail rows re-read row V-1 (masked later).
  const uint16_t* wrow[2 * VT];
#pragma unroll
  for (int i = 0; i < 2 * VT; ++i) {
    const int v = min(vwave + i * 8 + (lane >> 3), p.V - 1);
    wrow[i] = p.weight + (int64_t)v * p.ws + (lane & 7) * 8;
  }
  // Hidden rows >= M read row M-1 (in bounds); their results are dropped.
  const uint16_t* hrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    hrow[mt] = p.hidden + (int64_t)min(mt * 16 + r16, p.M - 1) * p.hs + g * 16;

  auto load = [&](LmStage<MT, VT>& st, int ks) {
    const int off = ks * kKStep;
#pragma unroll
    for (int i = 0; i < 2 * VT; ++i) st.a[i] = *reinterpret_cast<const u32x4*>(wrow[i] + off);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      st.b[mt][0] = *reinterpret_cast<const u32x4*>(hrow[mt] + off);
      st.b[mt][1] = *reinterpret_cast<const u32x4*>(hrow[mt] + off + 8);
    }
  };

  f32x4 acc[VT][MT];
#pragma unroll
  for (int vt = 0; vt < VT; ++vt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[vt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  unsigned char* tile_lds = atile[wave];

  const int nks = p.H / kKStep;
  LmStage<MT, VT> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nks) load(ring[d], d);

  for (int ks0 = 0; ks0 < nks; ks0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int ks = ks0 + d;
      if (ks < nks) {
        // Coalesced layout -> fragment layout through the wave's LDS tile.
#pragma unroll
        for (int i = 0; i < 2 * VT; ++i)
          *reinterpret_cast<u32x4*>(tile_lds + (i * 8 + (lane >> 3)) * kTileRowBytes + (lane & 7) * 16) =
              ring[d].a[i];
        u32x4 a[VT][2];
#pragma unroll
        for (int vt = 0; vt < VT; ++vt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            a[vt][h] = *reinterpret_cast<const u32x4*>(tile_lds + (vt * 16 + r16) * kTileRowBytes +
                                                       (2 * g + h) * 16);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(a[vt][0]), as_bf16x8(ring[d].b[mt][0]), acc[vt][mt], 0, 0, 0);
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(a[vt][1]), as_bf16x8(ring[d].b[mt][1]), acc[vt][mt], 0, 0, 0);
          }
        if (ks + D < nks) load(ring[d], ks + D);
      }
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    uint64_t best = 0;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const float vals[4] = {acc[vt][mt].x, acc[vt][mt].y, acc[vt][mt].z, acc[vt][mt].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = vwave + vt * 16 + g * 4 + i;
        if (v < p.V) best = u64_max(best, argmax_key(vals[i], v));
      }
    }
    // Merge the 4 lane groups holding the same hidden row.
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const uint32_t lo = __shfl_xor((unsigned)(best & 0xffffffffu), off, 64);
      const uint32_t hi = __shfl_xor((unsigned)(best >> 32), off, 64);
      best = u64_max(best, ((uint64_t)hi << 32) | lo);
    }
    if (g == 0) wkeys[wave][mt * 16 + r16] = best;
  }
  __syncthreads();
  if (threadIdx.x < MT * 16 && (int)threadIdx.x < p.M) {
    uint64_t m = wkeys[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < kLmThreads / 64; ++w) m = u64_max(m, wkeys[w][threadIdx.x]);
    p.keys[(int64_t)threadIdx.x * p.nwg + blockIdx.x] = m;
  }
}

// The same head over a fragment-tiled weight (dflash_weight_tile_bf16:
// [H/64][V/16][2][64 lanes][8], every 64-lane load 1 KB contiguous and
// already in A-fragment layout, so no LDS transpose).  The 4 wavefronts are
// kLmTiledKW k-parts of kLmTiledRG row groups of VT tiles: each k-part sums
// its share of H, the parts merge through LDS, then the argmax epilogue is
// the row-major kernel's.  The fragment loads are nontemporal (whole 1 KB
// runs, each read once): on MI355X at V = 151936, H = 2560, 16 rows this
// streams the 778 MB head at ~6.9 TB/s (~6.1 with ordinary loads) against
// ~5.3 row-major.
constexpr int kLmTiledKW = 2;
constexpr int kLmTiledRG = (kLmThreads / 64) / kLmTiledKW;
constexpr int kLmTiledVT = 4;
static_assert(kLmTiledRG * kLmTiledVT * 16 == kVocabRowsPerBlock,
              "both layouts give a workgroup the same vocab rows (one workspace size)");

template <int MT, int VT, int D, int KW>
__global__ __launch_bounds__(kLmThreads) void lm_head_argmax_tiled_kernel(const LmParams p) {
  constexpr int RG = (kLmThreads / 64) / KW;
  __shared__ uint64_t wkeys[RG][MT * 16];
  __shared__ f32x4 red[RG][KW - 1][VT * MT][64];  // per row group: its k-parts 1 .. KW-1
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int kpart = wave % KW;
  const int rg = wave / KW;
  const int vwave = (blockIdx.x * RG + rg) * VT * 16;
  const int nks_all = p.H / kKStep;
  const int part_len = (nks_all + KW - 1) / KW;
  const int ks_begin = min(kpart * part_len, nks_all);
  const int nks = min(part_len, nks_all - ks_begin);
  const int tiles = p.V / 16;

  // Fragment (k-step, row tile, half) is 1 KB at ((ks * V/16 + rt) * 2 + h) KB;
  // tail tiles re-read the last one (their rows are masked in the epilogue).
  const uint16_t* wrow[VT];
#pragma unroll
  for (int vt = 0; vt < VT; ++vt) {
    const int rt = min(vwave / 16 + vt, tiles - 1);
    wrow[vt] = p.weight + ((int64_t)ks_begin * tiles + rt) * 1024 + lane * 8;
  }
  // Hidden rows >= M read row M-1 (in bounds); their results are dropped.
  const uint16_t* hrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    hrow[mt] = p.hidden + (int64_t)min(mt * 16 + r16, p.M - 1) * p.hs + (int64_t)ks_begin * kKStep + g * 16;

  auto load = [&](LmStage<MT, VT>& st, int ks) {
    const int64_t woff = (int64_t)ks * tiles * 1024;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      st.a[2 * vt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[vt] + woff));
      st.a[2 * vt + 1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[vt] + woff + 512));
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      st.b[mt][0] = *reinterpret_cast<const u32x4*>(hrow[mt] + ks * kKStep);
      st.b[mt][1] = *reinterpret_cast<const u32x4*>(hrow[mt] + ks * kKStep + 8);
    }
  };

  f32x4 acc[VT][MT];
#pragma unroll
  for (int vt = 0; vt < VT; ++vt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[vt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  LmStage<MT, VT> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d < nks) load(ring[d], d);

  for (int ks0 = 0; ks0 < nks; ks0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int ks = ks0 + d;
      if (ks < nks) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(ring[d].a[2 * vt]), as_bf16x8(ring[d].b[mt][0]), acc[vt][mt], 0, 0, 0);
            acc[vt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                as_bf16x8(ring[d].a[2 * vt + 1]), as_bf16x8(ring[d].b[mt][1]), acc[vt][mt], 0, 0, 0);
          }
        if (ks + D < nks) load(ring[d], ks + D);
      }
    }
  }

  // Merge the k-parts into part 0 (every wavefront reaches both barriers).
  if (kpart > 0) {
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[rg][kpart - 1][vt * MT + mt][lane] = acc[vt][mt];
  }
  __syncthreads();
  if (kpart == 0) {
#pragma unroll
    for (int q = 0; q < KW - 1; ++q)
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[vt][mt] += red[rg][q][vt * MT + mt][lane];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      uint64_t best = 0;
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        const float vals[4] = {acc[vt][mt].x, acc[vt][mt].y, acc[vt][mt].z, acc[vt][mt].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = vwave + vt * 16 + g * 4 + i;
          if (v < p.V) best = u64_max(best, argmax_key(vals[i], v));
        }
      }
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const uint32_t lo = __shfl_xor((unsigned)(best & 0xffffffffu), off, 64);
        const uint32_t hi = __shfl_xor((unsigned)(best >> 32), off, 64);
        best = u64_max(best, ((uint64_t)hi << 32) | lo);
      }
      if (g == 0) wkeys[rg][mt * 16 + r16] = best;
    }
  }
  __syncthreads();
  if (threadIdx.x < MT * 16 && (int)threadIdx.x < p.M) {
    uint64_t m = wkeys[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < RG; ++w) m = u64_max(m, wkeys[w][threadIdx.x]);
    p.keys[(int64_t)threadIdx.x * p.nwg + blockIdx.x] = m;
  }
}

int lm_blocks(int V) { return (int)ceil_div(V, kVocabRowsPerBlock); }

// Prefetch depth of the tiled kernel per M-tile count.
template <int MT>
constexpr int lm_tiled_depth() { return MT == 1 ? 4 : (MT == 2 ? 3 : 2); }

template <int MT>
hipError_t launch_tiled_mt(const LmParams& p, hipStream_t s) {
  hipLaunchKernelGGL((lm_head_argmax_tiled_kernel<MT, kLmTiledVT, lm_tiled_depth<MT>(), kLmTiledKW>),
                     dim3(p.nwg), dim3(kLmThreads), 0, s, p);
  return hipGetLastError();
}

// Prefetch depth per M-tile count (operand ring of ~100 VGPRs per lane).
template <int MT>
constexpr int lm_depth() { return MT == 1 ? 6 : (MT == 2 ? 4 : 2); }

template <int MT>
hipError_t launch_mt(const LmParams& p, hipStream_t s) {
  hipLaunchKernelGGL((lm_head_argmax_kernel<MT, kVT, lm_depth<MT>()>), dim3(p.nwg),
                     dim3(kLmThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace
}  // namespace dflash

extern "C" size_t dflash_lm_head_accept_workspace_bytes(int B, int N, int V) {
  if (B <= 0 || N <= 0 || V <= 0) return 0;
  return sizeof(uint64_t) * (size_t)B * N * dflash::lm_blocks(V);
}

namespace dflash {
namespace {

// Shared by the row-major and tiled entry points: weight_row_stride < 0
// selects the tiled layout (which needs V % 16 == 0).
int lm_head_impl(const void* hidden, int64_t hidden_row_stride, const void* weight,
                 int64_t weight_row_stride, int H, int V, const int32_t* draft,
                 int64_t draft_stride, int n_draft, int32_t* posterior, int32_t* matched,
                 int32_t* bonus, int B, int N, void* workspace, size_t workspace_bytes,
                 void* stream) {
  const bool tiled = weight_row_stride < 0;
  if (B < 0 || N <= 0 || H <= 0 || V <= 0 || n_draft < 0) return DFLASH_ERR_SHAPE;
  if ((int64_t)B * N > kMaxLmRows) return DFLASH_ERR_UNSUPPORTED;
  if (H % kKStep != 0) return DFLASH_ERR_UNSUPPORTED;
  if (tiled && V % 16 != 0) return DFLASH_ERR_UNSUPPORTED;
  if (hidden_row_stride < H || (!tiled && weight_row_stride < H)) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  if (hidden == nullptr || weight == nullptr || workspace == nullptr) return DFLASH_ERR_NULL;
  if (n_draft > 0 && draft == nullptr) return DFLASH_ERR_NULL;
  if (posterior == nullptr && matched == nullptr && bonus == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)hidden & 15) || ((uintptr_t)weight & 15) || (hidden_row_stride % 8) ||
      (!tiled && (weight_row_stride % 8)) || ((uintptr_t)workspace & 7))
    return DFLASH_ERR_ALIGN;
  if (workspace_bytes < dflash_lm_head_accept_workspace_bytes(B, N, V)) return DFLASH_ERR_WORKSPACE;
  LmParams p{};
  p.hidden = static_cast<const uint16_t*>(hidden);
  p.hs = hidden_row_stride;
  p.weight = static_cast<const uint16_t*>(weight);
  p.ws = tiled ? 0 : weight_row_stride;
  p.M = B * N;
  p.H = H;
  p.V = V;
  p.nwg = lm_blocks(V);
  p.keys = static_cast<uint64_t*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch ((int)ceil_div(p.M, 16)) {
    case 1: e = tiled ? launch_tiled_mt<1>(p, s) : launch_mt<1>(p, s); break;
    case 2: e = tiled ? launch_tiled_mt<2>(p, s) : launch_mt<2>(p, s); break;
    case 3: e = tiled ? launch_tiled_mt<3>(p, s) : launch_mt<3>(p, s); break;
    default: e = tiled ? launch_tiled_mt<4>(p, s) : launch_mt<4>(p, s); break;
  }
  if (e != hipSuccess) return (int)e;
  return to_status(launch_accept_finalize(p.keys, p.nwg, B, N, draft, draft_stride, n_draft,
                                          posterior, matched, bonus, s));
}

}  // namespace
}  // namespace dflash

extern "C" int dflash_lm_head_greedy_accept(const void* hidden, int64_t hidden_row_stride,
                                            const void* weight, int64_t weight_row_stride,
                                            int H, int V, const int32_t* draft,
                                            int64_t draft_stride, int n_draft,
                                            int32_t* posterior, int32_t* matched,
                                            int32_t* bonus, int B, int N, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  if (weight_row_stride < 0) return DFLASH_ERR_SHAPE;
  return dflash::lm_head_impl(hidden, hidden_row_stride, weight, weight_row_stride, H, V, draft,
                              draft_stride, n_draft, posterior, matched, bonus, B, N, workspace,
                              workspace_bytes, stream);
}

extern "C" int dflash_lm_head_greedy_accept_tiled(const void* hidden, int64_t hidden_row_stride,
                                                  const void* weight_tiled, int H, int V,
                                                  const int32_t* draft, int64_t draft_stride,
                                                  int n_draft, int32_t* posterior,
                                                  int32_t* matched, int32_t* bonus, int B, int N,
                                                  void* workspace, size_t workspace_bytes,
                                                  void* stream) {
  return dflash::lm_head_impl(hidden, hidden_row_stride, weight_tiled, -1, H, V, draft,
                              draft_stride, n_draft, posterior, matched, bonus, B, N, workspace,
                              workspace_bytes, stream);
}
