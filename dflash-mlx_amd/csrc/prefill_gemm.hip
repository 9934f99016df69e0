// Prompt-sized GEMMs: out[M, N] = x[M, K] . W[N, K]^T with M = the prompt's
// token count (hundreds to thousands of rows).
//
// The prompt pass of the Qwen3.5 target (Qwen3_5TextModel.__call__ over the
// whole prompt, dflash_mlx/runtime.py:384-390 -> forward_dflash,
// custom_qwen35_model.py:883-1001) runs every projection of every layer (the
// gated-delta in_proj, out_proj, the attention q/k/v and o projections, the
// MLP gate/up and down; :726-736 and mlx-lm's Qwen3NextAttention /
// Qwen3NextMLP Linears) once over all P prompt rows.  There the weight is
// reused by every row, so the work is a dense contraction for the matrix
// cores, not a weight stream: the verify-sized GEMMs (M <= 64) would read
// the whole weight once per 16 rows.
//
// The weight is the verify GEMMs' fragment-tiled copy (dflash_weight_tile_bf16,
// made once at load time: [K/64 k-steps][N/16 row tiles][2 halves][64 lanes]
// [8]), so both GEMM families share one copy and its k-slot order:
//   - A workgroup (4 waves) computes 256 weight rows x 128 activation rows.
//     Wave w owns weight rows 64w .. 64w+63 (4 row tiles) against all 128
//     activation rows (8 column tiles): 32 accumulator tiles of
//     v_mfma_f32_16x16x32_bf16, 64 MFMAs per 64-wide k-step.
//   - A operand (weight): each wave loads its 4 row tiles' 8 fragments of a
//     k-step as 8 contiguous 1 KB loads straight into registers, two k-steps
//     ahead (no LDS: no other wave reads them).
//   - B operand (activations): the workgroup's 128 rows x 64 k of a k-step
//     are loaded once (8 lanes per 128-byte row segment, fully coalesced)
//     into LDS, double buffered with one barrier per k-step, and every wave
//     reads its fragments from there: lane (r16 = l % 16, g = l / 16) of
//     half h holds x[m = 16c + r16][64 ks + 16 g + 8 h .. +7], the k-slots
//     of the weight fragments.
//   - Workgroup -> tile order: consecutive workgroups go to different XCDs
//     (workgroup b runs on XCD b % 8), so each XCD is given a contiguous
//     range of tiles, walked in bands of 8 weight tiles x all activation
//     tiles (activation tile slowest within a band): the 64 workgroups an
//     XCD holds at once share 8 weight tiles and 8 activation tiles in its
//     L2.
//   - Epilogue: bf16 (round to nearest even) out[m][n], or (the _swiglu
//     form) the MLP gating silu(gate) * up of a weight whose 32-row blocks
//     are 16 gate rows then the 16 matching up rows (the verify GEMMs'
//     w_pairs layout): a wave's row tiles 2j and 2j+1 are the gate and up
//     of the same 16 output columns.
// fp32 accumulation in k order (one chain per output, k-steps in order,
// the two halves of a k-step in order).
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

constexpr int kPRows = 256;          // weight rows per workgroup (4 waves x 4 tiles x 16)
constexpr int kPCols = 128;          // activation rows per workgroup (8 tiles x 16)
constexpr int kPPitch = 64 + 8;      // LDS row pitch in bf16 (144 bytes: 16 bytes of padding)
constexpr int kPGroup = 8;           // weight tiles per band of the tile walk

struct PrefillGemmParams {
  const uint16_t* x;  // [M][xs]
  int64_t xs;
  const uint16_t* w;  // fragment-tiled [K/64][N/16][2][64][8]
  uint16_t* out;      // [M][os]
  int64_t os;
  int M, N, K;
  int n_tiles, m_tiles, total, per_xcd;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
  return u32x2{(uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16),
               (uint32_t)f32_to_bf16_rne(c) | ((uint32_t)f32_to_bf16_rne(d) << 16)};
}

// The wave's 8 weight fragments of k-step ks: tile i (clamped to the last row
// tile of the weight; clamped tiles' sums are never stored), half h.
__device__ __forceinline__ void load_a(const PrefillGemmParams& p, int ks, int rt0, int lane,
                                       u32x4 (&a)[8]) {
  const int NT = p.N >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rt = min(rt0 + i, NT - 1);
    const u32x4* src = reinterpret_cast<const u32x4*>(
        p.w + (((int64_t)ks * NT + rt) * 2) * 512 + lane * 8);
    a[2 * i] = __builtin_nontemporal_load(src);
    a[2 * i + 1] = __builtin_nontemporal_load(src + 64);
  }
}

// The workgroup's 128 activation rows of k-step ks: piece e = j * 256 + tid
// is row e / 8, 16-byte column e % 8 (rows past M read row M - 1; their
// sums are never stored).
__device__ __forceinline__ void load_b(const PrefillGemmParams& p, int ks, int m0, int tid,
                                       u32x4 (&b)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = j * 256 + tid;
    const int m = min(m0 + (e >> 3), p.M - 1);
    b[j] = *reinterpret_cast<const u32x4*>(p.x + (int64_t)m * p.xs + ks * 64 + (e & 7) * 8);
  }
}

__device__ __forceinline__ void store_b(uint16_t* sx, int tid, const u32x4 (&b)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = j * 256 + tid;
    *reinterpret_cast<u32x4*>(sx + (e >> 3) * kPPitch + (e & 7) * 8) = b[j];
  }
}

// One k-step: 8 column tiles x 4 row tiles x 2 halves.
__device__ __forceinline__ void mma_step(const uint16_t* sx, int lane, const u32x4 (&a)[8],
                                         f32x4 (&acc)[4][8]) {
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint16_t* row = sx + (16 * c + r16) * kPPitch + 16 * g;
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(row);
    const u32x4 b1 = *reinterpret_cast<const u32x4*>(row + 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[2 * i]), as_bf16x8(b0),
                                                          acc[i][c], 0, 0, 0);
      acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[2 * i + 1]), as_bf16x8(b1),
                                                          acc[i][c], 0, 0, 0);
    }
  }
}

template <bool SWIGLU>
__global__ __launch_bounds__(256, 1) void prefill_gemm_kernel(const PrefillGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sx[2][kPCols * kPPitch];
  const int t = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (t >= p.total) return;
  const int band_tiles = kPGroup * p.m_tiles;
  const int band = t / band_tiles;
  const int in_band = t - band * band_tiles;
  const int gsz = min(kPGroup, p.n_tiles - band * kPGroup);
  const int mt = in_band / gsz;
  const int nt = band * kPGroup + (in_band - mt * gsz);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n0 = nt * kPRows + wave * 64;  // the wave's first weight row
  const int rt0 = n0 >> 4;
  const int m0 = mt * kPCols;
  const int nks = p.K >> 6;

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 a0[8], a1[8], bx[4];
  load_b(p, 0, m0, tid, bx);
  load_a(p, 0, rt0, lane, a0);
  store_b(sx[0], tid, bx);
  if (nks > 1) {
    load_b(p, 1, m0, tid, bx);
    load_a(p, 1, rt0, lane, a1);
  }
  __syncthreads();
  // Two k-steps per trip, so each register ring slot has a fixed name.
  for (int ks = 0; ks < nks; ks += 2) {
    mma_step(sx[0], lane, a0, acc);
    if (ks + 2 < nks) load_a(p, ks + 2, rt0, lane, a0);
    if (ks + 1 < nks) {
      store_b(sx[1], tid, bx);
      if (ks + 2 < nks) load_b(p, ks + 2, m0, tid, bx);
    }
    __syncthreads();
    if (ks + 1 >= nks) break;
    mma_step(sx[1], lane, a1, acc);
    if (ks + 3 < nks) load_a(p, ks + 3, rt0, lane, a1);
    if (ks + 2 < nks) {
      store_b(sx[0], tid, bx);
      if (ks + 3 < nks) load_b(p, ks + 3, m0, tid, bx);
    }
    __syncthreads();
  }

  // Epilogue.  Lane (r16, g) of tile (i, c) holds out[m = m0 + 16c + r16]
  // [n = n0 + 16i + 4g .. +3].
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int m = m0 + 16 * c + r16;
    if (m >= p.M) continue;
    uint16_t* orow = p.out + (int64_t)m * p.os;
    if (SWIGLU) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + 32 * j;  // gate rows n .. n+15, up rows n+16 .. n+31
        if (n >= p.N) continue;
        const f32x4 gt = acc[2 * j][c], up = acc[2 * j + 1][c];
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = gt[e] / (1.f + __expf(-gt[e])) * up[e];
        *reinterpret_cast<u32x2*>(orow + (n >> 1) + 4 * g) = pack4(o[0], o[1], o[2], o[3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 16 * i;
        if (n >= p.N) continue;
        const f32x4 v = acc[i][c];
        *reinterpret_cast<u32x2*>(orow + n + 4 * g) = pack4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

int launch_prefill(const void* x, int64_t x_row_stride, const void* w_tiled, void* out,
                   int64_t out_row_stride, int M, int N, int K, bool swiglu, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || K % 64 != 0 || N % (swiglu ? 32 : 16) != 0)
    return DFLASH_ERR_SHAPE;
  if (x_row_stride < K || out_row_stride < (swiglu ? N / 2 : N)) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_tiled == nullptr || out == nullptr) return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || (x_row_stride % 8) || ((uintptr_t)w_tiled & 15) ||
      ((uintptr_t)out & 7) || (out_row_stride % 4))
    return DFLASH_ERR_ALIGN;
  PrefillGemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  p.w = static_cast<const uint16_t*>(w_tiled);
  p.out = static_cast<uint16_t*>(out);
  p.os = out_row_stride;
  p.M = M; p.N = N; p.K = K;
  p.n_tiles = (int)ceil_div(N, kPRows);
  p.m_tiles = (int)ceil_div(M, kPCols);
  const int64_t total = (int64_t)p.n_tiles * p.m_tiles;
  if (total > (int64_t)INT32_MAX / 2) return DFLASH_ERR_SHAPE;
  p.total = (int)total;
  p.per_xcd = (int)ceil_div(total, 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(8 * p.per_xcd));
  if (swiglu)
    hipLaunchKernelGGL(prefill_gemm_kernel<true>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(prefill_gemm_kernel<false>, grid, dim3(256), 0, s, p);
  return to_status(hipGetLastError());
}

}  // namespace
}  // namespace dflash

extern "C" int dflash_gemm_bf16_tiled_prefill(const void* x, int64_t x_row_stride,
                                              const void* w_tiled, void* out,
                                              int64_t out_row_stride, int M, int N, int K,
                                              void* stream) {
  return dflash::launch_prefill(x, x_row_stride, w_tiled, out, out_row_stride, M, N, K, false,
                                stream);
}

extern "C" int dflash_gemm_bf16_swiglu_tiled_prefill(const void* x, int64_t x_row_stride,
                                                     const void* w_pairs_tiled, void* out,
                                                     int64_t out_row_stride, int M, int N, int K,
                                                     void* stream) {
  return dflash::launch_prefill(x, x_row_stride, w_pairs_tiled, out, out_row_stride, M, N, K,
                                true, stream);
}
