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
// [8]), so both GEMM families share one copy and its k-slot order.
//
// Two workgroup tiles, chosen per launch: 256 weight rows x 256 activation
// rows (8 waves, both operands staged in LDS by direct loads; the wide tile
// below) or the 256 x 128 tile described here (twice the units, each about
// 0.7 of a wide unit's time), whichever takes fewer rounds of the compute
// units at those costs.  Both add each output's products in the same order,
// so the choice never changes a bit.  The 256 x 128 tile:
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
//   - Operand loads run kPDepth k-steps ahead in register rings, and the
//     activation tile sits in LDS with its 16-byte chunks XOR-swizzled by
//     row (chunk c of row r in slot c ^ (r % 8)), so the 16 rows a
//     fragment read touches fall in different banks.  Measured at the c4
//     shapes (4096 rows): depth 2 / padded rows 578 TFLOP/s over the
//     projections, depth 3 691, depth 3 swizzled 701, depth 4 653.
//   - Split-K (dflash_gemm_bf16_tiled_prefill_splitk): when the output
//     tiles would leave most compute units idle in the last round (N = 2560
//     at 4096 rows is 320 tiles on 256 CUs), each tile's k-range is split
//     and the fp32 partial sums go to the consumer that adds them into the
//     residual stream (dflash_add_rmsnorm_splitk).
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
#include <type_traits>

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
#ifndef DFLASH_PREFILL_DEPTH
#define DFLASH_PREFILL_DEPTH 3
#endif
#ifndef DFLASH_PREFILL_SWIZZLE
#define DFLASH_PREFILL_SWIZZLE 1
#endif
constexpr int kPDepth = DFLASH_PREFILL_DEPTH;      // k-steps of operand loads in flight
constexpr bool kPSwizzle = DFLASH_PREFILL_SWIZZLE;  // swizzled activation tile in LDS

struct PrefillGemmParams {
  const uint16_t* x;  // [M][xs]
  int64_t xs;
  const uint16_t* w;  // fragment-tiled [K/64][nt_w][2][64][8], at the launch's first row tile
  int nt_w;           // row tiles per k-step of the weight (its full row count / 16)
  uint16_t* out;      // [M][os]
  int64_t os;
  float* part;        // split-K: fp32 partial sums [nsplit][M][N] (out unused)
  int M, N, K;
  int n_tiles, m_tiles, tiles, total, per_xcd;
  int nsplit, ks_per_split;
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
        p.w + (((int64_t)ks * p.nt_w + rt) * 2) * 512 + lane * 8);
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

// LDS layout of the activation tile: row r (of kPCols) holds 64 bf16 of the
// k-step in 8 chunks of 16 bytes.  SWZ: chunk c of row r sits at chunk slot
// c ^ (r & 7) of a 128-byte row (no padding); else at slot c of a 144-byte
// row (16 bytes of padding).
template <bool SWZ>
__device__ __forceinline__ int b_off(int row, int chunk) {
  return SWZ ? row * 64 + ((chunk ^ (row & 7)) << 3) : row * kPPitch + (chunk << 3);
}

template <bool SWZ>
__device__ __forceinline__ void store_b(uint16_t* sx, int tid, const u32x4 (&b)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = j * 256 + tid;
    *reinterpret_cast<u32x4*>(sx + b_off<SWZ>(e >> 3, e & 7)) = b[j];
  }
}

// One k-step: 8 column tiles x 4 row tiles x 2 halves.  Lane (r16, g) of
// half h reads chunk 2g + h of row 16c + r16.
template <bool SWZ>
__device__ __forceinline__ void mma_step(const uint16_t* sx, int lane, const u32x4 (&a)[8],
                                         f32x4 (&acc)[4][8]) {
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int row = 16 * c + r16;
    const u32x4 b0 = *reinterpret_cast<const u32x4*>(sx + b_off<SWZ>(row, 2 * g));
    const u32x4 b1 = *reinterpret_cast<const u32x4*>(sx + b_off<SWZ>(row, 2 * g + 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[2 * i]), as_bf16x8(b0),
                                                          acc[i][c], 0, 0, 0);
      acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[2 * i + 1]), as_bf16x8(b1),
                                                          acc[i][c], 0, 0, 0);
    }
  }
}

template <int I>
using Slot = std::integral_constant<int, I>;

// SWIGLU: the gated epilogue.  D: depth of the operand rings (k-steps whose
// global loads are in flight ahead of the one being multiplied).  SWZ: the
// swizzled LDS layout.
template <bool SWIGLU, int D, bool SWZ>
__global__ __launch_bounds__(256, 1) void prefill_gemm_kernel(const PrefillGemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sx[2][kPCols * kPPitch];
  const int u = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (u >= p.total) return;
  // work unit u = split * tiles + t: k-range `split` of output tile t
  const int split = u / p.tiles;
  const int t = u - split * p.tiles;
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
  const int kb = split * p.ks_per_split;  // the unit's first k-step
  const int nks = min(p.ks_per_split, (p.K >> 6) - kb);

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Rings: slot s holds the operands of k-steps s, s + D, s + 2D, ...  Every
  // step issues the same loads, whatever nks is (k-steps past the unit's
  // last re-read the last one; nothing multiplies them), so the compiler's
  // count of loads in flight is exact at each wait.  Loads under a condition
  // make it wait for all of them once per turn of the ring instead.
  const int klast = kb + nks - 1;
  u32x4 a[D][8], bx[D][4];
#pragma unroll
  for (int s = 0; s < D; ++s) {
    load_b(p, min(kb + s, klast), m0, tid, bx[s]);
    load_a(p, min(kb + s, klast), rt0, lane, a[s]);
  }
  store_b<SWZ>(sx[0], tid, bx[0]);
  load_b(p, min(kb + D, klast), m0, tid, bx[0]);
  __syncthreads();
  // k-step i = ks + s multiplies LDS buffer i % 2 with a[s] (when i < nks);
  // then a[s] is refilled with step i + D, step i + 1's activations go from
  // bx[(s+1) % D] to the other LDS buffer, and that slot is refilled with
  // step i + 1 + D.
  auto step = [&](auto S, int ks) {
    constexpr int s = decltype(S)::value;
    constexpr int s1 = (s + 1) % D;
    const int i = ks + s;
    if (s == 0 || i < nks) mma_step<SWZ>(sx[i & 1], lane, a[s], acc);
    load_a(p, min(kb + i + D, klast), rt0, lane, a[s]);
    store_b<SWZ>(sx[(i + 1) & 1], tid, bx[s1]);
    load_b(p, min(kb + i + 1 + D, klast), m0, tid, bx[s1]);
    __syncthreads();
  };
  for (int ks = 0; ks < nks; ks += D) {
    step(Slot<0>{}, ks);
    if (D > 1) step(Slot<(D > 1 ? 1 : 0)>{}, ks);
    if (D > 2) step(Slot<(D > 2 ? 2 : 0)>{}, ks);
    if (D > 3) step(Slot<(D > 3 ? 3 : 0)>{}, ks);
  }

  // Epilogue.  Lane (r16, g) of tile (i, c) holds out[m = m0 + 16c + r16]
  // [n = n0 + 16i + 4g .. +3].
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int m = m0 + 16 * c + r16;
    if (m >= p.M) continue;
    if (p.part != nullptr) {  // split-K: this unit's fp32 sums
      float* prow = p.part + ((int64_t)split * p.M + m) * p.N;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 16 * i;
        if (n < p.N) *reinterpret_cast<f32x4*>(prow + n + 4 * g) = acc[i][c];
      }
      continue;
    }
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

// ---------------------------------------------------------------------------
// Wide tile: 256 weight rows x 256 activation rows per workgroup of 12 waves
// (8 that multiply, 4 that load), both operands staged in LDS by direct
// global -> LDS loads.
//
// Compute wave w < 8 (wr = w / 2, wc = w % 2) owns weight row tiles
// 4 wr .. 4 wr + 3 against activation column tiles 8 wc .. 8 wc + 7: 32
// accumulator tiles, 32 MFMAs per half k-step (32 k), and issues no global
// load.  Its fragments: the weight's straight from the tiled layout (lane
// (r16, g) of fragment (tile, h) holds W[16 tile + r16][64 ks + 16 g + 8 h ..
// +7]) and the activations' with the same k-slots, x[16 c + r16][64 ks +
// 16 g + 8 h .. +7].
//   - Weight stages: one half k-step's 16 fragments (16 KB), loaded by
//     loader waves 8-9 (eight 1 KB loads each, straight from the tiled
//     layout); three slots rotate, stage i + 2 loaded while stage i is
//     multiplied.
//   - Activation stages: one whole k-step of the 256 rows (32 KB, 128 bytes
//     a row), loaded by loader waves 10-11 in chunks of 128 rows: each load
//     takes 8 whole rows (8 lanes a row, 1 KB of whole 128-byte lines) where
//     a load in fragment order would take 16 rows of half lines (the k-slots
//     of half h are every other 16 bytes of the row); measured that way in
//     the prompt pass's own launch order (c4 shapes, 4096 rows, 32 layers)
//     the GEMMs took 25.9 ms against 23.9 ms now.  In LDS a 1 KB block holds
//     8 rows, 16-byte piece c of row r at slot 8 r + (c ^ r): the DMA puts
//     lane l's 16 bytes at slot l, so lane l loads piece (l % 8) ^ (l / 8) of
//     row l / 8, still 128 contiguous bytes a row; a compute wave's fragment
//     read (8 consecutive lanes = 8 rows of one piece) then touches 8
//     different 16-byte bank groups.  Three slots (96 KB): k-step v's two
//     chunks are issued 4 and 3 half k-steps before v is first multiplied.
//   - One barrier per half k-step, which all 12 waves keep; LDS 144 KB.
//     Per k-step the workgroup moves 64 KB for 2 * 256 * 256 * 64 flops,
//     half the bytes per flop of the 256 x 128 tile.
//
// Why loader waves: timing copies at gate|up (N 18432, K 2560, 8192 prompt
// rows; wrong sums) took 307 us with the loads alone, 395 us with the
// fragment reads and MFMAs alone, and 652-700 us with both in the same
// waves — almost no overlap, however deep the stage ring (four stages, the
// same) and even with no fragment reads at all (643 us).  Waves that issue
// loads and MFMAs both lose MFMA issue time to their loads; with the loads
// in waves of their own the same sums took 606-641 us (hipBLASLt on the
// same box 650-690 us).  Two loader waves of 16 loads each measured 1-2 %
// slower than four, wave priorities (either way) changed nothing, whole
// k-step stages for both operands in two slots were slower (674 us).
// Isolated back-to-back launches favour the loader waves by 8-17 %; in the
// prompt pass's launch order (different weights every launch) by ~1 %, and
// there the activation loads' whole lines are what gained (above): the
// GEMMs run at a power-held clock (zeroed activations ran the same
// launches 6 % faster), so fewer cache requests per byte pay.
//
// The first form of this tile (8 waves, each loading its share of every
// stage and multiplying; activation fragments gathered 16 rows of half
// lines a load), at the c4 projections (4096 prompt rows; TFLOP/s, that
// form / the 256 x 128 tile / hipBLASLt on the same box): in_proj 897 / 679
// / 909, q|k|v 790 / 682 / 1109, gate|up (SwiGLU) 1159 / 821 / 1047, out_proj
// split 3 999 / 691 / 1192, o_proj 793 / 568 / 960, down 1194 / 829 / 1333;
// the six shapes 1061 us against 1443 us and hipBLASLt's 1013 us, and the
// sums bit for bit the 256 x 128 tile's (as they are now).  Tried on that
// form: 4 waves of 128 x 128 (256 accumulator registers a lane: the
// compiler shuffles them between register files every step; with the
// accumulators held in AGPRs by the MFMA's own operand constraint, one wave
// a SIMD, 830 us against 712 at gate|up, 8192 rows), 2 / 4 / 5 stages
// (1296 / 1075 / 1097 us), bands of 4 / 8 / 16 weight tiles (within 2 %),
// fragments read a half k-step ahead into a second register set (no gain),
// the loads spread between groups of 8 MFMAs (9 % slower), half the
// fragment reads (wrong sums; 2 % faster: the LDS read bandwidth is not
// what bounds it); on the 12-wave form, 32 x 32 x 16 MFMAs over the same
// bytes (half the operand register reads a flop; a timing copy) ran the
// prompt pass's launch order 6 % slower.  Clocks under load (GRBM_GUI_ACTIVE over the dispatch,
// and rocm-smi during 400 back-to-back calls): that form ran at 1.6-2.2 GHz
// with the matrix cores busy 51 % of the cycles, hipBLASLt at 1.4-1.8 GHz
// with them busy 80-86 %: both are held below the 2.4 GHz peak clock by the
// power drawn.
constexpr int kWRows = 256;                  // weight rows per workgroup
constexpr int kWCols = 256;                  // activation rows per workgroup
constexpr int kWGroup = 16;                  // weight tiles per band of the tile walk
constexpr int kWThreads = 768;               // 8 compute waves + 4 loader waves
constexpr int kWWeightSlot = 16384;          // bytes: a half k-step's 16 weight fragments
constexpr int kWActSlot = 32768;             // bytes: a k-step of 256 activation rows
constexpr int kWActBase = 3 * kWWeightSlot;  // the activation slots follow the weight slots
constexpr int kWLdsU4 = (kWActBase + 3 * kWActSlot) / 16;  // 144 KB

// The 32-bit LDS address of a workgroup-shared object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One direct global -> LDS load of 16 bytes a lane: lane l reads
// sbase + voff (its own byte offset) and its 16 bytes land at LDS address
// lds + 16 l.  Written as an instruction of its own so that the compiler
// does not see a pending LDS write and hold every later LDS read behind all
// of the loads in flight: the waits for these loads are explicit (wait_vm).
// M0 (the LDS base of the load) is set inside the instruction pair; the
// compiler treats M0 as reserved and does not use it in these kernels (the
// generated code's only M0 writes are these), so nothing it holds is lost.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// Wait until at most N loads of this wave are outstanding (loads complete
// in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most n activation chunks (8 loads each) of this wave are
// outstanding; n <= 3.
__device__ __forceinline__ void wait_chunks(int n) {
  if (n <= 0) wait_vm<0>();
  else if (n == 1) wait_vm<8>();
  else if (n == 2) wait_vm<16>();
  else wait_vm<24>();
}

// Weight stage hs (k-step hs / 2, half hs % 2) into the slot at LDS byte
// address `st`, by weight loader l (0-1): fragments 8l .. 8l + 7 (row tiles
// past the weight's last are clamped to it; their sums are never stored),
// 16 bytes a lane in lane order.  l and rt0 are wave-uniform.
__device__ __forceinline__ void wide_load_weights(const PrefillGemmParams& p, int hs, int rt0,
                                                  int l, uint32_t voff, uint32_t st) {
  const int ks = hs >> 1, h = hs & 1;
  const int NT = p.N >> 4;
  const char* wb = reinterpret_cast<const char*>(p.w) + (int64_t)ks * p.nt_w * 2048 + h * 1024;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int f = 8 * l + i;
    dma16(wb + (int64_t)min(rt0 + f, NT - 1) * 2048, voff, st + f * 1024);
  }
}

// One half k-step of the wave's 4 x 8 accumulator tiles: weight fragments
// 4 wr .. 4 wr + 3 from the weight slot `wst`, activation column tiles
// 8 wc .. 8 wc + 7 from the activation slot `ast` (tile c's rows are blocks
// 2c and 2c + 1; boff = the lane's slot for this half, see the kernel), in
// two halves of four (so a compute wave fits three waves a SIMD).
__device__ __forceinline__ void wide_mma(const u32x4* wst, const u32x4* ast, int wr, int wc,
                                         int lane, int boff, f32x4 (&acc)[4][8]) {
  u32x4 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = wst[(4 * wr + i) * 64 + lane];
#pragma unroll
  for (int jh = 0; jh < 2; ++jh) {
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = ast[boff + 2 * (8 * wc + 4 * jh + j) * 64];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][4 * jh + j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(a[i]), as_bf16x8(b[j]), acc[i][4 * jh + j], 0, 0, 0);
  }
}

template <bool SWIGLU>
__global__ __launch_bounds__(kWThreads, 1) void prefill_gemm_wide_kernel(const PrefillGemmParams p) {
  __shared__ __attribute__((aligned(16))) u32x4 lds[kWLdsU4];
  const int u = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (u >= p.total) return;
  // work unit u = split * tiles + t: k-range `split` of output tile t
  const int split = u / p.tiles;
  const int t = u - split * p.tiles;
  const int band_tiles = kWGroup * p.m_tiles;
  const int band = t / band_tiles;
  const int in_band = t - band * band_tiles;
  const int gsz = min(kWGroup, p.n_tiles - band * kWGroup);
  const int mt = in_band / gsz;
  const int nt = band * kWGroup + (in_band - mt * gsz);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wr = wave >> 1, wc = wave & 1;
  const int rt0 = (nt * kWRows) >> 4;  // the workgroup's first weight row tile
  const int m0 = mt * kWCols;
  const int ks0 = split * p.ks_per_split;  // the unit's first k-step
  const int hb = 2 * ks0;                  // ... and half k-step
  const int nhs = 2 * min(p.ks_per_split, (p.K >> 6) - ks0);
  const uint32_t l0 = lds_addr(lds);

  // Half k-step i multiplies weight slot i % 3 and activation slot
  // (i / 2) % 3.  Before it each loader's loads of what it needs must be
  // done and every wave must have passed the barrier, which also frees the
  // slots read at half k-step i - 1 for what the loaders issue next (a
  // compute wave reaches the barrier only after the MFMAs that consumed its
  // reads).  The barrier is the bare instruction: its waits are explicit
  // (the loads by count, the fragment reads by the MFMAs that consumed
  // them), where a workgroup fence would also wait for the later loads.
  // Every wave runs nhs barriers; the loaders then exit and the compute
  // waves store their sums (no barrier after the loop).
  if (wave >= 10) {
    // Activation loader a: chunk j = 2 v + r (the unit's k-step v, rows
    // 128 r .. 128 r + 127) into activation slot v % 3, blocks 16 r + 8 a ..
    // +7 of 8 rows each.  Lane l loads piece (l % 8) ^ (l / 8) of the block's
    // row l / 8 (rows past the last clamped to it; their sums are never
    // stored).  Chunk j is issued at half k-step j - 4: its slot last held
    // k-step v - 3, multiplied up to half k-step 2v - 5.
    const int a = wave - 10;
    const int piece = (lane & 7) ^ (lane >> 3);
    uint32_t off0[8], off1[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int row = m0 + 8 * (8 * a + q) + (lane >> 3);
      off0[q] = (uint32_t)((int64_t)(min(row, p.M - 1) - m0) * p.xs * 2) + 16 * piece;
      off1[q] = (uint32_t)((int64_t)(min(row + 128, p.M - 1) - m0) * p.xs * 2) + 16 * piece;
    }
    const char* xb = reinterpret_cast<const char*>(p.x) + (int64_t)m0 * p.xs * 2;
    auto chunk = [&](int j) {
      const int v = j >> 1;
      const char* src = xb + (int64_t)(ks0 + v) * 128;
      const uint32_t dst = l0 + kWActBase + (v % 3) * kWActSlot + (16 * (j & 1) + 8 * a) * 1024;
      if (j & 1) {
#pragma unroll
        for (int q = 0; q < 8; ++q) dma16(src, off1[q], dst + q * 1024);
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) dma16(src, off0[q], dst + q * 1024);
      }
    };
    for (int j = 0; j < 4 && j < nhs; ++j) chunk(j);
    for (int i = 0; i < nhs; ++i) {
      // chunks issued: min(i + 4, nhs); k-step i / 2 needs chunks < 2 (i / 2) + 2
      wait_chunks(min(i + 4, nhs) - (2 * (i >> 1) + 2));
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (i + 4 < nhs) chunk(i + 4);
    }
    return;
  }
  if (wave >= 8) {
    // Weight loader l: its half of weight stage i + 2 after barrier i.
    // nhs >= 2 (K >= 64): stages 0 and 1 before the loop.
    const int l = wave - 8;
    const uint32_t voff = (uint32_t)(lane * 16);
    wide_load_weights(p, hb, rt0, l, voff, l0);
    wide_load_weights(p, hb + 1, rt0, l, voff, l0 + kWWeightSlot);
    int fill = 2;  // the slot of stage i + 2
    for (int i = 0; i < nhs; ++i) {
      if (i + 1 < nhs) wait_vm<8>();
      else wait_vm<0>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (i + 2 < nhs) wide_load_weights(p, hb + i + 2, rt0, l, voff, l0 + fill * kWWeightSlot);
      fill = fill == 2 ? 0 : fill + 1;
    }
    return;
  }

  f32x4 acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A compute wave whose weight row tiles all lie past the weight's last (in
  // the last weight tile of a launch whose N is not a multiple of 256) keeps
  // the barriers but multiplies nothing: its sums would never be stored.
  const bool live = rt0 + 4 * wr < (p.N >> 4);
  // Lane (r16, g) of an activation fragment of half h is piece 2g + h of the
  // tile's row r16: block r16 / 8 of the tile, slot 8 rr + ((2g + h) ^ rr)
  // with rr = r16 % 8 (in u32x4 units).
  const int r16 = lane & 15, g = lane >> 4, rr = r16 & 7;
  const int boff0 = (r16 >> 3) * 64 + 8 * rr + ((2 * g) ^ rr);
  const int boff1 = (r16 >> 3) * 64 + 8 * rr + ((2 * g + 1) ^ rr);
  auto pipeline = [&](auto MMA) {
    int ws = 0;  // the weight slot of stage i
    for (int i = 0; i < nhs; ++i) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const u32x4* ast = lds + (kWActBase + ((i >> 1) % 3) * kWActSlot) / 16;
      if (decltype(MMA)::value)
        wide_mma(lds + ws * (kWWeightSlot / 16), ast, wr, wc, lane, (i & 1) ? boff1 : boff0, acc);
      ws = ws == 2 ? 0 : ws + 1;
    }
  };
  if (live)
    pipeline(std::true_type{});
  else
    pipeline(std::false_type{});

  // Epilogue.  Lane (r16, g) of tile (i, j) holds out[m = m0 + 16 (8 wc + j)
  // + r16][n = n0 + 16 i + 4 g .. +3], n0 the wave's first weight row.
  const int n0 = nt * kWRows + wr * 64;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int m = m0 + 16 * (8 * wc + j) + r16;
    if (m >= p.M) continue;
    if (p.part != nullptr) {
      float* prow = p.part + ((int64_t)split * p.M + m) * p.N;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = n0 + 16 * i;
        if (n < p.N) *reinterpret_cast<f32x4*>(prow + n + 4 * g) = acc[i][j];
      }
      continue;
    }
    uint16_t* orow = p.out + (int64_t)m * p.os;
    if (SWIGLU) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int n = n0 + 32 * q;  // gate rows n .. n+15, up rows n+16 .. n+31
        if (n >= p.N) continue;
        const f32x4 gt = acc[2 * q][j], up = acc[2 * q + 1][j];
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
        const f32x4 v = acc[i][j];
        *reinterpret_cast<u32x2*>(orow + n + 4 * g) = pack4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

// Rows row0 .. row0+N-1 of a tiled weight of w_rows rows.  nsplit == 0:
// bf16 out (SwiGLU with swiglu); nsplit >= 1: fp32 partial sums of
// dflash_gemm_splits-style k-ranges into part [splits][M][N].
int launch_prefill(const void* x, int64_t x_row_stride, const void* w_tiled, int w_rows, int row0,
                   void* out, int64_t out_row_stride, float* part, int nsplit, int M, int N,
                   int K, bool swiglu, void* stream) {
  const int rows_unit = swiglu ? 32 : 16;
  if (M < 0 || N <= 0 || K <= 0 || K % 64 != 0 || N % rows_unit != 0 || nsplit < 0)
    return DFLASH_ERR_SHAPE;
  if (row0 < 0 || row0 % rows_unit != 0 || w_rows % 16 != 0 || (int64_t)row0 + N > w_rows)
    return DFLASH_ERR_SHAPE;
  if (x_row_stride < K || (nsplit == 0 && out_row_stride < (swiglu ? N / 2 : N)))
    return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (x == nullptr || w_tiled == nullptr || (nsplit == 0 ? out == nullptr : part == nullptr))
    return DFLASH_ERR_NULL;
  if (((uintptr_t)x & 15) || (x_row_stride % 8) || ((uintptr_t)w_tiled & 15))
    return DFLASH_ERR_ALIGN;
  if (nsplit == 0 ? (((uintptr_t)out & 7) || (out_row_stride % 4)) : ((uintptr_t)part & 15))
    return DFLASH_ERR_ALIGN;
  // The wide tile's activation offsets are 32-bit: (256 rows - 1) * row stride.
  if (x_row_stride > ((int64_t)1 << 22)) return DFLASH_ERR_SHAPE;
  PrefillGemmParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.xs = x_row_stride;
  // the first row tile of the range; k-steps stay w_rows / 16 tiles apart
  p.w = static_cast<const uint16_t*>(w_tiled) + (int64_t)(row0 / 16) * 1024;
  p.nt_w = w_rows / 16;
  p.out = static_cast<uint16_t*>(out);
  p.os = out_row_stride;
  p.part = nsplit > 0 ? part : nullptr;
  p.M = M; p.N = N; p.K = K;
  const int nks = K / 64;
  const int want = nsplit > 0 ? std::min(nsplit, nks) : 1;
  p.ks_per_split = (int)ceil_div(nks, want);
  p.nsplit = (int)ceil_div(nks, p.ks_per_split);
  // The tile whose units take less time on the compute units: whole rounds
  // of units, a 256 x 128 unit costing 0.7 of a 256 x 256 one (measured on
  // MI355X at the Qwen3.5-4B projection shapes, 512-2048 prompt rows: the
  // ratio of the two tiles' times at equal rounds was 1.35-1.43, and this
  // rule picked the faster tile in every case measured; the wide tile on a
  // tie).  Both add each output's products in the same order, so the
  // choice never changes a bit.
  const int64_t cus = std::max(device_cus(), 1);
  const int64_t wide_units = ceil_div(N, kWRows) * ceil_div(M, kWCols) * (int64_t)p.nsplit;
  const int64_t narrow_units = ceil_div(N, kPRows) * ceil_div(M, kPCols) * (int64_t)p.nsplit;
  const bool wide = 10 * ceil_div(wide_units, cus) <= 7 * ceil_div(narrow_units, cus);
  p.n_tiles = (int)ceil_div(N, wide ? kWRows : kPRows);
  p.m_tiles = (int)ceil_div(M, wide ? kWCols : kPCols);
  const int64_t tiles = (int64_t)p.n_tiles * p.m_tiles;
  const int64_t total = tiles * p.nsplit;
  if (total > (int64_t)INT32_MAX / 2) return DFLASH_ERR_SHAPE;
  p.tiles = (int)tiles;
  p.total = (int)total;
  p.per_xcd = (int)ceil_div(total, 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(8 * p.per_xcd));
  if (wide) {
    if (swiglu)
      hipLaunchKernelGGL((prefill_gemm_wide_kernel<true>), grid, dim3(kWThreads), 0, s, p);
    else
      hipLaunchKernelGGL((prefill_gemm_wide_kernel<false>), grid, dim3(kWThreads), 0, s, p);
  } else if (swiglu) {
    hipLaunchKernelGGL((prefill_gemm_kernel<true, kPDepth, kPSwizzle>), grid, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((prefill_gemm_kernel<false, kPDepth, kPSwizzle>), grid, dim3(256), 0, s, p);
  }
  return to_status(hipGetLastError());
}

}  // namespace
}  // namespace dflash

extern "C" int dflash_gemm_bf16_tiled_prefill(const void* x, int64_t x_row_stride,
                                              const void* w_tiled, void* out,
                                              int64_t out_row_stride, int M, int N, int K,
                                              void* stream) {
  return dflash::launch_prefill(x, x_row_stride, w_tiled, N, 0, out, out_row_stride, nullptr, 0,
                                M, N, K, false, stream);
}

extern "C" int dflash_gemm_bf16_swiglu_tiled_prefill(const void* x, int64_t x_row_stride,
                                                     const void* w_pairs_tiled, void* out,
                                                     int64_t out_row_stride, int M, int N, int K,
                                                     void* stream) {
  return dflash::launch_prefill(x, x_row_stride, w_pairs_tiled, N, 0, out, out_row_stride,
                                nullptr, 0, M, N, K, true, stream);
}

extern "C" int dflash_gemm_bf16_tiled_prefill_splitk(const void* x, int64_t x_row_stride,
                                                     const void* w_tiled, float* partials,
                                                     int nsplit, int M, int N, int K,
                                                     void* stream) {
  if (nsplit < 1) return DFLASH_ERR_SHAPE;
  return dflash::launch_prefill(x, x_row_stride, w_tiled, N, 0, nullptr, 0, partials, nsplit, M,
                                N, K, false, stream);
}

extern "C" int dflash_gemm_bf16_tiled_prefill_rows(const void* x, int64_t x_row_stride,
                                                   const void* w_tiled, int w_rows, int row0,
                                                   void* out, int64_t out_row_stride,
                                                   float* partials, int nsplit, int M, int N,
                                                   int K, int swiglu, void* stream) {
  if (nsplit < 0 || (nsplit > 0 && swiglu)) return DFLASH_ERR_SHAPE;
  return dflash::launch_prefill(x, x_row_stride, w_tiled, w_rows, row0, out, out_row_stride,
                                partials, nsplit, M, N, K, swiglu != 0, stream);
}
