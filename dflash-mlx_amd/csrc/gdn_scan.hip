// Gated-delta-rule verify scan with per-token state tape (gfx950).
//
// The recurrence is independent per state row (b, hv, dv): row dv of the
// [Dv, Dk] state needs only its own Dk values plus the per-token k, q (shared
// by the head), v[dv], g and beta.  The reference's Metal kernel exploits the
// same independence (dflash_mlx/custom_qwen35_model.py:33-74: one simdgroup
// per dv row, simd_sum over dk).
//
// CDNA4 mapping:
//   - 16 lanes (one DPP row) own one state row; lane s holds Dk/16 fp32 of the
//     row in VGPRs for the whole token loop.  The dk reductions (k.S and q.S)
//     are 4 DPP adds inside the 16-lane row: no LDS, no barriers.
//   - Element ownership is interleaved: chunk c of lane s covers
//     dk = c*16*VEC + s*VEC .. +VEC-1, so one store instruction of a row's 16
//     lanes writes 16*VEC*4 contiguous bytes (256 B for Dk % 64 == 0).
//   - A wavefront holds 4 row groups, each carrying R rows; a 256-thread
//     workgroup covers 16*R consecutive-by-stride rows of one (b, hv) head.
//   - The tape dominates the bytes (T state copies per head), so it is
//     written with non-temporal dwordx4 stores as soon as each token is done.
//   - The inputs of tokens t+1 .. t+4 are in flight while token t is computed.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "argmax_common.h"
#include "conv_window.h"
#include "dflash_gdn.h"
#include "device_common.h"
#include "gdn_prologue_math.h"
#include "host_common.h"

namespace dflash {
namespace {

struct ScanParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g;
  const float* beta;
  const float* state_in;
  uint16_t* out;
  float* final_state;
  float* tape;
  const int32_t* lengths;
  // Fused rollback of the previous verify (null sel_tape: off).  Sequence b
  // starts from sel_tape[a-1, b] with a = clamp(sel_accepted[b % sel_period],
  // 0, sel_T); for a >= 1 that state is also written to state_wb (= the
  // state buffer), so the buffer always ends holding the block's initial state.
  const float* sel_tape;
  const int32_t* sel_accepted;
  float* state_wb;
  int sel_period, sel_T;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int64_t g_sb, g_st;
  int64_t b_sb, b_st;
  int64_t tape_tstride;  // elements between tape[t] and tape[t+1] = B*Hv*Dv*Dk
  int B, T, Hv, Dv;
  int rep;         // Hv / Hk
  int row_blocks;  // Dv / (16 * R)
  int items;       // B * Hv * row_blocks
  // XCD-aware walk (gridDim % 8 == 0, items % 8 == 0): workgroups are
  // dispatched round-robin over the 8 XCDs, so workgroup w runs on XCD w % 8;
  // that XCD walks the contiguous item range [x*items/8, (x+1)*items/8), which
  // keeps all row blocks of a head (and its k/q/v) in one XCD's L2.
  int xcd_items;  // items / 8, or 0 for the plain grid-stride walk
  // Prologue on the fly (the PRO kernels): k, q, v, g and beta of an item
  // are computed from the raw in_proj rows at the item's start instead of
  // being read.  Channels of a row: q (Hk*Dk) | k (Hk*Dk) | v (Hv*Dv).
  const uint16_t* pro_qkv;  // [B, T, *] with the strides below
  int64_t pro_qkv_sb, pro_qkv_st;
  const uint16_t* pro_conv_state;  // [B, K-1, C]
  const uint16_t* pro_conv_w;      // [C, K]
  const uint16_t* pro_a;           // [B, T, Hv] with strides
  const uint16_t* pro_b;
  int64_t pro_a_sb, pro_a_st, pro_b_sb, pro_b_st;
  const float* pro_A_log;         // [Hv]
  const uint16_t* pro_dt_bias;    // [Hv]
  int pro_C, pro_K, pro_Hk;
  float pro_eps, pro_q_scale, pro_k_scale;
  // Greedy-accept argmax in the same launch: the last acc_blocks workgroups
  // (after the scan's, so the scan's dispatch and XCD walk are those of a
  // launch without them; the scan leaves room on every CU for them to run
  // alongside) each reduce one slice of one logits row to its key
  // (argmax_common.h).  acc_blocks == 0: no accept.
  int acc_blocks, acc_rows, acc_splits, acc_chunk, acc_N, acc_V, acc_bf16;
  const void* acc_logits;
  int64_t acc_bs, acc_rs;
  uint64_t* acc_keys;
  // The accept's finalize and the conv-window rollback in the same launch
  // (fin_count null: off; see accept_finish).  Sequence b's accepted count
  // a = clamp(matched + fin_offset, 0, fin_T) goes to fin_keep[b], which the
  // scan of this launch does not read (sel_accepted is another buffer).
  int* fin_count;  // [acc rows / acc_N] arrival counts, zero between calls
  const int32_t* fin_draft;
  int64_t fin_dstride;
  int fin_ndraft, fin_offset, fin_T;
  int32_t* fin_posterior;
  int32_t* fin_matched;
  int32_t* fin_bonus;
  int32_t* fin_keep;
  int fin_L, fin_K1;
  int64_t fin_Cu, fin_qbs, fin_qrs;  // 16-byte units
  ConvTable fin_conv;
};

// Tokens per block the on-the-fly prologue supports (its LDS is sized for it).
constexpr int kProMaxT = 32;

// The item's prologue outputs, rounded to bf16 as the standalone prologue
// stores them.
template <int DK, int ROWS>
struct ProLds {
  uint16_t qk[kProMaxT][2 * DK];  // q | k of the item's key head
  uint16_t v[kProMaxT][ROWS];     // the item's value rows
  float g[kProMaxT];
  float beta[kProMaxT];
};

template <int VEC>
struct BF16Vec;
template <>
struct BF16Vec<4> {
  typedef uint2 raw;
  __device__ static raw load(const uint16_t* p) {
    return *reinterpret_cast<const uint2*>(p);
  }
  __device__ static void unpack(raw r, float* f) {
    f[0] = bf16_lo(r.x);
    f[1] = bf16_hi(r.x);
    f[2] = bf16_lo(r.y);
    f[3] = bf16_hi(r.y);
  }
};
template <>
struct BF16Vec<2> {
  typedef uint32_t raw;
  __device__ static raw load(const uint16_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
  }
  __device__ static void unpack(raw r, float* f) {
    f[0] = bf16_lo(r);
    f[1] = bf16_hi(r);
  }
};

template <int VEC>
__device__ __forceinline__ void load_f32(const float* p, float* f) {
  if constexpr (VEC == 4) {
    f32x4 x = *reinterpret_cast<const f32x4*>(p);
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  } else {
    f32x2 x = *reinterpret_cast<const f32x2*>(p);
    f[0] = x.x; f[1] = x.y;
  }
}

template <int VEC>
__device__ __forceinline__ void store_f32(float* p, const float* f) {
  if constexpr (VEC == 4) {
    f32x4 x = {f[0], f[1], f[2], f[3]};
    *reinterpret_cast<f32x4*>(p) = x;
  } else {
    f32x2 x = {f[0], f[1]};
    *reinterpret_cast<f32x2*>(p) = x;
  }
}

template <int VEC>
__device__ __forceinline__ void store_f32_stream(float* p, const float* f) {
  if constexpr (VEC == 4) {
    f32x4 x = {f[0], f[1], f[2], f[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4*>(p));
  } else {
    f32x2 x = {f[0], f[1]};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x2*>(p));
  }
}

// PER consecutive bf16 channels (PER * 2 bytes, naturally aligned) as fp32.
template <int PER>
__device__ __forceinline__ void load_bf16_run(const uint16_t* p, float* f) {
  if constexpr (PER == 2) {
    const uint32_t r = *reinterpret_cast<const uint32_t*>(p);
    f[0] = bf16_lo(r);
    f[1] = bf16_hi(r);
  } else if constexpr (PER == 4) {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    f[0] = bf16_lo(r.x); f[1] = bf16_hi(r.x); f[2] = bf16_lo(r.y); f[3] = bf16_hi(r.y);
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) f[i] = bf16_bits_to_f32(p[i]);
  }
}

// The layer prologue of one item (sequence b, value head hv, row block rb)
// for its n tokens, into LDS.  Same arithmetic and lane layout as the
// standalone prologue kernel (gdn_layer_ops.hip), so the values are the ones
// it would store:
//   - q and k of key head hk: one wavefront per (head, run of consecutive
//     tokens), lane l owning channels l*PER .. l*PER+PER-1 with the head's
//     rms-norm summed by pro_wave_sum; the conv window of the run is loaded
//     once (rows t .. t+K-2 of the previous token are rows of the next);
//   - the ROWS value channels of the row block: one (token, channel) per
//     thread;
//   - g and beta of head hv: one token per thread.
// load() issues every load of the phase and consumes none; compute() does
// the arithmetic and the LDS stores.  KT: conv taps when fixed at compile
// time, 0 for the run-time K (<= kMaxConvTaps).
template <int DK, int ROWS, int KT>
struct ProPhase {
  static constexpr int PER = DK / 64;
  static constexpr int NT = KT > 0 ? KT : kMaxConvTaps;  // taps held in registers
  static constexpr int RUN = kProMaxT / 2;              // tokens per q/k wavefront
  static constexpr int XR = RUN + NT - 1;               // conv rows of a run
  static constexpr int VT = (kProMaxT * ROWS + 255) / 256;  // value tasks per thread

  float xq[XR][PER], wq[PER][NT];
  float xv[VT][NT], wv[VT][NT];
  float av, bv, A_log, dt_bias;
  int sel, t_begin, t_end;

  __device__ __forceinline__ int taps(const ScanParams& p) const { return KT > 0 ? KT : p.pro_K; }

  __device__ __forceinline__ void load(const ScanParams& p, int b, int hv, int hk, int rb, int n) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int K = taps(p), K1 = K - 1;
    const uint16_t* qkv = p.pro_qkv + b * p.pro_qkv_sb;
    const uint16_t* cst = p.pro_conv_state + (int64_t)b * K1 * p.pro_C;
    // Row s of concat(conv_state, qkv); s is clamped into [0, n - 1 + K1].
    auto row_ptr = [&](int s) -> const uint16_t* {
      s = min(s, n - 1 + K1);
      return s < K1 ? cst + (int64_t)s * p.pro_C : qkv + (int64_t)(s - K1) * p.pro_qkv_st;
    };
    // q / k: wavefronts 0, 2 take q, 1, 3 take k; wavefronts 0, 1 the first
    // half of the tokens, 2, 3 the second.
    sel = w & 1;
    const int half = (n + 1) >> 1;
    t_begin = (w >> 1) * half;
    t_end = min(n, t_begin + half);
    const int c0 = sel * p.pro_Hk * DK + hk * DK + lane * PER;
#pragma unroll
    for (int r = 0; r < XR; ++r) load_bf16_run<PER>(row_ptr(t_begin + r) + c0, xq[r]);
    // Taps j >= K (run-time K) are loaded from tap K-1 (a valid address, no
    // branch around the load) and never used: the tap sum stops at K.
#pragma unroll
    for (int i = 0; i < PER; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j)
        wq[i][j] = bf16_bits_to_f32(p.pro_conv_w[(int64_t)(c0 + i) * K + min(j, K1)]);
    // Value channels.
    const int vbase = 2 * p.pro_Hk * DK + hv * p.Dv + rb * ROWS;
#pragma unroll
    for (int k = 0; k < VT; ++k) {
      const int task = min(tid + k * 256, n * ROWS - 1);
      const int t = task / ROWS, ch = task - t * ROWS;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        xv[k][j] = bf16_bits_to_f32(row_ptr(t + min(j, K1))[vbase + ch]);
        wv[k][j] = bf16_bits_to_f32(p.pro_conv_w[(int64_t)(vbase + ch) * K + min(j, K1)]);
      }
    }
    // Decay and write strength.
    const int tg = min(tid, n - 1);
    av = bf16_bits_to_f32(p.pro_a[b * p.pro_a_sb + (int64_t)tg * p.pro_a_st + hv]);
    bv = bf16_bits_to_f32(p.pro_b[b * p.pro_b_sb + (int64_t)tg * p.pro_b_st + hv]);
    A_log = p.pro_A_log[hv];
    dt_bias = bf16_bits_to_f32(p.pro_dt_bias[hv]);
  }

  __device__ __forceinline__ void compute(const ScanParams& p, int n, ProLds<DK, ROWS>& L) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int K = taps(p);
    if (tid < n) {
      L.g[tid] = pro_decay(A_log, av, dt_bias);
      L.beta[tid] = pro_sigmoid(bv);
    }
#pragma unroll
    for (int k = 0; k < VT; ++k) {
      const int task = tid + k * 256;
      if (task < n * ROWS) {
        const int t = task / ROWS, ch = task - t * ROWS;
        L.v[t][ch] = f32_to_bf16_rne(pro_conv_silu_n<NT>(wv[k], xv[k], K));
      }
    }
    // Tokens in chunks of 8 with no branch inside a chunk, so that the eight
    // cross-lane reductions overlap (rows past the run are clamped copies).
    const float scale = sel ? p.pro_k_scale : p.pro_q_scale;
#pragma unroll
    for (int u0 = 0; u0 < RUN; u0 += 8) {
      if (t_begin + u0 < t_end) {  // uniform over the wavefront
        float vals[8][PER], ss[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          ss[u] = 0.f;
#pragma unroll
          for (int i = 0; i < PER; ++i) {
            float xi[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) xi[j] = xq[u0 + u + j][i];
            vals[u][i] = pro_conv_silu_n<NT>(wq[i], xi, K);
            ss[u] = fmaf(vals[u][i], vals[u][i], ss[u]);
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) ss[u] = pro_wave_sum(ss[u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int t = t_begin + u0 + u;
          const float r = pro_head_scale(ss[u], DK, p.pro_eps, scale);
          if (t < t_end) {
#pragma unroll
            for (int i = 0; i < PER; ++i)
              L.qk[t][sel * DK + lane * PER + i] = f32_to_bf16_rne(vals[u][i] * r);
          }
        }
      }
    }
  }
};

// PF: tokens of inputs in flight (register ring).  1 for launches that fill
// the chip with workgroups; 4 when there are at most as many work items as
// CUs (one layer of one sequence), where each step otherwise waits on its
// own loads.
// PRO: the layer prologue runs at each item's start (pro_phase) and the
// token loop reads its inputs from LDS.
// Rows of one sequence the in-launch accept finalize holds (its LDS), and
// the conv window rows it copies at most.
constexpr int kFinMaxRows = 64;
constexpr int kFinConvRows = 4;

// The accept's last step inside the scan's launch, run by each argmax
// workgroup after it stored its key (agent-scope): the workgroup waits for
// that store, counts itself in fin_count[b], and the last of sequence b's
// N * splits argmax workgroups to arrive puts the count back to zero and
// finishes the sequence alone, while the scan's workgroups run on:
//   - merges the N x splits keys (agent-scope loads: the other workgroups'
//     stores completed before they counted themselves), as
//     accept_conv_rollback_kernel does (16 lanes per row, order-free max);
//   - matched = the first position where the draft differs from the
//     posterior, bonus = posterior[matched] (dflash_mlx/runtime.py:41-47,
//     :145-147), posterior / matched / bonus and the keep count
//     a = clamp(matched + fin_offset, 0, fin_T) stored;
//   - the new conv window of every layer: rows a .. a+K1-1 of
//     concat(conv_in, qkv) (custom_qwen35_model.py:1044-1051), 16-byte
//     units, four units per lane loaded before any is stored.
// No workgroup waits on another.
__device__ __forceinline__ void accept_finish(const ScanParams& p, int row) {
  __shared__ int fin_last, fin_first;
  __shared__ int32_t post[kFinMaxRows];
  const int N = p.acc_N;
  const int b = row / N;
  // The last-arriver protocol of device_common.h: relaxed agent-scope
  // atomics ordered by the hardware (store acknowledged before the count,
  // loads issued after the count returns), not by happens-before edges of
  // the HIP memory model.
  if (threadIdx.x == 0) {
    __builtin_amdgcn_s_waitcnt(0);  // this workgroup's key store has completed
    const int old = __hip_atomic_fetch_add(p.fin_count + b, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    fin_last = old == N * p.acc_splits - 1;
  }
  __syncthreads();
  if (!fin_last) return;
  if (threadIdx.x == 0)
    __hip_atomic_store(p.fin_count + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int mlen = min(p.fin_ndraft, N);
  int draft0 = 0;  // draft token `lane` of the first 64 (wavefront 0)
  if (wave == 0 && lane < mlen) draft0 = p.fin_draft[(int64_t)b * p.fin_dstride + lane];
  const int sub = threadIdx.x & 15;
  const int splits = p.acc_splits;
  for (int r0 = 0; r0 < N; r0 += 16) {
    const int r = r0 + (threadIdx.x >> 4);
    uint64_t m = 0;
    if (r < N) {
      const uint64_t* kr = p.acc_keys + ((int64_t)b * N + r) * splits;
      for (int s0 = sub; s0 < splits; s0 += 16 * 8) {
        uint64_t v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = __hip_atomic_load(kr + min(s0 + 16 * i, splits - 1), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
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
      const int dj = base0 == 0 ? draft0 : (j < mlen ? p.fin_draft[(int64_t)b * p.fin_dstride + j] : 0);
      const bool mismatch = (j < mlen) && (dj != post[j]);
      const unsigned long long mask = __ballot(mismatch);
      if (mask != 0ull) {
        first = base0 + __ffsll(mask) - 1;
        break;
      }
    }
    if (lane == 0) fin_first = first;
  }
  __syncthreads();
  const int first = fin_first;
  const int a = min(max(first + p.fin_offset, 0), p.fin_T);
  if (p.fin_posterior != nullptr)
    for (int r = threadIdx.x; r < N; r += 256) p.fin_posterior[(int64_t)b * N + r] = post[r];
  if (threadIdx.x == 0) {
    if (p.fin_matched != nullptr) p.fin_matched[b] = first;
    if (p.fin_bonus != nullptr) p.fin_bonus[b] = first < N ? post[first] : -1;
    p.fin_keep[b] = a;
  }
  // conv windows: unit e of the flattened (layer, column unit) range
  const int K1 = p.fin_K1;
  const int64_t Cu = p.fin_Cu, units = (int64_t)p.fin_L * Cu;
  constexpr int kU = 4;
  for (int64_t e0 = threadIdx.x; e0 < units; e0 += 256 * kU) {
    u32x4 vals[kU][kFinConvRows];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t e = min(e0 + 256 * u, units - 1);
      const int l = (int)(e / Cu);
      const int64_t c = e - (int64_t)l * Cu;
      const u32x4* cin = reinterpret_cast<const u32x4*>(p.fin_conv.cin[l]) + (int64_t)b * K1 * Cu + c;
      const u32x4* qkv = reinterpret_cast<const u32x4*>(p.fin_conv.qkv[l]) + (int64_t)b * p.fin_qbs + c;
#pragma unroll
      for (int r = 0; r < kFinConvRows; ++r) {
        if (r < K1) {
          const int j = a + r;
          vals[u][r] = j < K1 ? cin[(int64_t)j * Cu] : qkv[(int64_t)(j - K1) * p.fin_qrs];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t e = e0 + 256 * u;
      if (e < units) {
        const int l = (int)(e / Cu);
        const int64_t c = e - (int64_t)l * Cu;
        u32x4* cout = reinterpret_cast<u32x4*>(p.fin_conv.cout[l]) + (int64_t)b * K1 * Cu + c;
#pragma unroll
        for (int r = 0; r < kFinConvRows; ++r)
          if (r < K1) cout[(int64_t)r * Cu] = vals[u][r];
      }
    }
  }
}

// FIN: the argmax workgroups finish the accept (accept_finish); its own
// instantiations, so the other scans keep their register budget.
template <int DK, int R, int PF, bool PRO = false, int KT = 0, bool FIN = false>
__global__ __launch_bounds__(256) void gdn_scan_kernel(const ScanParams p) {
  constexpr int VEC = (DK % 64 == 0) ? 4 : 2;
  constexpr int NCH = DK / (16 * VEC);
  constexpr int ROWS_WG = 16 * R;
  typedef BF16Vec<VEC> LD;
  __shared__ std::conditional_t<PRO, ProLds<DK, ROWS_WG>, int> pro_lds;

  const int sub = threadIdx.x & 15;  // lane within the 16-lane row group
  const int gi = threadIdx.x >> 4;   // row group within the workgroup, 0..15
  const bool has_q = PRO || p.q != nullptr;
  const bool has_tape = p.tape != nullptr;

  const int bid = blockIdx.x, nblk = gridDim.x - p.acc_blocks;
  if (bid >= nblk) {  // an accept workgroup (uniform over the workgroup)
    const int a = bid - nblk;
    const int row = a / p.acc_splits;
    const int split = a - row * p.acc_splits;
    const bool fin = FIN && p.fin_count != nullptr;
    if (p.acc_bf16)
      argmax_partial_block<uint16_t, true>(static_cast<const uint16_t*>(p.acc_logits), p.acc_bs,
                                           p.acc_rs, p.acc_N, p.acc_V, p.acc_chunk, p.acc_splits,
                                           p.acc_keys, row, split, fin);
    else
      argmax_partial_block<float, true>(static_cast<const float*>(p.acc_logits), p.acc_bs,
                                        p.acc_rs, p.acc_N, p.acc_V, p.acc_chunk, p.acc_splits,
                                        p.acc_keys, row, split, fin);
    if constexpr (FIN && !PRO) {
      if (fin) accept_finish(p, row);
    }
    return;
  }
  int item_begin = bid, item_end = p.items, item_step = nblk;
  if (p.xcd_items > 0) {
    const int x = bid & 7;
    item_begin = x * p.xcd_items + (bid >> 3);
    item_end = (x + 1) * p.xcd_items;
    item_step = nblk >> 3;
  }
  for (int item = item_begin; item < item_end; item += item_step) {
    const int rb = item % p.row_blocks;
    const int bh = item / p.row_blocks;
    const int b = bh / p.Hv;
    const int hv = bh - b * p.Hv;
    const int hk = hv / p.rep;
    int n = p.T;
    if (!PRO && p.lengths != nullptr) n = min(max(p.lengths[b], 0), p.T);

    int row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row[r] = rb * ROWS_WG + r * 16 + gi;

    // Load the state rows (from the previous tape when the rollback is fused).
    float S[R][NCH][VEC];
    const int64_t head_base = (int64_t)bh * p.Dv * DK;
    const float* s_src = p.state_in + head_base;
    bool writeback = false;
    int a_sel = 0;
    ProPhase<DK, ROWS_WG, KT> pro;
    if constexpr (PRO) {
      // The accepted count is loaded with no branch around it (from the state
      // buffer, a valid address, when there is no selection; then unused), and
      // the prologue's loads go out before it is waited on, ahead of the state
      // loads that need it.
      const bool has_sel = p.sel_tape != nullptr;
      const int32_t* ap = has_sel ? p.sel_accepted + b % max(p.sel_period, 1)
                                  : reinterpret_cast<const int32_t*>(p.state_in);
      const int a_raw = *ap;
      pro.load(p, b, hv, hk, rb, n);
      a_sel = has_sel ? min(max(a_raw, 0), p.sel_T) : 0;
    } else {
      if (p.sel_tape != nullptr) a_sel = min(max(p.sel_accepted[b % p.sel_period], 0), p.sel_T);
    }
    if (a_sel >= 1) {
      s_src = p.sel_tape + (int64_t)(a_sel - 1) * p.tape_tstride + head_base;
      writeback = true;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        load_f32<VEC>(s_src + (int64_t)row[r] * DK + c * 16 * VEC + sub * VEC, S[r][c]);
    if constexpr (PRO) {
      // The state loads stay in flight while the prologue computes.
      __syncthreads();  // the previous item's token loop is done with pro_lds
      pro.compute(p, n, pro_lds);
      __syncthreads();
    }
    if (writeback) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          store_f32<VEC>(p.state_wb + head_base + (int64_t)row[r] * DK + c * 16 * VEC + sub * VEC,
                         S[r][c]);
    }

    const uint16_t* kp = PRO ? nullptr : p.k + b * p.k_sb + hk * p.k_sh + sub * VEC;
    const uint16_t* qp =
        (has_q && !PRO) ? p.q + b * p.q_sb + hk * p.q_sh + sub * VEC : nullptr;
    const uint16_t* vp = PRO ? nullptr : p.v + b * p.v_sb + hv * p.v_sh;
    const float* gp = PRO ? nullptr : p.g + b * p.g_sb + hv;
    const float* bp = PRO ? nullptr : p.beta + b * p.b_sb + hv;
    float* tp = has_tape ? p.tape + head_base + sub * VEC : nullptr;

    // Inputs of the next PF tokens stay in flight in a register ring (slot
    // t % PF holds token t).
    typename LD::raw k_raw[PF][NCH], q_raw[PF][NCH];
    uint16_t v_raw[PF][R];
    float g_r[PF], b_r[PF];
    auto fetch = [&](int slot, int t) {
      if constexpr (PRO) {
        const uint16_t* qk = pro_lds.qk[t];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          k_raw[slot][c] = LD::load(qk + DK + c * 16 * VEC + sub * VEC);
          q_raw[slot][c] = LD::load(qk + c * 16 * VEC + sub * VEC);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) v_raw[slot][r] = pro_lds.v[t][r * 16 + gi];
        g_r[slot] = pro_lds.g[t];
        b_r[slot] = pro_lds.beta[t];
      } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c) k_raw[slot][c] = LD::load(kp + t * p.k_st + c * 16 * VEC);
        if (has_q) {
#pragma unroll
          for (int c = 0; c < NCH; ++c) q_raw[slot][c] = LD::load(qp + t * p.q_st + c * 16 * VEC);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) v_raw[slot][r] = vp[t * p.v_st + row[r]];
        g_r[slot] = gp[t * p.g_st];
        b_r[slot] = bp[t * p.b_st];
      }
    };
    if (n > 0) {
#pragma unroll
      for (int d = 0; d < PF; ++d) fetch(d, min(d, n - 1));
    }

    float okeep[R];
#pragma unroll
    for (int r = 0; r < R; ++r) okeep[r] = 0.f;

    for (int t0 = 0; t0 < n; t0 += PF) {
#pragma unroll
      for (int d = 0; d < PF; ++d) {
        const int t = t0 + d;
        if (t < n) {
          float kf[NCH][VEC], qf[NCH][VEC], vr[R];
#pragma unroll
          for (int c = 0; c < NCH; ++c) LD::unpack(k_raw[d][c], kf[c]);
          if (has_q) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) LD::unpack(q_raw[d][c], qf[c]);
          }
#pragma unroll
          for (int r = 0; r < R; ++r) vr[r] = bf16_bits_to_f32(v_raw[d][r]);
          const float gt = g_r[d];
          const float bt = b_r[d];
          fetch(d, min(t + PF, n - 1));

#pragma unroll
          for (int r = 0; r < R; ++r) {
            // S <- g*S ; kv = S.k
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
              for (int e = 0; e < VEC; ++e) {
                S[r][c][e] *= gt;
                acc = fmaf(S[r][c][e], kf[c][e], acc);
              }
            const float kv = row16_sum(acc);
            const float delta = (vr[r] - kv) * bt;
            // S += k (x) delta
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
              for (int e = 0; e < VEC; ++e) S[r][c][e] = fmaf(kf[c][e], delta, S[r][c][e]);
            if (has_q) {
              float o = 0.f;
#pragma unroll
              for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int e = 0; e < VEC; ++e) o = fmaf(S[r][c][e], qf[c][e], o);
              o = row16_sum(o);
              if (sub == (t & 15)) okeep[r] = o;
            }
            if (has_tape) {
              float* dst = tp + (int64_t)t * p.tape_tstride + (int64_t)row[r] * DK;
#pragma unroll
              for (int c = 0; c < NCH; ++c) store_f32_stream<VEC>(dst + c * 16 * VEC, S[r][c]);
            }
          }

          // Lane s of each row group holds out for token (t & ~15) + s; flush
          // every 16 tokens and at the end.
          if (has_q && (((t & 15) == 15) || (t == n - 1))) {
            const int tb = t & ~15;
            if (sub <= (t & 15)) {
              uint16_t* op = p.out + (((int64_t)b * p.T + tb + sub) * p.Hv + hv) * p.Dv;
#pragma unroll
              for (int r = 0; r < R; ++r) op[row[r]] = f32_to_bf16_rne(okeep[r]);
            }
          }
        }
      }
    }

    if (p.final_state != nullptr) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          store_f32<VEC>(p.final_state + head_base + (int64_t)row[r] * DK +
                             c * 16 * VEC + sub * VEC,
                         S[r][c]);
    }
  }
}

int scan_grid(int items);
int scan_cus();

template <int DK, bool PRO = false>
hipError_t launch_dk(const ScanParams& base, int R, int grid, int xcd, hipStream_t s) {
  ScanParams p = base;
  p.row_blocks = p.Dv / (16 * R);
  p.items = p.B * p.Hv * p.row_blocks;
  // grid < 0: the tuned default; 0: one workgroup per item; > 0: that many.
  const int blocks = grid < 0 ? scan_grid(p.items) : (grid > 0 ? min(grid, p.items) : p.items);
  // xcd < 0: XCD-aware walk whenever the shapes allow it; 0: off; > 0: on if allowed.
  const bool xcd_ok = blocks % 8 == 0 && p.items % 8 == 0 && blocks < p.items;
  p.xcd_items = (xcd != 0 && xcd_ok) ? p.items / 8 : 0;
  const bool deep = p.items <= scan_cus();
  const unsigned total = (unsigned)(blocks + p.acc_blocks);  // accept workgroups last
  if constexpr (PRO) {
    if (R != 1) return hipErrorInvalidValue;
    const dim3 g(total), b(256);
    if (p.pro_K == 4) {  // the Qwen3.5 conv width, taps fixed at compile time
      if (deep) hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 4, true, 4>), g, b, 0, s, p);
      else hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 1, true, 4>), g, b, 0, s, p);
    } else {
      if (deep) hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 4, true, 0>), g, b, 0, s, p);
      else hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 1, true, 0>), g, b, 0, s, p);
    }
    return hipGetLastError();
  }
  if (p.fin_count != nullptr) {
    if (R != 1) return hipErrorInvalidValue;
    if (deep) hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 4, false, 0, true>), dim3(total), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 1, false, 0, true>), dim3(total), dim3(256), 0, s, p);
    return hipGetLastError();
  }
  switch (R * (deep ? 10 : 1)) {
    case 1: hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 1>), dim3(total), dim3(256), 0, s, p); break;
    case 2: hipLaunchKernelGGL((gdn_scan_kernel<DK, 2, 1>), dim3(total), dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL((gdn_scan_kernel<DK, 4, 1>), dim3(total), dim3(256), 0, s, p); break;
    case 10: hipLaunchKernelGGL((gdn_scan_kernel<DK, 1, 4>), dim3(total), dim3(256), 0, s, p); break;
    case 20: hipLaunchKernelGGL((gdn_scan_kernel<DK, 2, 4>), dim3(total), dim3(256), 0, s, p); break;
    case 40: hipLaunchKernelGGL((gdn_scan_kernel<DK, 4, 4>), dim3(total), dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Rows per lane group (1, 2 or 4 are compiled).  Measured on MI355X at the
// Qwen3.5-4B verify shapes with the capped grid below, one row per group was
// fastest (R = 2 within 2 %, R = 4 slower: fewer waves in flight).
int pick_rows(int Dv) {
  (void)Dv;
  return 1;
}

// Workgroups launched: at most 3 per CU, each walking several (head, row
// block) items.  On MI355X this beat one workgroup per item by ~12 % on the
// tape-write-bound verify shapes (fewer concurrent write streams).
// CUs of the current device (0 if unknown).
int scan_cus() { return device_cus(); }

int scan_grid(int items) {
  const int cus = scan_cus();
  if (cus == 0) return items;
  const int cap = 3 * cus;
  return items < cap ? items : cap;
}

// Fused-rollback source of the initial states (see ScanParams::sel_tape).
struct Select {
  const float* prev_tape;
  const int32_t* prev_accepted;
  float* state;  // the state buffer: read for a == 0, written for a >= 1
  int prev_T;
  int period;
};

// The greedy accept's argmax run in the scan's launch (see ScanParams::acc_*).
struct AcceptArgs {
  const void* logits;
  int bf16;  // 0: fp32 logits, 1: bf16
  int64_t bs, rs;
  int B, N, V;
  uint64_t* keys;
};

// The accept's finalize + conv rollback run in the launch (ScanParams::fin_*).
struct FinishArgs {
  int* count;
  const int32_t* draft;
  int64_t dstride;
  int n_draft, offset, T;
  int32_t *posterior, *matched, *bonus, *keep;
  int L, K1;
  int64_t Cu, qbs, qrs;
  ConvTable conv;
};

int scan_impl(const void* q, const void* k, const void* v, const float* g,
              const float* beta, const float* state_in, void* out,
              float* final_state, float* tape, const int32_t* lengths, int B,
              int T, int Hk, int Hv, int Dk, int Dv, const int64_t* strides,
              const Select* sel, void* stream, const AcceptArgs* acc = nullptr,
              const FinishArgs* fin = nullptr) {
  if (B < 0 || T < 0 || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0) return DFLASH_ERR_SHAPE;
  if (Hv % Hk != 0) return DFLASH_ERR_SHAPE;
  if (Dv % 16 != 0) return DFLASH_ERR_UNSUPPORTED;
  if (!(Dk == 32 || Dk == 64 || Dk == 96 || Dk == 128 || Dk == 192 || Dk == 256))
    return DFLASH_ERR_UNSUPPORTED;
  if ((int64_t)B * Hv * (Dv / 16) > INT32_MAX) return DFLASH_ERR_SHAPE;
  if (sel != nullptr && (sel->prev_T < 0 || sel->period <= 0)) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  if (state_in == nullptr) return DFLASH_ERR_NULL;
  if (sel != nullptr && sel->prev_T > 0 && (sel->prev_tape == nullptr || sel->prev_accepted == nullptr))
    return DFLASH_ERR_NULL;
  if (T == 0 && sel == nullptr) {
    // Nothing to scan: the final state is the initial state.
    if (final_state != nullptr && final_state != state_in) {
      hipError_t e = hipMemcpyAsync(final_state, state_in,
                                    sizeof(float) * (size_t)B * Hv * Dv * Dk,
                                    hipMemcpyDeviceToDevice, (hipStream_t)stream);
      return e == hipSuccess ? DFLASH_OK : (int)e;
    }
    return DFLASH_OK;
  }
  if (T > 0 && (k == nullptr || v == nullptr || g == nullptr || beta == nullptr))
    return DFLASH_ERR_NULL;
  if ((q == nullptr) != (out == nullptr)) return DFLASH_ERR_NULL;
  if (sel == nullptr && out == nullptr && final_state == nullptr && tape == nullptr)
    return DFLASH_ERR_NULL;

  ScanParams p{};
  if (sel != nullptr && sel->prev_T > 0) {
    p.sel_tape = sel->prev_tape;
    p.sel_accepted = sel->prev_accepted;
    p.state_wb = sel->state;
    p.sel_period = sel->period;
    p.sel_T = sel->prev_T;
  }
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.g = g;
  p.beta = beta;
  p.state_in = state_in;
  p.out = static_cast<uint16_t*>(out);
  p.final_state = final_state;
  p.tape = tape;
  p.lengths = lengths;
  p.B = B;
  p.T = T;
  p.Hv = Hv;
  p.Dv = Dv;
  p.rep = Hv / Hk;
  p.tape_tstride = (int64_t)B * Hv * Dv * Dk;
  if (strides != nullptr) {
    p.q_sb = strides[0]; p.q_st = strides[1]; p.q_sh = strides[2];
    p.k_sb = strides[3]; p.k_st = strides[4]; p.k_sh = strides[5];
    p.v_sb = strides[6]; p.v_st = strides[7]; p.v_sh = strides[8];
    p.g_sb = strides[9]; p.g_st = strides[10];
    p.b_sb = strides[11]; p.b_st = strides[12];
  } else {
    p.q_sh = Dk; p.q_st = (int64_t)Hk * Dk; p.q_sb = (int64_t)T * Hk * Dk;
    p.k_sh = p.q_sh; p.k_st = p.q_st; p.k_sb = p.q_sb;
    p.v_sh = Dv; p.v_st = (int64_t)Hv * Dv; p.v_sb = (int64_t)T * Hv * Dv;
    p.g_st = Hv; p.g_sb = (int64_t)T * Hv;
    p.b_st = Hv; p.b_sb = (int64_t)T * Hv;
  }
  // Vector loads of q/k need VEC-element alignment of every row start;
  // state rows need 16-byte (or 8-byte) alignment.
  const int vec = (Dk % 64 == 0) ? 4 : 2;
  const uintptr_t kmask = (uintptr_t)(vec * 2 - 1);
  if (((uintptr_t)k & kmask) || (p.k_sb % vec) || (p.k_st % vec) || (p.k_sh % vec))
    return DFLASH_ERR_ALIGN;
  if (q != nullptr &&
      (((uintptr_t)q & kmask) || (p.q_sb % vec) || (p.q_st % vec) || (p.q_sh % vec)))
    return DFLASH_ERR_ALIGN;
  const uintptr_t smask = (uintptr_t)(vec * 4 - 1);
  if (((uintptr_t)state_in & smask) || ((uintptr_t)final_state & smask) ||
      ((uintptr_t)tape & smask) || ((uintptr_t)p.sel_tape & smask) || ((uintptr_t)p.state_wb & smask))
    return DFLASH_ERR_ALIGN;
  if (((uintptr_t)v & 1) || ((uintptr_t)out & 1) || ((uintptr_t)g & 3) || ((uintptr_t)beta & 3))
    return DFLASH_ERR_ALIGN;

  if (acc != nullptr) {
    const Split sp = plan_split(acc->B, acc->N, acc->V);
    p.acc_rows = acc->B * acc->N;
    p.acc_splits = sp.splits;
    p.acc_chunk = sp.chunk;
    p.acc_blocks = p.acc_rows * sp.splits;
    p.acc_N = acc->N;
    p.acc_V = acc->V;
    p.acc_bf16 = acc->bf16;
    p.acc_logits = acc->logits;
    p.acc_bs = acc->bs;
    p.acc_rs = acc->rs;
    p.acc_keys = acc->keys;
    if (fin != nullptr) {
      p.fin_count = fin->count;
      p.fin_draft = fin->draft;
      p.fin_dstride = fin->dstride;
      p.fin_ndraft = fin->n_draft;
      p.fin_offset = fin->offset;
      p.fin_T = fin->T;
      p.fin_posterior = fin->posterior;
      p.fin_matched = fin->matched;
      p.fin_bonus = fin->bonus;
      p.fin_keep = fin->keep;
      p.fin_L = fin->L;
      p.fin_K1 = fin->K1;
      p.fin_Cu = fin->Cu;
      p.fin_qbs = fin->qbs;
      p.fin_qrs = fin->qrs;
      p.fin_conv = fin->conv;
    }
  }
  const int R = pick_rows(Dv);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (Dk) {
    case 32: e = launch_dk<32>(p, R, -1, -1, s); break;
    case 64: e = launch_dk<64>(p, R, -1, -1, s); break;
    case 96: e = launch_dk<96>(p, R, -1, -1, s); break;
    case 128: e = launch_dk<128>(p, R, -1, -1, s); break;
    case 192: e = launch_dk<192>(p, R, -1, -1, s); break;
    default: e = launch_dk<256>(p, R, -1, -1, s); break;
  }
  return e == hipSuccess ? DFLASH_OK : (int)e;
}

// Verify scan with the layer prologue on the fly (Dk = 128, T <= kProMaxT).
int scan_pro_impl(const void* qkv, int64_t qkv_sb, int64_t qkv_st, const void* conv_state,
                  const void* conv_weight, const void* a, const void* b,
                  const int64_t* ab_strides, const float* A_log, const void* dt_bias,
                  const Select& sel, void* out, float* final_state, float* tape, int B, int T,
                  int K, int Hk, int Hv, int Dk, int Dv, float eps, void* stream) {
  if (B < 0 || T < 0 || K < 1 || K > kMaxConvTaps || Hk <= 0 || Hv <= 0 || Dk <= 0 || Dv <= 0)
    return DFLASH_ERR_SHAPE;
  if (Hv % Hk != 0) return DFLASH_ERR_SHAPE;
  if (Dk != 128 || Dv % 16 != 0 || T > kProMaxT) return DFLASH_ERR_UNSUPPORTED;
  if ((int64_t)B * Hv * (Dv / 16) > INT32_MAX) return DFLASH_ERR_SHAPE;
  if (sel.prev_T < 0 || sel.period <= 0) return DFLASH_ERR_SHAPE;
  if (sel.state == nullptr) return DFLASH_ERR_NULL;
  if (final_state != nullptr && final_state == sel.state) return DFLASH_ERR_SHAPE;
  if (sel.prev_T > 0 && (sel.prev_tape == nullptr || sel.prev_accepted == nullptr))
    return DFLASH_ERR_NULL;
  if (B == 0) return DFLASH_OK;
  if (T == 0)  // nothing to run the prologue on: the rollback alone
    return scan_impl(nullptr, nullptr, nullptr, nullptr, nullptr, sel.state, nullptr, final_state,
                     tape, nullptr, B, 0, Hk, Hv, Dk, Dv, nullptr, &sel, stream);
  if (qkv == nullptr || (K > 1 && conv_state == nullptr) || conv_weight == nullptr ||
      a == nullptr || b == nullptr || A_log == nullptr || dt_bias == nullptr || out == nullptr)
    return DFLASH_ERR_NULL;
  const int64_t C = 2LL * Hk * Dk + (int64_t)Hv * Dv;
  // q/k channel pairs are read as 4-byte words.
  if (((uintptr_t)qkv & 3) || (qkv_sb & 1) || (qkv_st & 1) || ((uintptr_t)conv_state & 3))
    return DFLASH_ERR_ALIGN;
  if (((uintptr_t)conv_weight | (uintptr_t)a | (uintptr_t)b | (uintptr_t)dt_bias |
       (uintptr_t)out) & 1)
    return DFLASH_ERR_ALIGN;
  if (((uintptr_t)sel.state & 15) || ((uintptr_t)final_state & 15) || ((uintptr_t)tape & 15) ||
      ((uintptr_t)sel.prev_tape & 15))
    return DFLASH_ERR_ALIGN;

  ScanParams p{};
  if (sel.prev_T > 0) {
    p.sel_tape = sel.prev_tape;
    p.sel_accepted = sel.prev_accepted;
    p.state_wb = sel.state;
    p.sel_period = sel.period;
    p.sel_T = sel.prev_T;
  }
  p.state_in = sel.state;
  p.out = static_cast<uint16_t*>(out);
  p.final_state = final_state;
  p.tape = tape;
  p.B = B;
  p.T = T;
  p.Hv = Hv;
  p.Dv = Dv;
  p.rep = Hv / Hk;
  p.tape_tstride = (int64_t)B * Hv * Dv * Dk;
  p.pro_qkv = static_cast<const uint16_t*>(qkv);
  p.pro_qkv_sb = qkv_sb;
  p.pro_qkv_st = qkv_st;
  p.pro_conv_state = static_cast<const uint16_t*>(conv_state);
  p.pro_conv_w = static_cast<const uint16_t*>(conv_weight);
  p.pro_a = static_cast<const uint16_t*>(a);
  p.pro_b = static_cast<const uint16_t*>(b);
  if (ab_strides != nullptr) {
    p.pro_a_sb = ab_strides[0]; p.pro_a_st = ab_strides[1];
    p.pro_b_sb = ab_strides[2]; p.pro_b_st = ab_strides[3];
  } else {
    p.pro_a_st = p.pro_b_st = Hv;
    p.pro_a_sb = p.pro_b_sb = (int64_t)T * Hv;
  }
  p.pro_A_log = A_log;
  p.pro_dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.pro_C = (int)C;
  p.pro_K = K;
  p.pro_Hk = Hk;
  p.pro_eps = eps;
  // The standalone prologue's scales: k by Dk^-1/2, q by Dk^-1.
  p.pro_k_scale = 1.0f / sqrtf((float)Dk);
  p.pro_q_scale = p.pro_k_scale * p.pro_k_scale;
  const hipError_t e = launch_dk<128, true>(p, 1, -1, -1, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? DFLASH_OK : (int)e;
}

}  // namespace
}  // namespace dflash

extern "C" int dflash_gdn_verify_scan(const void* q, const void* k, const void* v,
                                      const float* g, const float* beta,
                                      const float* state_in, void* out,
                                      float* final_state, float* tape,
                                      const int32_t* lengths, int B, int T,
                                      int Hk, int Hv, int Dk, int Dv,
                                      const int64_t* strides, void* stream) {
  return dflash::scan_impl(q, k, v, g, beta, state_in, out, final_state, tape,
                           lengths, B, T, Hk, Hv, Dk, Dv, strides, nullptr, stream);
}

extern "C" int dflash_gdn_verify_scan_rollback(
    const void* q, const void* k, const void* v, const float* g, const float* beta,
    float* state, const float* prev_tape, const int32_t* prev_accepted, int prev_T,
    int accepted_period, void* out, float* final_state, float* tape, int B, int T, int Hk,
    int Hv, int Dk, int Dv, const int64_t* strides, void* stream) {
  if (state == nullptr) return DFLASH_ERR_NULL;
  if (final_state != nullptr && final_state == state) return DFLASH_ERR_SHAPE;
  const dflash::Select sel{prev_tape, prev_accepted, state, prev_T, accepted_period};
  return dflash::scan_impl(q, k, v, g, beta, state, out, final_state, tape, nullptr, B, T, Hk,
                           Hv, Dk, Dv, strides, &sel, stream);
}

extern "C" int dflash_gdn_verify_scan_rollback_argmax(
    const void* q, const void* k, const void* v, const float* g, const float* beta,
    float* state, const float* prev_tape, const int32_t* prev_accepted, int prev_T,
    int accepted_period, void* out, float* final_state, float* tape, int B, int T, int Hk,
    int Hv, int Dk, int Dv, const int64_t* strides, const void* logits, int logits_dtype,
    int64_t logits_batch_stride, int64_t logits_row_stride, int accept_B, int N, int V,
    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dflash;
  if (state == nullptr) return DFLASH_ERR_NULL;
  if (final_state != nullptr && final_state == state) return DFLASH_ERR_SHAPE;
  if (accept_B <= 0 || N <= 0 || V <= 0 || (int64_t)accept_B * N > 16384) return DFLASH_ERR_SHAPE;
  if (B <= 0 || T <= 0) return DFLASH_ERR_SHAPE;  // the launch has scan work
  if (logits == nullptr || workspace == nullptr) return DFLASH_ERR_NULL;
  if (logits_dtype != DFLASH_DTYPE_F32 && logits_dtype != DFLASH_DTYPE_BF16)
    return DFLASH_ERR_UNSUPPORTED;
  if (workspace_bytes < dflash_greedy_accept_workspace_bytes(accept_B, N, V)) return DFLASH_ERR_WORKSPACE;
  // the vector path of the argmax: 16-byte aligned rows
  const int per = logits_dtype == DFLASH_DTYPE_F32 ? 4 : 8;
  if (((uintptr_t)logits & 15) || (logits_batch_stride % per) || (logits_row_stride % per) ||
      ((uintptr_t)workspace & 7))
    return DFLASH_ERR_ALIGN;
  const AcceptArgs acc{logits, logits_dtype == DFLASH_DTYPE_BF16 ? 1 : 0, logits_batch_stride,
                       logits_row_stride, accept_B, N, V, static_cast<uint64_t*>(workspace)};
  const Select sel{prev_tape, prev_accepted, state, prev_T, accepted_period};
  return scan_impl(q, k, v, g, beta, state, out, final_state, tape, nullptr, B, T, Hk, Hv, Dk, Dv,
                   strides, &sel, stream, &acc);
}

namespace dflash {
namespace {
// Bytes of the argmax keys in the single-launch step's workspace (the arrival
// counts follow, 256-byte aligned).
size_t step_keys_bytes(int B, int N, int V) {
  return (size_t)ceil_div((int64_t)dflash_greedy_accept_workspace_bytes(B, N, V), 256) * 256;
}
}  // namespace
}  // namespace dflash

extern "C" size_t dflash_gdn_verify_step_workspace_bytes(int B, int N, int V) {
  if (B <= 0 || N <= 0 || V <= 0) return 0;
  return dflash::step_keys_bytes(B, N, V) + sizeof(int) * (size_t)B;
}

extern "C" int dflash_gdn_verify_step(
    const void* q, const void* k, const void* v, const float* g, const float* beta,
    float* state, const float* prev_tape, const int32_t* prev_accepted, int prev_T,
    int accepted_period, void* out, float* final_state, float* tape, int B, int T, int Hk,
    int Hv, int Dk, int Dv, const int64_t* strides, const void* logits, int logits_dtype,
    int64_t logits_batch_stride, int64_t logits_row_stride, int accept_B, int N, int V,
    const int32_t* draft, int64_t draft_stride, int n_draft, int32_t* posterior,
    int32_t* matched, int32_t* bonus, int accepted_offset, int32_t* accepted_out,
    const void* const* conv_in, const void* const* qkv, void* const* conv_out, int L, int K1,
    int64_t C, int64_t qkv_batch_stride, int64_t qkv_row_stride, void* workspace,
    size_t workspace_bytes, void* stream) {
  using namespace dflash;
  if (state == nullptr || accepted_out == nullptr) return DFLASH_ERR_NULL;
  if (final_state != nullptr && final_state == state) return DFLASH_ERR_SHAPE;
  if (accept_B <= 0 || N <= 0 || V <= 0 || (int64_t)accept_B * N > 16384 || n_draft < 0)
    return DFLASH_ERR_SHAPE;
  if (B <= 0 || T <= 0 || L < 0 || (L > 0 && (K1 <= 0 || C <= 0))) return DFLASH_ERR_SHAPE;
  // the keep count this launch writes must not be the one its scan reads
  if (prev_T > 0 && accepted_out == prev_accepted) return DFLASH_ERR_SHAPE;
  if (N > kFinMaxRows || K1 > kFinConvRows || L > kMaxLayersPerLaunch) return DFLASH_ERR_UNSUPPORTED;
  if (logits == nullptr || workspace == nullptr) return DFLASH_ERR_NULL;
  if (n_draft > 0 && draft == nullptr) return DFLASH_ERR_NULL;
  if (logits_dtype != DFLASH_DTYPE_F32 && logits_dtype != DFLASH_DTYPE_BF16)
    return DFLASH_ERR_UNSUPPORTED;
  if (workspace_bytes < dflash_gdn_verify_step_workspace_bytes(accept_B, N, V))
    return DFLASH_ERR_WORKSPACE;
  const int per = logits_dtype == DFLASH_DTYPE_F32 ? 4 : 8;
  if (((uintptr_t)logits & 15) || (logits_batch_stride % per) || (logits_row_stride % per) ||
      ((uintptr_t)workspace & 255) || ((uintptr_t)accepted_out & 3))
    return DFLASH_ERR_ALIGN;
  // conv windows (L > 0): bf16 rows copied as 16-byte units
  ConvPlan pl{16, 0, 0, 0};
  if (L > 0) {
    const int cst = conv_plan(conv_in, qkv, conv_out, L, T, K1, C, qkv_batch_stride,
                              qkv_row_stride, 2, &pl);
    if (cst != DFLASH_OK) return cst;
    if (pl.unit != 16) return DFLASH_ERR_ALIGN;
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const AcceptArgs acc{logits, logits_dtype == DFLASH_DTYPE_BF16 ? 1 : 0, logits_batch_stride,
                       logits_row_stride, accept_B, N, V, reinterpret_cast<uint64_t*>(ws)};
  FinishArgs fin{};
  fin.count = reinterpret_cast<int*>(ws + step_keys_bytes(accept_B, N, V));
  fin.draft = draft;
  fin.dstride = draft_stride;
  fin.n_draft = n_draft;
  fin.offset = accepted_offset;
  fin.T = T;
  fin.posterior = posterior;
  fin.matched = matched;
  fin.bonus = bonus;
  fin.keep = accepted_out;
  fin.L = L;
  fin.K1 = K1;
  fin.Cu = pl.Cu;
  fin.qbs = pl.qbs;
  fin.qrs = pl.qrs;
  if (L > 0) fin.conv = conv_table(conv_in, qkv, conv_out, 0, L);
  const Select sel{prev_tape, prev_accepted, state, prev_T, accepted_period};
  return scan_impl(q, k, v, g, beta, state, out, final_state, tape, nullptr, B, T, Hk, Hv, Dk, Dv,
                   strides, &sel, stream, &acc, &fin);
}

extern "C" int dflash_gdn_replay(const void* k, const void* v, const float* g,
                                 const float* beta, const float* state_in,
                                 float* state_out, const int32_t* lengths, int B,
                                 int T, int Hk, int Hv, int Dk, int Dv,
                                 const int64_t* strides, void* stream) {
  if (state_out == nullptr) return DFLASH_ERR_NULL;
  return dflash::scan_impl(nullptr, k, v, g, beta, state_in, nullptr, state_out,
                           nullptr, lengths, B, T, Hk, Hv, Dk, Dv, strides, nullptr, stream);
}

extern "C" int dflash_gdn_prologue_scan_rollback(
    const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride, const void* conv_state,
    const void* conv_weight, const void* a, const void* b, const int64_t* ab_strides,
    const float* A_log, const void* dt_bias, float* state, const float* prev_tape,
    const int32_t* prev_accepted, int prev_T, int accepted_period, void* out, float* final_state,
    float* tape, int B, int T, int K, int Hk, int Hv, int Dk, int Dv, float eps, void* stream) {
  const dflash::Select sel{prev_tape, prev_accepted, state, prev_T, accepted_period};
  return dflash::scan_pro_impl(qkv, qkv_batch_stride, qkv_row_stride, conv_state, conv_weight, a,
                               b, ab_strides, A_log, dt_bias, sel, out, final_state, tape, B, T, K,
                               Hk, Hv, Dk, Dv, eps, stream);
}
