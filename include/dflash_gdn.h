/*
 * dflash_gdn.h — C ABI of the MI355X (gfx950) gated-delta verify hot path.
 *
 * One shared library, libdflash_gfx950.so, exports these entry points.  They
 * take plain device pointers, sizes and element strides; no C++ or framework
 * types cross the boundary.  Every entry point:
 *   - returns 0 on success, a negative DFLASH_ERR_* code when the arguments are
 *     rejected before any launch, or a positive hipError_t when the launch
 *     itself fails;
 *   - allocates nothing, synchronises nothing and keeps no state between calls
 *     (so it is reentrant and ordered only by the stream it is given), except
 *     dflash_greedy_accept_noalloc, whose scratch is one static device array
 *     per device;
 *   - enqueues its kernels on `stream` (a hipStream_t; NULL = the null stream).
 *
 * Tensor conventions (row-major, innermost index last):
 *   q, k    [B, T, Hk, Dk]  bf16, Dk contiguous, other dims strided
 *   v       [B, T, Hv, Dv]  bf16, Dv contiguous, other dims strided
 *   g, beta [B, T, Hv]      fp32, Hv contiguous, other dims strided
 *   state   [B, Hv, Dv, Dk] fp32, contiguous (the reference's recurrent-state
 *                           orientation: dk fastest)
 *   out     [B, T, Hv, Dv]  bf16, contiguous
 *   tape    [T, B, Hv, Dv, Dk] fp32, contiguous; tape[t] is the state after
 *                           token t, so tape[T-1] equals the final state.
 * GQA: value head hv reads key head hv / (Hv / Hk).
 */
#ifndef DFLASH_GDN_H
#define DFLASH_GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFLASH_ABI_VERSION 4

/* Argument-validation codes (negative).  Positive values are hipError_t. */
#define DFLASH_OK 0
#define DFLASH_ERR_NULL (-1)        /* a required pointer is NULL              */
#define DFLASH_ERR_SHAPE (-2)       /* a size is out of range or inconsistent
                                       (also: a row or workgroup count that
                                       would not fit in int)                 */
#define DFLASH_ERR_UNSUPPORTED (-3) /* head dim / dtype not compiled in        */
#define DFLASH_ERR_ALIGN (-4)       /* pointer or stride breaks vector access  */
#define DFLASH_ERR_WORKSPACE (-5)   /* workspace smaller than required         */

/* dtype tags used where an entry point accepts more than one element type. */
#define DFLASH_DTYPE_F32 0
#define DFLASH_DTYPE_BF16 1
#define DFLASH_DTYPE_F16 2

/* Returns DFLASH_ABI_VERSION.  No reference counterpart (ABI handshake). */
int dflash_abi_version(void);

/* Human-readable text for a return code (static storage). */
const char* dflash_strerror(int code);

/*
 * Gated-delta-rule scan over a verify block, emitting the per-token state tape.
 *
 * Replaces the forward scan the reference calls per linear-attention layer,
 * mlx_lm gated_delta_kernel(q, k, v, g, beta, state) -> (out, state)
 * (call sites dflash_mlx/custom_qwen35_model.py:457-466 and :365-374,
 * dflash_mlx/adapters.py:202-211), and adds the tape that the reference
 * rebuilds by replay on rollback (custom_qwen35_model.py:1029-1074).
 *
 * Per (b, hv) with S = state_in[b, hv] and for t = 0 .. n_b - 1:
 *   S      <- g[b,t,hv] * S
 *   kv[dv]  = sum_dk S[dv,dk] * k[b,t,hk,dk]
 *   d[dv]   = (v[b,t,hv,dv] - kv[dv]) * beta[b,t,hv]
 *   S[dv,dk] += k[b,t,hk,dk] * d[dv]
 *   out[b,t,hv,dv] = bf16(sum_dk S[dv,dk] * q[b,t,hk,dk])   (if q and out)
 *   tape[t,b,hv] = S                                          (if tape)
 * and final_state[b,hv] = S after n_b tokens (if final_state), where
 * n_b = lengths ? clamp(lengths[b], 0, T) : T.  Entries of out and tape at
 * t >= n_b are left untouched.
 *
 * q and out are optional together (both NULL gives the state-only replay);
 * tape, final_state and lengths are each optional.  At least one of out,
 * tape, final_state must be given.
 *
 * strides: NULL for contiguous inputs, else 13 int64 element strides:
 *   { q_b, q_t, q_h,  k_b, k_t, k_h,  v_b, v_t, v_h,  g_b, g_t,  beta_b, beta_t }
 *
 * Supported: Dk in {32, 64, 96, 128, 192, 256}; Dv % 16 == 0; Hv % Hk == 0.
 * final_state may alias state_in (each state row is read before it is
 * written by the same lanes); tape and out must not alias any input.
 */
int dflash_gdn_verify_scan(const void* q, const void* k, const void* v,
                           const float* g, const float* beta,
                           const float* state_in, void* out,
                           float* final_state, float* tape,
                           const int32_t* lengths, int B, int T, int Hk,
                           int Hv, int Dk, int Dv, const int64_t* strides,
                           void* stream);

/*
 * The scan above with the previous verify step's rollback fused into its
 * state load, for device-driven serving loops (no host sync, no separate
 * gather launch).
 *
 * Replaces the pair rollback_linear_caches(..., accepted_inputs)
 * (dflash_mlx/custom_qwen35_model.py:1029-1074) + next verify scan
 * (custom_qwen35_model.py:457-466): the reference replays the accepted prefix
 * and then scans the next block from the rebuilt state; here the next scan
 * reads that state straight from the previous tape.
 *
 * For sequence b, with a = clamp(prev_accepted[b % accepted_period], 0, prev_T):
 *   S0[b] = a >= 1 ? prev_tape[a-1, b] : state[b]
 * and when a >= 1, S0[b] is also written to state[b], so on return `state`
 * holds every sequence's rolled-back initial state (the state an accept of
 * zero tokens in this block would roll back to).  The scan then runs from S0
 * exactly as dflash_gdn_verify_scan (out, final_state, tape optional; no
 * lengths).  prev_tape is [prev_T, B, Hv, Dv, Dk] fp32 and may be the same
 * buffer as tape (each state row is read before the same lanes write it).
 * prev_T = 0 disables the selection (prev_tape and prev_accepted unused).
 * final_state must not alias state.  accepted_period lets layers stacked as
 * batch entries (index l*B + b) share one accepted count per sequence
 * (accepted_period = B).
 */
int dflash_gdn_verify_scan_rollback(const void* q, const void* k, const void* v,
                                    const float* g, const float* beta,
                                    float* state, const float* prev_tape,
                                    const int32_t* prev_accepted, int prev_T,
                                    int accepted_period, void* out,
                                    float* final_state, float* tape, int B,
                                    int T, int Hk, int Hv, int Dk, int Dv,
                                    const int64_t* strides, void* stream);

/*
 * dflash_gdn_verify_scan_rollback with the argmax phase of the greedy accept
 * (dflash_greedy_accept's first launch: per-slice argmax keys of the verify
 * logits into `workspace`) run by extra workgroups of the same launch,
 * dispatched after the scan's; the keys are then merged by
 * dflash_accept_keys_conv_rollback.  The verify step's scan and the accept
 * read disjoint inputs, so sharing the launch changes nothing but the launch
 * count (the reference's verify_block_parallel_replay runs them in order,
 * dflash_mlx/runtime.py:117-147).  Scan arguments as
 * dflash_gdn_verify_scan_rollback (B, T > 0); logits fp32 or bf16 [accept_B,
 * N, V] with 16-byte aligned rows (strides in elements); workspace as for
 * dflash_greedy_accept(accept_B, N, V).
 */
int dflash_gdn_verify_scan_rollback_argmax(
    const void* q, const void* k, const void* v, const float* g,
    const float* beta, float* state, const float* prev_tape,
    const int32_t* prev_accepted, int prev_T, int accepted_period, void* out,
    float* final_state, float* tape, int B, int T, int Hk, int Hv, int Dk,
    int Dv, const int64_t* strides, const void* logits, int logits_dtype,
    int64_t logits_batch_stride, int64_t logits_row_stride, int accept_B,
    int N, int V, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The whole fused verify step in one launch: dflash_gdn_verify_scan_rollback_argmax
 * followed by dflash_accept_keys_conv_rollback (the reference's
 * verify_block_parallel_replay after the target forward: greedy accept, keep
 * = matched + accepted_offset, conv-window rollback; dflash_mlx/runtime.py:
 * 117-163, adapters.py:505-560), with the same outputs bit for bit.  The last
 * of each sequence's argmax workgroups to finish (counted in the workspace)
 * merges that sequence's keys, writes posterior / matched / bonus and
 * accepted_out[b] = clamp(matched + accepted_offset, 0, T), and copies its
 * conv windows of all L layers, while the scan's workgroups run on; no
 * workgroup waits on another.  accepted_out must not be prev_accepted (the
 * scan of the same launch reads that one): a serving loop alternates two
 * buffers.  Scan and logits arguments as dflash_gdn_verify_scan_rollback_argmax;
 * draft / draft_stride / n_draft / posterior / matched / bonus as
 * dflash_greedy_accept (posterior, matched, bonus may be NULL); conv_in /
 * qkv / conv_out as dflash_conv_rollback with bf16 elements whose rows and
 * pointers are 16-byte aligned.  L = 0: no conv windows (the caller runs
 * dflash_conv_rollback with accepted_out after it: one workgroup copies
 * the windows here, at one CU's streaming rate, which only pays while the
 * copy is small).  Supported: N <= 64, K1 <= 4, L <= 32.
 * workspace: dflash_gdn_verify_step_workspace_bytes(accept_B, N, V) bytes,
 * 256-byte aligned, zeroed once before the first call (every call leaves its
 * counts zeroed again); calls sharing it must not overlap (one stream).
 */
size_t dflash_gdn_verify_step_workspace_bytes(int B, int N, int V);
int dflash_gdn_verify_step(
    const void* q, const void* k, const void* v, const float* g,
    const float* beta, float* state, const float* prev_tape,
    const int32_t* prev_accepted, int prev_T, int accepted_period, void* out,
    float* final_state, float* tape, int B, int T, int Hk, int Hv, int Dk,
    int Dv, const int64_t* strides, const void* logits, int logits_dtype,
    int64_t logits_batch_stride, int64_t logits_row_stride, int accept_B,
    int N, int V, const int32_t* draft, int64_t draft_stride, int n_draft,
    int32_t* posterior, int32_t* matched, int32_t* bonus, int accepted_offset,
    int32_t* accepted_out, const void* const* conv_in, const void* const* qkv,
    void* const* conv_out, int L, int K1, int64_t C, int64_t qkv_batch_stride,
    int64_t qkv_row_stride, void* workspace, size_t workspace_bytes,
    void* stream);

/*
 * State-only replay of the first n_b tokens: the same recurrence without q,
 * out or tape.  Replaces advance_gated_delta_states(initial_states, keys,
 * values, g, beta) (dflash_mlx/custom_qwen35_model.py:97-139, duplicate at
 * dflash_mlx/adapters.py:93-135) and its Metal kernel
 * gated_delta_state_update (custom_qwen35_model.py:29-89).  The reference
 * passes keys already repeated to Hv heads; pass Hk == Hv for that layout,
 * or Hk < Hv to read un-repeated keys.  strides as for the scan (q entries
 * ignored).  state_out may alias state_in.
 */
int dflash_gdn_replay(const void* k, const void* v, const float* g,
                      const float* beta, const float* state_in,
                      float* state_out, const int32_t* lengths, int B, int T,
                      int Hk, int Hv, int Dk, int Dv, const int64_t* strides,
                      void* stream);

/*
 * Prompt prefill of one gated-delta layer in chunked (WY / UT-transform) form.
 *
 * Replaces the prompt-pass scan mlx_lm gated_delta_update(q, k, v, a, b,
 * A_log, dt_bias, state) (dflash_mlx/custom_qwen35_model.py:790-801, reached
 * from the prefill at dflash_mlx/runtime.py:384-388) for long prompts: the
 * same recurrence as dflash_gdn_verify_scan (same q/k/v/g/beta/state layouts
 * and strides; out and final_state; no tape, no lengths), evaluated over
 * chunks of 64 tokens so the token-token and token-state products run on the
 * matrix cores.  Results agree with the sequential scan to fp32 rounding
 * (the order of the sums differs), not bit for bit.
 *
 * workspace: device memory of at least
 * dflash_gdn_chunked_prefill_workspace_bytes(B, T, Hv, Dk, Dv) bytes,
 * 16-byte aligned, no initial contents needed (about 82 KB per head per
 * 64 tokens).  final_state may be NULL and must not alias state_in.
 * Supported: Dk == Dv == 128, Hv % Hk == 0.
 */
size_t dflash_gdn_chunked_prefill_workspace_bytes(int B, int T, int Hv,
                                                  int Dk, int Dv);
int dflash_gdn_chunked_prefill(const void* q, const void* k, const void* v,
                               const float* g, const float* beta,
                               const float* state_in, void* out,
                               float* final_state, int B, int T, int Hk,
                               int Hv, int Dk, int Dv, const int64_t* strides,
                               void* workspace, size_t workspace_bytes,
                               void* stream);

/*
 * Greedy verify accept: argmax over the vocabulary, then the longest prefix of
 * the draft that agrees with it.
 *
 * Replaces sample_tokens(logits, temperature=0) (dflash_mlx/runtime.py:22-29)
 * followed by longest_prefix_match(block[1:], posterior[:-1]) and the bonus
 * pick posterior[matched] (runtime.py:41-47, :145-147, :163).
 *
 *   posterior[b,i] = argmax_v logits[b,i,v]   (lowest index wins ties; NaN
 *                    counts as larger than every number, first NaN wins)
 *   matched[b]     = largest m <= min(n_draft, N) with
 *                    draft[b,j] == posterior[b,j] for all j < m
 *   bonus[b]       = posterior[b, matched[b]] if matched[b] < N, else -1
 * The reference wiring is draft = block[1:] (n_draft = T-1) against N = T
 * logit rows; accepted_inputs = matched + 1.  n_draft = 0 gives the plain
 * greedy sample (matched = 0, bonus = posterior[b,0]).
 *
 * logits: [B, N, V] of logits_dtype (DFLASH_DTYPE_F32 / _BF16 / _F16),
 * innermost contiguous, batch and row strides in elements.  draft: int32
 * [B, n_draft] with batch stride draft_stride.  posterior (int32 [B, N],
 * contiguous; may be NULL), matched and bonus (int32 [B]) are outputs.
 * matched and bonus may be NULL when only posterior is wanted.
 * workspace: device memory of at least
 * dflash_greedy_accept_workspace_bytes(B, N, V) bytes, 8-byte aligned, no
 * initial contents needed (it holds the per-slice partial maxima between the
 * two launches).  Calls that overlap in time must use different workspaces.
 */
size_t dflash_greedy_accept_workspace_bytes(int B, int N, int V);
int dflash_greedy_accept(const void* logits, int logits_dtype,
                         int64_t logits_batch_stride, int64_t logits_row_stride,
                         const int32_t* draft, int64_t draft_stride,
                         int n_draft, int32_t* posterior, int32_t* matched,
                         int32_t* bonus, int B, int N, int V, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * dflash_greedy_accept without a workspace argument and without allocating:
 * no reference counterpart; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The argmax keys go to a static device array of
 * dflash_greedy_accept_noalloc_max_bytes() bytes (1 MiB) that each device
 * holds until the process ends; shapes whose
 * dflash_greedy_accept_workspace_bytes(B, N, V) exceeds it are refused with
 * DFLASH_ERR_WORKSPACE before any launch (that is B * N > 131072 logits
 * rows, at any vocabulary size).  Calls on one device share the array, so
 * calls that overlap in time on one device race.  The first call with a
 * device current resolves the array's address on that device
 * (hipGetSymbolAddress).  Arguments and outputs as dflash_greedy_accept,
 * bit for bit.
 */
size_t dflash_greedy_accept_noalloc_max_bytes(void);
int dflash_greedy_accept_noalloc(const void* logits, int logits_dtype,
                                 int64_t logits_batch_stride,
                                 int64_t logits_row_stride,
                                 const int32_t* draft, int64_t draft_stride,
                                 int n_draft, int32_t* posterior,
                                 int32_t* matched, int32_t* bonus, int B, int N,
                                 int V, void* stream);

/*
 * Gated-delta layer prologue: everything between the input projections and
 * the scan, in one launch.
 *
 * Replaces the layer body at dflash_mlx/custom_qwen35_model.py:431-450:
 * conv_input = concat(conv_state, qkv); causal depthwise conv1d (weight
 * [C, K, 1], :718-725) + silu; split into q | k | v heads; q <- Dk^-1 *
 * rms_norm(q, eps), k <- Dk^-1/2 * rms_norm(k, eps); beta = sigmoid(b);
 * g = compute_g(A_log, a, dt_bias) = exp(-exp(A_log) * softplus(a + dt_bias))
 * (mlx-lm 0.31.2, the published Qwen3-Next decay); new conv window
 * conv_input[:, -(K-1):] (:434).
 *
 * qkv: bf16 [B, T, C], C = 2*Hk*Dk + Hv*Dv contiguous, batch/row strides in
 * elements; conv_state bf16 [B, K-1, C] contiguous; conv_weight bf16 [C, K];
 * a, b bf16 [B, T, Hv] with strides {a_b, a_t, b_b, b_t} (NULL: contiguous);
 * A_log fp32 [Hv]; dt_bias bf16 [Hv].  Outputs: act bf16 [B, T, C] holding
 * q | k | v (the scan reads them as strided views), g and beta fp32
 * [B, T, Hv], new_conv_state bf16 [B, K-1, C], which must not alias
 * conv_state.  All arithmetic is fp32; only act is rounded (to bf16).
 * Supported: Dk % 64 == 0, Dk <= 256, 1 <= K <= 8.
 */
int dflash_gdn_prologue(const void* qkv, int64_t qkv_batch_stride,
                        int64_t qkv_row_stride, const void* conv_state,
                        const void* conv_weight, const void* a, const void* b,
                        const int64_t* ab_strides, const float* A_log,
                        const void* dt_bias, void* act, float* g, float* beta,
                        void* new_conv_state, int B, int T, int K, int Hk,
                        int Hv, int Dk, int Dv, float eps, void* stream);

/*
 * dflash_gdn_prologue followed by dflash_gdn_verify_scan_rollback, in one
 * launch: the scan's workgroups compute the prologue of their own head from
 * the raw projection rows (into LDS) instead of reading act, g and beta.
 *
 * Replaces the same reference span as the pair: the layer body at
 * dflash_mlx/custom_qwen35_model.py:431-466 (conv + silu, q/k rms-norm, g and
 * beta, then the gated-delta kernel of :33-74 with its tape), with the
 * rollback of the previous verify fused into the state load as in
 * dflash_gdn_verify_scan_rollback.  The reference has no single call for it.
 *
 * Arguments as the two calls it stands for: the prologue's inputs (qkv,
 * conv_state, conv_weight, a, b, A_log, dt_bias, K, eps), then the rollback
 * scan's state / tape / selection and outputs (out is required).  q, k, v, g
 * and beta are bit-identical to what dflash_gdn_prologue would store, so
 * out, final_state and tape are bit-identical to the two-call path.  No new
 * conv window is written (the pair's new_conv_state output is dropped; the
 * verify path rebuilds the window at commit, dflash_conv_rollback).
 * Supported: Dk == 128, Dv % 16 == 0, 1 <= K <= 8, T <= 32; qkv 4-byte
 * aligned with even strides, conv_state 4-byte aligned.
 */
int dflash_gdn_prologue_scan_rollback(
    const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
    const void* conv_state, const void* conv_weight, const void* a,
    const void* b, const int64_t* ab_strides, const float* A_log,
    const void* dt_bias, float* state, const float* prev_tape,
    const int32_t* prev_accepted, int prev_T, int accepted_period, void* out,
    float* final_state, float* tape, int B, int T, int K, int Hk, int Hv,
    int Dk, int Dv, float eps, void* stream);

/*
 * Gated-delta layer epilogue: y = weight * x * rsqrt(mean(x^2) + eps) *
 * silu(z) over each (b, t, h) row of D channels.
 *
 * Replaces RMSNormGated(out, z) (dflash_mlx/custom_qwen35_model.py:478;
 * mlx-lm qwen3_next, the published Qwen3-Next gated norm).
 * x bf16 [B, T, H, D] contiguous (the scan's out); z bf16 [B, T, H, D] with
 * element strides {b, t, h} (NULL: contiguous), D contiguous; weight bf16
 * [D]; y bf16 [B, T, H, D] contiguous.  Supported: D % 64 == 0, D <= 256.
 */
int dflash_gdn_gated_rmsnorm(const void* x, const void* z,
                             const int64_t* z_strides, const void* weight,
                             void* y, int B, int T, int H, int D, float eps,
                             void* stream);

/*
 * Fused greedy LM head + accept: the same outputs as dflash_greedy_accept on
 * logits = hidden . weight^T, without materialising the logits.
 *
 * Replaces MLXTargetAdapter.lm_head_argmax(model, hidden_states)
 * (dflash_mlx/adapters.py:267-271) and the prefix compare that follows it in
 * verify_block_parallel_greedy_argmax (dflash_mlx/runtime.py:246-292).
 *
 * hidden: bf16 [B*N, H] (row b*N + i is sequence b, position i), row stride
 * hidden_row_stride; weight: bf16 [V, H] (the LM head / tied embedding
 * matrix), row stride weight_row_stride.  Logits are accumulated in fp32 from
 * bf16 products (MFMA); posterior/matched/bonus and the draft follow
 * dflash_greedy_accept.  Supported: B*N <= 64, H % 64 == 0, 16-byte aligned
 * rows.  workspace: dflash_lm_head_accept_workspace_bytes(B, N, V) bytes,
 * 8-byte aligned, no initial contents needed.
 */
size_t dflash_lm_head_accept_workspace_bytes(int B, int N, int V);
int dflash_lm_head_greedy_accept(const void* hidden, int64_t hidden_row_stride,
                                 const void* weight, int64_t weight_row_stride,
                                 int H, int V, const int32_t* draft,
                                 int64_t draft_stride, int n_draft,
                                 int32_t* posterior, int32_t* matched,
                                 int32_t* bonus, int B, int N,
                                 void* workspace, size_t workspace_bytes,
                                 void* stream);

/*
 * dflash_lm_head_greedy_accept over the head's fragment-tiled copy
 * (dflash_weight_tile_bf16(weight, H, weight_tiled, V, H, stream), made once
 * at load time): the same reference call replaced, the same outputs and
 * workspace.  The contraction is split over two k-halves summed in fp32, so
 * a logit may differ from the row-major kernel's in its last bits (ties
 * within fp32 rounding may pick either token).  Supported: V % 16 == 0 and
 * the limits above.
 */
int dflash_lm_head_greedy_accept_tiled(const void* hidden,
                                       int64_t hidden_row_stride,
                                       const void* weight_tiled, int H, int V,
                                       const int32_t* draft,
                                       int64_t draft_stride, int n_draft,
                                       int32_t* posterior, int32_t* matched,
                                       int32_t* bonus, int B, int N,
                                       void* workspace, size_t workspace_bytes,
                                       void* stream);

/*
 * Recurrent-state rollback by tape gather, for L layers in one launch.
 *
 * Replaces the replay in Qwen3_5TextModel.rollback_linear_caches
 * (dflash_mlx/custom_qwen35_model.py:1053-1074; adapter copy
 * dflash_mlx/adapters.py:537-560), which re-runs the accepted prefix; with
 * the tape the state after a accepted tokens is already stored.
 *
 * For layer l < L and sequence b < B with a = clamp(accepted[b], 0, T):
 *   states_out[l][b] = a >= 1 ? tapes[l][a-1, b] : states_in[l][b]
 * tapes[l] is [T, B, S] fp32 whose token index has stride tape_token_stride
 * elements (0 means B*S, a contiguous per-layer tape; layers stacked as batch
 * entries of one scan pass L*B*S), states_in[l] / states_out[l] are [B, S]
 * fp32 with S = state_elems (= Hv*Dv*Dk).  The three arguments are host
 * arrays of L device pointers.  states_out[l] may alias states_in[l].
 */
int dflash_tape_select(const float* const* tapes,
                       const float* const* states_in, float* const* states_out,
                       const int32_t* accepted, int L, int B, int T,
                       int64_t state_elems, int64_t tape_token_stride,
                       void* stream);

/*
 * Convolution-window rollback for L layers in one launch.
 *
 * Replaces the conv-state half of rollback_linear_caches
 * (dflash_mlx/custom_qwen35_model.py:1044-1051; adapters.py:530-536):
 *   conv_out[l][b] = concat(conv_in[l][b], qkv[l][b, :a], axis=0)[-K1:]
 * with a = clamp(accepted[b], 0, T) and K1 = conv kernel size - 1, i.e. row r
 * of the window is conv_in row a+r when a+r < K1, else qkv row a+r-K1.
 * conv_in[l] / conv_out[l]: [B, K1, C] contiguous; qkv[l]: [B, T, C] with
 * batch / row strides in elements and C contiguous.  elem_bytes is 2 or 4.
 * conv_out[l] may alias conv_in[l].  Host arrays of L device pointers.
 */
int dflash_conv_rollback(const void* const* conv_in, const void* const* qkv,
                         void* const* conv_out, const int32_t* accepted, int L,
                         int B, int T, int K1, int64_t C,
                         int64_t qkv_batch_stride, int64_t qkv_row_stride,
                         int elem_bytes, void* stream);

/*
 * dflash_greedy_accept followed by dflash_conv_rollback with
 * accepted[b] = matched[b] + accepted_offset, in two launches instead of
 * three: the accept's finalize (key merge, prefix compare, bonus) runs inside
 * the conv-window copy's workgroups, each of which needs its sequence's
 * accepted count anyway.
 *
 * Replaces the accept of verify_block_parallel_replay (dflash_mlx/runtime.py:
 * 134-147: argmax, longest_prefix_match, bonus) and the conv half of the
 * rollback that follows it (custom_qwen35_model.py:1044-1051); the reference
 * has no single call for the pair.  accepted_offset is 1 to roll back to
 * accepted_inputs = matched + 1 (runtime.py:146), 0 to keep matched tokens.
 * Arguments and outputs as the two calls (posterior and bonus may be NULL);
 * the outputs are bit-identical to theirs.  accepted_out ([B] int32, or
 * NULL) receives clamp(matched + accepted_offset, 0, T), the keep count that
 * dflash_gdn_verify_scan_rollback of the next step reads as prev_accepted.
 * With L, K1 or C zero only the accept runs (accepted_out must be NULL).
 */
int dflash_greedy_accept_conv_rollback(
    const void* logits, int logits_dtype, int64_t logits_batch_stride,
    int64_t logits_row_stride, const int32_t* draft, int64_t draft_stride,
    int n_draft, int32_t* posterior, int32_t* matched, int32_t* bonus, int B,
    int N, int V, void* workspace, size_t workspace_bytes,
    const void* const* conv_in, const void* const* qkv, void* const* conv_out,
    int accepted_offset, int32_t* accepted_out, int L, int T, int K1, int64_t C,
    int64_t qkv_batch_stride, int64_t qkv_row_stride, int elem_bytes,
    void* stream);

/*
 * The second launch of dflash_greedy_accept_conv_rollback alone: the same
 * finalize + conv-window rollback from argmax keys already in `workspace`
 * (written by dflash_gdn_verify_scan_rollback_argmax for the same B, N, V).
 * Arguments and outputs as dflash_greedy_accept_conv_rollback, the same bits.
 */
int dflash_accept_keys_conv_rollback(
    const int32_t* draft, int64_t draft_stride, int n_draft, int32_t* posterior,
    int32_t* matched, int32_t* bonus, int B, int N, int V,
    const void* workspace, size_t workspace_bytes, const void* const* conv_in,
    const void* const* qkv, void* const* conv_out, int accepted_offset,
    int32_t* accepted_out, int L, int T, int K1, int64_t C,
    int64_t qkv_batch_stride, int64_t qkv_row_stride, int elem_bytes,
    void* stream);

/*
 * ---- The rest of the hybrid target's verify step (config c4) ----
 * Cache lengths `lens` are int32 [B] in device memory, so a whole verify step
 * (append, attend, accept, commit) needs no host round trip.
 */

/*
 * Residual add + RMSNorm of the decoder layers: DecoderLayer.__call__
 * (dflash_mlx/custom_qwen35_model.py:841-845) with nn.RMSNorm input /
 * post-attention layernorms (:824-827) and the final norm (:881).
 *   h = bf16(x + r) -> h_out;  y = bf16(h * rsqrt(mean(h^2) + eps) * weight)
 * r may be NULL (then h = x and h_out is not written).  x, r, h_out, y are
 * bf16 [M, H] contiguous, weight bf16 [H]; h_out may alias x.  fp32
 * arithmetic.  Supported: H % 8 == 0, H <= 8192.
 */
int dflash_add_rmsnorm(const void* x, const void* r, const void* weight,
                       void* h_out, void* y, int M, int H, float eps,
                       void* stream);

/*
 * dflash_add_rmsnorm with the branch given as the fp32 split-K partial sums
 * of the projection that produced it (dflash_gemm_bf16 with nsplit > 1):
 *   r = bf16(sum_s r_partials[s][m][:]),  h = bf16(x + r),  y as above.
 * r_partials is fp32 [nsplit, M, H] contiguous, 16-byte aligned.
 */
int dflash_add_rmsnorm_splitk(const void* x, const float* r_partials,
                              int nsplit, const void* weight, void* h_out,
                              void* y, int M, int H, float eps, void* stream);

/*
 * dflash_add_rmsnorm (r_partials NULL) or dflash_add_rmsnorm_splitk (r NULL)
 * that also stores the new residual stream h to h_copy (row m at
 * h_copy + m * h_copy_row_stride, bf16; stride % 8 == 0, >= H).
 *
 * Replaces the capture of the target hidden states the drafter reads:
 * `selected_hidden_states.append(hidden_states)` after each layer in
 * layer_ids and the concatenation along the feature axis
 * (dflash_mlx/custom_qwen35_model.py:984-991, adapters.py:402-414).  The
 * residual stream after layer i is complete in the add that opens layer
 * i + 1 (or the final norm), so the caller points h_copy at that layer's
 * column block of the [M, n_layers * H] capture buffer.
 */
int dflash_add_rmsnorm_capture(const void* x, const void* r,
                               const float* r_partials, int nsplit,
                               const void* weight, void* h_out, void* h_copy,
                               int64_t h_copy_row_stride, void* y, int M,
                               int H, float eps, void* stream);

/*
 * The step's first norm with the embedding lookup folded in
 * (Qwen3_5TextModel: embed_tokens(inputs) then layer 0's input_layernorm,
 * custom_qwen35_model.py:866-869, :841):
 *   h_out[m] = table[tokens[m]],  y = bf16(h * rsqrt(mean(h^2) + eps) * weight).
 * table bf16 [vocab, H], tokens int32 [M] on the device (ids outside
 * [0, vocab) are clamped: the kernel cannot raise, and must stay in bounds).
 */
int dflash_embed_rmsnorm(const void* table, const int32_t* tokens, int vocab,
                         const void* weight, void* h_out, void* y, int M,
                         int H, float eps, void* stream);

/*
 * Verify-sized projection GEMM: out[M, N] = x[M, K] . w[N, K]^T, bf16 in,
 * fp32 accumulation, M <= 64 (the block rows of a verify step).  Every
 * Linear of the target's layers at verify time (custom_qwen35_model.py:726-
 * 736; mlx-lm Qwen3NextAttention / Qwen3NextMLP projections) has this shape:
 * a stream of the weight against 16 rows, which library GEMMs tuned for
 * large M serve at a fraction of HBM bandwidth.
 * nsplit: split-K factor requested; dflash_gemm_splits(K, nsplit) is the
 * number of splits actually used.  With nsplit == 1, out is bf16 [M, N] with
 * row stride out_row_stride (elements; multiple of 4, 8-byte aligned).  With
 * nsplit > 1, out is fp32 partial sums [dflash_gemm_splits(K, nsplit), M, N]
 * (16-byte aligned) for dflash_add_rmsnorm_splitk or dflash_splitk_reduce.
 * rows_per_wave (16 or 32) sets the weight rows a wavefront streams; k_waves
 * (1 or 4) how many of a workgroup's 4 wavefronts share those rows, each
 * streaming a quarter of the k-range (4: a workgroup covers rows_per_wave
 * rows, merged through LDS; 1: it covers 4 * rows_per_wave rows).
 * Supported: K % 64 == 0, row strides multiples of 8 elements, 16-byte
 * aligned x and w.
 */
int dflash_gemm_bf16(const void* x, int64_t x_row_stride, const void* w,
                     int64_t w_row_stride, void* out, int64_t out_row_stride,
                     int M, int N, int K, int nsplit, int rows_per_wave,
                     int k_waves, void* stream);
int dflash_gemm_splits(int K, int nsplit);

/*
 * The MLP's gate/up projection with its gating fused (Qwen3NextMLP,
 * custom_qwen35_model.py:845: down(silu(gate(x)) * up(x)) up to the down
 * projection): out[M, N/2] = bf16(silu(x . G^T) * (x . U^T)) where w_pairs
 * [N, K] holds 32-row blocks of 16 gate rows followed by the 16 up rows of the
 * same output columns (block j: gate rows 16j .. 16j+15, then up rows 16j ..
 * 16j+15).  Supported: N % 32 == 0, K % 64 == 0; k_waves as above.
 */
int dflash_gemm_bf16_swiglu(const void* x, int64_t x_row_stride,
                            const void* w_pairs, int64_t w_row_stride,
                            void* out, int64_t out_row_stride, int M, int N,
                            int K, int k_waves, void* stream);

/*
 * The same projections with the weight stored once, at load time, as MFMA
 * fragments (the nn.Linear weight [N, K] of custom_qwen35_model.py:726-736
 * and mlx-lm's attention / MLP Linears, re-laid out for streaming):
 *   w_tiled[((ks * (N/16) + rt) * 2 + h) * 512 + l * 8 + e]
 *     = w[16 rt + l % 16][64 ks + 16 (l / 16) + 8 h + e],
 * so every 64-lane load is 1 KB of contiguous memory going straight into
 * matrix-core registers, and workgroups in flight read close together.  dflash_weight_tile_bf16 builds it (N % 16 == 0,
 * K % 64 == 0; dflash_weight_tile_bytes(N, K) bytes, 16-byte aligned); the
 * _tiled GEMMs take it in place of (w, w_row_stride) and return the same sums
 * bit for bit as their row-major counterparts.  rows_per_wave may also be 64
 * here.  dflash_gemm_bf16_swiglu_tiled takes the tiled form of its w_pairs.
 */
size_t dflash_weight_tile_bytes(int N, int K);
int dflash_weight_tile_bf16(const void* w, int64_t w_row_stride, void* w_tiled,
                            int N, int K, void* stream);
int dflash_gemm_bf16_tiled(const void* x, int64_t x_row_stride,
                           const void* w_tiled, void* out,
                           int64_t out_row_stride, int M, int N, int K,
                           int nsplit, int rows_per_wave, int k_waves,
                           void* workspace, size_t workspace_bytes,
                           void* stream);
int dflash_gemm_bf16_swiglu_tiled(const void* x, int64_t x_row_stride,
                                  const void* w_pairs_tiled, void* out,
                                  int64_t out_row_stride, int M, int N, int K,
                                  int k_waves, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * Workspace of the tiled GEMMs' tail split (dflash_gemm_bf16_tiled,
 * _swiglu_tiled, _tiled_normed, _swiglu_tiled_normed; k_waves 4, one
 * K split): bytes to pass, 256-byte aligned.  Its first 1 KB holds arrival
 * counters: zero them once before the first call (every call leaves them
 * zero again); the rest holds partial sums and needs no clearing.  With it,
 * when the row groups
 * (N / rows_per_wave; 32 rows for the SwiGLU forms) leave a last round of
 * T groups on the device's compute units with 4T <= CUs (and T <= 64),
 * those T groups run as 4T single-wavefront units of a k-quarter each,
 * merged through the workspace in the workgroup's own k order: the same
 * bits as without it (NULL workspace), in less time.  Calls sharing a
 * workspace must not overlap (one stream).  No reference counterpart
 * (scheduling of the verify-sized projections).
 */
size_t dflash_gemm_tail_workspace_bytes(void);

/*
 * The decoder layer's residual add and the next RMSNorm folded into the two
 * projections around them, with no launch of their own (the residual adds
 * `h = h + r` and norms `input_layernorm` / `post_attention_layernorm` of the
 * decoder layer, custom_qwen35_model.py:836-846, and the RMSNorm of mlx-lm):
 *
 * dflash_gemm_bf16_tiled_residual_norm: the tiled projection r = bf16(x .
 * w^T) (no K split across workgroups: 16 wavefronts of a workgroup share
 * each 16-column tile's k-range), then
 *   h = bf16(resid + r),  h_out = h (h_copy = h too, row stride
 *   h_copy_row_stride, when not NULL),
 *   row_sumsq[t, m] = sum of h[m, n]^2 over the tile's columns n in
 *   [16t, 16t + 16)   (fp32 [N / 16, M]).
 * resid may alias h_out.  Supported: N % 16 == 0, K % 64 == 0.
 *
 * dflash_gemm_bf16_tiled_normed / dflash_gemm_bf16_swiglu_tiled_normed: the
 * tiled projections (k_waves 4, K <= 16384) whose activation rows are the
 * RMSNorm output of h over its K columns,
 *   y = bf16((h[m, k] * inv[m]) * norm_weight[k]),
 *   inv[m] = 1 / sqrt(sum_t row_sumsq[t, m] / K + eps)
 * (the row sums of the producing call, norm_tiles = its N / 16, added in a
 * fixed order that depends on neither M nor the launch), computed on load.
 * row_inv_out (fp32 [M]) receives inv when not NULL.  Apart from inv's
 * summation order, y is what dflash_add_rmsnorm computes.
 */
int dflash_gemm_bf16_tiled_residual_norm(const void* x, int64_t x_row_stride,
                                         const void* w_tiled, int M, int N,
                                         int K, const void* resid, void* h_out,
                                         void* h_copy, int64_t h_copy_row_stride,
                                         float* row_sumsq, void* stream);
int dflash_gemm_bf16_tiled_normed(const void* h, int64_t h_row_stride,
                                  const void* norm_weight,
                                  const float* row_sumsq, int norm_tiles,
                                  float eps, float* row_inv_out,
                                  const void* w_tiled, void* out,
                                  int64_t out_row_stride, int M, int N, int K,
                                  int nsplit, int rows_per_wave, int k_waves,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);
int dflash_gemm_bf16_swiglu_tiled_normed(const void* h, int64_t h_row_stride,
                                         const void* norm_weight,
                                         const float* row_sumsq, int norm_tiles,
                                         float eps, float* row_inv_out,
                                         const void* w_pairs_tiled, void* out,
                                         int64_t out_row_stride, int M, int N,
                                         int K, int k_waves, void* workspace,
                                         size_t workspace_bytes, void* stream);

/*
 * Prompt-sized projection GEMMs over the same fragment-tiled weights:
 * out[M, N] = bf16(x[M, K] . w[N, K]^T) for M = the rows of a prompt pass
 * (any M >= 0; built for hundreds to thousands of rows), fp32 accumulation
 * with one chain per output in k order.
 *
 * Replaces every nn.Linear of the target's layers during the prompt pass
 * (Qwen3_5TextModel over the whole prompt, dflash_mlx/runtime.py:384-390 ->
 * forward_dflash, custom_qwen35_model.py:883-1001; the Linears of :726-736
 * and mlx-lm Qwen3NextAttention / Qwen3NextMLP), where each weight is
 * contracted against all P rows at once on the matrix cores instead of
 * being streamed once per 16-row verify block.
 * w_tiled is dflash_weight_tile_bf16's layout (N % 16 == 0, K % 64 == 0).
 * dflash_gemm_bf16_swiglu_tiled_prefill takes the tiled w_pairs of
 * dflash_gemm_bf16_swiglu (N % 32 == 0) and writes out[M, N/2] =
 * bf16(silu(x . G^T) * (x . U^T)).  x: 16-byte aligned, row stride a
 * multiple of 8 elements (>= K, <= 2^22); out: 8-byte aligned, row stride a
 * multiple of 4 (>= N, or N/2).  Workgroups own 256 x 256 or 256 x 128
 * output tiles, whichever takes fewer rounds of the compute units (a
 * 256 x 128 tile counted at 0.7); the sums are the same bits either way.
 */
int dflash_gemm_bf16_tiled_prefill(const void* x, int64_t x_row_stride,
                                   const void* w_tiled, void* out,
                                   int64_t out_row_stride, int M, int N, int K,
                                   void* stream);
int dflash_gemm_bf16_swiglu_tiled_prefill(const void* x, int64_t x_row_stride,
                                          const void* w_pairs_tiled, void* out,
                                          int64_t out_row_stride, int M, int N,
                                          int K, void* stream);
/*
 * dflash_gemm_bf16_tiled_prefill with the k-range split nsplit ways (for
 * output shapes with too few tiles to fill the device): fp32 partial sums
 * [dflash_gemm_splits(K, nsplit), M, N] (16-byte aligned) for
 * dflash_add_rmsnorm_splitk / dflash_splitk_reduce, which add them in split
 * order.
 */
int dflash_gemm_bf16_tiled_prefill_splitk(const void* x, int64_t x_row_stride,
                                          const void* w_tiled, float* partials,
                                          int nsplit, int M, int N, int K,
                                          void* stream);

/*
 * The prompt-sized GEMMs over rows row0 .. row0+N-1 of a tiled weight of
 * w_rows rows (the same projections of custom_qwen35_model.py:726-736 as
 * above; a launch over part of a projection, so that a projection's last
 * output tiles can run split-K apart from the rest): nsplit == 0 writes
 * bf16 out[M, N] (swiglu != 0: the gated out[M, N/2] of a w_pairs weight),
 * nsplit >= 1 writes fp32 partials [dflash_gemm_splits(K, nsplit), M, N]
 * (swiglu must be 0; dflash_splitk_swiglu_reduce gates a w_pairs range).
 * Each output's sums are the bits of the whole-weight launch.  Needs
 * w_rows % 16 == 0, row0 and N multiples of 16 (32 with swiglu),
 * row0 + N <= w_rows; otherwise as dflash_gemm_bf16_tiled_prefill(_splitk).
 */
int dflash_gemm_bf16_tiled_prefill_rows(const void* x, int64_t x_row_stride,
                                        const void* w_tiled, int w_rows, int row0,
                                        void* out, int64_t out_row_stride,
                                        float* partials, int nsplit, int M, int N,
                                        int K, int swiglu, void* stream);

/*
 * out[m, n] = bf16(sum_s partials[s, m, n]) for partials fp32 [nsplit, M, N]
 * (N % 4 == 0), out bf16 with row stride out_row_stride.
 */
int dflash_splitk_reduce(const float* partials, int nsplit, int M, int N,
                         void* out, int64_t out_row_stride, void* stream);

/*
 * The MLP's gating over split-K partials (mlx-lm Qwen3NextMLP, called at
 * dflash_mlx/custom_qwen35_model.py:845; the partials of a
 * dflash_gemm_bf16_tiled_prefill_splitk over the tiled w_pairs of
 * dflash_gemm_bf16_swiglu): out[m, j] = bf16(silu(g) * u) with g and u the
 * split sums (in split order) of partials columns 32 (j / 16) + j % 16 and
 * that column + 16.  partials fp32 [nsplit, M, N] (16-byte aligned,
 * N % 32 == 0), out bf16 [M, N/2] with row stride out_row_stride (a
 * multiple of 4, >= N/2).
 */
int dflash_splitk_swiglu_reduce(const float* partials, int nsplit, int M, int N,
                                void* out, int64_t out_row_stride, void* stream);

/*
 * The MLP's gating (mlx-lm Qwen3NextMLP, called at
 * dflash_mlx/custom_qwen35_model.py:845): out = bf16(silu(gate) * up) with
 * gate_up bf16 [M, 2I] = [gate | up] (one GEMM of the stacked gate/up
 * projections) and out bf16 [M, I].  Supported: I % 8 == 0.
 */
int dflash_swiglu(const void* gate_up, void* out, int M, int I, void* stream);

/*
 * Gated full-attention layer, before the attention itself
 * (forward_full_attention_layer_explicit, custom_qwen35_model.py:496-522):
 * from the stacked q/k/v projection rows proj [B*T, proj_row_stride] bf16,
 * laid out [Hq x (query D | gate D), Hkv x key D, Hkv x value D]:
 *   q = rope(rms_norm(query) * q_norm_w)      -> q_out [B, T, Hq, D] bf16
 *   k = rope(rms_norm(key) * k_norm_w)        -> k_cache[b, h, pos]
 *   v                                          -> vt_cache[b, h, :, pos]
 * with pos = lens[b] + t.  k_cache is [B, Hkv, Smax, D], vt_cache is the
 * value cache transposed, [B, Hkv, D, Smax] (keys contiguous per feature).
 * Rotary (nn.RoPE, traditional=False): feature i < rot_dims/2 pairs with
 * i + rot_dims/2 at angle pos * rope_base^(-2i/rot_dims); features past
 * rot_dims pass through.  Positions outside [0, Smax) are never written: the
 * caller keeps 0 <= lens[b] and lens[b] + T <= Smax, and when overflow is not
 * NULL ([B] int32, cleared by the caller) the kernel sets overflow[b] = 1 for
 * every sequence that had a position outside the cache, so the host can
 * refuse that step's output at its next synchronisation.
 * Supported: D == 128, rot_dims in {0,16,32,64,128}.
 */
int dflash_attn_prep(const void* proj, int64_t proj_row_stride,
                     const void* q_norm_w, const void* k_norm_w,
                     const int32_t* lens, void* k_cache, void* vt_cache,
                     void* q_out, int32_t* overflow, int B, int T, int Hq,
                     int Hkv, int D, int Smax, int rot_dims, float rope_base,
                     float eps, void* stream);

/*
 * Verify attention over the cache (custom_qwen35_model.py:524-534): causal
 * SDPA of the T block queries against the lens[b] + T cached keys (query t
 * sees keys 0 .. lens[b] + t), output * sigmoid(gate) with the gate read from
 * the projection rows (head h at h*2D + D of row b*T + t).
 *   out[b, t, h*D .. h*D+D) = bf16(softmax(scale * q k^T) v * sigmoid(gate))
 * Split over 64-key ranges on MFMA, then one merge.  max_len is a host-side
 * upper bound of lens[b] + T (it sizes the grid; max_len <= Smax).  Cache
 * positions past lens[b] + T are read and given zero weight, so the caches
 * must hold finite values there (allocate them zero-filled).  workspace: at
 * least dflash_attn_verify_workspace_bytes(B, Hq, Hkv, max_len) bytes.
 * Supported: D == 128, T <= 16, Hq / Hkv <= 4, Smax % 64 == 0, B <= 65535.
 */
size_t dflash_attn_verify_workspace_bytes(int B, int Hq, int Hkv, int max_len);
int dflash_attn_verify(const void* q, const void* k_cache,
                       const void* vt_cache, const int32_t* lens,
                       const void* gate_src, int64_t gate_row_stride,
                       void* out, int B, int T, int Hq, int Hkv, int D,
                       int Smax, int max_len, float scale, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * The same gated attention over a prompt pass of one sequence (the SDPA +
 * sigmoid gate of custom_qwen35_model.py:524-534 with the whole prompt as
 * queries, reached from the prefill at dflash_mlx/runtime.py:384-390): the
 * prompt's keys and values are already in the cache (dflash_attn_prep with
 * B = 1, T = P), and prompt row i attends to cache positions 0 .. lens[0] + i.
 *   out[i, h*D .. h*D+D) = bf16(softmax(scale * q_i k^T) v * sigmoid(gate_i))
 * q: [P, Hq, D] bf16 (dflash_attn_prep's q_out); k_cache [Hkv, Smax, D] and
 * vt_cache [Hkv, D, Smax] of the sequence; lens: device int32 [1], the
 * cache length before the prompt (the kernel clamps it to [0, Smax] and reads
 * no position at or past Smax); gate_src: the projection rows (row i's gate of
 * head h at i * gate_row_stride + h*2D + D); out [P, Hq*D] bf16.  Online
 * softmax over 64-key tiles on MFMA, no workspace.
 * Supported: D == 128, Hq / Hkv <= 4, Smax % 64 == 0.
 */
int dflash_attn_prefill(const void* q, const void* k_cache, const void* vt_cache,
                        const int32_t* lens, const void* gate_src,
                        int64_t gate_row_stride, void* out, int P, int Hq,
                        int Hkv, int D, int Smax, float scale, void* stream);

/*
 * Commit a greedy accept on the device: keep[b] = clamp(matched[b], 0, T-1)
 * + 1 (the block's first token plus the accepted drafts, accepted_inputs of
 * runtime.py:146) and, if lens is not NULL, lens[b] += keep[b] (the KV trim
 * of adapters.py:505-508 seen from the other side: the caches keep the
 * accepted positions).  keep feeds dflash_gdn_verify_scan_rollback and
 * dflash_conv_rollback of the next step.
 */
int dflash_commit_accept(const int32_t* matched, int32_t* keep, int32_t* lens,
                         int B, int T, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DFLASH_GDN_H */
