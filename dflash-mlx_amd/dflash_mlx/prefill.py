"""The prompt pass of the hybrid target on MI355X.

The reference runs the prompt through the target in one forward
(dflash_mlx/runtime.py:384-390 -> forward_with_hidden_states ->
Qwen3_5TextModel.forward_dflash, custom_qwen35_model.py:883-1001): every
decoder layer sees all P prompt rows at once, each gated-delta layer runs
gated_delta_update over the P tokens (:790-801) from the cached state, and
each attention layer appends P keys and attends causally (:487-540).

``HybridPrefill`` does the same over the caches of a ``HybridVerifyRunner``
(one sequence), with launches sized to the prompt:

* the projections on the prompt-sized MFMA GEMMs
  (``dflash_gemm_bf16_tiled_prefill``, the MLP gating fused:
  ``dflash_gemm_bf16_swiglu_tiled_prefill``) over the verify GEMMs'
  fragment-tiled weights (a stacked projection whose row count is not a
  multiple of 16 gets a zero-padded tiled copy of its own);
* per gated-delta layer: the prologue over the P tokens
  (``dflash_gdn_prologue``: conv1d + silu from the cached window, q/k norms,
  g and beta, the new window), the chunked WY-form scan on the matrix cores
  (``dflash_gdn_chunked_prefill``) from the cached state, the gated RMSNorm;
* per attention layer: q/k norm + rotary + KV append at the cached length
  (``dflash_attn_prep`` with T = P), causal attention over cache + prompt
  (``dflash_attn_prefill``);
* residual adds and norms (``dflash_embed_rmsnorm``, ``dflash_add_rmsnorm``,
  ``dflash_add_rmsnorm_capture`` for the target hidden states at the
  runner's capture layers); a projection into the residual stream whose
  output tiles would leave most compute units idle in the last round runs
  split-K (``dflash_gemm_bf16_tiled_prefill_splitk``) and the add + norm
  sums its fp32 partials (``dflash_add_rmsnorm_splitk``); a projection with
  a bf16 output (the gated-delta in_proj, q|k|v, gate|up) whose tiles would
  leave most compute units idle runs split-K too, its partials summed and
  cast by ``dflash_splitk_reduce`` (gate|up: ``dflash_splitk_swiglu_reduce``).

Before the pass the recurrent states the runner would roll back on its next
load (tape[keep - 1] when keep >= 1) are gathered into its state buffers
(``dflash_tape_select``); each layer's final state is written to its tape's
slab 0 and keep becomes 1, so the next verify scan starts from it with no
copy.  Prompts longer than ``max_rows`` run as consecutive passes over the
caches the previous one left.  No launch here has a CPU counterpart: every
call goes to this package's gfx950 library.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .gdn_layer import QK_NORM_EPS


MAX_SPLITS = 4
# Residual projections of short prompts split further (see residual_splits).
MAX_RESIDUAL_SPLITS = 16
# The split model's rates (MI355X, measured): one compute unit's MFMA rate
# on a 256 x 256 prompt GEMM tile (about 1 PFLOP/s over 256 units), and the
# rate at which split partials are written and read back.
UNIT_FLOPS = 4.0e12
PARTIAL_BYTES_PER_S = 5.0e12


def residual_splits(N: int, P: int, cus: int, K: int) -> int:
    """K splits for a prompt-sized projection of N output columns over P rows
    and K inputs, whose fp32 partials the residual add + norm sums.

    While the 256 x 128 tiles fill at most half the compute units, each
    streams its weight rows on one unit at a rate that does not grow with
    the units left idle: the largest count whose units (tiles x splits) still
    fit the compute units once wins, with at least 8 k-steps of 64 a split
    (more splits cost more in partials than they save) and at most
    MAX_RESIDUAL_SPLITS (measured on MI355X for out_proj / o_proj / down at
    128-1024 prompt rows, the add + norm included: within 6 % of the fastest
    count, up to 3x faster than one launch).
    Past that the count up to MAX_SPLITS with the least estimated time wins
    (the smallest on a tie), 1 when the wide tiles alone fill two rounds.
    The GEMM runs 256 x 256 or 256 x 128 output tiles, whichever takes fewer
    whole rounds of the compute units with a 256 x 128 unit costing 0.7 of a
    256 x 256 one (half the products at the smaller tile's lower rate); a
    256 x 256 unit over all K takes 2 * 256 * 256 * K / UNIT_FLOPS and a
    split's unit 1/s of that; the partials add 8 * s * P * N bytes (written
    by the GEMM, read by the add + norm) at PARTIAL_BYTES_PER_S against
    4 * P * N for one launch's bf16 output.  Measured on MI355X (GEMM + add +
    norm at 2048 and 4096 prompt rows) this picked the fastest count for
    every projection: 3 at 2048 rows, and at 4096 rows 3 for down, 1 for
    o_proj (75 against 86 us split 3 ways), a tie for out_proj."""
    wide = -(-N // 256) * -(-P // 256)
    narrow = -(-N // 256) * -(-P // 128)
    if 2 * narrow <= cus:
        return max(1, min(cus // narrow, (K // 64) // 8, MAX_RESIDUAL_SPLITS))
    if wide >= 2 * cus:
        return 1
    unit_us = 2 * 256 * 256 * K / UNIT_FLOPS * 1e6
    best, best_cost = 1, None
    for s in range(1, MAX_SPLITS + 1):
        rounds = min(-(-(wide * s) // cus), 0.7 * -(-(narrow * s) // cus))
        traffic = (8 * s if s > 1 else 4) * P * N / PARTIAL_BYTES_PER_S * 1e6
        cost = rounds * unit_us / s + traffic
        if best_cost is None or cost < best_cost - 1e-9:
            best, best_cost = s, cost
    return best


def prompt_splits(N: int, P: int, cus: int) -> int:
    """K splits for a prompt-sized projection with a bf16 output, summed and
    cast afterwards by dflash_splitk_reduce / dflash_splitk_swiglu_reduce.

    One launch when the 256 x 256 tile's units give every compute unit one.
    Otherwise each 256 x 128 tile streams its 256 weight rows on one compute
    unit, at a rate that does not grow with the units left idle, so a launch
    of few tiles is as long as one tile: the largest count up to MAX_SPLITS
    whose units (tiles x splits) still fit the compute units once wins.
    Measured on MI355X (in_proj, q|k|v and gate|up at 128-1024 prompt rows,
    partials and reduce included) that count was the fastest or within 4 %
    of it."""
    if -(-N // 256) * -(-P // 256) >= cus:
        return 1
    tiles = -(-N // 256) * -(-P // 128)
    return max(1, min(MAX_SPLITS, cus // tiles))


MAX_TAIL_SPLITS = 16


def tail_split(N: int, P: int, cus: int, K: int) -> tuple[int, int] | None:
    """(rows of the main launch, k-splits of the rest) for a bf16 prompt
    projection whose 256 x 256 units end in a mostly empty round, else None.

    U units of 256 x 256 on the compute units run as U // cus whole rounds
    and a last one of U % cus; when that last round is at most half full the
    GEMM runs as two launches (dflash_gemm_bf16_tiled_prefill_rows): the
    weight rows of the whole rounds as usual, and the last n-tiles' rows
    split-K into enough units to fill one round of 1/s of the time (at least
    4 k-steps of 64 a split, at most MAX_TAIL_SPLITS), their partials summed
    and cast by the reduce.  None where the kernel would take the 256 x 128
    tile (see dflash_gemm_bf16_tiled_prefill) or nothing is gained."""
    n_tiles, m_tiles = -(-N // 256), -(-P // 256)
    wide = n_tiles * m_tiles
    narrow = n_tiles * -(-P // 128)
    if 10 * -(-wide // cus) > 7 * -(-narrow // cus):
        return None
    rounds, last = divmod(wide, cus)
    if rounds < 1 or last == 0 or 2 * last > cus:
        return None
    n_tail = -(-last // m_tiles)
    rows_main = (n_tiles - n_tail) * 256
    if rows_main <= 0 or rows_main >= N:
        return None
    s = min(MAX_TAIL_SPLITS, cus // (n_tail * m_tiles), (K // 64) // 4)
    return (rows_main, s) if s >= 2 else None


class HybridPrefill:
    """Prompt pass over the caches of ``runner`` (B = 1)."""

    def __init__(self, runner, max_rows: int = 8192):
        if runner.B != 1:
            raise ValueError("the prompt pass runs one sequence (runner.B == 1)")
        cfg = runner.cfg
        lc = cfg.linear
        if lc.linear_key_head_dim != 128 or lc.linear_value_head_dim != 128 or cfg.head_dim != 128:
            raise ValueError("the prompt pass needs 128-wide gated-delta and attention heads")
        self.run, self.cfg = runner, cfg
        self.max_rows = int(max_rows)
        self.rows_cap = 0
        self._lib = _lib.load()
        self.cus = torch.cuda.get_device_properties(runner.device).multi_processor_count
        self._weights()

    # ------------------------------------------------------------ weights
    def _tiled(self, lw, name):
        """(fragment-tiled weight, its row count): the verify GEMMs' copy when
        there is one, else a tiled copy zero-padded to whole 16-row tiles."""
        w = lw[name]
        n, k = w.shape
        if n % 16 == 0:
            key = name + "_tiled"
            src = w
        else:
            key = name + "_ptiled"
            src = None
        if key not in lw:
            if src is None:
                src = torch.zeros(-(-n // 16) * 16, k, dtype=w.dtype, device=w.device)
                src[:n].copy_(w)
            npad = src.shape[0]
            t = torch.empty(int(self._lib.dflash_weight_tile_bytes(npad, k)) // 2,
                            dtype=torch.bfloat16, device=w.device)
            _lib.call("dflash_weight_tile_bf16", src.data_ptr(), src.stride(0), t.data_ptr(), npad,
                      k, _lib.stream_handle(w.device))
            lw[key] = t
        return lw[key], -(-n // 16) * 16

    def _weights(self):
        cfg = self.cfg
        self.w = []
        for i, lw in enumerate(self.run.w.layers):
            names = ["w_gu_pairs", "w_down"] + (["w_in", "w_out"] if cfg.is_linear(i)
                                                else ["w_qkv", "w_o"])
            self.w.append({n: self._tiled(lw, n) for n in names})
        torch.cuda.synchronize(self.run.device)
        # the stacked gated-delta projection's (padded) row count: the row
        # stride of its output
        self.in_stride = max((d["w_in"][1] for d in self.w if "w_in" in d), default=0)

    # ------------------------------------------------------------ buffers
    def _ensure(self, P: int) -> None:
        if P <= self.rows_cap:
            return
        cfg, lc, dev = self.cfg, self.cfg.linear, self.run.device
        H, I = cfg.hidden_size, cfg.intermediate_size
        Hv, Dv, C = lc.linear_num_value_heads, lc.linear_value_head_dim, lc.conv_dim
        Hq, D = cfg.num_attention_heads, cfg.head_dim
        bf, f32 = torch.bfloat16, torch.float32
        e = lambda *s, dt=bf: torch.empty(*s, dtype=dt, device=dev)  # noqa: E731
        self.tokens = e(P, dt=torch.int32)
        self.h, self.xn, self.r = e(P, H), e(P, H), e(P, H)
        self.mlp_act = e(P, I)
        self.proj = e(P, max(self.in_stride, 16))
        self.act = e(P, C)
        self.g, self.beta = e(P, Hv, dt=f32), e(P, Hv, dt=f32)
        self.scan_out, self.gnorm = e(P, Hv, Dv), e(P, Hv, Dv)
        self.aproj = e(P, cfg.attn_proj_rows)
        self.q = e(P, Hq, D)
        self.attn_out = e(P, Hq * D)
        self.conv_new = e(1, lc.linear_conv_kernel_dim - 1, C)
        ws = int(self._lib.dflash_gdn_chunked_prefill_workspace_bytes(
            1, P, Hv, lc.linear_key_head_dim, Dv))
        self.chunk_ws = e(max(ws, 16), dt=torch.uint8)
        # fp32 partials of the split projections at the split counts this
        # prompt length plans: the residual ones (N = H) and the bf16 ones
        need = 0
        for d in self.w:
            for name, (wt, n) in d.items():
                K = wt.numel() // n
                if name in ("w_out", "w_o", "w_down"):
                    ns = residual_splits(n, P, self.cus, K)
                else:
                    ns = prompt_splits(n, P, self.cus)
                    tail = tail_split(n, P, self.cus, K) if ns == 1 else None
                    if tail is not None:
                        rows_main, ts = tail
                        need = max(need, int(self._lib.dflash_gemm_splits(K, ts)) * P
                                   * (n - rows_main))
                if ns > 1:
                    need = max(need, int(self._lib.dflash_gemm_splits(K, ns)) * P * n)
        self.part = e(max(need, 4), dt=f32)
        self.rows_cap = P

    # ------------------------------------------------------------ the pass
    def resolve_states(self, stream) -> None:
        """state[l] = tape[l][keep - 1] where keep >= 1 (the rollback the next
        verify scan would have done on load), then keep = 0."""
        run = self.run
        n = len(run.state)
        if n == 0:
            return
        lc = self.cfg.linear
        S = lc.linear_num_value_heads * lc.linear_value_head_dim * lc.linear_key_head_dim
        for l0 in range(0, n, 32):
            m = min(32, n - l0)
            states = _lib.ptr_array(run.state[l0:l0 + m])
            _lib.call("dflash_tape_select", _lib.ptr_array(run.tape[l0:l0 + m]), states, states,
                      run.keep.data_ptr(), m, 1, run.T, S, 0, stream)
        run.keep.zero_()

    def forward(self, tokens: torch.Tensor, norm_out: torch.Tensor,
                capture_out: torch.Tensor | None) -> None:
        """Run the prompt `tokens` (int32 [P] on the device) from the caches at
        the runner's device-side length (run.lens[0]); write the normed hidden
        states to norm_out [P, H] and, with capture layers set on the runner,
        the residual stream after each of them to capture_out [P, n * H].
        Leaves run.lens advanced by P, keep = 1 (state = tape[0]), the conv
        windows advanced."""
        P = int(tokens.numel())
        stream = _lib.stream_handle(self.run.device)
        self.resolve_states(stream)
        for p0 in range(0, P, self.max_rows):
            Pp = min(self.max_rows, P - p0)
            cap = None if capture_out is None else capture_out[p0:p0 + Pp]
            self._pass(tokens[p0:p0 + Pp], Pp, cap, stream)
            norm_out[p0:p0 + Pp].copy_(self.xn[:Pp])
            if p0 + Pp < P:
                self._carry(stream)
            self.run.lens.add_(Pp)

    def _carry(self, stream) -> None:
        """Between passes: the states the last pass wrote to tape slab 0
        (keep = 1) become the next pass's initial states."""
        self.resolve_states(stream)

    def _pass(self, tokens, P, capture, stream):
        run, cfg, lc = self.run, self.cfg, self.cfg.linear
        self._ensure(P)
        H, I = cfg.hidden_size, cfg.intermediate_size
        C, Hk, Hv = lc.conv_dim, lc.linear_num_key_heads, lc.linear_num_value_heads
        Dk, Dv, K = lc.linear_key_head_dim, lc.linear_value_head_dim, lc.linear_conv_kernel_dim
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = float(cfg.rms_norm_eps)
        call = _lib.call
        L = cfg.num_hidden_layers
        h, xn = self.h.data_ptr(), self.xn.data_ptr()
        self.tokens[:P].copy_(tokens)
        layers = run.w.layers
        call("dflash_embed_rmsnorm", run.w.embed.data_ptr(), self.tokens.data_ptr(), cfg.vocab_size,
             layers[0]["ln_in"].data_ptr(), h, xn, P, H, eps, stream)
        cap_ids = {layer: j for j, layer in enumerate(run.capture_layers)}
        n_cap = len(run.capture_layers)
        rs = self.in_stride
        base = self.proj.data_ptr()
        ab = (ctypes.c_int64 * 4)(P * rs, rs, P * rs, rs)
        zs = (ctypes.c_int64 * 3)(P * rs, rs, Dv)
        act = self.act.data_ptr()
        scan_strides = (ctypes.c_int64 * 13)(P * C, C, Dk, P * C, C, Dk, P * C, C, Dv,
                                             P * Hv, Hv, P * Hv, Hv)
        arows = cfg.attn_proj_rows
        gi = ai = 0
        for i in range(L):
            lw, tw = layers[i], self.w[i]
            if cfg.is_linear(i):
                gw = lw["gdn"]
                self._bf16_proj(tw["w_in"], xn, H, P, base, rs, False, stream)
                a_ptr, b_ptr = base + 2 * (C + Hv * Dv + Hv), base + 2 * (C + Hv * Dv)
                call("dflash_gdn_prologue", base, P * rs, rs, run.conv[gi].data_ptr(),
                     gw.conv_weight.data_ptr(), a_ptr, b_ptr, ab, gw.A_log.data_ptr(),
                     gw.dt_bias.data_ptr(), act, self.g.data_ptr(), self.beta.data_ptr(),
                     self.conv_new.data_ptr(), 1, P, K, Hk, Hv, Dk, Dv, QK_NORM_EPS, stream)
                run.conv[gi].copy_(self.conv_new)
                call("dflash_gdn_chunked_prefill", act, act + 2 * Hk * Dk, act + 4 * Hk * Dk,
                     self.g.data_ptr(), self.beta.data_ptr(), run.state[gi].data_ptr(),
                     self.scan_out.data_ptr(), run.tape[gi][0].data_ptr(), 1, P, Hk, Hv, Dk, Dv,
                     scan_strides, self.chunk_ws.data_ptr(), self.chunk_ws.numel(), stream)
                call("dflash_gdn_gated_rmsnorm", self.scan_out.data_ptr(), base + 2 * C, zs,
                     gw.norm_weight.data_ptr(), self.gnorm.data_ptr(), 1, P, Hv, Dv, eps, stream)
                branch = self._to_residual(tw["w_out"], self.gnorm.data_ptr(), Hv * Dv, P, stream)
                gi += 1
            else:
                ap = self.aproj.data_ptr()
                self._bf16_proj(tw["w_qkv"], xn, H, P, ap, arows, False, stream)
                call("dflash_attn_prep", ap, arows, lw["q_norm"].data_ptr(), lw["k_norm"].data_ptr(),
                     run.lens.data_ptr(), run.k_cache[ai].data_ptr(), run.vt_cache[ai].data_ptr(),
                     self.q.data_ptr(), run.overflow.data_ptr(), 1, P, Hq, Hkv, D, run.Smax,
                     cfg.rot_dims, float(cfg.rope_theta), eps, stream)
                call("dflash_attn_prefill", self.q.data_ptr(), run.k_cache[ai].data_ptr(),
                     run.vt_cache[ai].data_ptr(), run.lens.data_ptr(), ap, arows,
                     self.attn_out.data_ptr(), P, Hq, Hkv, D, run.Smax, float(D ** -0.5), stream)
                branch = self._to_residual(tw["w_o"], self.attn_out.data_ptr(), Hq * D, P, stream)
                ai += 1
            self._add_norm(branch, lw["ln_post"], None, P, stream)
            self._bf16_proj(tw["w_gu_pairs"], xn, H, P, self.mlp_act.data_ptr(), I, True, stream)
            branch = self._to_residual(tw["w_down"], self.mlp_act.data_ptr(), I, P, stream)
            nw = layers[i + 1]["ln_in"] if i + 1 < L else run.w.final_norm
            j = cap_ids.get(i)
            cap = None if j is None else (capture.data_ptr() + 2 * j * H, n_cap * H)
            self._add_norm(branch, nw, cap, P, stream)
        # every layer's final state is in its tape's slab 0
        run.keep.fill_(1)

    def _bf16_proj(self, weight, x_ptr, K, P, out_ptr, out_stride, swiglu, stream):
        """out = bf16(x . W^T) (swiglu: the gated form over the w_pairs rows,
        N / 2 output columns) in one launch; or split-K (prompt_splits) with
        the partials summed and cast by the reduce; or the rows of the whole
        rounds in one launch and the last n-tiles' rows split-K (tail_split)."""
        wt, n = weight
        ns = prompt_splits(n, P, self.cus)
        used = int(self._lib.dflash_gemm_splits(K, ns)) if ns > 1 else 1
        tail = tail_split(n, P, self.cus, K) if ns == 1 else None
        reduce = "dflash_splitk_swiglu_reduce" if swiglu else "dflash_splitk_reduce"
        if used > 1 and used * P * n <= self.part.numel():
            part = self.part.data_ptr()
            _lib.call("dflash_gemm_bf16_tiled_prefill_splitk", x_ptr, K, wt.data_ptr(), part, ns,
                      P, n, K, stream)
            _lib.call(reduce, part, used, P, n, out_ptr, out_stride, stream)
            return
        if tail is not None:
            rows_main, ts = tail
            n_tail = n - rows_main
            tused = int(self._lib.dflash_gemm_splits(K, ts))
            if tused > 1 and tused * P * n_tail <= self.part.numel():
                part = self.part.data_ptr()
                _lib.call("dflash_gemm_bf16_tiled_prefill_rows", x_ptr, K, wt.data_ptr(), n, 0,
                          out_ptr, out_stride, None, 0, P, rows_main, K, int(swiglu), stream)
                _lib.call("dflash_gemm_bf16_tiled_prefill_rows", x_ptr, K, wt.data_ptr(), n,
                          rows_main, None, 0, part, ts, P, n_tail, K, 0, stream)
                out_col = rows_main // 2 if swiglu else rows_main
                _lib.call(reduce, part, tused, P, n_tail, out_ptr + 2 * out_col, out_stride,
                          stream)
                return
        if swiglu:
            _lib.call("dflash_gemm_bf16_swiglu_tiled_prefill", x_ptr, K, wt.data_ptr(), out_ptr,
                      out_stride, P, n, K, stream)
        else:
            _lib.call("dflash_gemm_bf16_tiled_prefill", x_ptr, K, wt.data_ptr(), out_ptr,
                      out_stride, P, n, K, stream)

    def _to_residual(self, weight, x_ptr, K, P, stream):
        """A projection whose output the residual stream adds: bf16 into r,
        or split-K fp32 partials into part; returns the split count (0: r)."""
        wt, n = weight
        ns = residual_splits(n, P, self.cus, K)
        if ns > 1 and int(self._lib.dflash_gemm_splits(K, ns)) * P * n > self.part.numel():
            ns = 1
        if ns == 1:
            _lib.call("dflash_gemm_bf16_tiled_prefill", x_ptr, K, wt.data_ptr(), self.r.data_ptr(),
                      self.cfg.hidden_size, P, n, K, stream)
            return 0
        _lib.call("dflash_gemm_bf16_tiled_prefill_splitk", x_ptr, K, wt.data_ptr(),
                  self.part.data_ptr(), ns, P, n, K, stream)
        return int(self._lib.dflash_gemm_splits(K, ns))

    def _add_norm(self, splits, weight, capture, P, stream):
        """h += the branch (r, or the sum of `splits` fp32 partials), xn =
        RMSNorm(h) * weight; capture = (pointer, row stride) also receives h."""
        H, eps = self.cfg.hidden_size, float(self.cfg.rms_norm_eps)
        h, xn = self.h.data_ptr(), self.xn.data_ptr()
        r = None if splits else self.r.data_ptr()
        part = self.part.data_ptr() if splits else None
        if capture is not None:
            _lib.call("dflash_add_rmsnorm_capture", h, r, part, splits, weight.data_ptr(), h,
                      capture[0], capture[1], xn, P, H, eps, stream)
        elif splits:
            _lib.call("dflash_add_rmsnorm_splitk", h, part, splits, weight.data_ptr(), h, xn, P, H,
                      eps, stream)
        else:
            _lib.call("dflash_add_rmsnorm", h, r, weight.data_ptr(), h, xn, P, H, eps, stream)
