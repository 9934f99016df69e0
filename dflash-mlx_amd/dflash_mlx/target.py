"""The hybrid target behind the reference's model interface.

The reference's decode loop talks to its Qwen3.5 target through a model
object with ``forward_dflash`` (custom_qwen35_model.py:883-1001 for the text
model, :1099-1126 with the LM head), ``rollback_linear_caches`` (:1029-1074),
``snapshot_linear_caches`` / ``restore_linear_caches`` (:1004-1027) and
``make_cache`` (:1153-1154), wrapped by Qwen35TargetAdapter and the
LoadedTargetModel facade (adapters.py:341-570, :729-826).
``HybridTargetModel`` is that model object for the MI355X hybrid runner:

* ``make_cache()`` makes one ``HybridVerifyRunner`` (B = 1, block length up
  to ``block_size``, ``max_seq_len`` cache positions) and returns its caches
  as the reference's per-layer list: an ``ArraysCache`` [conv window, state]
  per gated-delta layer and a ``DeviceKVCache`` per attention layer, all views
  of the runner's device buffers.
* ``forward_dflash(inputs, cache, layer_ids, return_rollback_records)`` runs
  a verify block (at most ``block_size`` tokens) through the runner, and a
  longer input (a prompt) in one pass with launches sized to it
  (``prefill.HybridPrefill``: prompt-sized MFMA projections, the chunked
  gated-delta scan, causal prompt attention; ``prompt_pass="blocks"`` runs
  it through the runner ``block_size`` tokens at a time instead), and
  leaves the caches as after accepting every input, like the reference.
  It returns the normed hidden states, the target hidden states at
  ``layer_ids`` (the residual stream
  after each of those layers, concatenated in layer order on the feature
  axis) and, for one block, the rollback records: {initial_conv_state,
  initial_state, qkv, state_tape} per gated-delta layer.  Records, like the
  tape they hold, are valid until the next forward on the same cache.
* ``rollback_linear_caches(cache, records, a)`` keeps a of the block's
  tokens: the conv windows are rebuilt from the block's initial windows and
  qkv rows (one launch), and the recurrent state becomes the view
  ``state_tape[a-1]``; the next forward's scan reads that tape entry as its
  initial state (no copy).

Cache entries replaced from outside (``restore_linear_caches``, or a caller
assigning ``cache[i][1]``) are copied into the runner's buffers before the
next forward.  Every launch goes to this package's gfx950 library; there is
no CPU path.
"""
from __future__ import annotations

from typing import Any

import torch

from . import _lib
from .adapters import make_rollback_record
from .cache import ArraysCache, KVCache
from .hybrid_model import HybridConfig, HybridVerifyRunner, HybridWeights
from .prefill import HybridPrefill


class DeviceKVCache(KVCache):
    """A full-attention layer's KV cache held in a runner's device buffers:
    keys [B, Hkv, Smax, D] and values stored transposed [B, Hkv, D, Smax].
    ``offset`` (host) counts the valid positions; the runner appends at it
    and ``trim`` (the reference's KVCache.trim, called from adapters.py:
    505-508) only lowers it."""

    def __init__(self, k_cache: torch.Tensor, vt_cache: torch.Tensor):
        self._k = k_cache
        self._vt = vt_cache
        self.offset = 0

    @property
    def capacity(self) -> int:
        return self._k.shape[2]

    @property
    def keys(self) -> torch.Tensor:
        return self._k[:, :, : self.offset]

    @property
    def values(self) -> torch.Tensor:
        return self._vt[:, :, :, : self.offset].transpose(2, 3)

    def update_and_fetch(self, keys, values):
        raise NotImplementedError("the runner's attention kernels append to this cache")


class HybridCache(list):
    """The per-layer cache list of one sequence, bound to its runner."""

    runner: HybridVerifyRunner
    linear_idx: list[int]
    attn_idx: list[int]


class HybridTargetModel:
    """The Qwen3.5-shaped hybrid target on MI355X with the reference model's
    DFlash methods (see the module docstring)."""

    def __init__(self, cfg: HybridConfig, weights: HybridWeights, device: torch.device,
                 max_seq_len: int = 4096, block_size: int = 16, weight_layout: str = "tiled",
                 eos_token_ids: set[int] | None = None, prompt_pass: str = "prefill",
                 prefill_rows: int = 8192):
        """prompt_pass: "prefill" runs inputs longer than block_size in one
        pass (prefill.HybridPrefill, up to prefill_rows rows per pass);
        "blocks" runs them through the verify runner block_size tokens at a
        time."""
        if prompt_pass not in ("prefill", "blocks"):
            raise ValueError(f"prompt_pass must be 'prefill' or 'blocks', got {prompt_pass!r}")
        self.cfg, self.weights, self.device = cfg, weights, torch.device(device)
        self.block_size = int(block_size)
        self.max_seq_len = int(max_seq_len)
        self.weight_layout = weight_layout
        self.prompt_pass = prompt_pass
        self.prefill_rows = int(prefill_rows)
        self.eos_token_ids = set(eos_token_ids or ())
        self._smax = -(-(self.max_seq_len + self.block_size) // 64) * 64

    # ------------------------------------------------------------- caches
    def make_cache(self) -> HybridCache:
        """Model.make_cache (custom_qwen35_model.py:1153-1154): ArraysCache(2)
        for gated-delta layers, KV caches for attention layers, on one fresh
        runner."""
        cfg = self.cfg
        run = HybridVerifyRunner(cfg, self.weights, 1, self.block_size, self._smax, self.device,
                                 weight_layout=self.weight_layout)
        run.snapshot_conv()
        cache = HybridCache()
        cache.runner = run
        cache.linear_idx, cache.attn_idx = [], []
        gi = ai = 0
        for i in range(cfg.num_hidden_layers):
            if cfg.is_linear(i):
                c = ArraysCache(size=2)
                c[0], c[1] = run.conv[gi], run.state[gi]
                cache.linear_idx.append(i)
                gi += 1
            else:
                c = DeviceKVCache(run.k_cache[ai], run.vt_cache[ai])
                cache.attn_idx.append(i)
                ai += 1
            cache.append(c)
        cache._installed = [(cache[i][0], cache[i][1]) for i in cache.linear_idx]
        cache._records = None
        cache._block = 0
        return cache

    @staticmethod
    def _runner_of(cache) -> HybridVerifyRunner:
        run = getattr(cache, "runner", None)
        if run is None:
            raise TypeError("the cache must come from HybridTargetModel.make_cache()")
        return run

    def _sync_in(self, cache: HybridCache, n_new: int) -> int:
        """Copy cache entries replaced from outside into the runner (then the
        next scan starts from `state`), check the KV offsets, and return the
        live KV length."""
        run = cache.runner
        foreign = any(cache[i][0] is not c or cache[i][1] is not s
                      for i, (c, s) in zip(cache.linear_idx, cache._installed))
        if foreign:
            for gi, i in enumerate(cache.linear_idx):
                conv, state = cache[i][0], cache[i][1]
                for dst, src in ((run.conv[gi], conv), (run.state[gi], state)):
                    if src is None:
                        dst.zero_()
                    elif src.data_ptr() != dst.data_ptr():
                        dst.copy_(src.reshape(dst.shape))
                cache[i][0], cache[i][1] = run.conv[gi], run.state[gi]
            run.keep.zero_()
            cache._installed = [(cache[i][0], cache[i][1]) for i in cache.linear_idx]
        offsets = {cache[i].offset for i in cache.attn_idx}
        if len(offsets) > 1:
            raise RuntimeError(f"attention caches disagree on their length: {sorted(offsets)}")
        off = offsets.pop() if offsets else 0
        if off < 0 or off + n_new > run.Smax:
            raise ValueError(f"{n_new} new tokens at cache length {off} exceed the "
                             f"{run.Smax}-position cache (max_seq_len {self.max_seq_len} "
                             f"+ one block, rounded up to 64)")
        return off

    def _install(self, cache: HybridCache, states) -> None:
        run = cache.runner
        for gi, i in enumerate(cache.linear_idx):
            cache[i][0], cache[i][1] = run.conv[gi], states[gi]
        cache._installed = [(cache[i][0], cache[i][1]) for i in cache.linear_idx]

    # ------------------------------------------------------------ forward
    def forward_dflash(self, inputs: torch.Tensor, cache: HybridCache, layer_ids: list[int],
                       return_rollback_records: bool = False):
        """Qwen3_5TextModel.forward_dflash (custom_qwen35_model.py:883-1001):
        (norm_hidden [1, P, H], target_hidden [1, P, n*H][, records])."""
        run = self._runner_of(cache)
        toks = torch.as_tensor(inputs)
        if toks.dim() == 1:
            toks = toks[None]
        if toks.dim() != 2 or toks.shape[0] != 1:
            raise ValueError(f"inputs must be [1, P] token ids, got {tuple(toks.shape)}")
        P = toks.shape[1]
        if P == 0:
            raise ValueError("inputs hold no tokens")
        if return_rollback_records and P > run.T:
            raise ValueError(f"a block with rollback records holds at most {run.T} tokens, got {P}")
        toks = toks.to(device=self.device, dtype=torch.int32)
        off = self._sync_in(cache, P)
        run.set_capture(layer_ids)
        H = self.cfg.hidden_size
        if P > run.T and self.prompt_pass == "prefill":
            return self._forward_prompt(cache, run, toks[0], off)
        norm_parts, hid_parts = [], []
        pos = 0
        while pos < P:
            Tp = min(run.T, P - pos)
            run.tokens.view(-1)[:Tp].copy_(toks[0, pos:pos + Tp])
            run.lens.fill_(off)
            if return_rollback_records:
                run.snapshot_conv()
            run.forward(Tp, lm_head=False)
            norm_parts.append(run.xn[:Tp].clone())
            if run.captured is not None:
                hid_parts.append(run.captured[:Tp].clone())
            # every input accepted: states follow tape[Tp-1] on the next load,
            # conv windows advance in place, the KV caches hold Tp more
            run.accept_all(Tp)
            off += Tp
            pos += Tp
        for i in cache.attn_idx:
            cache[i].offset = off
        self._install(cache, [run.tape[gi][Tp - 1, 0:1] for gi in range(len(cache.linear_idx))])
        norm_hidden = torch.cat(norm_parts).view(1, P, H)
        if hid_parts:
            target_hidden = torch.cat(hid_parts).view(1, P, -1)
        else:
            target_hidden = norm_hidden.new_empty((1, P, 0))
        if not return_rollback_records:
            cache._records = None
            return norm_hidden, target_hidden
        C = self.cfg.linear.conv_dim
        records = {}
        for gi, i in enumerate(cache.linear_idx):
            records[i] = make_rollback_record(
                run.conv_snap[gi], run.state[gi], run.proj[gi][:P, :C].view(1, P, C),
                run.tape[gi][:P])
        cache._records = records
        cache._block = P
        return norm_hidden, target_hidden, records

    def _forward_prompt(self, cache: HybridCache, run: HybridVerifyRunner, toks: torch.Tensor,
                        off: int):
        """forward_dflash of a prompt in one pass (prefill.HybridPrefill):
        the caches end as after accepting every token (states in tape slab 0
        with keep = 1, windows advanced, KV lengths += P)."""
        pre = getattr(cache, "_prefill", None)
        if pre is None:
            pre = cache._prefill = HybridPrefill(run, max_rows=self.prefill_rows)
        P, H = toks.numel(), self.cfg.hidden_size
        run.lens.fill_(off)
        norm = torch.empty(P, H, dtype=torch.bfloat16, device=self.device)
        n_cap = len(run.capture_layers)
        cap = torch.empty(P, n_cap * H, dtype=torch.bfloat16, device=self.device) if n_cap else None
        pre.forward(toks, norm, cap)
        for i in cache.attn_idx:
            cache[i].offset = off + P
        self._install(cache, [run.tape[gi][0, 0:1] for gi in range(len(cache.linear_idx))])
        cache._records = None
        target_hidden = cap.view(1, P, -1) if cap is not None else norm.new_empty((1, P, 0))
        return norm.view(1, P, H), target_hidden

    def rollback_linear_caches(self, cache: HybridCache, rollback_records: dict[int, dict[str, Any]],
                               accepted_inputs: int) -> None:
        """Qwen3_5TextModel.rollback_linear_caches (custom_qwen35_model.py:
        1029-1074) with the tape: keep accepted_inputs tokens of the last
        block (one conv-window launch; the state is tape[a-1])."""
        run = self._runner_of(cache)
        if rollback_records is not cache._records or not rollback_records:
            from .adapters import rollback_linear_caches as generic

            generic(cache, rollback_records, accepted_inputs)
            return
        a = int(accepted_inputs)
        T = cache._block
        if not 0 <= a <= T:
            raise ValueError(f"accepted_inputs={a} outside [0, {T}]")
        run.keep.fill_(a)
        run.rollback_to(T)
        self._install(cache, [run.tape[gi][a - 1, 0:1] if a >= 1 else run.state[gi]
                              for gi in range(len(cache.linear_idx))])

    def snapshot_linear_caches(self, cache: HybridCache) -> dict[int, list[torch.Tensor | None]]:
        """custom_qwen35_model.py:1004-1014: copies of every linear layer's
        [conv window, state]."""
        return {i: [None if v is None else v.clone() for v in (cache[i][0], cache[i][1])]
                for i in cache.linear_idx}

    def restore_linear_caches(self, cache: HybridCache,
                              snapshots: dict[int, list[torch.Tensor | None]]) -> None:
        """custom_qwen35_model.py:1016-1027: put the snapshots back (copied
        into the runner before the next forward)."""
        for i, values in snapshots.items():
            cache[i][0], cache[i][1] = values[0], values[1]

    # ------------------------------------------------------------ LM head
    def embed_tokens(self, tokens: torch.Tensor) -> torch.Tensor:
        """embed_tokens (custom_qwen35_model.py:853): bf16 rows of the table."""
        t = torch.as_tensor(tokens).to(device=self.device, dtype=torch.long)
        return torch.nn.functional.embedding(t, self.weights.embed)

    def lm_head_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """lm_head(hidden) (custom_qwen35_model.py:1090-1097): bf16 logits
        [..., V] from this package's GEMMs: the prompt-sized GEMM over the
        fragment-tiled head for more than 64 rows, else the verify-sized
        GEMM, 64 rows a launch."""
        H, V = self.cfg.hidden_size, self.cfg.vocab_size
        lead = hidden.shape[:-1]
        x = hidden.reshape(-1, H).to(torch.bfloat16)
        if x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
            x = x.contiguous()
        out = torch.empty((x.shape[0], V), dtype=torch.bfloat16, device=self.device)
        w = self.weights
        stream = _lib.stream_handle(self.device)
        if x.shape[0] > 64 and w.lm_head_tiled is not None:
            _lib.call("dflash_gemm_bf16_tiled_prefill", x.data_ptr(), x.stride(0),
                      w.lm_head_tiled.data_ptr(), out.data_ptr(), V, x.shape[0], V, H, stream)
            return out.view(*lead, V)
        for m0 in range(0, x.shape[0], 64):
            m = min(64, x.shape[0] - m0)
            xp, op = x[m0:].data_ptr(), out[m0:].data_ptr()
            if w.lm_head_tiled is not None and self.weight_layout == "tiled":
                _lib.call("dflash_gemm_bf16_tiled", xp, x.stride(0), w.lm_head_tiled.data_ptr(),
                          op, V, m, V, H, 1, 64, 4, None, 0, stream)
            else:
                _lib.call("dflash_gemm_bf16", xp, x.stride(0), w.lm_head.data_ptr(), H, op, V, m, V,
                          H, 1, 32, 4, stream)
        return out.view(*lead, V)

    def lm_head_argmax(self, hidden: torch.Tensor) -> torch.Tensor:
        """The lm_head_argmax hook (adapters.py:267-271) as the fused LM-head
        greedy kernel: int32 argmax ids [..., N], no logits."""
        from .runtime import lm_head_argmax

        tiled = self.weights.lm_head_tiled if self.weight_layout == "tiled" else None
        return lm_head_argmax(hidden, self.weights.lm_head, weight_tiled=tiled)
