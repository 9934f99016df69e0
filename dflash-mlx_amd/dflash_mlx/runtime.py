"""Verify-step accept and rollback orchestration on MI355X.

Mirrors the reference's decode-runtime pieces on the hot path
(dflash_mlx/runtime.py):

* ``sample_tokens`` (:22-29) — greedy argmax runs in the gfx950 accept kernel;
* ``longest_prefix_match`` (:41-47) — the host-list primitive, unchanged;
* ``greedy_accept`` — argmax + prefix compare + bonus fused on the device, so
  only (matched, bonus) cross to the host;
* ``verify_block_parallel_replay`` (:117-163) — same arguments and return
  tuple; the rollback it triggers is a tape gather instead of a replay.

Token ids are int32 on the device (the reference uses uint32; vocabularies
here are far below 2**31).
"""
from __future__ import annotations

import time
from typing import Any, Sequence

import torch

from . import _lib
from .gated_delta import _require_device


def _as_3d(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() == 1:
        return logits.reshape(1, 1, -1)
    if logits.dim() == 2:
        return logits.unsqueeze(0)
    if logits.dim() == 3:
        return logits
    return logits.reshape(-1, logits.shape[-2], logits.shape[-1])


def greedy_accept(
    logits: torch.Tensor,
    draft: torch.Tensor | Sequence[int] | Sequence[Sequence[int]] | None = None,
    *,
    want_posterior: bool = True,
) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor]:
    """Fused greedy verify on the device.

    logits: [B,N,V] (or [N,V]) fp32/bf16/fp16; draft: [B,n] token ids (host or
    device) or None.  Returns device int32 tensors
    (posterior [B,N] or None, matched [B], bonus [B]) with
    posterior = argmax(logits, -1) (lowest index on ties),
    matched = leading positions where draft == posterior (<= min(n, N)),
    bonus = posterior[matched] or -1 when matched == N."""
    _require_device("logits", logits, None)
    lg = _as_3d(logits)
    if lg.stride(-1) != 1:
        lg = lg.contiguous()
    B, N, V = lg.shape
    dev = lg.device
    if draft is None:
        d = None
        n = 0
    else:
        if isinstance(draft, torch.Tensor):
            _require_device("draft", draft, dev)
            d = draft.to(torch.int32)
        else:
            d = torch.tensor(draft, dtype=torch.int32).to(dev)
        if d.dim() == 1:
            d = d.unsqueeze(0)
        if d.shape[0] != B:
            raise ValueError(f"draft batch {d.shape[0]} != logits batch {B}")
        if d.stride(-1) != 1:
            d = d.contiguous()
        n = d.shape[1]
    post = torch.empty((B, N), dtype=torch.int32, device=dev) if want_posterior else None
    matched = torch.empty((B,), dtype=torch.int32, device=dev)
    bonus = torch.empty((B,), dtype=torch.int32, device=dev)
    if B == 0:
        return post, matched, bonus
    if N == 0 or V == 0:
        raise ValueError(f"logits need at least one row and one vocabulary entry, got {tuple(lg.shape)}")
    lib = _lib.load()
    ws_bytes = int(lib.dflash_greedy_accept_workspace_bytes(B, N, V))
    ws = torch.empty((max(ws_bytes, 8),), dtype=torch.uint8, device=dev)
    _lib.call(
        "dflash_greedy_accept",
        lg.data_ptr(), _lib.dtype_tag(lg.dtype), lg.stride(0), lg.stride(1),
        _lib.ptr(d), d.stride(0) if d is not None else 0, n,
        _lib.ptr(post), matched.data_ptr(), bonus.data_ptr(), B, N, V,
        ws.data_ptr(), ws.numel(), _lib.stream_handle(dev),
    )
    return post, matched, bonus


def lm_head_greedy_accept(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    draft: torch.Tensor | Sequence[int] | Sequence[Sequence[int]] | None = None,
    *,
    want_posterior: bool = True,
    weight_tiled: torch.Tensor | None = None,
) -> tuple[torch.Tensor | None, torch.Tensor, torch.Tensor]:
    """greedy_accept(hidden @ weight.T, draft) without materialising logits.

    hidden: [B,N,H] (or [N,H]) bf16; weight: [V,H] bf16 (LM head or tied
    embedding).  B*N <= 64 (verify-sized), H % 64 == 0.  Fuses the reference's
    lm_head_argmax hook (dflash_mlx/adapters.py:267-271) with the accept.
    weight_tiled: the head's fragment-tiled copy (tile_weight(weight), made
    once; V % 16 == 0), streamed instead of weight when given."""
    _require_device("hidden", hidden, None)
    dev = hidden.device
    _require_device("weight", weight, dev)
    h = hidden.unsqueeze(0) if hidden.dim() == 2 else hidden
    if h.dim() != 3 or weight.dim() != 2 or h.shape[-1] != weight.shape[1]:
        raise ValueError(f"hidden [B,N,H] and weight [V,H] disagree: {tuple(hidden.shape)}, "
                         f"{tuple(weight.shape)}")
    if h.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("hidden and weight must be bfloat16")
    B, N, H = h.shape
    V = weight.shape[0]
    h2 = h.reshape(B * N, H)
    if h2.stride(-1) != 1 or h2.stride(0) % 8 or h2.data_ptr() % 16:
        h2 = h2.contiguous()
    w = weight if (weight.stride(-1) == 1 and weight.stride(0) % 8 == 0) else weight.contiguous()
    d, n = None, 0
    if draft is not None:
        d = draft.to(torch.int32) if isinstance(draft, torch.Tensor) else \
            torch.tensor(draft, dtype=torch.int32).to(dev)
        if isinstance(draft, torch.Tensor):
            _require_device("draft", draft, dev)
        if d.dim() == 1:
            d = d.unsqueeze(0)
        d = d.contiguous()
        if d.shape[0] != B:
            raise ValueError(f"draft batch {d.shape[0]} != hidden batch {B}")
        n = d.shape[1]
    post = torch.empty((B, N), dtype=torch.int32, device=dev) if want_posterior else None
    matched = torch.empty((B,), dtype=torch.int32, device=dev)
    bonus = torch.empty((B,), dtype=torch.int32, device=dev)
    if B == 0:
        return post, matched, bonus
    lib = _lib.load()
    ws = torch.empty((max(int(lib.dflash_lm_head_accept_workspace_bytes(B, N, V)), 8),),
                     dtype=torch.uint8, device=dev)
    if weight_tiled is not None:
        _require_device("weight_tiled", weight_tiled, dev)
        if weight_tiled.numel() * weight_tiled.element_size() < \
                int(lib.dflash_weight_tile_bytes(V, H)) or not weight_tiled.is_contiguous():
            raise ValueError("weight_tiled must be the contiguous tile_weight(weight) copy")
        _lib.call(
            "dflash_lm_head_greedy_accept_tiled",
            h2.data_ptr(), h2.stride(0), weight_tiled.data_ptr(), H, V,
            _lib.ptr(d), d.stride(0) if d is not None else 0, n,
            _lib.ptr(post), matched.data_ptr(), bonus.data_ptr(), B, N,
            ws.data_ptr(), ws.numel(), _lib.stream_handle(dev),
        )
        return post, matched, bonus
    _lib.call(
        "dflash_lm_head_greedy_accept",
        h2.data_ptr(), h2.stride(0), w.data_ptr(), w.stride(0), H, V,
        _lib.ptr(d), d.stride(0) if d is not None else 0, n,
        _lib.ptr(post), matched.data_ptr(), bonus.data_ptr(), B, N,
        ws.data_ptr(), ws.numel(), _lib.stream_handle(dev),
    )
    return post, matched, bonus


def tile_weight(weight: torch.Tensor) -> torch.Tensor:
    """The fragment-tiled copy of a bf16 [N, K] weight (dflash_weight_tile_bf16:
    [K/64][N/16][2][64][8], the layout the tiled GEMMs and LM head stream);
    N % 16 == 0, K % 64 == 0.  Made once per weight at load time."""
    _require_device("weight", weight, None)
    if weight.dim() != 2 or weight.dtype != torch.bfloat16 or weight.stride(-1) != 1:
        raise ValueError("weight must be a bf16 [N, K] matrix with contiguous rows")
    N, K = weight.shape
    lib = _lib.load()
    nbytes = int(lib.dflash_weight_tile_bytes(N, K))
    if nbytes <= 0:
        raise ValueError(f"[{N}, {K}] cannot be tiled (needs N % 16 == 0, K % 64 == 0)")
    t = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=weight.device)
    _lib.call("dflash_weight_tile_bf16", weight.data_ptr(), weight.stride(0), t.data_ptr(), N, K,
              _lib.stream_handle(weight.device))
    return t


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor,
                   weight_tiled: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's lm_head_argmax hook (adapters.py:267-271):
    argmax(hidden @ weight.T, -1) as int32 [..., N], fused (no logits)."""
    post, _, _ = lm_head_greedy_accept(hidden, weight, None, weight_tiled=weight_tiled)
    return post.reshape(hidden.shape[:-1])


def sample_tokens(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """runtime.py:22-29: greedy argmax over the last axis when temperature is
    ~0 (gfx950 kernel), else a categorical draw (torch on the device; outside
    the verify hot path).  Returns int32 of shape logits.shape[:-1]."""
    V = logits.shape[-1]
    flat = logits.reshape(-1, V)
    if temperature < 1e-5:
        post, _, _ = greedy_accept(flat.unsqueeze(0), None)
        sampled = post[0]
    else:
        probs = torch.softmax(flat.float() / temperature, dim=-1)
        sampled = torch.multinomial(probs, 1).squeeze(-1).to(torch.int32)
    return sampled.reshape(logits.shape[:-1])


def longest_prefix_match(draft_tokens: list[int], verifier_tokens: list[int]) -> int:
    """runtime.py:41-47: number of leading positions where the lists agree."""
    matched = 0
    for draft_token, verifier_token in zip(draft_tokens, verifier_tokens):
        if draft_token != verifier_token:
            break
        matched += 1
    return matched


def profile_start(profile: dict[str, float] | None) -> float:
    return time.perf_counter() if profile is not None else 0.0


def add_profile_elapsed(profile: dict[str, float] | None, key: str, start: float) -> None:
    if profile is not None:
        profile[key] = profile.get(key, 0.0) + time.perf_counter() - start


def verify_block_parallel_replay(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    draft_block_size: int,
    temperature: float,
    layer_ids: list[int],
    profile: dict[str, float] | None = None,
) -> tuple[int, int, torch.Tensor]:
    """One verify step (runtime.py:117-163).

    ``target`` follows the reference's LoadedTargetModel facade:
    forward_with_hidden_states(inputs, cache, layer_ids,
    return_rollback_records=True) -> (logits, hidden, records),
    rewind_kv_caches(cache, n) and rollback_linear_caches(cache, records, a).
    Returns (accepted_inputs, bonus_token, verifier_hidden[:, :accepted_inputs]).
    """
    if temperature >= 1e-5:
        raise NotImplementedError("the fused verify accepts greedy decoding only (temperature 0)")
    verifier_start = profile_start(profile)
    dev = target.device
    block = torch.tensor(block_tokens, dtype=torch.int32).to(dev)
    logits, verifier_hidden, rollback_records = target.forward_with_hidden_states(
        block[None], target_cache, layer_ids, return_rollback_records=True
    )
    # draft = block[1:] against posterior rows 0..T-2; the bonus may come from
    # row `matched` <= T-1, so all T rows are argmax'ed (runtime.py:145-147).
    _, matched_t, bonus_t = greedy_accept(logits[:1], block[None, 1:], want_posterior=False)
    host = torch.stack([matched_t, bonus_t]).cpu()  # the one device->host sync
    matched, bonus = int(host[0, 0]), int(host[1, 0])
    accepted_inputs = matched + 1
    add_profile_elapsed(profile, "verify_forward_logits_time_s", verifier_start)

    if accepted_inputs < draft_block_size:
        rollback_start = profile_start(profile)
        target.rewind_kv_caches(target_cache, draft_block_size - accepted_inputs)
        target.rollback_linear_caches(target_cache, rollback_records, accepted_inputs)
        add_profile_elapsed(profile, "verify_rollback_time_s", rollback_start)

    return accepted_inputs, bonus, verifier_hidden[:, :accepted_inputs, :]
