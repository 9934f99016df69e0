"""DFlash decode runtime on MI355X: the verify step, its accept and
rollback, and the speculative decode loop.

Mirrors the reference's dflash_mlx/runtime.py:

* ``sample_tokens`` (:22-29) — greedy argmax runs in the gfx950 accept kernel;
* ``longest_prefix_match`` (:41-47) — the host-list primitive, unchanged;
* ``greedy_accept`` — argmax + prefix compare + bonus fused on the device, so
  only (matched, bonus) cross to the host;
* the verify modes ``verify_block_stream`` (:86-114),
  ``verify_block_parallel_replay`` (:117-163),
  ``verify_block_parallel_lazy_logits`` (:166-243),
  ``verify_block_parallel_greedy_argmax`` (:246-292) and
  ``verify_block_chunked`` (:295-357), same arguments and return tuples; the
  rollback they trigger is a tape gather instead of a replay;
* ``dflash_generate_stream`` / ``dflash_generate`` (:360-589): prefill,
  draft a block, verify, accept, roll back, repeat, with the same events and
  metrics.

``target`` is the LoadedTargetModel facade (adapters.py) over the MI355X
hybrid target; ``draft`` is any object with the DFlash drafter's interface
(``block_size``, ``mask_token_id``, ``target_layer_ids``, ``make_cache()``,
``__call__(noise_embedding=, target_hidden=, cache=)`` returning draft hidden
states, dflash_mlx/draft.py:190-223).  The drafter network itself is not part
of this package.

Token ids are int32 on the device (the reference uses uint32; vocabularies
here are far below 2**31).
"""
from __future__ import annotations

import time
from collections.abc import Iterator
from dataclasses import dataclass
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


@dataclass
class DFlashRuntimeEvent:
    """runtime.py:14-19: tokens added since the last event, the whole output
    so far, and the metrics on the final event."""

    token_ids: list[int]
    output_tokens: list[int]
    metrics: dict[str, Any] | None = None
    finished: bool = False


def trim_draft_cache(cache: list[Any], num_tokens: int) -> None:
    """runtime.py:32-34."""
    for layer_cache in cache:
        layer_cache.trim(num_tokens)


def generated_token_count(output_tokens: list[int], prompt_len: int) -> int:
    return max(len(output_tokens) - prompt_len, 0)


def stop_position(tokens: list[int], start_idx: int, stop_token_ids: set[int]) -> int | None:
    """runtime.py:50-54: index of the first stop token at or after start_idx."""
    for idx in range(start_idx, len(tokens)):
        if tokens[idx] in stop_token_ids:
            return idx
    return None


def peak_memory_gb() -> float:
    """runtime.py:57-58, as the device allocator's high-water mark."""
    if not torch.cuda.is_available():
        return 0.0
    return torch.cuda.max_memory_allocated() / 1e9


def _block_tensor(block_tokens: Sequence[int], device) -> torch.Tensor:
    return torch.tensor([list(block_tokens)], dtype=torch.int32).to(device)


def _target_device(target: Any):
    model = getattr(target, "model", None)
    return getattr(model, "device", None) or getattr(target, "device", None) or "cuda"


def _posterior(logits: torch.Tensor, temperature: float) -> list[int]:
    """Posterior tokens of row 0 of [1, N, V] logits on the host."""
    return sample_tokens(logits[:1], temperature)[0].cpu().tolist()


def _rollback(target, target_cache, rollback_records, draft_block_size, accepted_inputs,
              profile) -> None:
    """runtime.py:150-161: rewind the KV caches and roll the linear caches
    back when only part of the block was accepted."""
    if accepted_inputs < draft_block_size:
        rollback_start = profile_start(profile)
        target.rewind_kv_caches(target_cache, draft_block_size - accepted_inputs)
        target.rollback_linear_caches(target_cache, rollback_records, accepted_inputs)
        add_profile_elapsed(profile, "verify_rollback_time_s", rollback_start)


def verify_block_stream(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    temperature: float,
    layer_ids: list[int],
) -> tuple[int, int, torch.Tensor]:
    """runtime.py:86-114: verify token by token, stopping at the first
    mismatch (no rollback needed)."""
    dev = _target_device(target)
    verified_hidden_steps: list[torch.Tensor] = []
    for idx, token in enumerate(block_tokens):
        logits_step, hidden_step = target.forward_with_hidden_states(
            _block_tensor([token], dev), target_cache, layer_ids)
        next_token = _posterior(logits_step[:, -1:, :], temperature)[0]
        verified_hidden_steps.append(hidden_step)
        if idx == len(block_tokens) - 1:
            return len(block_tokens), next_token, torch.cat(verified_hidden_steps, dim=1)
        if next_token != block_tokens[idx + 1]:
            return idx + 1, next_token, torch.cat(verified_hidden_steps, dim=1)
    raise RuntimeError("Streaming verifier reached an impossible state.")


def verify_block_parallel_replay(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    draft_block_size: int,
    temperature: float,
    layer_ids: list[int],
    profile: dict[str, float] | None = None,
) -> tuple[int, int, torch.Tensor]:
    """One verify step (runtime.py:117-163): the whole block in one forward
    with rollback records, the posterior from its logits, the accept, and the
    rollback of a partial accept.

    Greedy (temperature 0): argmax, prefix compare and bonus run in one
    device kernel pair and only (matched, bonus) cross to the host.  Else
    the posterior is sampled (sample_tokens) and compared on the host.
    Returns (accepted_inputs, bonus_token, verifier_hidden[:, :accepted_inputs])."""
    verifier_start = profile_start(profile)
    block = _block_tensor(block_tokens, _target_device(target))
    logits, verifier_hidden, rollback_records = target.forward_with_hidden_states(
        block, target_cache, layer_ids, return_rollback_records=True
    )
    if temperature < 1e-5:
        # draft = block[1:] against posterior rows 0..T-2; the bonus may come
        # from row `matched` <= T-1, so all T rows are argmax'ed (runtime.py:145-147).
        _, matched_t, bonus_t = greedy_accept(logits[:1], block.to(logits.device)[:, 1:],
                                              want_posterior=False)
        host = torch.stack([matched_t, bonus_t]).cpu()  # the one device->host sync
        matched, bonus = int(host[0, 0]), int(host[1, 0])
    else:
        posterior = _posterior(logits, temperature)
        matched = longest_prefix_match(block_tokens[1:], posterior[:-1])
        bonus = posterior[matched]
    accepted_inputs = matched + 1
    add_profile_elapsed(profile, "verify_forward_logits_time_s", verifier_start)
    _rollback(target, target_cache, rollback_records, draft_block_size, accepted_inputs, profile)
    return accepted_inputs, bonus, verifier_hidden[:, :accepted_inputs, :]


def verify_block_parallel_lazy_logits(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    draft_block_size: int,
    temperature: float,
    layer_ids: list[int],
    logit_chunk_size: int,
    profile: dict[str, float] | None = None,
) -> tuple[int, int, torch.Tensor]:
    """runtime.py:166-243: the verifier's normed hidden states first, then
    the LM head chunk by chunk until the first mismatch."""
    state_start = profile_start(profile)
    norm_hidden_states, verifier_hidden, rollback_records = target.forward_verifier_states(
        _block_tensor(block_tokens, _target_device(target)), target_cache, layer_ids)
    add_profile_elapsed(profile, "verify_state_time_s", state_start)

    matched = 0
    accepted_inputs = draft_block_size
    posterior_token: int | None = None
    chunk_size = max(1, logit_chunk_size)
    for chunk_start in range(0, draft_block_size, chunk_size):
        chunk_end = min(chunk_start + chunk_size, draft_block_size)
        logit_start = profile_start(profile)
        logits_chunk = target.lm_head_logits(norm_hidden_states[:, chunk_start:chunk_end, :])
        posterior_chunk = _posterior(logits_chunk, temperature)
        add_profile_elapsed(profile, "verify_lazy_logits_time_s", logit_start)
        prefix_start = profile_start(profile)
        for local_idx, token in enumerate(posterior_chunk):
            pos = chunk_start + local_idx
            if pos == draft_block_size - 1:
                posterior_token = token
                accepted_inputs = draft_block_size
                break
            if token == block_tokens[pos + 1]:
                matched += 1
                continue
            posterior_token = token
            accepted_inputs = matched + 1
            break
        add_profile_elapsed(profile, "verify_prefix_time_s", prefix_start)
        if posterior_token is not None:
            break
    if posterior_token is None:
        raise RuntimeError("Lazy-logit verifier failed to produce a posterior token.")
    _rollback(target, target_cache, rollback_records, draft_block_size, accepted_inputs, profile)
    return accepted_inputs, posterior_token, verifier_hidden[:, :accepted_inputs, :]


def verify_block_parallel_greedy_argmax(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    draft_block_size: int,
    temperature: float,
    layer_ids: list[int],
    profile: dict[str, float] | None = None,
) -> tuple[int, int, torch.Tensor]:
    """runtime.py:246-292: the verifier's normed hidden states, then the
    target's lm_head_argmax hook (here the fused LM-head greedy kernel: no
    logits are materialised), the prefix compare and the rollback."""
    if temperature >= 1e-5:
        raise ValueError("parallel-greedy-argmax only supports temperature=0.")
    state_start = profile_start(profile)
    norm_hidden_states, verifier_hidden, rollback_records = target.forward_verifier_states(
        _block_tensor(block_tokens, _target_device(target)), target_cache, layer_ids)
    add_profile_elapsed(profile, "verify_state_time_s", state_start)

    argmax_start = profile_start(profile)
    posterior = target.lm_head_argmax(norm_hidden_states)[0].cpu().tolist()
    add_profile_elapsed(profile, "verify_argmax_time_s", argmax_start)

    prefix_start = profile_start(profile)
    matched = longest_prefix_match(block_tokens[1:], posterior[:-1])
    accepted_inputs = matched + 1
    add_profile_elapsed(profile, "verify_prefix_time_s", prefix_start)
    _rollback(target, target_cache, rollback_records, draft_block_size, accepted_inputs, profile)
    return accepted_inputs, posterior[matched], verifier_hidden[:, :accepted_inputs, :]


def verify_block_chunked(
    target: Any,
    target_cache: list[Any],
    block_tokens: list[int],
    draft_block_size: int,
    temperature: float,
    layer_ids: list[int],
    verify_chunk_size: int,
) -> tuple[int, int, torch.Tensor]:
    """runtime.py:295-357: verify in chunks; on a mismatch restore the
    chunk's linear caches from a snapshot and re-run only its accepted
    prefix."""
    dev = _target_device(target)
    verified_hidden_chunks: list[torch.Tensor] = []
    cursor = 0
    while cursor < draft_block_size:
        chunk_end = min(cursor + verify_chunk_size, draft_block_size)
        chunk_tokens = block_tokens[cursor:chunk_end]
        linear_snapshots = target.snapshot_linear_caches(target_cache)
        chunk_logits, chunk_hidden = target.forward_with_hidden_states(
            _block_tensor(chunk_tokens, dev), target_cache, layer_ids)
        posterior_chunk = _posterior(chunk_logits, temperature)

        max_compare = min(len(chunk_tokens), draft_block_size - cursor - 1)
        local_matches = 0
        while local_matches < max_compare:
            if posterior_chunk[local_matches] != block_tokens[cursor + local_matches + 1]:
                break
            local_matches += 1

        if local_matches == max_compare and chunk_end < draft_block_size:
            verified_hidden_chunks.append(chunk_hidden)
            cursor = chunk_end
            continue
        if local_matches == max_compare and chunk_end == draft_block_size:
            verified_hidden_chunks.append(chunk_hidden)
            return (draft_block_size, posterior_chunk[-1],
                    torch.cat(verified_hidden_chunks, dim=1))

        accepted_local_inputs = local_matches + 1
        target.rewind_kv_caches(target_cache, len(chunk_tokens))
        target.restore_linear_caches(target_cache, linear_snapshots)
        replay_hidden = target.forward_with_hidden_states(
            _block_tensor(chunk_tokens[:accepted_local_inputs], dev), target_cache, layer_ids)[1]
        verified_hidden_chunks.append(replay_hidden)
        return (cursor + accepted_local_inputs, posterior_chunk[local_matches],
                torch.cat(verified_hidden_chunks, dim=1))
    raise RuntimeError("Chunked verifier reached an impossible state.")


VERIFY_MODES = ("parallel-replay", "parallel-greedy-argmax", "parallel-lazy-logits", "stream",
                "chunked")


def dflash_generate_stream(
    target: Any,
    draft: Any,
    prompt_tokens: torch.Tensor | Sequence[int],
    max_new_tokens: int,
    temperature: float,
    stop_token_ids: set[int],
    layer_ids: list[int],
    speculative_tokens: int | None,
    verify_mode: str,
    verify_chunk_size: int,
    profile: bool = False,
) -> Iterator[DFlashRuntimeEvent]:
    """The DFlash decode loop (runtime.py:360-555): prefill the prompt, then
    repeatedly draft a block [last token, drafts...] from the target hidden
    states, verify it, keep the accepted prefix plus the posterior's bonus
    token, and stop at max_new_tokens or a stop token.  Yields the new tokens
    after the prefill and after every block, then a final event with the
    metrics."""
    if verify_mode not in VERIFY_MODES:
        raise ValueError(f"unknown verify_mode {verify_mode!r}; one of {VERIFY_MODES}")
    prompt = torch.as_tensor(prompt_tokens).reshape(-1)
    dev = _target_device(target)
    target_cache = target.make_cache()
    draft_cache = draft.make_cache()
    profile_times: dict[str, float] | None = {} if profile else None
    prompt_len = int(prompt.shape[0])
    total_max_tokens = prompt_len + max_new_tokens
    if speculative_tokens is None:
        block_size = draft.block_size
    else:
        block_size = max(1, min(speculative_tokens, draft.block_size))

    sync_start = time.perf_counter()
    # runtime.py:384-390 takes forward_with_hidden_states' logits of every
    # prompt row and samples the last; the facade's last-position form
    # (forward_accept_all_block) gives that row and the same target hidden
    # states without the other P - 1 rows of the LM head (3.2 ms of a
    # 4096-token prompt at the c4 shape), which nothing reads.
    logits, target_hidden = target.forward_accept_all_block(
        prompt.to(device=dev, dtype=torch.int32)[None], target_cache, layer_ids)
    first_token = _posterior(logits[:, -1:, :], temperature)[0]
    prefill_time = time.perf_counter() - sync_start

    output_tokens = prompt.tolist() + [first_token]
    start = prompt_len
    streamed_len = prompt_len
    acceptance_lengths: list[int] = []

    if max_new_tokens > 0:
        yield DFlashRuntimeEvent(token_ids=output_tokens[streamed_len:],
                                 output_tokens=list(output_tokens))
        streamed_len = len(output_tokens)

    decode_start = time.perf_counter()
    while start < total_max_tokens:
        draft_start = profile_start(profile_times)
        block_tokens = [output_tokens[start]] + [draft.mask_token_id] * (block_size - 1)
        noise_embedding = target.embed_tokens(_block_tensor(block_tokens, dev))
        draft_hidden = draft(noise_embedding=noise_embedding, target_hidden=target_hidden,
                             cache=draft_cache)
        draft_logits = target.lm_head_logits(draft_hidden[:, 1:, :])
        drafted_suffix = sample_tokens(draft_logits, temperature)[0].cpu().tolist()
        trim_draft_cache(draft_cache, block_size)
        block_tokens[1:] = drafted_suffix[: block_size - 1]
        add_profile_elapsed(profile_times, "draft_time_s", draft_start)

        verify_start = profile_start(profile_times)
        if verify_mode == "stream":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_stream(
                target, target_cache, block_tokens, temperature, layer_ids)
        elif verify_mode == "chunked":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_chunked(
                target, target_cache, block_tokens, block_size, temperature, layer_ids,
                verify_chunk_size)
        elif verify_mode == "parallel-lazy-logits":
            accepted_inputs, posterior_token, verifier_hidden = verify_block_parallel_lazy_logits(
                target, target_cache, block_tokens, block_size, temperature, layer_ids,
                verify_chunk_size, profile=profile_times)
        elif verify_mode == "parallel-greedy-argmax":
            accepted_inputs, posterior_token, verifier_hidden = \
                verify_block_parallel_greedy_argmax(target, target_cache, block_tokens, block_size,
                                                    temperature, layer_ids, profile=profile_times)
        else:
            accepted_inputs, posterior_token, verifier_hidden = verify_block_parallel_replay(
                target, target_cache, block_tokens, block_size, temperature, layer_ids,
                profile=profile_times)
        acceptance_lengths.append(accepted_inputs)
        target_hidden = verifier_hidden[:, :accepted_inputs, :]
        add_profile_elapsed(profile_times, "verify_time_s", verify_start)

        bookkeeping_start = profile_start(profile_times)
        output_tokens = output_tokens[:start]
        output_tokens.extend(block_tokens[:accepted_inputs])
        output_tokens.append(posterior_token)
        start += accepted_inputs
        add_profile_elapsed(profile_times, "bookkeeping_time_s", bookkeeping_start)

        stop_idx = stop_position(output_tokens, prompt_len, stop_token_ids)
        finished = False
        if stop_idx is not None:
            output_tokens = output_tokens[: stop_idx + 1]
            finished = True
        if len(output_tokens) > total_max_tokens:
            output_tokens = output_tokens[:total_max_tokens]
            finished = True

        token_ids = output_tokens[streamed_len:]
        if token_ids:
            yield DFlashRuntimeEvent(token_ids=token_ids, output_tokens=list(output_tokens))
            streamed_len = len(output_tokens)
        if finished:
            break

    decode_time = time.perf_counter() - decode_start
    output_tokens = output_tokens[:total_max_tokens]
    generated_tokens = generated_token_count(output_tokens, prompt_len)
    total_time = prefill_time + decode_time
    metrics: dict[str, Any] = {
        "num_input_tokens": prompt_len,
        "num_output_tokens": generated_tokens,
        "prefill_time_s": prefill_time,
        "decode_time_s": decode_time,
        "total_time_s": total_time,
        "prompt_tps": prompt_len / max(prefill_time, 1e-9),
        "generation_tps": generated_tokens / max(decode_time, 1e-9),
        "end_to_end_tps": generated_tokens / max(total_time, 1e-9),
        "avg_acceptance_length": sum(acceptance_lengths) / max(len(acceptance_lengths), 1),
        "acceptance_lengths": acceptance_lengths,
        "peak_memory_gb": peak_memory_gb(),
        "target_cache_summary": target.cache_summary(target_cache),
        "speculative_tokens": block_size,
    }
    if profile_times is not None:
        profiled_time = sum(profile_times.get(key, 0.0)
                            for key in ("draft_time_s", "verify_time_s", "bookkeeping_time_s"))
        metrics["profile"] = {**profile_times,
                              "unattributed_decode_time_s": decode_time - profiled_time,
                              "steps": len(acceptance_lengths)}
    yield DFlashRuntimeEvent(token_ids=[], output_tokens=list(output_tokens), metrics=metrics,
                             finished=True)


def dflash_generate(
    target: Any,
    draft: Any,
    prompt_tokens: torch.Tensor | Sequence[int],
    max_new_tokens: int,
    temperature: float,
    stop_token_ids: set[int],
    layer_ids: list[int],
    speculative_tokens: int | None,
    verify_mode: str,
    verify_chunk_size: int,
    profile: bool = False,
) -> tuple[list[int], dict[str, Any]]:
    """runtime.py:558-589: run the stream to the end; (output_tokens, metrics)."""
    final_event: DFlashRuntimeEvent | None = None
    for event in dflash_generate_stream(
        target=target, draft=draft, prompt_tokens=prompt_tokens, max_new_tokens=max_new_tokens,
        temperature=temperature, stop_token_ids=stop_token_ids, layer_ids=layer_ids,
        speculative_tokens=speculative_tokens, verify_mode=verify_mode,
        verify_chunk_size=verify_chunk_size, profile=profile,
    ):
        if event.finished:
            final_event = event
    if final_event is None or final_event.metrics is None:
        raise RuntimeError("DFlash generation did not produce a final event.")
    return final_event.output_tokens, final_event.metrics
