"""Cache rollback for the Qwen3.5 hybrid target, driven by the state tape.

Reference: Qwen35TargetAdapter.rewind_kv_caches / rollback_linear_caches
(dflash_mlx/adapters.py:505-560) and Qwen3_5TextModel.rollback_linear_caches
(dflash_mlx/custom_qwen35_model.py:1029-1074).  The reference's rollback
record holds {initial_conv_state, initial_state, qkv, k, v, g, beta,
repeat_factor} (:295-304) and replays the accepted prefix.  Here the verify
scan already wrote the per-token state tape, so the record holds
{initial_conv_state, initial_state, qkv, state_tape} and the rollback is a
gather:

* accepted_inputs given as a host int (the reference's signature): the new
  recurrent state is the view state_tape[a-1] (no bytes move), and the conv
  windows of all layers are rebuilt by one gfx950 launch;
* accepted_inputs given as a device int32 tensor [B] (batched serving, no host
  sync): one launch gathers every layer's state from its tape and one
  launch rebuilds every conv window.
"""
from __future__ import annotations

from typing import Any

import torch

from .cache import ArraysCache, KVCache
from .gated_delta import conv_rollback, tape_select


def rewind_kv_caches(cache: list[Any], num_tokens: int) -> None:
    """adapters.py:505-508: trim every full-attention cache by num_tokens."""
    for layer_cache in cache:
        if isinstance(layer_cache, KVCache):
            layer_cache.trim(num_tokens)


def make_rollback_record(initial_conv_state, initial_state, qkv, state_tape) -> dict[str, Any]:
    """The per-layer record the verify forward returns with the tape."""
    return {
        "initial_conv_state": initial_conv_state,
        "initial_state": initial_state,
        "qkv": qkv,
        "state_tape": state_tape,
    }


def rollback_linear_caches(
    cache: list[Any],
    rollback_records: dict[int, dict[str, Any]],
    accepted_inputs: int | torch.Tensor,
) -> None:
    """Restore every gated-delta layer's [conv_state, state] to what it was
    after ``accepted_inputs`` tokens of the verified block."""
    if not rollback_records:
        return
    idxs = list(rollback_records.keys())
    recs = [rollback_records[i] for i in idxs]
    conv_ins = [r["initial_conv_state"] for r in recs]
    qkvs = [r["qkv"] for r in recs]
    new_convs = conv_rollback(conv_ins, qkvs, accepted_inputs)
    if isinstance(accepted_inputs, torch.Tensor):
        new_states = tape_select(
            [r["state_tape"] for r in recs], [r["initial_state"] for r in recs], accepted_inputs
        )
    else:
        a = int(accepted_inputs)
        T = recs[0]["state_tape"].shape[0]
        if not 0 <= a <= T:
            raise ValueError(f"accepted_inputs={a} outside [0, {T}]")
        new_states = [r["state_tape"][a - 1] if a >= 1 else r["initial_state"] for r in recs]
    for idx, conv, state in zip(idxs, new_convs, new_states):
        cache[idx][0] = conv
        cache[idx][1] = state


class Qwen35TargetAdapter:
    """Rollback half of the reference's Qwen35TargetAdapter
    (adapters.py:341-570).  Model loading, prompting and the LM head are
    outside the verify hot path and are not provided here."""

    family = "qwen3_5"

    def make_cache(self, num_layers: int, full_attention_interval: int = 4) -> list[Any]:
        """custom_qwen35_model.py:818, :1153-1154: layer i is linear
        attention unless (i + 1) % full_attention_interval == 0."""
        return [
            ArraysCache(size=2) if (i + 1) % full_attention_interval != 0 else KVCache()
            for i in range(num_layers)
        ]

    def rewind_kv_caches(self, cache: list[Any], num_tokens: int) -> None:
        rewind_kv_caches(cache, num_tokens)

    def rollback_linear_caches(self, model, cache, rollback_records, accepted_inputs) -> None:
        rollback_linear_caches(cache, rollback_records, accepted_inputs)

    def cache_summary(self, cache: list[Any]) -> str:
        parts: list[str] = []
        for idx, layer_cache in enumerate(cache):
            if isinstance(layer_cache, KVCache):
                parts.append(f"{idx}:kv={layer_cache.offset}")
            elif isinstance(layer_cache, ArraysCache):
                st = layer_cache[1]
                parts.append(f"{idx}:ssm={None if st is None else tuple(st.shape)}")
        return " ".join(parts)


ADAPTERS = {"qwen3_5": Qwen35TargetAdapter}


def adapter_for_model_type(model_type: str):
    return ADAPTERS.get(model_type)
