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

from dataclasses import dataclass, field
from pathlib import Path
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
    """The reference's Qwen35TargetAdapter (adapters.py:341-570) over a model
    object with the DFlash methods (``target.HybridTargetModel``).  Loading a
    checkpoint and the chat template are outside the verify hot path: the
    model is built by the caller and the tokenizer, when there is one, is
    any object with the Hugging Face ``encode`` / ``decode`` /
    ``apply_chat_template`` / ``eos_token_ids`` surface."""

    family = "qwen3_5"

    def build_prompt(self, tokenizer, prompt_text: str) -> torch.Tensor:
        """adapters.py:356-365: the chat template with thinking disabled."""
        if tokenizer is None:
            raise ValueError("building a prompt from text needs a tokenizer")
        messages = [{"role": "user", "content": prompt_text}]
        prompt = tokenizer.apply_chat_template(messages, tokenize=False,
                                               add_generation_prompt=True, enable_thinking=False)
        return torch.tensor(tokenizer.encode(prompt, add_special_tokens=False), dtype=torch.int32)

    def stop_token_ids(self, tokenizer, model=None) -> set[int]:
        """adapters.py:367-371 (the tokenizer's eos ids); without a tokenizer,
        the model's configured eos ids."""
        if tokenizer is None:
            return set(getattr(model, "eos_token_ids", ()))
        eos = tokenizer.eos_token_ids
        return {eos} if isinstance(eos, int) else set(eos)

    def make_cache(self, model=None, num_layers: int | None = None,
                   full_attention_interval: int = 4) -> list[Any]:
        """The model's cache list (custom_qwen35_model.py:1153-1154); without
        a model, host-side cache objects for num_layers layers (layer i is
        linear attention unless (i + 1) % full_attention_interval == 0, :818)."""
        if model is not None and hasattr(model, "make_cache"):
            return model.make_cache()
        return [
            ArraysCache(size=2) if (i + 1) % full_attention_interval != 0 else KVCache()
            for i in range(int(num_layers))
        ]

    def embed_tokens(self, model, tokens):
        return model.embed_tokens(tokens)

    def lm_head_logits(self, model, hidden_states):
        return model.lm_head_logits(hidden_states)

    def lm_head_argmax(self, model, hidden_states):
        """The hook of adapters.py:267-271, served by the fused LM-head
        greedy kernel (no logits)."""
        return model.lm_head_argmax(hidden_states)

    def forward_with_hidden_states(self, model, inputs, cache, layer_ids,
                                   return_rollback_records: bool = False):
        """adapters.py:373-418 via the model's forward_dflash: (logits,
        target_hidden[, records])."""
        out = model.forward_dflash(inputs, cache, layer_ids,
                                   return_rollback_records=return_rollback_records)
        logits = model.lm_head_logits(out[0])
        return (logits,) + tuple(out[1:])

    def forward_verifier_states(self, model, inputs, cache, layer_ids):
        """adapters.py:420-437: (norm_hidden, target_hidden, records)."""
        return model.forward_dflash(inputs, cache, layer_ids, return_rollback_records=True)

    def forward_accept_all_block(self, model, inputs, cache, layer_ids):
        """adapters.py:439-456: logits of the last position only."""
        norm_hidden, target_hidden = model.forward_dflash(inputs, cache, layer_ids,
                                                          return_rollback_records=False)
        return model.lm_head_logits(norm_hidden[:, -1:, :]), target_hidden

    def snapshot_linear_caches(self, model, cache):
        return model.snapshot_linear_caches(cache)

    def restore_linear_caches(self, model, cache, snapshots) -> None:
        model.restore_linear_caches(cache, snapshots)

    def rewind_kv_caches(self, cache: list[Any], num_tokens: int) -> None:
        rewind_kv_caches(cache, num_tokens)

    def rollback_linear_caches(self, model, cache, rollback_records, accepted_inputs) -> None:
        """adapters.py:510-520: the model's own rollback when it has one, else
        the generic tape gather."""
        if model is not None and hasattr(model, "rollback_linear_caches"):
            model.rollback_linear_caches(cache, rollback_records, accepted_inputs)
            return
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


@dataclass
class LoadedTargetModel:
    """The reference's LoadedTargetModel facade (adapters.py:729-826): the
    decode runtime calls these methods, each delegating to the adapter with
    the model.  ``model`` is a built model object (no checkpoint loading)."""

    model: Any
    adapter: Qwen35TargetAdapter = field(default_factory=Qwen35TargetAdapter)
    tokenizer: Any = None
    requested_model: str = "random-init"
    resolved_model_path: Path | None = None

    def build_prompt(self, prompt_text: str) -> torch.Tensor:
        return self.adapter.build_prompt(self.tokenizer, prompt_text)

    def stop_token_ids(self) -> set[int]:
        return self.adapter.stop_token_ids(self.tokenizer, self.model)

    def make_cache(self) -> list[Any]:
        return self.adapter.make_cache(self.model)

    def embed_tokens(self, tokens):
        return self.adapter.embed_tokens(self.model, tokens)

    def lm_head_logits(self, hidden_states):
        return self.adapter.lm_head_logits(self.model, hidden_states)

    def lm_head_argmax(self, hidden_states):
        return self.adapter.lm_head_argmax(self.model, hidden_states)

    def forward_with_hidden_states(self, inputs, cache, layer_ids,
                                   return_rollback_records: bool = False):
        return self.adapter.forward_with_hidden_states(
            self.model, inputs, cache, layer_ids, return_rollback_records=return_rollback_records)

    def forward_verifier_states(self, inputs, cache, layer_ids):
        return self.adapter.forward_verifier_states(self.model, inputs, cache, layer_ids)

    def forward_accept_all_block(self, inputs, cache, layer_ids):
        return self.adapter.forward_accept_all_block(self.model, inputs, cache, layer_ids)

    def snapshot_linear_caches(self, cache):
        return self.adapter.snapshot_linear_caches(self.model, cache)

    def restore_linear_caches(self, cache, snapshots) -> None:
        self.adapter.restore_linear_caches(self.model, cache, snapshots)

    def rewind_kv_caches(self, cache: list[Any], num_tokens: int) -> None:
        self.adapter.rewind_kv_caches(cache, num_tokens)

    def rollback_linear_caches(self, cache, rollback_records, accepted_inputs) -> None:
        self.adapter.rollback_linear_caches(self.model, cache, rollback_records, accepted_inputs)

    def cache_summary(self, cache: list[Any]) -> str:
        return self.adapter.cache_summary(cache)
