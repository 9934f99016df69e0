"""The reference's public generation API (dflash_mlx/api.py:20-212) over the
MI355X target.

``DFlashGenerator`` keeps the reference's methods, arguments and results
(``generate`` / ``stream`` from text, ``generate_from_tokens`` /
``stream_from_tokens`` from token ids, ``DFlashResult`` /
``DFlashStreamEvent``) and runs ``runtime.dflash_generate(_stream)``.  The
reference constructor downloads and loads an MLX target and a DFlash drafter
by name; here both are passed in already built: ``target`` is a
``LoadedTargetModel`` (or a model object with the DFlash methods, such as
``target.HybridTargetModel``, which is wrapped in one) and ``draft`` is any
object with the drafter interface described in runtime.py.  Checkpoint
loading, quantisation of the drafter and the MLX memory wiring are outside
the verify hot path.
"""
from __future__ import annotations

from collections.abc import Iterator
from dataclasses import dataclass
from typing import Any

import torch

from .adapters import LoadedTargetModel
from .runtime import dflash_generate, dflash_generate_stream


@dataclass
class DFlashResult:
    text: str
    output_tokens: list[int]
    generated_tokens: list[int]
    metrics: dict[str, Any]


@dataclass
class DFlashStreamEvent:
    delta: str
    text: str
    token_ids: list[int]
    output_tokens: list[int]
    generated_tokens: list[int]
    metrics: dict[str, Any] | None = None
    finished: bool = False


class DFlashGenerator:
    """api.py:39-212 with the target and drafter injected."""

    def __init__(self, target: Any, draft: Any, tokenizer: Any = None,
                 draft_attention_mask: str = "auto", seed: int = 0):
        torch.manual_seed(seed)
        if not isinstance(target, LoadedTargetModel):
            target = LoadedTargetModel(model=target, tokenizer=tokenizer)
        elif tokenizer is not None:
            target.tokenizer = tokenizer
        self.target: LoadedTargetModel = target
        self.draft = draft
        if draft_attention_mask == "auto":  # api.py:57-60
            draft_attention_mask = "causal" if self.target.adapter.family == "qwen3_5" else "none"
        self.draft_attention_mask = draft_attention_mask
        if hasattr(draft, "attention_mask_mode"):
            draft.attention_mask_mode = draft_attention_mask

    @property
    def target_model_path(self):
        return self.target.resolved_model_path

    def encode_prompt(self, prompt_text: str) -> torch.Tensor:
        return self.target.build_prompt(prompt_text)

    def _decode(self, tokens: list[int], skip_special_tokens: bool) -> str:
        tok = self.target.tokenizer
        if tok is None:
            return ""
        return tok.decode(tokens, skip_special_tokens=skip_special_tokens)

    def generate_from_tokens(
        self,
        prompt_tokens: torch.Tensor,
        max_new_tokens: int = 256,
        temperature: float = 0.0,
        speculative_tokens: int | None = None,
        verify_mode: str = "parallel-replay",
        verify_chunk_size: int = 4,
        reset_peak_memory: bool = True,
        skip_special_tokens: bool = False,
        profile: bool = False,
    ) -> DFlashResult:
        if reset_peak_memory and torch.cuda.is_available():
            torch.cuda.reset_peak_memory_stats()
        output_tokens, metrics = dflash_generate(
            target=self.target,
            draft=self.draft,
            prompt_tokens=prompt_tokens,
            max_new_tokens=max_new_tokens,
            temperature=temperature,
            stop_token_ids=self.target.stop_token_ids(),
            layer_ids=self.draft.target_layer_ids,
            speculative_tokens=speculative_tokens,
            verify_mode=verify_mode,
            verify_chunk_size=verify_chunk_size,
            profile=profile,
        )
        generated_tokens = output_tokens[metrics["num_input_tokens"]:]
        return DFlashResult(
            text=self._decode(generated_tokens, skip_special_tokens),
            output_tokens=output_tokens,
            generated_tokens=generated_tokens,
            metrics=metrics,
        )

    def stream_from_tokens(
        self,
        prompt_tokens: torch.Tensor,
        max_new_tokens: int = 256,
        temperature: float = 0.0,
        speculative_tokens: int | None = None,
        verify_mode: str = "parallel-replay",
        verify_chunk_size: int = 4,
        reset_peak_memory: bool = True,
        skip_special_tokens: bool = False,
        profile: bool = False,
    ) -> Iterator[DFlashStreamEvent]:
        prompt_len = int(torch.as_tensor(prompt_tokens).reshape(-1).shape[0])
        decoded_text = ""
        if reset_peak_memory and torch.cuda.is_available():
            torch.cuda.reset_peak_memory_stats()
        for event in dflash_generate_stream(
            target=self.target,
            draft=self.draft,
            prompt_tokens=prompt_tokens,
            max_new_tokens=max_new_tokens,
            temperature=temperature,
            stop_token_ids=self.target.stop_token_ids(),
            layer_ids=self.draft.target_layer_ids,
            speculative_tokens=speculative_tokens,
            verify_mode=verify_mode,
            verify_chunk_size=verify_chunk_size,
            profile=profile,
        ):
            generated_tokens = event.output_tokens[prompt_len:]
            text = self._decode(generated_tokens, skip_special_tokens)
            delta = text[len(decoded_text):] if text.startswith(decoded_text) else text
            decoded_text = text
            yield DFlashStreamEvent(
                delta=delta,
                text=text,
                token_ids=list(event.token_ids),
                output_tokens=list(event.output_tokens),
                generated_tokens=list(generated_tokens),
                metrics=event.metrics,
                finished=event.finished,
            )

    def generate(self, prompt_text: str, **kwargs) -> DFlashResult:
        """api.py:170-190: generate_from_tokens on the chat-templated prompt."""
        return self.generate_from_tokens(prompt_tokens=self.encode_prompt(prompt_text), **kwargs)

    def stream(self, prompt_text: str, **kwargs) -> Iterator[DFlashStreamEvent]:
        """api.py:192-212: stream_from_tokens on the chat-templated prompt."""
        return self.stream_from_tokens(prompt_tokens=self.encode_prompt(prompt_text), **kwargs)
