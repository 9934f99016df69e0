"""Per-layer caches of the hybrid target, as the verify path sees them.

Mirrors the two cache kinds the reference's Qwen3.5 model makes
(dflash_mlx/custom_qwen35_model.py:1153-1154): an ``ArraysCache(size=2)`` per
gated-delta layer holding [conv_state, recurrent_state], and a ``KVCache`` per
full-attention layer whose rollback is an offset decrement (mlx_lm
``KVCache.trim``, called from dflash_mlx/adapters.py:505-508).  Tensors live
on the ROCm device; only the KV offset is host state.
"""
from __future__ import annotations

import torch


class ArraysCache:
    """Fixed-size list of device tensors: [conv_state [B,K-1,C], state [B,Hv,Dv,Dk]]."""

    def __init__(self, size: int = 2):
        self.cache: list[torch.Tensor | None] = [None] * size

    def __getitem__(self, idx: int) -> torch.Tensor | None:
        return self.cache[idx]

    def __setitem__(self, idx: int, value: torch.Tensor | None) -> None:
        self.cache[idx] = value

    def __len__(self) -> int:
        return len(self.cache)


class KVCache:
    """Growing key/value cache; ``offset`` counts the valid positions."""

    def __init__(self):
        self.keys: torch.Tensor | None = None
        self.values: torch.Tensor | None = None
        self.offset = 0

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Append [B,H,L,D] keys/values at ``offset`` and return the valid prefix."""
        L = keys.shape[2]
        need = self.offset + L
        if self.keys is None or self.keys.shape[2] < need:
            cap = max(need, 2 * (self.keys.shape[2] if self.keys is not None else 0), 256)
            shape = (keys.shape[0], keys.shape[1], cap, keys.shape[3])
            vshape = (values.shape[0], values.shape[1], cap, values.shape[3])
            new_k = keys.new_zeros(shape)
            new_v = values.new_zeros(vshape)
            if self.keys is not None and self.offset:
                new_k[:, :, : self.offset] = self.keys[:, :, : self.offset]
                new_v[:, :, : self.offset] = self.values[:, :, : self.offset]
            self.keys, self.values = new_k, new_v
        self.keys[:, :, self.offset : need] = keys
        self.values[:, :, self.offset : need] = values
        self.offset = need
        return self.keys[:, :, :need], self.values[:, :, :need]

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        """Drop the last n positions (no data moves); returns how many were dropped."""
        n = min(self.offset, max(int(n), 0))
        self.offset -= n
        return n
