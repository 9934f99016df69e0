"""Seeded synthetic workloads of the verify hot path (the benchmark configs).

Draw order per config, on a CPU ``torch.Generator`` seeded with the config
index: q, k, v, x_g, x_beta, S0, logits, accept lengths.  q and k rows are
L2-normalised over Dk in fp32, then rounded to bf16; v is bf16 N(0,1);
g = exp(-softplus(x_g)) and beta = sigmoid(x_beta) in fp32 (the reference's
compute_g with A_log = 0, dt_bias = 0, and its beta = sigmoid(b)).  Stacked
independent layers (config 1's 24-layer sweep) are drawn as extra batch
entries: batch index = layer * B + b.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class ScanConfig:
    name: str
    B: int
    T: int
    Hk: int
    Hv: int
    Dk: int
    Dv: int
    layers: int = 1
    state_std: float = 0.0  # 0 -> zero initial state
    V: int = 0              # vocabulary of the accept logits
    fixed_accept: int | None = None  # known accept length (config 0)
    seed: int = 0

    @property
    def batch(self) -> int:
        """Scan batch: independent (layer, sequence) problems in one launch."""
        return self.layers * self.B

    def scan_bytes(self, with_final: bool = True) -> int:
        """Algorithmic HBM bytes of one scan launch over all stacked layers:
        bf16 q, k, v, out; fp32 g, beta; fp32 state_in + tape (+ final)."""
        Bt, T = self.batch, self.T
        qkvo = 2 * Bt * T * (2 * self.Hk * self.Dk + 2 * self.Hv * self.Dv)
        gb = 8 * Bt * T * self.Hv
        states = 4 * Bt * self.Hv * self.Dv * self.Dk * (1 + T + (1 if with_final else 0))
        return qkvo + gb + states


CONFIGS: dict[int, ScanConfig] = {
    0: ScanConfig("c0-tiny", B=1, T=16, Hk=4, Hv=4, Dk=64, Dv=64, V=1024, fixed_accept=7, seed=0),
    1: ScanConfig("c1-qwen35-4b-24layer", B=1, T=16, Hk=16, Hv=32, Dk=128, Dv=128, layers=24,
                  state_std=0.05, V=151936, seed=1),
    2: ScanConfig("c2-batched-b32", B=32, T=16, Hk=16, Hv=32, Dk=128, Dv=128, state_std=0.05,
                  V=151936, seed=2),
    3: ScanConfig("c3-prefill-8k", B=1, T=8192, Hk=16, Hv=32, Dk=128, Dv=128, seed=3),
}


def _unit_rows(x: torch.Tensor) -> torch.Tensor:
    return x / torch.linalg.vector_norm(x, dim=-1, keepdim=True).clamp_min(1e-12)


def make_scan_inputs(cfg: ScanConfig, seed: int | None = None) -> dict[str, torch.Tensor]:
    """CPU tensors q, k [Bt,T,Hk,Dk] bf16; v [Bt,T,Hv,Dv] bf16; g, beta
    [Bt,T,Hv] fp32; state [Bt,Hv,Dv,Dk] fp32, with Bt = layers * B."""
    gen = torch.Generator().manual_seed(cfg.seed if seed is None else seed)
    Bt, T = cfg.batch, cfg.T
    q = _unit_rows(torch.randn(Bt, T, cfg.Hk, cfg.Dk, generator=gen)).to(torch.bfloat16)
    k = _unit_rows(torch.randn(Bt, T, cfg.Hk, cfg.Dk, generator=gen)).to(torch.bfloat16)
    v = torch.randn(Bt, T, cfg.Hv, cfg.Dv, generator=gen).to(torch.bfloat16)
    xg = torch.randn(Bt, T, cfg.Hv, generator=gen)
    xb = torch.randn(Bt, T, cfg.Hv, generator=gen)
    g = torch.exp(-torch.nn.functional.softplus(xg))
    beta = torch.sigmoid(xb)
    if cfg.state_std > 0:
        state = cfg.state_std * torch.randn(Bt, cfg.Hv, cfg.Dv, cfg.Dk, generator=gen)
    else:
        state = torch.zeros(Bt, cfg.Hv, cfg.Dv, cfg.Dk)
    return {"q": q, "k": k, "v": v, "g": g, "beta": beta, "state": state, "_gen": gen}


def make_accept_inputs(cfg: ScanConfig, gen: torch.Generator | None = None,
                       B: int | None = None) -> dict[str, torch.Tensor]:
    """CPU fp32 logits [B,T,V] ~ N(0,1) and int32 draft [B,T] agreeing with the
    argmax on exactly the first accept[b] positions (then argmax+1 mod V).
    Config 0 uses its fixed accept length; others draw a ~ U{0..T}."""
    if gen is None:
        gen = make_scan_inputs(cfg)["_gen"]
    B = cfg.B if B is None else B
    logits = torch.randn(B, cfg.T, cfg.V, generator=gen)
    if cfg.fixed_accept is not None:
        accept = torch.full((B,), cfg.fixed_accept, dtype=torch.int32)
    else:
        accept = torch.randint(0, cfg.T + 1, (B,), generator=gen, dtype=torch.int32)
    am = logits.argmax(dim=-1).to(torch.int32)
    pos = torch.arange(cfg.T, dtype=torch.int32)[None, :]
    draft = torch.where(pos < accept[:, None], am, (am + 1) % cfg.V).to(torch.int32)
    return {"logits": logits, "draft": draft, "accept": accept}


def make_verify_block(acc: dict[str, torch.Tensor], first_token: int = 0) -> torch.Tensor:
    """The verify block [B, T] of the reference's wiring (runtime.py:145-147):
    block[0] is the last accepted token, block[1:] the drafts, compared with
    posterior rows 0..T-2.  Here block[1+i] = draft[i], so an accept length
    a drawn by make_accept_inputs gives matched = min(a, T-1) and
    accepted_inputs = matched + 1."""
    draft = acc["draft"]
    block = torch.empty_like(draft)
    block[:, 0] = first_token
    block[:, 1:] = draft[:, :-1]
    return block
