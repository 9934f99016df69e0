"""Pins the chunked (WY / UT-transform) statement of the scan on the CPU.

The chunked prefill kernel evaluates the recurrence of
dflash_mlx/custom_qwen35_model.py:129-139 in a different order (64-token
chunks, token-token products, a triangular inverse).  Its fp64 restatement,
oracle.scan_chunked_form, must agree with both independent sequential
statements (the C op loop and the fp64 matrix form) to fp64 rounding, across
chunk boundaries, partial last chunks, GQA and strong decays; the triangular
inverse must be an inverse; and a planted mistake in the chunk algebra (a
dropped decay, an off-by-one mask) must fail the comparison.
"""
from __future__ import annotations

import numpy as np
import pytest



def _rand_inputs(rng, B, T, Hk, Hv, Dk, Dv, state_std=0.3):
    q = rng.standard_normal((B, T, Hk, Dk))
    k = rng.standard_normal((B, T, Hk, Dk))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, Dv))
    g = np.exp(-np.log1p(np.exp(rng.standard_normal((B, T, Hv)))))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))
    s0 = state_std * rng.standard_normal((B, Hv, Dv, Dk))
    return tuple(x.astype(np.float32) for x in (q, k, v, g, beta, s0))


def _max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("shape", [
    dict(B=1, T=200, Hk=2, Hv=4, Dk=16, Dv=8),    # 3 full chunks + a partial one
    dict(B=2, T=64, Hk=1, Hv=2, Dk=8, Dv=8),      # exactly one chunk
    dict(B=1, T=1, Hk=1, Hv=1, Dk=4, Dv=4),       # a single token
    dict(B=1, T=129, Hk=1, Hv=1, Dk=32, Dv=16),   # one token past two chunks
])
def test_chunked_form_matches_sequential_fp64(oracle, shape):
    rng = np.random.default_rng(5)
    ins = _rand_inputs(rng, **shape)
    out_c, fin_c, _ = oracle.scan_c(*ins, acc64=True)
    out_k, fin_k = oracle.scan_chunked_form(*ins)
    assert _max_rel(out_k, out_c) < 1e-10
    assert _max_rel(fin_k, fin_c) < 1e-10
    if shape["T"] <= 64:
        out_m, fin_m, _ = oracle.scan_matrix_form(*ins)
        assert _max_rel(fin_k, fin_m) < 1e-10


def test_chunked_form_strong_decay_and_zero_state(oracle):
    """g near 0 underflows gamma over a chunk: the form must stay finite."""
    rng = np.random.default_rng(6)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=150, Hk=1, Hv=2, Dk=16, Dv=16)
    g = np.where(rng.random(g.shape) < 0.3, 1e-12, g).astype(np.float32)
    s0 = np.zeros_like(s0)
    out_c, fin_c, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    out_k, fin_k = oracle.scan_chunked_form(q, k, v, g, beta, s0)
    assert np.all(np.isfinite(out_k)) and np.all(np.isfinite(fin_k))
    assert _max_rel(out_k, out_c) < 1e-9
    assert _max_rel(fin_k, fin_c) < 1e-9


def test_triangular_inverse(oracle):
    """(I + A) U~ = diag(beta) V with A rebuilt entry by entry here."""
    rng = np.random.default_rng(7)
    q, k, v, g, beta, _ = _rand_inputs(rng, B=1, T=100, Hk=1, Hv=1, Dk=16, Dv=8)
    chunks = oracle.chunk_intermediates(k[0, :, 0], v[0, :, 0], g[0, :, 0], beta[0, :, 0])
    assert len(chunks) == 2 and chunks[1]["n"] == 36
    for ci, ch in enumerate(chunks):
        c0, n, G, K = ci * 64, ch["n"], ch["G"], ch["K"]
        btv = np.zeros(64)
        btv[:n] = beta[0, c0:c0 + n, 0]
        V = np.zeros((64, 8))
        V[:n] = v[0, c0:c0 + n, 0]
        A = np.zeros((64, 64))
        for r in range(64):
            for c in range(r):
                A[r, c] = btv[r] * np.exp(G[r] - G[c]) * float(K[r] @ K[c])
        lhs = (np.eye(64) + A) @ ch["Ut"]
        assert np.max(np.abs(lhs - btv[:, None] * V)) < 1e-10


@pytest.mark.parametrize("kind", ["no_gamma_in_W", "halved_delta", "no_state_decay"])
def test_planted_chunk_mistakes_are_caught(oracle, kind, monkeypatch):
    rng = np.random.default_rng(8)
    ins = _rand_inputs(rng, B=1, T=100, Hk=1, Hv=2, Dk=8, Dv=8)
    out_c, fin_c, _ = oracle.scan_c(*ins, acc64=True)
    orig = oracle.chunk_intermediates

    def broken(k, v, g, beta, chunk=64):
        res = orig(k, v, g, beta, chunk)
        for ch in res:
            if kind == "no_gamma_in_W":
                ch["W"] = ch["W"] / np.maximum(np.exp(ch["G"])[:, None], 1e-300)
            elif kind == "halved_delta":
                ch["Ut"] = ch["Ut"] * 0.5
            elif kind == "no_state_decay":
                ch["G"] = np.zeros_like(ch["G"])
        return res

    monkeypatch.setattr(oracle, "chunk_intermediates", broken)
    out_k, fin_k = oracle.scan_chunked_form(*ins)
    assert _max_rel(out_k, out_c) > 1e-4 or _max_rel(fin_k, fin_c) > 1e-4
