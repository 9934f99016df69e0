"""Pins the hybrid-model oracle (oracle/hybrid_oracle.py) on the CPU.

The reference's attention, MLP and norms are MLX / mlx-lm code that cannot run
here, so each restatement is pinned by what the mathematics fixes:

* rotary: equal to the complex-product statement; identity at position 0;
  norm-preserving; scores depend only on the position difference; the
  non-interleaved pairing (i, i + dims/2) is told apart from the interleaved
  one (i, i + 1);
* attention: the vectorised masked softmax equals a query-by-query online
  softmax; all-zero queries give the mean of the visible values; a query that
  sees one key returns that key's value; an off-by-one causal mask is caught;
* RMSNorm: unit RMS output, invariance to input scale; SwiGLU closed forms.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import hybrid_oracle as ho


@pytest.mark.parametrize("dims", [16, 32, 64, 128])
def test_rope_equals_complex_form(dims):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 5, 128))
    pos = rng.integers(0, 5000, size=(3, 5))
    a = ho.rope(x, pos, dims, 100000.0)
    b = ho.rope_complex(x, pos, dims, 100000.0)
    assert np.max(np.abs(a - b)) < 1e-12
    assert np.array_equal(a[..., dims:], x[..., dims:])


def test_rope_identity_at_zero_and_norm_preserving():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 128))
    assert np.max(np.abs(ho.rope(x, np.zeros(4), 32, 1e5) - x)) == 0.0
    y = ho.rope(x, np.arange(4) * 997, 32, 1e5)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), atol=1e-12)


def test_rope_scores_depend_on_position_difference_only():
    rng = np.random.default_rng(3)
    q, k = rng.standard_normal(128), rng.standard_normal(128)
    s1 = ho.rope(q, np.array(40), 32, 1e5) @ ho.rope(k, np.array(13), 32, 1e5)
    s2 = ho.rope(q, np.array(4040), 32, 1e5) @ ho.rope(k, np.array(4013), 32, 1e5)
    assert abs(s1 - s2) < 1e-9 * (1 + abs(s1))


def test_rope_half_split_pairing_is_not_interleaved():
    """A feature pair (0, 16) rotates together for dims = 32; (0, 1) does not."""
    x = np.zeros(128)
    x[0] = 1.0
    y = ho.rope(x, np.array(1), 32, 1e5)  # angle 1 rad on pair (0, 16)
    assert abs(y[0] - np.cos(1.0)) < 1e-12 and abs(y[16] - np.sin(1.0)) < 1e-12
    assert y[1] == 0.0


def _attn_case(rng, B=2, T=5, Hq=4, Hkv=2, D=8, S=40, lens=(3, 17)):
    q = rng.standard_normal((B, T, Hq, D))
    k = rng.standard_normal((B, Hkv, S, D))
    v = rng.standard_normal((B, Hkv, S, D))
    gate = rng.standard_normal((B, T, Hq, D))
    return q, k, v, np.array(lens), gate


def test_attention_vectorised_equals_online_loop():
    rng = np.random.default_rng(4)
    q, k, v, lens, gate = _attn_case(rng)
    a = ho.attention_verify(q, k, v, lens, gate, 8 ** -0.5)
    b = ho.attention_verify_loop(q, k, v, lens, gate, 8 ** -0.5)
    assert np.max(np.abs(a - b)) < 1e-12


def test_attention_zero_queries_average_visible_values():
    rng = np.random.default_rng(5)
    q, k, v, lens, gate = _attn_case(rng)
    q[:] = 0.0
    gate[:] = 50.0  # sigmoid -> 1
    out = ho.attention_verify(q, k, v, lens, gate, 1.0).reshape(q.shape)
    for b in range(2):
        for t in range(5):
            n = lens[b] + t + 1
            for h in range(4):
                assert np.allclose(out[b, t, h], v[b, h // 2, :n].mean(axis=0), atol=1e-12)


def test_attention_single_visible_key():
    rng = np.random.default_rng(6)
    q, k, v, _, gate = _attn_case(rng)
    lens = np.array([0, 0])
    out = ho.attention_verify(q, k, v, lens, gate, 0.3).reshape(q.shape)
    sig = 1 / (1 + np.exp(-gate))
    assert np.allclose(out[:, 0], v[:, [0, 0, 1, 1], 0] * sig[:, 0], atol=1e-12)


def test_attention_off_by_one_mask_is_caught(monkeypatch):
    rng = np.random.default_rng(7)
    q, k, v, lens, gate = _attn_case(rng)
    good = ho.attention_verify(q, k, v, lens, gate, 0.4)

    def leaky(q, k_cache, v_cache, lens, gate, scale):  # query t also sees key lens+t+1
        q = np.asarray(q, np.float64)
        B, T, Hq, D = q.shape
        rep = Hq // k_cache.shape[1]
        out = np.zeros((B, T, Hq, D))
        for b in range(B):
            L = int(lens[b]) + T
            for h in range(Hq):
                s = scale * q[b, :, h] @ k_cache[b, h // rep, :L].T
                mask = np.arange(L)[None, :] <= (int(lens[b]) + np.arange(T) + 1)[:, None]
                s = np.where(mask, s, -np.inf)
                p = np.exp(s - s.max(1, keepdims=True))
                out[b, :, h] = (p / p.sum(1, keepdims=True)) @ v_cache[b, h // rep, :L]
        return (out / (1 + np.exp(-gate))).reshape(B, T, Hq * D)

    bad = leaky(q, k, v, lens, gate, 0.4)
    assert np.max(np.abs(bad - good)) > 1e-3


def test_rmsnorm_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 256))
    y = ho.rms_norm_w(x, np.ones(256), 0.0)
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=1e-12)
    assert np.allclose(ho.rms_norm_w(7.5 * x, np.ones(256), 0.0), y, atol=1e-12)
    h, y2 = ho.add_rmsnorm(x, -x, np.ones(256), 1e-6)
    assert np.all(h == 0.0) and np.all(y2 == 0.0)


def test_swiglu_closed_forms():
    g = np.array([0.0, 30.0, -30.0, 1.0])
    u = np.array([5.0, 2.0, 3.0, 4.0])
    out = ho.swiglu(np.concatenate([g, u]))
    assert out[0] == 0.0
    assert abs(out[1] - 60.0) < 1e-9
    assert abs(out[2]) < 1e-10
    assert abs(out[3] - 4.0 / (1 + np.exp(-1.0))) < 1e-12
