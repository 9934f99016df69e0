"""Pins the oracle's layer prologue/epilogue (CPU).

The conv, norm, decay and gated-norm restatements are checked against forms
the mathematics fixes: identity conv taps, the conv window vs the rollback
gather, unit RMS after normalisation, the benchmark's decay special case
(A_log = 0, dt_bias = 0 gives exp(-softplus(a))), limits of silu, and a
planted mistake per piece.
"""
from __future__ import annotations

import numpy as np
import pytest


def _layer_inputs(rng, B=2, T=5, Hk=2, Hv=4, Dk=64, Dv=64, K=4):
    C = 2 * Hk * Dk + Hv * Dv
    return dict(
        qkv=rng.standard_normal((B, T, C)),
        conv_state=rng.standard_normal((B, K - 1, C)),
        conv_w=rng.standard_normal((C, K)) * 0.5,
        a=rng.standard_normal((B, T, Hv)),
        b=rng.standard_normal((B, T, Hv)),
        A_log=np.log(rng.uniform(0.5, 16, Hv)),
        dt_bias=rng.standard_normal(Hv),
        Hk=Hk, Hv=Hv, Dk=Dk, Dv=Dv,
    )


def test_identity_taps_give_silu_of_current_row(oracle):
    rng = np.random.default_rng(1)
    x = _layer_inputs(rng)
    x["conv_w"] = np.zeros_like(x["conv_w"])
    x["conv_w"][:, -1] = 1.0  # last tap multiplies the current token
    q, k, v, *_ = oracle.gdn_prologue(**x)
    B, T, C = x["qkv"].shape
    act = oracle.silu(x["qkv"])
    np.testing.assert_allclose(v.reshape(B, T, -1), act[..., 2 * 2 * 64:], rtol=0, atol=1e-12)


def test_first_tap_reads_the_conv_state(oracle):
    rng = np.random.default_rng(2)
    x = _layer_inputs(rng, T=2)
    x["conv_w"] = np.zeros_like(x["conv_w"])
    x["conv_w"][:, 0] = 1.0  # token t sees stream row t = conv_state row t
    _, _, v, *_ = oracle.gdn_prologue(**x)
    want = oracle.silu(x["conv_state"][:, :2, 256:])
    np.testing.assert_allclose(v.reshape(2, 2, -1), want, rtol=0, atol=1e-12)


def test_new_conv_window_equals_rollback_gather(oracle):
    rng = np.random.default_rng(3)
    for T in (1, 2, 5):
        x = _layer_inputs(rng, T=T)
        *_, new_state = oracle.gdn_prologue(**x)
        ref = oracle.conv_rollback(x["conv_state"], x["qkv"], [T] * 2)
        np.testing.assert_array_equal(new_state, ref)


def test_qk_have_unit_rms_times_scale(oracle):
    rng = np.random.default_rng(4)
    x = _layer_inputs(rng, Dk=128)
    q, k, *_ = oracle.gdn_prologue(**x, eps=0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(q * q, -1)), 128 ** -1.0, rtol=1e-12)
    np.testing.assert_allclose(np.sqrt(np.mean(k * k, -1)), 128 ** -0.5, rtol=1e-12)


def test_decay_special_cases(oracle):
    a = np.linspace(-8, 8, 33)
    np.testing.assert_allclose(oracle.compute_g(0.0, a, 0.0), np.exp(-np.log1p(np.exp(a))),
                               rtol=1e-13)
    assert np.all(oracle.compute_g(-50.0, a, 0.0) > 1 - 1e-12)   # exp(A_log) -> 0: no decay
    g = oracle.compute_g(np.log(2.0), np.array([0.0]), np.array([0.0]))
    np.testing.assert_allclose(g, np.exp(-2.0 * np.log(2.0)), rtol=1e-13)  # = 1/4


def test_gated_norm_limits(oracle):
    x = np.array([[3.0, -3.0, 3.0, -3.0]])
    w = np.array([1.0, 2.0, 1.0, 1.0])
    big = np.full_like(x, 40.0)
    y = oracle.gated_rmsnorm(x, big, w, eps=0.0)
    np.testing.assert_allclose(y, w * np.sign(x) * 40.0, rtol=1e-12)  # silu(40) ~ 40
    assert np.allclose(oracle.gated_rmsnorm(x, np.zeros_like(x), w), 0.0)  # silu(0) = 0


@pytest.mark.parametrize("mistake", ["flipped_taps", "k_scale_on_q", "no_softplus"])
def test_planted_prologue_mistakes_are_caught(oracle, mistake):
    rng = np.random.default_rng(5)
    x = _layer_inputs(rng)
    q, k, v, g, beta, _ = oracle.gdn_prologue(**x)
    y = dict(x)
    if mistake == "flipped_taps":
        y["conv_w"] = x["conv_w"][:, ::-1]
        _, _, v2, *_ = oracle.gdn_prologue(**y)
        assert np.max(np.abs(v2 - v)) > 1e-2
    elif mistake == "k_scale_on_q":
        assert np.max(np.abs(q * np.sqrt(64) - q)) > 1e-3  # Dk^-1 vs Dk^-1/2 differ
        np.testing.assert_allclose(np.sqrt(np.mean(q * q, -1)), 64 ** -1.0, rtol=1e-3)
    else:
        g2 = np.exp(-np.exp(x["A_log"]) * (x["a"] + x["dt_bias"]))
        assert np.max(np.abs(g2 - g)) > 1e-2


def test_decay_with_dt_bias_closed_form(oracle):
    """compute_g with dt_bias != 0: a = -dt_bias zeroes the softplus
    argument, so g = exp(-exp(A_log) * ln 2): 1/2 at A_log = 0, 1/8 at
    A_log = ln 3, whatever dt_bias is."""
    dt_bias = np.array([1.7, -0.6, 3.0, 0.25])
    a = -dt_bias
    np.testing.assert_allclose(oracle.compute_g(0.0, a, dt_bias), 0.5, rtol=1e-14)
    np.testing.assert_allclose(oracle.compute_g(np.log(3.0), a, dt_bias), 0.125, rtol=1e-14)
    # A planted sign slip, softplus(a - dt_bias), misses the closed form.
    slip = np.exp(-np.log1p(np.exp(a - dt_bias)))
    assert np.max(np.abs(slip - 0.5)) > 1e-2


def test_gated_norm_weight_hand_row(oracle):
    """RMSNormGated with a non-unit weight against a row worked by hand:
    x = [3, 4] has rms sqrt(12.5); silu(z) = z / (1 + e^-z)."""
    x = np.array([[3.0, 4.0]])
    z = np.array([[1.0, -2.0]])
    w = np.array([2.0, 0.5])
    r = np.sqrt(12.5)
    silu = z / (1 + np.exp(-z))
    want = np.array([[2.0 * 3.0 / r, 0.5 * 4.0 / r]]) * silu
    np.testing.assert_allclose(oracle.gated_rmsnorm(x, z, w, eps=0.0), want, rtol=1e-14)
    # A (1 + w) weight shift (a load-time transform of some checkpoints, never
    # applied at run time) misses the hand row.
    shifted = oracle.gated_rmsnorm(x, z, 1.0 + w, eps=0.0)
    assert np.max(np.abs(shifted - want)) > 1e-2
