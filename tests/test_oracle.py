"""Pins the CPU oracle before it is trusted as the parity checker.

The reference ships no numeric tests, golden vectors or fixtures for this path
(its tests/ only check imports, CLI parsing and server JSON), and its maths
runs only under MLX on Apple GPUs, which this image cannot import.  So every
oracle function here is pinned by what the mathematics fixes:

* two independent restatements must agree: the C op loop (reference op order,
  custom_qwen35_model.py:129-139) and the fp64 matrix form
  S_t = S_{t-1} g_t (I - beta_t k_t k_t^T) + beta_t v_t k_t^T;
* closed forms: g=1,beta=0 leaves S unchanged; g=0 gives S_1 = beta v k^T;
  S_0=0, beta=1, |k|=1 gives S_1 = v k^T and out_1 = v (k.q); a hand-written
  T=1 formula;
* invariants: tape[T-1] == final state; tape[a-1] == replay of the first a
  tokens (the reference's rollback equivalence); GQA head mapping equals an
  explicit repeat of the key heads;
* planted mistakes (in the oracle, on the CPU) must fail those checks, which
  shows the checks can tell.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx.workloads import CONFIGS, make_accept_inputs, make_scan_inputs


def _rand_inputs(rng, B=2, T=5, Hk=2, Hv=4, Dk=8, Dv=6, state_std=0.3, unit=True):
    q = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32)
    k = rng.standard_normal((B, T, Hk, Dk)).astype(np.float32)
    if unit:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, Hv, Dv)).astype(np.float32)
    g = np.exp(-np.log1p(np.exp(rng.standard_normal((B, T, Hv))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, Hv))))).astype(np.float32)
    s0 = (state_std * rng.standard_normal((B, Hv, Dv, Dk))).astype(np.float32)
    return q, k, v, g, beta, s0


def _max_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("shape", [
    dict(B=2, T=5, Hk=2, Hv=4, Dk=8, Dv=6),
    dict(B=1, T=16, Hk=4, Hv=4, Dk=64, Dv=64),
    dict(B=1, T=3, Hk=1, Hv=3, Dk=12, Dv=5),
])
def test_c_oploop_matches_matrix_form_fp64(oracle, shape):
    rng = np.random.default_rng(11)
    ins = _rand_inputs(rng, **shape)
    out_c, fin_c, tape_c = oracle.scan_c(*ins, acc64=True)
    out_m, fin_m, tape_m = oracle.scan_matrix_form(*ins)
    assert _max_rel(fin_c, fin_m) < 1e-12
    assert _max_rel(tape_c, tape_m) < 1e-12
    assert _max_rel(out_c, out_m) < 1e-12


def test_numpy_oploop_matches_c(oracle):
    rng = np.random.default_rng(12)
    ins = _rand_inputs(rng, B=2, T=7, Hk=2, Hv=4, Dk=16, Dv=8)
    o1, f1, t1 = oracle.scan_c(*ins, acc64=True)
    o2, f2, t2 = oracle.scan_oploop(*ins, dtype=np.float64)
    assert _max_rel(f1, f2) < 1e-12 and _max_rel(t1, t2) < 1e-12 and _max_rel(o1, o2) < 1e-12


def test_fp32_oracle_close_to_fp64(oracle):
    cfg = CONFIGS[0]
    x = make_scan_inputs(cfg)
    ins = [x[n].float().numpy() for n in ("q", "k", "v", "g", "beta", "state")]
    o32, f32, t32 = oracle.scan_c(*ins, acc64=False)
    o64, f64, t64 = oracle.scan_c(*ins, acc64=True)
    assert _max_rel(f32, f64) < 1e-5
    assert _max_rel(t32, t64) < 1e-5
    assert np.max(np.abs(o32 - o64)) < 1e-5


def test_closed_form_identity_step(oracle):
    """g = 1, beta = 0: the state never changes and out_t = S0 q_t."""
    rng = np.random.default_rng(13)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=4, Hk=2, Hv=2, Dk=8, Dv=8)
    g[:] = 1.0
    beta[:] = 0.0
    out, fin, tape = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    np.testing.assert_array_equal(fin, s0.astype(np.float64))
    for t in range(4):
        np.testing.assert_array_equal(tape[t], s0.astype(np.float64))
        ref = np.einsum("bhvk,bhk->bhv", s0.astype(np.float64), q[:, t].astype(np.float64))
        np.testing.assert_allclose(out[:, t], ref, rtol=0, atol=1e-12)


def test_closed_form_full_decay(oracle):
    """g = 0 forgets the state: S_1 = beta v k^T whatever S_0 is."""
    rng = np.random.default_rng(14)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=1, Hk=1, Hv=2, Dk=8, Dv=4)
    g[:] = 0.0
    _, fin, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    kk = np.repeat(k, 2, axis=2)[0, 0].astype(np.float64)
    expect = beta[0, 0, :, None, None] * v[0, 0][:, :, None].astype(np.float64) * kk[:, None, :]
    np.testing.assert_allclose(fin[0], expect, rtol=0, atol=1e-12)


def test_closed_form_unit_key_write(oracle):
    """S_0 = 0, beta = 1, |k| = 1: S_1 = v k^T and out_1 = v (k . q)."""
    rng = np.random.default_rng(15)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=1, Hk=1, Hv=1, Dk=16, Dv=8)
    beta[:] = 1.0
    s0[:] = 0.0
    out, fin, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    k64, q64, v64 = (a[0, 0, 0].astype(np.float64) for a in (k, q, v))
    np.testing.assert_allclose(fin[0, 0], np.outer(v64, k64), rtol=0, atol=1e-7)
    np.testing.assert_allclose(out[0, 0, 0], v64 * (k64 @ q64), rtol=0, atol=1e-7)


def test_closed_form_single_token_by_hand(oracle):
    """T = 1 written out: S1 = g S0 + beta (v - g S0 k) k^T, out = S1 q."""
    rng = np.random.default_rng(16)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=1, Hk=1, Hv=1, Dk=6, Dv=3, unit=False)
    out, fin, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    S0 = s0[0, 0].astype(np.float64)
    kk, qq, vv = (a[0, 0, 0].astype(np.float64) for a in (k, q, v))
    gg, bb = float(g[0, 0, 0]), float(beta[0, 0, 0])
    S1 = gg * S0 + bb * np.outer(vv - gg * S0 @ kk, kk)
    np.testing.assert_allclose(fin[0, 0], S1, rtol=0, atol=1e-12)
    np.testing.assert_allclose(out[0, 0, 0], S1 @ qq, rtol=0, atol=1e-12)


def test_tape_invariants_and_replay_equivalence(oracle):
    """final == tape[T-1]; tape[a-1] == replay(S0, first a tokens), which is
    the reference's rollback contract (custom_qwen35_model.py:1053-1074)."""
    rng = np.random.default_rng(17)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=2, T=6, Hk=2, Hv=4, Dk=8, Dv=8)
    _, fin, tape = oracle.scan_c(q, k, v, g, beta, s0)
    np.testing.assert_array_equal(fin, tape[-1])
    for a in range(1, 7):
        kr = np.repeat(k[:, :a], 2, axis=2)  # the reference repeats keys to Hv heads
        rep = oracle.advance_gated_delta_states(s0, kr, v[:, :a], g[:, :a], beta[:, :a])
        assert _max_rel(rep, tape[a - 1]) < 1e-6
        lens = np.full(2, a, np.int32)
        _, fin_a, _ = oracle.scan_c(None, k, v, g, beta, s0, lengths=lens, with_out=False,
                                    with_tape=False)
        np.testing.assert_array_equal(fin_a, tape[a - 1])


def test_gqa_mapping_equals_explicit_repeat(oracle):
    rng = np.random.default_rng(18)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=4, Hk=2, Hv=6, Dk=8, Dv=8)
    o1, f1, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    o2, f2, _ = oracle.scan_c(np.repeat(q, 3, axis=2), np.repeat(k, 3, axis=2), v, g, beta, s0,
                              acc64=True)
    np.testing.assert_array_equal(f1, f2)
    np.testing.assert_array_equal(o1, o2)
    # A different mapping (hv % Hk instead of hv // rep) must not match.
    kw = np.tile(k, (1, 1, 3, 1))
    qw = np.tile(q, (1, 1, 3, 1))
    o3, f3, _ = oracle.scan_c(qw, kw, v, g, beta, s0, acc64=True)
    assert _max_rel(f3, f1) > 1e-2


def _mutant_scan(q, k, v, g, beta, s0, kind):
    """The matrix form with one planted mistake (oracle-side, CPU only)."""
    Hv = v.shape[2]
    rep = Hv // k.shape[2]
    kf = np.repeat(k.astype(np.float64), rep, axis=2)
    qf = np.repeat(q.astype(np.float64), rep, axis=2)
    S = s0.astype(np.float64).copy()
    outs = []
    for t in range(k.shape[1]):
        kt, qt, vt = kf[:, t], qf[:, t], v[:, t].astype(np.float64)
        gt, bt = g[:, t, :, None, None].astype(np.float64), beta[:, t, :, None, None]
        if kind == "no_decay":
            gt = np.ones_like(gt)
        kv = np.einsum("bhvk,bhk->bhv", gt * S, kt)
        d = (vt - kv) * bt[..., 0]
        if kind == "sign":
            d = (vt + kv) * bt[..., 0]
        S = gt * S + d[..., :, None] * kt[..., None, :]
        if kind == "q_for_k":
            outs.append(np.einsum("bhvk,bhk->bhv", S, kt))
        else:
            outs.append(np.einsum("bhvk,bhk->bhv", S, qt))
    return np.stack(outs, axis=1), S


@pytest.mark.parametrize("kind", ["no_decay", "sign", "q_for_k"])
def test_planted_mistakes_are_caught(oracle, kind):
    rng = np.random.default_rng(19)
    ins = _rand_inputs(rng, B=1, T=6, Hk=2, Hv=4, Dk=16, Dv=16)
    out_ok, fin_ok, _ = oracle.scan_matrix_form(*ins)
    out_bad, fin_bad = _mutant_scan(*ins, kind)
    worst = max(_max_rel(fin_bad, fin_ok), _max_rel(out_bad, out_ok))
    assert worst > 1e-2, f"planted mistake {kind} went unnoticed"


def test_transposed_state_is_caught(oracle):
    """With Dk != Dv the state orientation is a shape fact; with Dk == Dv a
    transposed state gives different numbers."""
    rng = np.random.default_rng(20)
    q, k, v, g, beta, s0 = _rand_inputs(rng, B=1, T=3, Hk=1, Hv=1, Dk=8, Dv=8)
    _, f_ok, _ = oracle.scan_c(q, k, v, g, beta, s0, acc64=True)
    _, f_tr, _ = oracle.scan_c(q, k, v, g, beta, np.swapaxes(s0, -1, -2).copy(), acc64=True)
    assert _max_rel(np.swapaxes(f_tr, -1, -2), f_ok) > 1e-2


# ---------------------------------------------------------------- accept

def test_accept_known_answer_config0(oracle):
    cfg = CONFIGS[0]
    acc = make_accept_inputs(cfg)
    logits = acc["logits"].numpy()
    draft = acc["draft"].numpy()
    post, matched, bonus = oracle.greedy_accept(logits, draft)
    assert matched.tolist() == [7]
    assert bonus[0] == int(np.argmax(logits[0, 7]))
    post_c, matched_c, bonus_c = oracle.greedy_accept_c(logits, draft)
    np.testing.assert_array_equal(post, post_c)
    assert matched_c.tolist() == [7] and bonus_c.tolist() == bonus.tolist()


def test_accept_reference_wiring(oracle):
    """runtime.py:145-147: compare block[1:] with posterior[:-1]; bonus is
    posterior[matched]; accepted_inputs = matched + 1 in [1, T]."""
    rng = np.random.default_rng(21)
    T, V = 16, 300
    for a_true in range(0, T):
        logits = rng.standard_normal((1, T, V)).astype(np.float32)
        post = np.argmax(logits[0], axis=-1)
        block = [5] + [int(post[i]) if i < a_true else int((post[i] + 1) % V) for i in range(T - 1)]
        matched = oracle.longest_prefix_match(block[1:], post[:-1].tolist())
        assert matched == a_true
        _, m_c, b_c = oracle.greedy_accept_c(logits, np.array([block[1:]], np.int32))
        assert m_c[0] == matched and b_c[0] == post[matched]


def test_accept_ties_nan_and_signed_zero(oracle):
    V = 64
    logits = np.zeros((1, 4, V), np.float32)
    logits[0, 0, [3, 9, 40]] = 2.0                 # tie -> lowest index 3
    logits[0, 1, :] = -0.0
    logits[0, 1, 5] = 0.0                          # -0 == +0 -> index 0
    logits[0, 2, [7, 30]] = np.nan                 # first NaN wins
    logits[0, 2, 1] = np.inf
    logits[0, 3, :] = -np.inf                      # all -inf -> 0
    post, _, _ = oracle.greedy_accept(logits, np.zeros((1, 0), np.int32))
    assert post[0].tolist() == [3, 0, 7, 0]
    post_c, _, _ = oracle.greedy_accept_c(logits, np.zeros((1, 0), np.int32))
    assert post_c[0].tolist() == [3, 0, 7, 0]


def test_accept_matched_equals_n_gives_no_bonus(oracle):
    logits = np.random.default_rng(22).standard_normal((2, 3, 10)).astype(np.float32)
    post = np.argmax(logits, axis=-1).astype(np.int32)
    _, m, b = oracle.greedy_accept_c(logits, post)
    assert m.tolist() == [3, 3] and b.tolist() == [-1, -1]


# ------------------------------------------------------------- rollback

def test_tape_select_semantics(oracle):
    rng = np.random.default_rng(23)
    T, B = 5, 3
    tape = rng.standard_normal((T, B, 2, 3, 4)).astype(np.float32)
    s0 = rng.standard_normal((B, 2, 3, 4)).astype(np.float32)
    out = oracle.tape_select(tape, s0, [0, 3, 5])
    np.testing.assert_array_equal(out[0], s0[0])
    np.testing.assert_array_equal(out[1], tape[2, 1])
    np.testing.assert_array_equal(out[2], tape[4, 2])


def test_conv_rollback_semantics(oracle):
    """Row r of the window is stream row a + r of [conv_in; qkv]."""
    B, K1, T, C = 2, 3, 6, 5
    conv = np.arange(B * K1 * C, dtype=np.float32).reshape(B, K1, C)
    qkv = 1000 + np.arange(B * T * C, dtype=np.float32).reshape(B, T, C)
    for a in range(0, T + 1):
        out = oracle.conv_rollback(conv, qkv, [a, a])
        stream = np.concatenate([conv, qkv], axis=1)
        np.testing.assert_array_equal(out, stream[:, a:a + K1])


def test_bf16_round_matches_torch(oracle):
    x = np.random.default_rng(24).standard_normal(10000).astype(np.float32) * 50
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ours = oracle.bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, ref)
