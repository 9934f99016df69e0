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


def test_rmsnorm_weight_hand_row():
    """nn.RMSNorm with a non-unit weight against a row worked by hand
    (x = [3, 4]: rms sqrt(12.5)), and the residual add before it.  The
    reference shifts norm weights by 1 only when loading some checkpoints
    (custom_qwen35_model.py:1156-1180); at run time y = w * x / rms, so a
    planted (1 + w) misses the row."""
    x = np.array([[3.0, 4.0]])
    w = np.array([2.0, 0.5])
    r = np.sqrt(12.5)
    want = np.array([[2.0 * 3.0 / r, 0.5 * 4.0 / r]])
    np.testing.assert_allclose(ho.rms_norm_w(x, w, 0.0), want, rtol=1e-14)
    h, y = ho.add_rmsnorm(np.array([[1.0, 5.0]]), np.array([[2.0, -1.0]]), w, 0.0)
    np.testing.assert_array_equal(h, [[3.0, 4.0]])
    np.testing.assert_allclose(y, want, rtol=1e-14)
    assert np.max(np.abs(ho.rms_norm_w(x, 1.0 + w, 0.0) - want)) > 1e-2


# ---------------------------------------------------------------- model wiring
from dflash_mlx.gdn_layer import GatedDeltaConfig  # noqa: E402
from dflash_mlx.hybrid_model import HybridConfig  # noqa: E402

TINY = HybridConfig(hidden_size=128, num_hidden_layers=4, intermediate_size=256, vocab_size=96,
                    num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                    linear=GatedDeltaConfig(linear_num_key_heads=1, linear_num_value_heads=2,
                                            linear_key_head_dim=64, linear_value_head_dim=64))


def _tiny_weights(rng, scale=0.05):
    cfg, lc = TINY, TINY.linear
    H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    bf = ho.bf16
    layers = []
    for i in range(cfg.num_hidden_layers):
        lw = {"ln_in": bf(1 + 0.2 * rng.standard_normal(H)),
              "ln_post": bf(1 + 0.2 * rng.standard_normal(H)),
              "w_gu": bf(scale * rng.standard_normal((2 * I, H))),
              "w_down": bf(scale * rng.standard_normal((H, I)))}
        if cfg.is_linear(i):
            lw.update(w_in=bf(scale * rng.standard_normal((cfg.in_proj_rows, H))),
                      w_out=bf(scale * rng.standard_normal((H, lc.value_dim))),
                      conv_w=bf(0.5 * rng.standard_normal((lc.conv_dim, lc.linear_conv_kernel_dim))),
                      A_log=np.log(rng.uniform(0.5, 8, lc.linear_num_value_heads)),
                      dt_bias=bf(rng.standard_normal(lc.linear_num_value_heads)),
                      norm_w=bf(1 + 0.2 * rng.standard_normal(lc.linear_value_head_dim)))
        else:
            lw.update(w_qkv=bf(scale * rng.standard_normal((cfg.attn_proj_rows, H))),
                      w_o=bf(scale * rng.standard_normal((H, cfg.num_attention_heads * D))),
                      q_norm=bf(1 + 0.2 * rng.standard_normal(D)),
                      k_norm=bf(1 + 0.2 * rng.standard_normal(D)))
        layers.append(lw)
    return dict(embed=bf(rng.standard_normal((cfg.vocab_size, H))),
                final_norm=bf(1 + 0.2 * rng.standard_normal(H)),
                lm_head=bf(scale * rng.standard_normal((cfg.vocab_size, H))), layers=layers)


def _empty_state(B=1):
    lc = TINY.linear
    return dict(lens=np.zeros(B, np.int64),
                conv=[np.zeros((B, lc.linear_conv_kernel_dim - 1, lc.conv_dim))] * TINY.n_linear,
                rec=[np.zeros((B, lc.linear_num_value_heads, lc.linear_value_head_dim,
                               lc.linear_key_head_dim))] * TINY.n_linear,
                k=[np.zeros((B, TINY.num_key_value_heads, 0, TINY.head_dim))] * TINY.n_attention,
                v=[np.zeros((B, TINY.num_key_value_heads, 0, TINY.head_dim))] * TINY.n_attention)


def _carry(state, res, T, conv_shift=0, lens_shift=0):
    """The caches after a model_step over T tokens (the runtime's
    all-accepted hand-off): conv windows advanced, recurrent state =
    tape[T-1], keys / values appended, lengths += T.  The shifts plant
    hand-off mistakes."""
    K1 = TINY.linear.linear_conv_kernel_dim - 1
    out = dict(lens=state["lens"] + T + lens_shift, conv=[], rec=[], k=[], v=[])
    for gi in range(TINY.n_linear):
        x = np.concatenate([state["conv"][gi], res["qkv"][gi]], axis=1)
        end = x.shape[1] - conv_shift
        out["conv"].append(x[:, end - K1:end])
        out["rec"].append(res["tape"][gi][T - 1])
    for ai in range(TINY.n_attention):
        out["k"].append(np.concatenate([state["k"][ai], res["k_new"][ai].transpose(0, 2, 1, 3)], 2))
        out["v"].append(np.concatenate([state["v"][ai], res["v_new"][ai].transpose(0, 2, 1, 3)], 2))
    return out


def test_model_step_zero_projections_pass_the_residual_through():
    """With every projection zero each layer adds nothing: the residual
    stream after every layer is the embedding row, the normed hidden is
    final_norm * rms_norm(embedding) and the logits are its LM-head
    product.  A dropped residual, a norm on the wrong stream or a missing
    final norm all break this."""
    rng = np.random.default_rng(11)
    w = _tiny_weights(rng)
    for lw in w["layers"]:
        for k in ("w_gu", "w_down", "w_in", "w_out", "w_qkv", "w_o"):
            if k in lw:
                lw[k] = np.zeros_like(lw[k])
    tokens = rng.integers(0, TINY.vocab_size, (2, 5))
    st = _empty_state(2)
    st["conv"] = [rng.standard_normal(c.shape) for c in st["conv"]]  # nonzero windows
    res = ho.model_step(TINY, w, st, tokens, 1e-6)
    emb = w["embed"][tokens]
    for lh in res["layer_hidden"]:
        np.testing.assert_array_equal(lh, emb)
    want = ho.rms_norm_w(emb, w["final_norm"], 1e-6)
    np.testing.assert_allclose(res["hidden"], ho.bf16(want), rtol=1e-14)  # rounded as the GPU
    np.testing.assert_allclose(res["logits"], ho.bf16(want) @ w["lm_head"].T, rtol=1e-12)


@pytest.mark.parametrize("split", [1, 3, 5])
def test_model_step_one_block_equals_two_blocks(split, oracle):
    """A block of 8 tokens in one model_step equals the same tokens in two
    steps with the caches carried between them (conv windows, recurrent
    state from the tape, keys / values and lengths): the layer wiring, the
    causal masks and the position offsets agree across the boundary."""
    rng = np.random.default_rng(12)
    w = _tiny_weights(rng)
    tokens = rng.integers(0, TINY.vocab_size, (1, 8))
    one = ho.model_step(TINY, w, _empty_state(), tokens, 1e-6)
    st0 = _empty_state()
    a = ho.model_step(TINY, w, st0, tokens[:, :split], 1e-6)
    b = ho.model_step(TINY, w, _carry(st0, a, split), tokens[:, split:], 1e-6)
    scale = np.max(np.abs(one["logits"]))
    for i in range(TINY.num_hidden_layers):
        got = np.concatenate([a["layer_hidden"][i], b["layer_hidden"][i]], axis=1)
        err = np.max(np.abs(got - one["layer_hidden"][i]))
        assert err <= 1e-6 * np.max(np.abs(one["layer_hidden"][i])), (i, err)
    got = np.concatenate([a["logits"], b["logits"]], axis=1)
    assert np.max(np.abs(got - one["logits"])) <= 1e-6 * scale  # (equal in fp64 here)


@pytest.mark.parametrize("mistake", ["conv_window", "kv_length"])
def test_model_step_split_catches_a_wrong_hand_off(mistake, oracle):
    rng = np.random.default_rng(12)
    w = _tiny_weights(rng)
    tokens = rng.integers(0, TINY.vocab_size, (1, 8))
    one = ho.model_step(TINY, w, _empty_state(), tokens, 1e-6)
    st0 = _empty_state()
    a = ho.model_step(TINY, w, st0, tokens[:, :3], 1e-6)
    bad = _carry(st0, a, 3, conv_shift=1 if mistake == "conv_window" else 0,
                 lens_shift=-1 if mistake == "kv_length" else 0)
    if mistake == "kv_length":  # the last key is overwritten at the wrong position
        bad["k"] = [k[:, :, :-1] for k in bad["k"]]
        bad["v"] = [v[:, :, :-1] for v in bad["v"]]
    b = ho.model_step(TINY, w, bad, tokens[:, 3:], 1e-6)
    got = np.concatenate([a["logits"], b["logits"]], axis=1)
    assert np.max(np.abs(got - one["logits"])) > 1e-2 * np.max(np.abs(one["logits"]))
