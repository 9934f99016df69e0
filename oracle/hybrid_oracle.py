"""CPU oracle for the hybrid target's verify step (config c4).

TEST INFRASTRUCTURE ONLY.  Only tests/ (and bench.py's cpu_baseline leg) may
import this module, and only as the checker; the product package never
imports it and has no CPU fallback.

Restates, in numpy (fp64 arithmetic, bf16 rounding where the GPU path rounds),
the pieces of the Qwen3.5 hybrid target's forward that surround the gated
delta layers:

* ``rms_norm_w``: nn.RMSNorm (custom_qwen35_model.py:824-827) — x *
  rsqrt(mean(x^2) + eps) * w;
* ``add_rmsnorm``: DecoderLayer's residual add then norm (:841-845);
* ``swiglu``: mlx-lm Qwen3NextMLP's silu(gate) * up (not vendored; the
  published SwiGLU MLP), called at :845;
* ``rope``: nn.RoPE(dims, traditional=False, base) on the first ``dims``
  features (non-interleaved halves), as Qwen3NextAttention applies it at the
  cache offset (:519-520);
* ``attn_prep`` / ``attention_verify``: forward_full_attention_layer_explicit
  (:487-540): q/k RMSNorm, rotary, KV append, causal SDPA over the cache
  (query t of the block sees keys 0 .. offset + t), output * sigmoid(gate);
* ``model_step``: the whole verify step of a (small) hybrid model built from
  the above and the gated-delta oracle (oracle.py), for end-to-end parity.
  Run over a whole generated sequence at once (teacher forcing), it checks
  each greedy choice of a decode (the reference's exactness gate compares
  DFlash output with plain greedy generation, ADDING_MODELS.md:76-137).
"""
from __future__ import annotations

import numpy as np

from . import oracle as gdn


def bf16(x):
    return gdn.bf16_round(np.asarray(x, np.float64)).astype(np.float64)


def rms_norm_w(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def add_rmsnorm(x, r, w, eps):
    """(h, y): h = bf16(x + r) (x alone when r is None), y = rms_norm_w(h)."""
    h = np.asarray(x, np.float64) if r is None else bf16(np.asarray(x, np.float64) + r)
    return h, rms_norm_w(h, w, eps)


def silu(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def swiglu(gate_up):
    gu = np.asarray(gate_up, np.float64)
    inter = gu.shape[-1] // 2
    return silu(gu[..., :inter]) * gu[..., inter:]


def rope(x, pos, dims, base):
    """nn.RoPE(dims, traditional=False, base): x [..., D] at integer positions
    pos (broadcast over the leading axes).  Feature i < dims/2 pairs with
    i + dims/2 at angle pos * base^(-2i/dims)."""
    x = np.asarray(x, np.float64)
    if dims == 0:
        return x.copy()
    half = dims // 2
    inv = base ** (-2.0 * np.arange(half) / dims)
    ang = np.asarray(pos, np.float64)[..., None] * inv
    c, s = np.cos(ang), np.sin(ang)
    out = x.copy()
    a, b = x[..., :half], x[..., half:dims]
    out[..., :half] = a * c - b * s
    out[..., half:dims] = b * c + a * s
    return out


def rope_complex(x, pos, dims, base):
    """The same rotation written as a complex product (x_i + i x_{i+half}) *
    exp(i * angle): an independent statement used to pin ``rope``."""
    x = np.asarray(x, np.float64)
    if dims == 0:
        return x.copy()
    half = dims // 2
    z = x[..., :half] + 1j * x[..., half:dims]
    ang = np.asarray(pos, np.float64)[..., None] * base ** (-2.0 * np.arange(half) / dims)
    z = z * np.exp(1j * ang)
    out = x.copy()
    out[..., :half] = z.real
    out[..., half:dims] = z.imag
    return out


def attn_prep(proj, q_norm_w, k_norm_w, lens, B, T, Hq, Hkv, D, rot, base, eps):
    """proj [B*T, >= (2Hq + 2Hkv) D] -> (q [B,T,Hq,D], k [B,T,Hkv,D],
    v [B,T,Hkv,D], gate [B,T,Hq,D]), q/k normed and rotated at lens[b] + t."""
    proj = np.asarray(proj, np.float64).reshape(B, T, -1)
    qg = proj[..., :2 * Hq * D].reshape(B, T, Hq, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = proj[..., 2 * Hq * D:2 * Hq * D + Hkv * D].reshape(B, T, Hkv, D)
    v = proj[..., 2 * Hq * D + Hkv * D:2 * Hq * D + 2 * Hkv * D].reshape(B, T, Hkv, D)
    pos = np.asarray(lens)[:, None] + np.arange(T)[None, :]  # [B, T]
    q = rope(rms_norm_w(q, q_norm_w, eps), pos[:, :, None], rot, base)
    k = rope(rms_norm_w(k, k_norm_w, eps), pos[:, :, None], rot, base)
    return q, k, v, gate


def attention_verify(q, k_cache, v_cache, lens, gate, scale):
    """q [B,T,Hq,D]; k_cache/v_cache [B,Hkv,S,D] holding lens[b] + T valid
    positions; gate [B,T,Hq,D].  Returns [B, T, Hq*D]:
    softmax(scale q k^T) v * sigmoid(gate), query t seeing keys <= lens+t."""
    q = np.asarray(q, np.float64)
    B, T, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    rep = Hq // Hkv
    out = np.zeros((B, T, Hq, D))
    for b in range(B):
        L = int(lens[b]) + T
        for h in range(Hq):
            kk = np.asarray(k_cache[b, h // rep, :L], np.float64)
            vv = np.asarray(v_cache[b, h // rep, :L], np.float64)
            s = scale * q[b, :, h] @ kk.T                       # [T, L]
            mask = np.arange(L)[None, :] <= (int(lens[b]) + np.arange(T))[:, None]
            s = np.where(mask, s, -np.inf)
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, h] = p @ vv
    sig = 1.0 / (1.0 + np.exp(-np.asarray(gate, np.float64)))
    return (out * sig).reshape(B, T, Hq * D)


def attention_verify_loop(q, k_cache, v_cache, lens, gate, scale):
    """Query-by-query restatement of attention_verify (explicit visible-key
    range, running max and sum): a second formulation that pins it."""
    q = np.asarray(q, np.float64)
    B, T, Hq, D = q.shape
    rep = Hq // k_cache.shape[1]
    out = np.zeros((B, T, Hq * D))
    for b in range(B):
        for t in range(T):
            n_vis = int(lens[b]) + t + 1
            for h in range(Hq):
                m, l, acc = -np.inf, 0.0, np.zeros(D)
                for j in range(n_vis):
                    sj = scale * float(q[b, t, h] @ np.asarray(k_cache[b, h // rep, j], np.float64))
                    m_new = max(m, sj)
                    c = np.exp(m - m_new) if np.isfinite(m) else 0.0
                    w = np.exp(sj - m_new)
                    l = l * c + w
                    acc = acc * c + w * np.asarray(v_cache[b, h // rep, j], np.float64)
                    m = m_new
                g = 1.0 / (1.0 + np.exp(-np.asarray(gate[b, t, h], np.float64)))
                out[b, t, h * D:(h + 1) * D] = acc / l * g
    return out


def model_step(cfg, weights, state, tokens, eps=1e-6):
    """One verify step of a hybrid model through the final norm and greedy
    accept, mirroring the GPU runner's rounding points (bf16 after every GEMM
    and every kernel output).

    cfg: the runner's HybridConfig; weights: dict of numpy arrays (fp64 values
    of the bf16 weights); state: dict with 'conv' [Lg][B,K-1,C], 'rec'
    [Lg][B,Hv,Dv,Dk], 'k'/'v' [La][B,Hkv,S,D], 'lens' [B]; tokens [B, T].
    Returns dict(hidden [B,T,H] (final normed), posterior, matched, bonus,
    qkv [Lg][B,T,C], k_new/v_new [La][B,T,Hkv,D], tape [Lg][T,B,Hv,Dv,Dk],
    layer_hidden [L][B,T,H] (the residual stream after each layer, what
    forward_dflash captures at layer_ids, custom_qwen35_model.py:984-991)).
    The gated-delta q/k RMSNorm uses eps 1e-6 whatever ``eps`` is
    (custom_qwen35_model.py:446-447); ``eps`` sets every other norm."""
    lc = cfg.linear
    B, T = tokens.shape
    H = cfg.hidden_size
    h = weights["embed"][tokens.reshape(-1)].reshape(B * T, H)
    r = None
    res = dict(qkv=[], tape=[], k_new=[], v_new=[], layer_hidden=[])
    gi = ai = 0
    for i in range(cfg.num_hidden_layers):
        lw = weights["layers"][i]
        h, x = add_rmsnorm(h, r, lw["ln_in"], eps)
        x = bf16(x)
        if cfg.is_linear(i):
            proj = bf16(x @ lw["w_in"].T)
            C, Hv, Dv = lc.conv_dim, lc.linear_num_value_heads, lc.linear_value_head_dim
            qkv = proj[:, :C].reshape(B, T, C)
            z = proj[:, C:C + Hv * Dv].reshape(B, T, Hv, Dv)
            bb = proj[:, C + Hv * Dv:C + Hv * Dv + Hv].reshape(B, T, Hv)
            aa = proj[:, C + Hv * Dv + Hv:C + Hv * Dv + 2 * Hv].reshape(B, T, Hv)
            q, k, v, g, beta, _ = gdn.gdn_prologue(
                qkv, state["conv"][gi], lw["conv_w"], aa, bb, lw["A_log"], lw["dt_bias"],
                lc.linear_num_key_heads, Hv, lc.linear_key_head_dim, Dv, 1e-6)
            q, k, v = bf16(q), bf16(k), bf16(v)
            out, _, tape = gdn.scan_c(q, k, v, g, beta, state["rec"][gi], acc64=True)
            y = bf16(gdn.gated_rmsnorm(bf16(out), z, lw["norm_w"], eps))
            r = bf16(y.reshape(B * T, Hv * Dv) @ lw["w_out"].T)
            res["qkv"].append(qkv)
            res["tape"].append(tape)
            gi += 1
        else:
            D, Hq, Hkv = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
            proj = bf16(x @ lw["w_qkv"].T)
            q, k, v, gate = attn_prep(proj, lw["q_norm"], lw["k_norm"], state["lens"], B, T, Hq,
                                      Hkv, D, cfg.rot_dims, cfg.rope_theta, eps)
            q, k = bf16(q), bf16(k)
            k0 = np.asarray(state["k"][ai], np.float64)
            S = max(k0.shape[2], int(np.max(state["lens"])) + T)
            kc = np.zeros(k0.shape[:2] + (S, D))
            vc = np.zeros(k0.shape[:2] + (S, D))
            kc[:, :, :k0.shape[2]] = k0
            vc[:, :, :k0.shape[2]] = state["v"][ai]
            for b in range(B):
                p0 = int(state["lens"][b])
                kc[b, :, p0:p0 + T] = k[b].transpose(1, 0, 2)
                vc[b, :, p0:p0 + T] = v[b].transpose(1, 0, 2)
            o = bf16(attention_verify(q, kc, vc, state["lens"], gate, D ** -0.5))
            r = bf16(o.reshape(B * T, Hq * D) @ lw["w_o"].T)
            res["k_new"].append(k)
            res["v_new"].append(v)
            ai += 1
        h, x = add_rmsnorm(h, r, lw["ln_post"], eps)
        x = bf16(x)
        act = bf16(swiglu(x @ lw["w_gu"].T))  # gating fused into the gate|up GEMM: one rounding
        r = bf16(act @ lw["w_down"].T)
        res["layer_hidden"].append(bf16(h + r).reshape(B, T, H))
    h, x = add_rmsnorm(h, r, weights["final_norm"], eps)
    x = bf16(x)
    logits = x @ weights["lm_head"].T
    posterior = logits.reshape(B, T, -1).argmax(-1)
    matched = np.array([gdn.longest_prefix_match(tokens[b, 1:], posterior[b, :-1]) for b in range(B)])
    bonus = posterior[np.arange(B), matched]
    res.update(hidden=x.reshape(B, T, H), logits=logits.reshape(B, T, -1), posterior=posterior,
               matched=matched, bonus=bonus)
    return res

