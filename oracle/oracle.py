"""CPU oracle for the gated-delta verify hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the checker (or the timed
CPU baseline); the product package never imports it and has no CPU fallback.

What is here, each restating a piece of the reference (Aryagm/dflash-mlx):

* ``scan_c``: ctypes binding of gdn_oracle.c — the recurrence in the op order
  of dflash_mlx/custom_qwen35_model.py:129-139 (fp32, or fp64 accumulation),
  with ``out`` and the per-token state tape.
* ``scan_oploop``: numpy restatement of the same pure-op loop, vectorised over
  (B, Hv, Dv, Dk) the way the reference's MLX op loop is
  (custom_qwen35_model.py:129-139; mlx_lm gated_delta_ops is the same maths).
* ``scan_matrix_form``: an algebraically different statement of the same
  recurrence, S_t = S_{t-1} (g_t (I - beta_t k_t k_t^T)) + beta_t v_t k_t^T,
  computed with fp64 matrix products.  It shares no code with the loops, so a
  dropped term, a wrong sign or a transposed operand in either one fails the
  comparison.
* ``advance_gated_delta_states``: the replay contract of
  custom_qwen35_model.py:97-139 (keys already repeated to Hv heads).
* ``tape_select`` / ``conv_rollback``: the rollback gathers that replace the
  replay (custom_qwen35_model.py:1044-1051 for the conv window).
* ``longest_prefix_match`` (runtime.py:41-47) and ``greedy_accept``
  (runtime.py:22-29 argmax + :145-147 wiring).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle_gdn.so"

_lib = None


def build(force: bool = True) -> Path:
    """Compile gdn_oracle.c with gcc via oracle/Makefile."""
    cmd = ["make", "-C", str(ORACLE_DIR)] + (["-B"] if force else []) + ["liboracle_gdn.so"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}")
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build(force=False)
        L = ctypes.CDLL(str(LIB_PATH))
        fp = ctypes.POINTER(ctypes.c_float)
        dp = ctypes.POINTER(ctypes.c_double)
        ip = ctypes.POINTER(ctypes.c_int32)
        i = ctypes.c_int
        L.oracle_gdn_scan_f32.argtypes = [fp, fp, fp, fp, fp, fp, fp, fp, fp, ip, i, i, i, i, i, i]
        L.oracle_gdn_scan_f32.restype = i
        L.oracle_gdn_scan_f64.argtypes = [fp, fp, fp, fp, fp, fp, dp, dp, dp, ip, i, i, i, i, i, i]
        L.oracle_gdn_scan_f64.restype = i
        L.oracle_greedy_accept_f32.argtypes = [fp, ip, i, ip, ip, ip, i, i, i]
        L.oracle_greedy_accept_f32.restype = i
        L.oracle_num_threads.restype = i
        L.oracle_set_num_threads.argtypes = [i]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray | None, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def scan_c(q, k, v, g, beta, state, lengths=None, acc64: bool = False, with_out=True,
           with_tape=True, threads: int | None = None):
    """Scan via the C oracle.  Shapes: q,k [B,T,Hk,Dk]; v [B,T,Hv,Dv];
    g,beta [B,T,Hv]; state [B,Hv,Dv,Dk].  Returns (out [B,T,Hv,Dv] or None,
    final_state [B,Hv,Dv,Dk], tape [T,B,Hv,Dv,Dk] or None)."""
    k = _f32(k)
    v = _f32(v)
    g = _f32(g)
    beta = _f32(beta)
    state = _f32(state)
    B, T, Hk, Dk = k.shape
    Hv, Dv = v.shape[2], v.shape[3]
    qa = _f32(q) if (with_out and q is not None) else None
    dt = np.float64 if acc64 else np.float32
    out = np.zeros((B, T, Hv, Dv), dt) if qa is not None else None
    final = np.zeros((B, Hv, Dv, Dk), dt)
    tape = np.zeros((T, B, Hv, Dv, Dk), dt) if with_tape else None
    lens = None if lengths is None else np.ascontiguousarray(lengths, dtype=np.int32)
    L = lib()
    if threads is not None:
        L.oracle_set_num_threads(int(threads))
    fn = L.oracle_gdn_scan_f64 if acc64 else L.oracle_gdn_scan_f32
    ot = ctypes.c_double if acc64 else ctypes.c_float
    rc = fn(_ptr(qa, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
            _ptr(g, ctypes.c_float), _ptr(beta, ctypes.c_float), _ptr(state, ctypes.c_float),
            _ptr(out, ot), _ptr(final, ot), _ptr(tape, ot), _ptr(lens, ctypes.c_int32),
            B, T, Hk, Hv, Dk, Dv)
    if rc != 0:
        raise ValueError(f"oracle_gdn_scan rejected the shapes (rc={rc})")
    return out, final, tape


def _repeat_heads(x: np.ndarray, Hv: int) -> np.ndarray:
    """[B,T,Hk,D] -> [B,T,Hv,D] with value head hv reading key head hv // (Hv/Hk)
    (the mx.repeat(..., repeat_factor, axis=2) of custom_qwen35_model.py:1054-1057)."""
    Hk = x.shape[2]
    return np.repeat(x, Hv // Hk, axis=2)


def scan_oploop(q, k, v, g, beta, state, dtype=np.float64):
    """Vectorised op loop (custom_qwen35_model.py:129-139) plus out = S.q."""
    Hv = v.shape[2]
    kf = _repeat_heads(np.asarray(k, dtype), Hv)
    qf = _repeat_heads(np.asarray(q, dtype), Hv) if q is not None else None
    vf = np.asarray(v, dtype)
    gf = np.asarray(g, dtype)
    bf = np.asarray(beta, dtype)
    S = np.array(state, dtype=dtype, copy=True)
    B, T = kf.shape[:2]
    outs, tape = [], []
    for t in range(T):
        S = S * gf[:, t, :, None, None]
        kv_mem = np.sum(S * kf[:, t, :, None, :], axis=-1)
        delta = (vf[:, t] - kv_mem) * bf[:, t, :, None]
        S = S + delta[..., None] * kf[:, t, :, None, :]
        if qf is not None:
            outs.append(np.sum(S * qf[:, t, :, None, :], axis=-1))
        tape.append(S.copy())
    out = np.stack(outs, axis=1) if qf is not None else None
    tape_arr = np.stack(tape, axis=0) if T else np.zeros((0,) + S.shape, dtype)
    return out, S, tape_arr


def scan_matrix_form(q, k, v, g, beta, state):
    """fp64 matrix statement: S_t = S_{t-1} A_t + beta_t v_t k_t^T with
    A_t = g_t (I - beta_t k_t k_t^T); out_t = S_t q_t."""
    Hv = v.shape[2]
    kf = _repeat_heads(np.asarray(k, np.float64), Hv)
    qf = _repeat_heads(np.asarray(q, np.float64), Hv) if q is not None else None
    vf = np.asarray(v, np.float64)
    gf = np.asarray(g, np.float64)
    bf = np.asarray(beta, np.float64)
    S = np.array(state, dtype=np.float64, copy=True)  # [B,Hv,Dv,Dk]
    B, T, _, Dk = kf.shape
    eye = np.eye(Dk)
    outs, tape = [], []
    for t in range(T):
        kt = kf[:, t]                                   # [B,Hv,Dk]
        outer_kk = kt[..., :, None] * kt[..., None, :]  # [B,Hv,Dk,Dk]
        A = gf[:, t, :, None, None] * (eye - bf[:, t, :, None, None] * outer_kk)
        S = S @ A + bf[:, t, :, None, None] * (vf[:, t][..., :, None] * kt[..., None, :])
        if qf is not None:
            outs.append((S @ qf[:, t][..., :, None])[..., 0])
        tape.append(S.copy())
    out = np.stack(outs, axis=1) if qf is not None else None
    return out, S, (np.stack(tape, axis=0) if T else None)


def chunk_intermediates(k, v, g, beta, chunk: int = 64):
    """Per-chunk quantities of the chunked (WY / UT-transform) evaluation of
    the scan, fp64, for one head: k [T, Dk], v [T, Dv], g, beta [T].

    Per chunk of C tokens (the last one zero-padded: k = v = 0, beta = 0,
    g = 1) with G = cumsum(log g) and gamma = exp(G):
      A[i,j] = beta_i exp(G_i - G_j) k_i.k_j (j < i),  T = (I + A)^-1 by
      forward substitution, W = T diag(beta gamma) K, U~ = T diag(beta) V.
    Returns a list of dicts with G, W, Ut, K per chunk."""
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T_len, Dk = k.shape
    Dv = v.shape[1]
    res = []
    for c0 in range(0, T_len, chunk):
        n = min(chunk, T_len - c0)
        K = np.zeros((chunk, Dk)); V = np.zeros((chunk, Dv))
        bt = np.zeros(chunk); lg = np.zeros(chunk)
        K[:n] = k[c0:c0 + n]; V[:n] = v[c0:c0 + n]
        bt[:n] = beta[c0:c0 + n]; lg[:n] = np.log(np.asarray(g[c0:c0 + n], np.float64))
        G = np.cumsum(lg)
        i, j = np.indices((chunk, chunk))
        A = np.where(j < i, bt[:, None] * np.exp(G[:, None] - G[None, :]) * (K @ K.T), 0.0)
        Tm = np.zeros((chunk, chunk))
        for r in range(chunk):
            Tm[r] = -(A[r, :r] @ Tm[:r])
            Tm[r, r] = 1.0
        res.append(dict(n=n, G=G, K=K, W=Tm @ ((bt * np.exp(G))[:, None] * K),
                        Ut=Tm @ (bt[:, None] * V)))
    return res


def scan_chunked_form(q, k, v, g, beta, state, chunk: int = 64):
    """fp64 chunked statement of the scan (the evaluation order the chunked
    prefill kernel uses), returning (out, final_state).  Per chunk, from S0:
      U = U~ - W S0^T,  O = diag(gamma) Q S0^T + P U with
      P[i,j] = exp(G_i - G_j) q_i.k_j (j <= i),
      S = gamma_C S0 + (diag(exp(G_C - G)) U)^T K.
    Agrees with the token-by-token recurrence up to rounding; the CPU tests
    check that against scan_c and scan_matrix_form."""
    q = np.asarray(q, np.float64)
    B, T_len, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    rep = Hv // Hk
    out = np.zeros((B, T_len, Hv, Dv))
    fin = np.array(state, dtype=np.float64, copy=True)
    for b in range(B):
        for hv in range(Hv):
            hk = hv // rep
            S = fin[b, hv]
            chunks = chunk_intermediates(k[b, :, hk], v[b, :, hv], g[b, :, hv], beta[b, :, hv],
                                         chunk)
            for ci, ch in enumerate(chunks):
                c0, n, G = ci * chunk, ch["n"], ch["G"]
                Q = np.zeros((chunk, Dk))
                Q[:n] = q[b, c0:c0 + n, hk]
                i, j = np.indices((chunk, chunk))
                P = np.where(j <= i, np.exp(G[:, None] - G[None, :]) * (Q @ ch["K"].T), 0.0)
                U = ch["Ut"] - ch["W"] @ S.T
                O = np.exp(G)[:, None] * (Q @ S.T) + P @ U
                S = np.exp(G[-1]) * S + (np.exp(G[-1] - G)[:, None] * U).T @ ch["K"]
                out[b, c0:c0 + n, hv] = O[:n]
            fin[b, hv] = S
    return out, fin


def advance_gated_delta_states(initial_states, keys, values, g, beta):
    """Replay contract of custom_qwen35_model.py:97-139: keys are already
    repeated to Hv heads; returns the state after all keys.shape[1] tokens
    (fp32 compute, cast back to the state dtype as at :139)."""
    _, S, _ = scan_oploop(None, keys, values, g, beta, initial_states, dtype=np.float32)
    return S.astype(np.asarray(initial_states).dtype)


def tape_select(tape, state_in, accepted):
    """state after a_b tokens: tape[a_b-1, b] for a_b >= 1, else state_in[b]."""
    tape = np.asarray(tape)
    state_in = np.asarray(state_in)
    T = tape.shape[0]
    out = np.empty_like(state_in)
    for b, a in enumerate(np.asarray(accepted).tolist()):
        a = min(max(int(a), 0), T)
        out[b] = tape[a - 1, b] if a >= 1 else state_in[b]
    return out


def conv_rollback(conv_in, qkv, accepted):
    """concat(conv_in[b], qkv[b, :a], axis=0)[-K1:] per sequence
    (custom_qwen35_model.py:1044-1051)."""
    conv_in = np.asarray(conv_in)
    qkv = np.asarray(qkv)
    K1 = conv_in.shape[1]
    T = qkv.shape[1]
    out = np.empty_like(conv_in)
    for b, a in enumerate(np.asarray(accepted).tolist()):
        a = min(max(int(a), 0), T)
        out[b] = np.concatenate([conv_in[b], qkv[b, :a]], axis=0)[-K1:] if K1 else conv_in[b]
    return out


def longest_prefix_match(draft_tokens, verifier_tokens) -> int:
    """runtime.py:41-47: count of leading positions where the lists agree."""
    matched = 0
    for d, p in zip(draft_tokens, verifier_tokens):
        if d != p:
            break
        matched += 1
    return matched


def argmax_rows(logits) -> np.ndarray:
    """numpy argmax over the last axis: first maximum, NaN wins (first NaN)."""
    x = np.asarray(logits, dtype=np.float32)
    return np.argmax(x, axis=-1).astype(np.int32)


def greedy_accept(logits, draft):
    """logits [B,N,V], draft [B,n] -> (posterior [B,N], matched [B], bonus [B])."""
    post = argmax_rows(logits)
    draft = np.asarray(draft)
    B, N = post.shape
    matched = np.zeros(B, np.int32)
    bonus = np.zeros(B, np.int32)
    for b in range(B):
        m = longest_prefix_match(draft[b].tolist(), post[b].tolist())
        matched[b] = m
        bonus[b] = post[b, m] if m < N else -1
    return post, matched, bonus


def greedy_accept_c(logits, draft):
    """C oracle of greedy_accept (fp32 logits)."""
    lg = _f32(logits)
    B, N, V = lg.shape
    dr = np.ascontiguousarray(draft, dtype=np.int32).reshape(B, -1)
    n = dr.shape[1]
    post = np.zeros((B, N), np.int32)
    matched = np.zeros(B, np.int32)
    bonus = np.zeros(B, np.int32)
    rc = lib().oracle_greedy_accept_f32(_ptr(lg, ctypes.c_float), _ptr(dr, ctypes.c_int32), n,
                                        _ptr(post, ctypes.c_int32), _ptr(matched, ctypes.c_int32),
                                        _ptr(bonus, ctypes.c_int32), B, N, V)
    if rc != 0:
        raise ValueError(f"oracle_greedy_accept rejected the shapes (rc={rc})")
    return post, matched, bonus


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def bf16_round(x) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even), returned as fp32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


# ------------------------------------------------ gated-delta layer prologue

def silu(x):
    return x / (1.0 + np.exp(-x))


def softplus(x):
    return np.logaddexp(0.0, x)


def rms_norm(x, eps):
    """mx.fast.rms_norm(x, None, eps): x / sqrt(mean(x^2, -1) + eps)."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def compute_g(A_log, a, dt_bias):
    """mlx-lm compute_g (not vendored; the published Qwen3-Next decay):
    exp(-exp(A_log) * softplus(a + dt_bias))."""
    return np.exp(-np.exp(np.asarray(A_log, np.float64)) *
                  softplus(np.asarray(a, np.float64) + np.asarray(dt_bias, np.float64)))


def gdn_prologue(qkv, conv_state, conv_w, a, b, A_log, dt_bias, Hk, Hv, Dk, Dv, eps=1e-6):
    """fp64 restatement of custom_qwen35_model.py:431-450.

    qkv [B,T,C], conv_state [B,K-1,C], conv_w [C,K] (MLX [C,K,1] layout),
    a, b [B,T,Hv], A_log, dt_bias [Hv].  Returns (q [B,T,Hk,Dk],
    k [B,T,Hk,Dk], v [B,T,Hv,Dv], g, beta [B,T,Hv], new_conv_state)."""
    qkv = np.asarray(qkv, np.float64)
    st = np.asarray(conv_state, np.float64)
    w = np.asarray(conv_w, np.float64)
    B, T, C = qkv.shape
    K = w.shape[1]
    x = np.concatenate([st, qkv], axis=1)                    # [B, K-1+T, C]
    new_state = x[:, x.shape[1] - (K - 1):] if K > 1 else st
    conv = np.zeros((B, T, C))
    for j in range(K):                                        # cross-correlation, no flip
        conv += w[None, None, :, j] * x[:, j:j + T]
    act = silu(conv)
    kd = Hk * Dk
    q = act[..., :kd].reshape(B, T, Hk, Dk)
    k = act[..., kd:2 * kd].reshape(B, T, Hk, Dk)
    v = act[..., 2 * kd:].reshape(B, T, Hv, Dv)
    inv = Dk ** -0.5
    q = inv * inv * rms_norm(q, eps)
    k = inv * rms_norm(k, eps)
    g = compute_g(A_log, a, dt_bias)
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, np.float64)))
    return q, k, v, g, beta, new_state


def gated_rmsnorm(x, z, weight, eps=1e-6):
    """RMSNormGated (mlx-lm qwen3_next, not vendored; published Qwen3-Next
    form): weight * rms_norm(x) * silu(z) over the last axis."""
    x = np.asarray(x, np.float64)
    return np.asarray(weight, np.float64) * rms_norm(x, eps) * silu(np.asarray(z, np.float64))
