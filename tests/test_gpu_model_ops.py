"""GPU parity of the hybrid step's non-GEMM kernels against the CPU oracle, at
the config-c4 shapes (hidden 2560, MLP 9216, 16 query / 4 KV heads of 128,
a 4096-token cache) and ragged batches.

Tolerances: bf16 outputs within 2 bf16 ulps of the fp64 oracle's value
(|x - ref| <= 2^-7 |ref| + 1e-6, all arithmetic fp32 on the GPU); attention
output max-abs <= 2e-2 (bf16 output, fp32 softmax, bf16 P into the MFMA);
copies (V into the cache, the residual add) exact or within one ulp.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from dflash_mlx import _lib
from oracle import hybrid_oracle as ho

pytestmark = pytest.mark.gpu

ULP2 = 2.0 ** -7


def _np(x):
    return x.float().cpu().numpy().astype(np.float64)


def _within_ulps(got, ref, rel=ULP2, floor=1e-6):
    err = np.abs(got - ref)
    return float(np.max(err - (rel * np.abs(ref) + floor)))


@pytest.mark.parametrize("M,H,with_r", [(16, 2560, True), (16, 2560, False), (37, 1024, True),
                                        (3, 4096, True)])
def test_add_rmsnorm(device, M, H, with_r):
    gen = torch.Generator().manual_seed(M + H)
    x = torch.randn(M, H, generator=gen).bfloat16()
    r = torch.randn(M, H, generator=gen).bfloat16() if with_r else None
    w = (1 + 0.1 * torch.randn(H, generator=gen)).bfloat16()
    xd, wd = x.to(device), w.to(device)
    rd = r.to(device) if with_r else None
    h = torch.empty_like(xd)
    y = torch.empty_like(xd)
    print(f"[add_rmsnorm] M={M} H={H} r={with_r}", flush=True)
    _lib.call("dflash_add_rmsnorm", xd.data_ptr(), None if rd is None else rd.data_ptr(),
              wd.data_ptr(), h.data_ptr(), y.data_ptr(), M, H, 1e-6, _lib.stream_handle(device))
    torch.cuda.synchronize()
    h_ref, y_ref = ho.add_rmsnorm(_np(x), None if r is None else _np(r), _np(w), 1e-6)
    if with_r:
        # bf16(x + r): exact RNE of an fp32 sum that is itself exact for
        # nearby exponents; allow one ulp where double rounding can differ.
        hd = _np(h)
        assert np.mean(hd == h_ref) > 0.999
        assert _within_ulps(hd, h_ref, rel=2.0 ** -8) <= 0
    assert _within_ulps(_np(y), y_ref) <= 0


@pytest.mark.parametrize("M,I", [(16, 9216), (5, 512)])
def test_swiglu(device, M, I):
    gen = torch.Generator().manual_seed(I)
    gu = (2 * torch.randn(M, 2 * I, generator=gen)).bfloat16()
    out = torch.empty(M, I, dtype=torch.bfloat16, device=device)
    gd = gu.to(device)
    _lib.call("dflash_swiglu", gd.data_ptr(), out.data_ptr(), M, I, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert _within_ulps(_np(out), ho.swiglu(_np(gu))) <= 0


C4 = dict(Hq=16, Hkv=4, D=128, rot=32, base=100000.0)


def _attn_prep(device, B, T, lens, Smax, seed):
    Hq, Hkv, D = C4["Hq"], C4["Hkv"], C4["D"]
    rows = (2 * Hq + 2 * Hkv) * D
    gen = torch.Generator().manual_seed(seed)
    proj = torch.randn(B * T, rows, generator=gen).bfloat16()
    qn = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    kn = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    pd = proj.to(device)
    # device copies held in names: a temporary's pointer could be handed to
    # the next allocation before the kernel runs
    qnd, knd = qn.to(device), kn.to(device)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=device)
    kc = torch.zeros(B, Hkv, Smax, D, dtype=torch.bfloat16, device=device)
    vtc = torch.zeros(B, Hkv, D, Smax, dtype=torch.bfloat16, device=device)
    q = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=device)
    _lib.call("dflash_attn_prep", pd.data_ptr(), rows, qnd.data_ptr(),
              knd.data_ptr(), lens_d.data_ptr(), kc.data_ptr(), vtc.data_ptr(),
              q.data_ptr(), None, B, T, Hq, Hkv, D, Smax, C4["rot"], C4["base"], 1e-6,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    ref = ho.attn_prep(_np(proj), _np(qn), _np(kn), np.array(lens), B, T, Hq, Hkv, D, C4["rot"],
                       C4["base"], 1e-6)
    return q, kc, vtc, ref, proj


@pytest.mark.parametrize("B,T,lens", [(1, 16, [4096]), (2, 16, [0, 1000]), (3, 5, [7, 63, 64]),
                                    (1, 200, [37]), (2, 130, [0, 4001]), (1, 64, [3000])])
def test_attn_prep_norm_rope_and_cache_append(device, B, T, lens):
    """q / k normed and rotated, V copied into the transposed cache at
    lens[b] + t, nothing else written; T >= 64 takes the value heads through
    64-token tiles (a last partial tile, odd start positions)."""
    Smax = 4160
    print(f"[attn_prep] B={B} T={T} lens={lens}", flush=True)
    q, kc, vtc, (q_ref, k_ref, v_ref, _), _ = _attn_prep(device, B, T, lens, Smax, seed=B * 7 + T)
    assert _within_ulps(_np(q), q_ref) <= 0
    kc_np, vtc_np = _np(kc), _np(vtc)
    for b in range(B):
        p0 = lens[b]
        got_k = kc_np[b, :, p0:p0 + T].transpose(1, 0, 2)        # [T, Hkv, D]
        assert _within_ulps(got_k, k_ref[b]) <= 0
        got_v = vtc_np[b, :, :, p0:p0 + T].transpose(2, 0, 1)    # [T, Hkv, D]
        assert np.array_equal(got_v, v_ref[b])                   # a copy
        # nothing else written
        mask = np.ones(Smax, bool)
        mask[p0:p0 + T] = False
        assert np.all(kc_np[b][:, mask] == 0) and np.all(vtc_np[b][:, :, mask] == 0)


@pytest.mark.parametrize("B,T,lens", [(1, 16, [4096]), (2, 16, [37, 1000]), (2, 7, [0, 130])])
def test_attn_verify(device, B, T, lens):
    Hq, Hkv, D = C4["Hq"], C4["Hkv"], C4["D"]
    Smax = 4160
    print(f"[attn_verify] B={B} T={T} lens={lens}", flush=True)
    gen = torch.Generator().manual_seed(B * 100 + T)
    k = torch.randn(B, Hkv, Smax, D, generator=gen).bfloat16()
    v = torch.randn(B, Hkv, Smax, D, generator=gen).bfloat16()
    q = torch.randn(B, T, Hq, D, generator=gen).bfloat16()
    rows = (2 * Hq + 2 * Hkv) * D
    proj = torch.randn(B * T, rows, generator=gen).bfloat16()
    kd, vtd = k.to(device), v.transpose(2, 3).contiguous().to(device)
    qd, pd = q.to(device), proj.to(device)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=device)
    out = torch.empty(B * T, Hq * D, dtype=torch.bfloat16, device=device)
    lib = _lib.load()
    for max_len in (Smax, max(lens) + T):
        ws = torch.empty(int(lib.dflash_attn_verify_workspace_bytes(B, Hq, Hkv, max_len)),
                         dtype=torch.uint8, device=device)
        _lib.call("dflash_attn_verify", qd.data_ptr(), kd.data_ptr(), vtd.data_ptr(),
                  lens_d.data_ptr(), pd.data_ptr(), rows, out.data_ptr(), B, T, Hq, Hkv, D, Smax,
                  max_len, D ** -0.5, ws.data_ptr(), ws.numel(), _lib.stream_handle(device))
        torch.cuda.synchronize()
        gate = _np(proj).reshape(B, T, -1)[..., :2 * Hq * D].reshape(B, T, Hq, 2 * D)[..., D:]
        ref = ho.attention_verify(_np(q), _np(k), _np(v), np.array(lens), gate, D ** -0.5)
        err = float(np.max(np.abs(_np(out).reshape(B, T, -1) - ref)))
        print(f"  max_len={max_len}: out max-abs {err:.3e} (|ref| max {np.max(np.abs(ref)):.3f})",
              flush=True)
        assert err <= 2e-2


def test_attn_verify_rejects_bad_arguments(device):
    lib = _lib.load()
    rc = lib.dflash_attn_verify(None, None, None, None, None, 0, None, 1, 17, 16, 4, 128, 4160,
                                4160, 0.1, None, 0, None)
    assert rc == -2  # T > 16
    rc = lib.dflash_attn_verify(None, None, None, None, None, 0, None, 1, 16, 16, 4, 128, 4100,
                                4100, 0.1, None, 0, None)
    assert rc == -2  # Smax % 64
    rc = lib.dflash_attn_verify(None, None, None, None, None, 0, None, 1, 16, 16, 4, 64, 4160,
                                4160, 0.1, None, 0, None)
    assert rc == -3  # head dim


def test_commit_accept(device):
    matched = torch.tensor([0, 3, 15, 99, -4], dtype=torch.int32, device=device)
    keep = torch.empty(5, dtype=torch.int32, device=device)
    lens = torch.tensor([10, 10, 10, 10, 10], dtype=torch.int32, device=device)
    _lib.call("dflash_commit_accept", matched.data_ptr(), keep.data_ptr(), lens.data_ptr(), 5, 16,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert keep.cpu().tolist() == [1, 4, 16, 16, 1]
    assert lens.cpu().tolist() == [11, 14, 26, 26, 11]


@pytest.mark.parametrize("nsplit", [1, 2, 3, 5, 8, 11])
def test_add_rmsnorm_splitk_every_split_count(device, nsplit):
    """The compile-time split counts (1..8) and the generic loop (11) sum the
    partials in split order, as dflash_splitk_reduce does: bit-identical to
    the bf16-branch kernel fed that reduce."""
    M, H = 16, 2560
    g = torch.Generator(device=device).manual_seed(nsplit)
    part = torch.randn(nsplit, M, H, generator=g, device=device)
    x = torch.randn(M, H, generator=g, device=device).bfloat16()
    w = (1 + 0.1 * torch.randn(H, generator=g, device=device)).bfloat16()
    r = torch.empty(M, H, dtype=torch.bfloat16, device=device)
    st = _lib.stream_handle(device)
    _lib.call("dflash_splitk_reduce", part.data_ptr(), nsplit, M, H, r.data_ptr(), H, st)
    h1, y1 = x.clone(), torch.empty_like(x)
    h2, y2 = x.clone(), torch.empty_like(x)
    _lib.call("dflash_add_rmsnorm_splitk", h1.data_ptr(), part.data_ptr(), nsplit, w.data_ptr(),
              h1.data_ptr(), y1.data_ptr(), M, H, 1e-6, st)
    _lib.call("dflash_add_rmsnorm", h2.data_ptr(), r.data_ptr(), w.data_ptr(), h2.data_ptr(),
              y2.data_ptr(), M, H, 1e-6, st)
    torch.cuda.synchronize()
    assert torch.equal(h1, h2) and torch.equal(y1, y2)


def test_add_rmsnorm_widest_row(device):
    M, H = 4, 8192
    gen = torch.Generator().manual_seed(81)
    x = torch.randn(M, H, generator=gen).bfloat16()
    r = torch.randn(M, H, generator=gen).bfloat16()
    w = (1 + 0.1 * torch.randn(H, generator=gen)).bfloat16()
    xd, rd, wd = x.to(device), r.to(device), w.to(device)
    h = torch.empty_like(xd)
    y = torch.empty_like(xd)
    _lib.call("dflash_add_rmsnorm", xd.data_ptr(), rd.data_ptr(), wd.data_ptr(), h.data_ptr(),
              y.data_ptr(), M, H, 1e-6, _lib.stream_handle(device))
    torch.cuda.synchronize()
    h_ref, y_ref = ho.add_rmsnorm(_np(x), _np(r), _np(w), 1e-6)
    assert _within_ulps(_np(h), h_ref, rel=2.0 ** -8) <= 0
    assert _within_ulps(_np(y), y_ref) <= 0
    lib = _lib.load()
    assert lib.dflash_add_rmsnorm(None, None, None, None, None, 1, 8200, 1e-6, None) == -2


def test_embed_rmsnorm(device):
    """Embedding lookup folded into the first norm: h = table[tokens] exactly,
    y as the oracle's RMSNorm of those rows; ids out of range clamp."""
    V, H = 1000, 2560
    gen = torch.Generator().manual_seed(5)
    table = (0.02 * torch.randn(V, H, generator=gen)).bfloat16()
    w = (1 + 0.1 * torch.randn(H, generator=gen)).bfloat16()
    tokens = torch.tensor([0, 999, 17, 123, -5, 1000, 4242, 500], dtype=torch.int32)
    td, wd, tokd = table.to(device), w.to(device), tokens.to(device)
    M = tokens.numel()
    h = torch.empty(M, H, dtype=torch.bfloat16, device=device)
    y = torch.empty_like(h)
    _lib.call("dflash_embed_rmsnorm", td.data_ptr(), tokd.data_ptr(), V, wd.data_ptr(), h.data_ptr(),
              y.data_ptr(), M, H, 1e-6, _lib.stream_handle(device))
    torch.cuda.synchronize()
    ids = tokens.clamp(0, V - 1).long()
    assert torch.equal(h.cpu(), table[ids])
    _, y_ref = ho.add_rmsnorm(_np(table[ids]), None, _np(w), 1e-6)
    assert _within_ulps(_np(y), y_ref) <= 0
