"""GPU parity of the gated-delta layer prologue / epilogue and the composite
layer verify (prologue -> scan -> gated norm) against the fp64 CPU oracle.

Tolerances: bf16 outputs within 1e-2 of the reference's max |value|
(bf16 keeps 8 mantissa bits: 2^-8 ~ 4e-3 relative); fp32 g/beta within
1e-5 relative; the new conv window bit-exact (a copy); the layer output y
within the verify tolerance, max-abs 2e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import _lib
from dflash_mlx.adapters import rollback_linear_caches
from dflash_mlx.cache import ArraysCache
from dflash_mlx.gdn_layer import (
    GatedDeltaConfig,
    GatedDeltaWeights,
    gated_rmsnorm,
    gdn_layer_verify,
    gdn_prologue,
)

pytestmark = pytest.mark.gpu


def _inputs(cfg: GatedDeltaConfig, B, T, seed):
    gen = torch.Generator().manual_seed(seed)
    C, K, Hv = cfg.conv_dim, cfg.linear_conv_kernel_dim, cfg.linear_num_value_heads
    qkv = torch.randn(B, T, C, generator=gen).bfloat16()
    conv_state = torch.randn(B, K - 1, C, generator=gen).bfloat16()
    a = torch.randn(B, T, Hv, generator=gen).bfloat16()
    b = torch.randn(B, T, Hv, generator=gen).bfloat16()
    z = torch.randn(B, T, Hv * cfg.linear_value_head_dim, generator=gen).bfloat16()
    w = GatedDeltaWeights.random(cfg, "cpu", gen)
    w.norm_weight = (1 + 0.1 * torch.randn(cfg.linear_value_head_dim, generator=gen)).bfloat16()
    w.dt_bias = (torch.randn(Hv, generator=gen) * 0.5).bfloat16()
    return dict(qkv=qkv, conv_state=conv_state, a=a, b=b, z=z), w


def _w_dev(w, dev):
    return GatedDeltaWeights(*(t.to(dev) for t in (w.conv_weight, w.A_log, w.dt_bias, w.norm_weight)))


def _oracle_prologue(oracle, x, w, cfg):
    f = lambda t: t.float().numpy()
    return oracle.gdn_prologue(f(x["qkv"]), f(x["conv_state"]), f(w.conv_weight), f(x["a"]),
                               f(x["b"]), w.A_log.numpy(), f(w.dt_bias),
                               cfg.linear_num_key_heads, cfg.linear_num_value_heads,
                               cfg.linear_key_head_dim, cfg.linear_value_head_dim,
                               cfg.rms_norm_eps)


def _rel_max(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


CFGS = [
    (GatedDeltaConfig(), 2, 16),                                        # Qwen3.5-4B shape
    (GatedDeltaConfig(), 1, 1),
    (GatedDeltaConfig(), 3, 2),                                         # T < K-1
    (GatedDeltaConfig(linear_num_key_heads=16, linear_num_value_heads=64,
                      linear_key_head_dim=192, linear_value_head_dim=128), 1, 16),
    (GatedDeltaConfig(linear_num_key_heads=2, linear_num_value_heads=4,
                      linear_key_head_dim=64, linear_value_head_dim=64,
                      linear_conv_kernel_dim=2), 2, 5),
]


@pytest.mark.parametrize("cfg,B,T", CFGS, ids=lambda x: str(x) if not isinstance(x, GatedDeltaConfig)
                         else f"Hk{x.linear_num_key_heads}Dk{x.linear_key_head_dim}K{x.linear_conv_kernel_dim}")
def test_prologue_matches_oracle(oracle, device, cfg, B, T):
    x, w = _inputs(cfg, B, T, seed=B * 100 + T)
    print(f"[prologue {cfg} B={B} T={T}]", flush=True)
    q, k, v, g, beta, new_conv = gdn_prologue(x["qkv"].to(device), x["conv_state"].to(device),
                                              x["a"].to(device), x["b"].to(device),
                                              _w_dev(w, device), cfg)
    torch.cuda.synchronize()
    rq, rk, rv, rg, rb, rst = _oracle_prologue(oracle, x, w, cfg)
    for name, got, ref in (("q", q, rq), ("k", k, rk), ("v", v, rv)):
        err = _rel_max(got.float().cpu().numpy(), ref)
        assert err <= 1e-2, f"{name}: {err}"
    assert _rel_max(g.cpu().numpy(), rg) <= 1e-5
    assert _rel_max(beta.cpu().numpy(), rb) <= 1e-5
    np.testing.assert_array_equal(new_conv.float().cpu().numpy(), rst)


@pytest.mark.parametrize("zoff", [0, 1])
@pytest.mark.parametrize("B,T,H,D", [(2, 16, 32, 128), (1, 3, 5, 64), (1, 16, 7, 192), (2, 1, 3, 256),
                                     (1, 161, 32, 128), (1, 129, 40, 64), (2, 33, 64, 256),
                                     (1, 100, 41, 192)])
def test_gated_rmsnorm_matches_oracle(oracle, device, B, T, H, D, zoff):
    """Every compiled channel count (D / 64 = 1..4), rows not a multiple of the
    rows per workgroup, the gate as a strided view of a wider projection row.
    Launches of 4096 rows or more with zoff = 0 (16-byte aligned rows and
    gates) take the 16-byte form (D = 64, 128, 256), the rest and zoff = 1
    (the gate one element off) the one-wave-a-row form."""
    gen = torch.Generator().manual_seed(7 + D)
    print(f"[gated_rmsnorm B={B} T={T} H={H} D={D} zoff={zoff}]", flush=True)
    x = torch.randn(B, T, H, D, generator=gen).bfloat16()
    zfull = torch.randn(B, T, H * D + 64, generator=gen).bfloat16()
    z = zfull[..., zoff:zoff + H * D].unflatten(-1, (H, D))  # strided view, as out of a projection
    wgt = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    y = gated_rmsnorm(x.to(device), zfull.to(device)[..., zoff:zoff + H * D].unflatten(-1, (H, D)),
                      wgt.to(device), 1e-6)
    torch.cuda.synchronize()
    ref = oracle.gated_rmsnorm(x.float().numpy(), z.float().numpy(), wgt.float().numpy(), 1e-6)
    assert _rel_max(y.float().cpu().numpy(), ref) <= 1e-2


def test_layer_verify_and_rollback(oracle, device):
    cfg = GatedDeltaConfig()
    B, T = 2, 16
    x, w = _inputs(cfg, B, T, seed=11)
    gen = torch.Generator().manual_seed(12)
    Hv, Dv, Dk = cfg.linear_num_value_heads, cfg.linear_value_head_dim, cfg.linear_key_head_dim
    state = 0.05 * torch.randn(B, Hv, Dv, Dk, generator=gen)
    d = {kk: t.to(device) for kk, t in x.items()}
    y, new_conv, final, tape, record = gdn_layer_verify(
        d["qkv"], d["z"], d["a"], d["b"], d["conv_state"], state.to(device), _w_dev(w, device), cfg)
    torch.cuda.synchronize()
    # Oracle: prologue (fp64), q/k/v rounded to bf16 as the scan's interface,
    # fp64 scan, fp64 gated norm.
    rq, rk, rv, rg, rb, rst = _oracle_prologue(oracle, x, w, cfg)
    bf = lambda t: oracle.bf16_round(np.asarray(t, np.float32))
    out, fin, tp = oracle.scan_c(bf(rq), bf(rk), bf(rv), rg, rb, state.numpy(), acc64=True)
    ref_y = oracle.gated_rmsnorm(bf(out), x["z"].float().numpy().reshape(B, T, Hv, Dv),
                                 w.norm_weight.float().numpy(), cfg.rms_norm_eps).reshape(B, T, -1)
    # y = weight * rms_norm(out) * silu(z) reaches |y| ~ 8, so one bf16 ulp of
    # out is ~3e-2 absolute in y: y is held to the relative bf16 bound, and
    # the scan's own out to the verify contract (max-abs 2e-2).
    y_err = _rel_max(y.float().cpu().numpy(), ref_y)
    fin_err = _rel_max(final.cpu().numpy(), fin)
    from dflash_mlx import gated_delta_verify
    from dflash_mlx.gdn_layer import gdn_prologue as _pro
    q, k, v, g, beta, _ = _pro(d["qkv"], d["conv_state"], d["a"], d["b"], _w_dev(w, device), cfg)
    out_gpu, _, _ = gated_delta_verify(q, k, v, g, beta, state.to(device))
    out_err = float(np.max(np.abs(out_gpu.float().cpu().numpy() - out)))
    print(f"[layer] y rel {y_err:.3e} out max-abs {out_err:.3e} final rel {fin_err:.3e}", flush=True)
    assert y_err <= 1e-2
    assert out_err <= 2e-2
    assert fin_err <= 1e-3
    np.testing.assert_array_equal(new_conv.float().cpu().numpy(), rst)
    # The record rolls the layer back to any accepted length.
    cache = [ArraysCache(2)]
    cache[0][0], cache[0][1] = new_conv, final
    acc = torch.tensor([3, 16], dtype=torch.int32, device=device)
    rollback_linear_caches(cache, {0: record}, acc)
    torch.cuda.synchronize()
    ref_conv = oracle.conv_rollback(x["conv_state"].float().numpy(), x["qkv"].float().numpy(), [3, 16])
    np.testing.assert_array_equal(cache[0][0].float().cpu().numpy(), ref_conv)
    assert torch.equal(cache[0][1][0], tape[2, 0]) and torch.equal(cache[0][1][1], tape[15, 1])


def test_prologue_rejects_aliasing_and_bad_dims(device):
    cfg = GatedDeltaConfig(linear_num_key_heads=1, linear_num_value_heads=1,
                           linear_key_head_dim=48, linear_value_head_dim=64)
    x, w = _inputs(cfg, 1, 2, seed=1)
    with pytest.raises(_lib.DFlashError):
        gdn_prologue(x["qkv"].to(device), x["conv_state"].to(device), x["a"].to(device),
                     x["b"].to(device), _w_dev(w, device), cfg)


FUSED_CFGS = [
    (GatedDeltaConfig(), 2, 16),                                        # Qwen3.5-4B shape
    (GatedDeltaConfig(), 1, 1),
    (GatedDeltaConfig(), 3, 2),                                         # T < K-1
    (GatedDeltaConfig(), 1, 32),                                        # the largest block
    (GatedDeltaConfig(linear_num_key_heads=4, linear_num_value_heads=16,
                      linear_conv_kernel_dim=2), 2, 7),                 # 4 value heads per key head
    (GatedDeltaConfig(linear_num_key_heads=2, linear_num_value_heads=2,
                      linear_value_head_dim=64, linear_conv_kernel_dim=8), 1, 9),
]


@pytest.mark.parametrize("inplace", [False, True], ids=["tape_out", "tape_in_place"])
@pytest.mark.parametrize("cfg,B,T", FUSED_CFGS, ids=lambda x: str(x) if not isinstance(x, GatedDeltaConfig)
                         else f"Hk{x.linear_num_key_heads}Hv{x.linear_num_value_heads}"
                              f"Dv{x.linear_value_head_dim}K{x.linear_conv_kernel_dim}")
def test_fused_prologue_scan_matches_two_calls(device, cfg, B, T, inplace):
    """dflash_gdn_prologue_scan_rollback gives the bits of dflash_gdn_prologue
    + dflash_gdn_verify_scan_rollback: out, tape and the rolled-back state,
    with q/k/v/a/b read as strided views of projection rows."""
    from dflash_mlx import gated_delta_verify_rollback
    from dflash_mlx.gdn_layer import gdn_prologue_verify_rollback

    print(f"[fused prologue+scan {cfg} B={B} T={T} inplace={inplace}]", flush=True)
    x, w = _inputs(cfg, B, T, seed=B * 1000 + T)
    C, Hv = cfg.conv_dim, cfg.linear_num_value_heads
    Dk, Dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    gen = torch.Generator().manual_seed(T + 77)
    rows = C + 2 * Hv + 6
    proj = torch.randn(B, T, rows, generator=gen).bfloat16()
    proj[..., :C] = x["qkv"]
    proj[..., C:C + Hv] = x["b"]
    proj[..., C + Hv:C + 2 * Hv] = x["a"]
    proj = proj.to(device)
    qkv, bb, aa = proj[..., :C], proj[..., C:C + Hv], proj[..., C + Hv:C + 2 * Hv]
    conv_state = x["conv_state"].to(device)
    wd = _w_dev(w, device)
    prev_T = T if inplace else 5
    state0 = (0.05 * torch.randn(B, Hv, Dv, Dk, generator=gen)).to(device)
    tape0 = (0.05 * torch.randn(prev_T, B, Hv, Dv, Dk, generator=gen)).to(device)
    acc = torch.tensor([0, 3, prev_T][:B], dtype=torch.int32, device=device)

    st_a, tp_a = state0.clone(), tape0.clone()
    q, k, v, g, beta, _ = gdn_prologue(qkv, conv_state, aa, bb, wd, cfg)
    out_a, tape_a = gated_delta_verify_rollback(q, k, v, g, beta, st_a, tp_a, acc,
                                                tape_out=tp_a if inplace else None)
    st_b, tp_b = state0.clone(), tape0.clone()
    out_b, tape_b = gdn_prologue_verify_rollback(qkv, conv_state, aa, bb, wd, cfg, st_b, tp_b, acc,
                                                 tape_out=tp_b if inplace else None)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(tape_a, tape_b)
    assert torch.equal(st_a, st_b)
    assert torch.isfinite(out_b.float()).all()


def test_fused_prologue_scan_rejects_unsupported(device):
    from dflash_mlx.gdn_layer import gdn_prologue_verify_rollback

    def run(cfg, T, offset=0):
        x, w = _inputs(cfg, 1, T, seed=3)
        Hv, Dv, Dk = cfg.linear_num_value_heads, cfg.linear_value_head_dim, cfg.linear_key_head_dim
        flat = torch.cat([torch.zeros(offset, dtype=torch.bfloat16), x["qkv"].flatten()]).to(device)
        qkv = flat[offset:].view(1, T, cfg.conv_dim)
        st = torch.zeros(1, Hv, Dv, Dk, device=device)
        tape = torch.zeros(1, 1, Hv, Dv, Dk, device=device)
        acc = torch.zeros(1, dtype=torch.int32, device=device)
        gdn_prologue_verify_rollback(qkv, x["conv_state"].to(device), x["a"].to(device),
                                     x["b"].to(device), _w_dev(w, device), cfg, st, tape, acc)
        torch.cuda.synchronize()

    small = dict(linear_num_key_heads=1, linear_num_value_heads=1, linear_value_head_dim=64)
    run(GatedDeltaConfig(**small), 4)                                   # supported: runs
    with pytest.raises(_lib.DFlashError):                               # Dk != 128
        run(GatedDeltaConfig(linear_key_head_dim=64, **small), 4)
    with pytest.raises(_lib.DFlashError):                               # T > 32
        run(GatedDeltaConfig(**small), 33)
    with pytest.raises(_lib.DFlashError):                               # qkv not 4-byte aligned
        run(GatedDeltaConfig(**small), 4, offset=1)


@pytest.mark.parametrize("cfg,B,T", [
    (GatedDeltaConfig(), 1, 300),                                       # K = 4: the 4-tap tile kernel
    (GatedDeltaConfig(linear_num_key_heads=2, linear_num_value_heads=4,
                      linear_conv_kernel_dim=6), 2, 77),               # any other K
], ids=["qwen35-4b-T300", "K6-B2-T77"])
def test_prompt_prologue_tiles(oracle, device, cfg, B, T):
    """Inputs longer than 32 tokens take the tiled prologue (token tiles, each
    stream row read once): against the oracle, and bit for bit against the
    same tokens fed as consecutive calls of at most 32 tokens (the per-token
    kernel), each starting from the window the previous one left."""
    x, w = _inputs(cfg, B, T, seed=T)
    print(f"[prompt prologue {cfg} B={B} T={T}]", flush=True)
    wd = _w_dev(w, device)
    d = {k: v.to(device) for k, v in x.items()}
    q, k, v, g, beta, new_conv = gdn_prologue(d["qkv"], d["conv_state"], d["a"], d["b"], wd, cfg)
    torch.cuda.synchronize()
    rq, rk, rv, rg, rb, rst = _oracle_prologue(oracle, x, w, cfg)
    for name, got, ref in (("q", q, rq), ("k", k, rk), ("v", v, rv)):
        assert _rel_max(got.float().cpu().numpy(), ref) <= 1e-2, name
    assert _rel_max(g.cpu().numpy(), rg) <= 1e-5
    np.testing.assert_array_equal(new_conv.float().cpu().numpy(), rst)
    parts, conv = [], d["conv_state"]
    for t0 in range(0, T, 32):
        t1 = min(T, t0 + 32)
        part = gdn_prologue(d["qkv"][:, t0:t1].contiguous(), conv, d["a"][:, t0:t1].contiguous(),
                            d["b"][:, t0:t1].contiguous(), wd, cfg)
        parts.append(part)
        conv = part[5]
    torch.cuda.synchronize()
    for i, whole in enumerate((q, k, v, g, beta)):
        assert torch.equal(whole, torch.cat([p[i] for p in parts], dim=1)), i
    assert torch.equal(new_conv, conv)
