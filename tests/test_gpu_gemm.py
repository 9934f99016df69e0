"""GPU parity of the verify-sized projection GEMM (dflash_gemm_bf16) and its
split-K consumers against an fp32 torch reference of the same bf16 inputs.

out = bf16(x . w^T): within one bf16 rounding of the fp32 reference
(|err| <= 2^-8 |ref| + 1e-3 * rms(ref), fp32 accumulation in a different
order); split-K partials summed in fp32: within 1e-4 of the reference's
scale.  Shapes: every projection of the config-c4 step at M = 16, other M up
to 64, N tails, both wave widths.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib

pytestmark = pytest.mark.gpu

C4_SHAPES = [  # (N, K, nsplit): in_proj, out_proj, attn qkv, o_proj, gate|up, down
    (12352, 2560, 1), (2560, 4096, 8), (5120, 2560, 4), (2560, 2048, 8), (18432, 2560, 1),
    (2560, 9216, 8)]


def _ref(x, w):
    return x.float() @ w.float().t()


def _run(device, M, N, K, nsplit, rpw, seed, kw=4):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
    lib = _lib.load()
    used = int(lib.dflash_gemm_splits(K, nsplit))
    if nsplit > 1:
        out = torch.full((used, M, N), float("nan"), device=device)
    else:
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_gemm_bf16", x.data_ptr(), K, w.data_ptr(), K, out.data_ptr(), N, M, N, K,
              nsplit, rpw, kw, _lib.stream_handle(device))
    torch.cuda.synchronize()
    return x, w, out, used


@pytest.mark.parametrize("kw", [1, 4])
@pytest.mark.parametrize("N,K,nsplit", C4_SHAPES)
def test_gemm_c4_shapes(device, N, K, nsplit, kw):
    M = 16
    print(f"[gemm] M={M} N={N} K={K} nsplit={nsplit} k_waves={kw}", flush=True)
    x, w, out, used = _run(device, M, N, K, nsplit, 16 if kw == 1 else 32, seed=N + K, kw=kw)
    ref = _ref(x, w)
    scale = ref.pow(2).mean().sqrt().item()
    if nsplit > 1:
        assert used == min(nsplit, K // 64) or used <= nsplit
        got = out.sum(0)
        err = (got - ref).abs().max().item()
        assert err <= 1e-4 * scale + 1e-5, err
    else:
        err = ((out.float() - ref).abs() - (2 ** -8) * ref.abs()).max().item()
        assert err <= 1e-3 * scale, err


@pytest.mark.parametrize("M,N,K,rpw,nsplit,kw", [
    (1, 100, 64, 16, 1, 1), (37, 1000, 640, 32, 1, 1), (64, 777, 1024, 16, 3, 1),
    (23, 300, 4096, 32, 5, 1), (16, 5120, 2560, 32, 4, 1), (1, 100, 64, 16, 1, 4),
    (37, 1000, 640, 32, 1, 4), (64, 777, 1024, 16, 3, 4), (23, 300, 192, 32, 5, 4),
    (16, 40, 128, 16, 1, 4)])
def test_gemm_ragged(device, M, N, K, rpw, nsplit, kw):
    x, w, out, used = _run(device, M, N, K, nsplit, rpw, seed=M * 7 + N, kw=kw)
    ref = _ref(x, w)
    scale = ref.pow(2).mean().sqrt().item()
    got = out.sum(0) if nsplit > 1 else out.float()
    tol = (1e-4 * scale + 1e-5) if nsplit > 1 else None
    if nsplit > 1:
        assert (got - ref).abs().max().item() <= tol
        assert torch.isfinite(out).all()  # every used split's every element written
    else:
        assert ((got - ref).abs() - (2 ** -8) * ref.abs()).max().item() <= 1e-3 * scale


def test_splitk_consumers(device):
    """add+RMSNorm and the reduce read the same partials the GEMM wrote:
    bf16(sum) then the residual add, as the unsplit path does."""
    M, N, K, H = 16, 2560, 4096, 2560
    x, w, part, used = _run(device, M, N, K, 8, 16, seed=5)
    r_bf = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    _lib.call("dflash_splitk_reduce", part.data_ptr(), used, M, N, r_bf.data_ptr(), N,
              _lib.stream_handle(device))
    resid = torch.randn(M, H, device=device).bfloat16()
    wn = torch.ones(H, dtype=torch.bfloat16, device=device)
    h1, y1 = resid.clone(), torch.empty_like(resid)
    h2, y2 = resid.clone(), torch.empty_like(resid)
    _lib.call("dflash_add_rmsnorm_splitk", h1.data_ptr(), part.data_ptr(), used, wn.data_ptr(),
              h1.data_ptr(), y1.data_ptr(), M, H, 1e-6, _lib.stream_handle(device))
    _lib.call("dflash_add_rmsnorm", h2.data_ptr(), r_bf.data_ptr(), wn.data_ptr(), h2.data_ptr(),
              y2.data_ptr(), M, H, 1e-6, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert torch.equal(r_bf, part.sum(0).bfloat16()) or \
        (r_bf.float() - part.sum(0)).abs().max().item() <= 2 ** -7 * part.sum(0).abs().max().item()
    assert torch.equal(h1, h2) and torch.equal(y1, y2)


def test_gemm_rejects_bad_arguments(device):
    lib = _lib.load()
    assert lib.dflash_gemm_bf16(None, 64, None, 64, None, 8, 65, 8, 64, 1, 16, 1, None) == -2  # M>64
    assert lib.dflash_gemm_bf16(None, 64, None, 64, None, 8, 16, 8, 100, 1, 16, 1, None) == -2  # K%64
    assert lib.dflash_gemm_bf16(None, 64, None, 64, None, 8, 16, 8, 64, 1, 24, 1, None) == -3  # width
    assert lib.dflash_gemm_bf16(None, 64, None, 64, None, 8, 16, 8, 64, 1, 16, 2, None) == -3  # k_waves
    assert lib.dflash_gemm_splits(4096, 8) == 8 and lib.dflash_gemm_splits(128, 8) == 2


@pytest.mark.parametrize("M,I,K,kw", [(16, 9216, 2560, 4), (16, 9216, 2560, 1), (37, 64, 128, 4)])
def test_gemm_swiglu_fused(device, M, I, K, kw):
    """Paired gate/up weight: out = bf16(silu(x G^T) * (x U^T)) within two
    bf16 ulps of the fp32 reference (silu of an fp32 product, one rounding)."""
    g = torch.Generator(device=device).manual_seed(I + M)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.05 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()  # [gate; up]
    pairs = w.view(2, I // 16, 16, K).transpose(0, 1).reshape(2 * I, K).contiguous()
    out = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_gemm_bf16_swiglu", x.data_ptr(), K, pairs.data_ptr(), K, out.data_ptr(), I, M,
              2 * I, K, kw, _lib.stream_handle(device))
    torch.cuda.synchronize()
    gu = x.float() @ w.float().t()
    ref = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
    scale = ref.pow(2).mean().sqrt().item()
    err = ((out.float() - ref).abs() - 2 ** -7 * ref.abs()).max().item()
    print(f"[gemm swiglu] M={M} I={I} K={K} kw={kw}: excess {err:.3e} (rms {scale:.3e})", flush=True)
    assert err <= 1e-3 * scale


def _tile(device, w):
    N, K = w.shape
    lib = _lib.load()
    t = torch.empty(int(lib.dflash_weight_tile_bytes(N, K)) // 2, dtype=torch.bfloat16, device=device)
    _lib.call("dflash_weight_tile_bf16", w.data_ptr(), w.stride(0), t.data_ptr(), N, K,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    return t


def test_weight_tile_layout(device):
    """The fragment layout entry by entry, from its defining formula."""
    N, K = 48, 192
    w = torch.arange(N * K, dtype=torch.float32).remainder(251).reshape(N, K).bfloat16().to(device)
    t = _tile(device, w).cpu().float().numpy()
    wn = w.cpu().float().numpy()
    nks = K // 64
    for rt in range(N // 16):
        for ks in range(nks):
            for h in range(2):
                for lane in range(64):
                    base = ((ks * (N // 16) + rt) * 2 + h) * 512 + lane * 8
                    row = 16 * rt + lane % 16
                    col = 64 * ks + 16 * (lane // 16) + 8 * h
                    assert (t[base:base + 8] == wn[row, col:col + 8]).all(), (rt, ks, h, lane)


@pytest.mark.parametrize("N,K,nsplit", C4_SHAPES)
@pytest.mark.parametrize("rpw,kw", [(16, 4), (32, 4), (32, 1)])
def test_gemm_tiled_bit_identical(device, N, K, nsplit, rpw, kw):
    """Tiled weights give the row-major kernel's sums bit for bit (same k-slots)."""
    M = 16
    print(f"[gemm tiled] N={N} K={K} nsplit={nsplit} rpw={rpw} kw={kw}", flush=True)
    x, w, out, used = _run(device, M, N, K, nsplit, rpw, seed=N * 3 + K, kw=kw)
    t = _tile(device, w)
    out_t = torch.full_like(out, float("nan"))
    _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), K, t.data_ptr(), out_t.data_ptr(), N, M, N, K,
              nsplit, rpw, kw, None, 0, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert torch.equal(out_t, out)


@pytest.mark.parametrize("M,N,K,nsplit,kw", [(16, 12352, 2560, 1, 4), (16, 5120, 2560, 1, 1),
                                              (37, 1008, 640, 1, 4), (64, 784, 1024, 3, 1),
                                              (1, 48, 64, 1, 4)])
def test_gemm_tiled_64_rows_per_wave(device, M, N, K, nsplit, kw):
    """rows_per_wave 64 (tiled only) against the fp32 reference, M and N tails."""
    g = torch.Generator(device=device).manual_seed(M + N)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
    t = _tile(device, w)
    lib = _lib.load()
    used = int(lib.dflash_gemm_splits(K, nsplit))
    out = (torch.full((used, M, N), float("nan"), device=device) if nsplit > 1 else
           torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device))
    _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), K, t.data_ptr(), out.data_ptr(), N, M, N, K,
              nsplit, 64, kw, None, 0, _lib.stream_handle(device))
    torch.cuda.synchronize()
    ref = _ref(x, w)
    scale = ref.pow(2).mean().sqrt().item()
    if nsplit > 1:
        assert torch.isfinite(out).all()
        assert (out.sum(0) - ref).abs().max().item() <= 1e-4 * scale + 1e-5
    else:
        assert ((out.float() - ref).abs() - (2 ** -8) * ref.abs()).max().item() <= 1e-3 * scale


@pytest.mark.parametrize("M", [16, 37])
@pytest.mark.parametrize("kw", [1, 4])
@pytest.mark.parametrize("steps", [1, 2, 3, 4, 5, 6, 7])
def test_gemm_tiled_every_ring_remainder(device, M, kw, steps):
    """Each wave's k-range of 1 .. 7 k-steps: every remainder modulo the
    load ring's depth (4 k-steps at M <= 32, 2 above), so the last turn of
    the ring skips 0 .. 3 steps.  Against the fp32 reference."""
    K = 64 * kw * steps
    N = 272
    print(f"[gemm tiled] ring remainder M={M} k_waves={kw} steps={steps}", flush=True)
    g = torch.Generator(device=device).manual_seed(100 * M + 10 * kw + steps)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
    t = _tile(device, w)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), K, t.data_ptr(), out.data_ptr(), N, M, N, K,
              1, 16, kw, None, 0, _lib.stream_handle(device))
    torch.cuda.synchronize()
    ref = _ref(x, w)
    scale = ref.pow(2).mean().sqrt().item()
    assert ((out.float() - ref).abs() - (2 ** -8) * ref.abs()).max().item() <= 1e-3 * scale


@pytest.mark.parametrize("M,I,K,kw", [(16, 9216, 2560, 4), (37, 64, 128, 1)])
def test_gemm_swiglu_tiled_bit_identical(device, M, I, K, kw):
    g = torch.Generator(device=device).manual_seed(I + M)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()
    pairs = w.view(2, I // 16, 16, K).transpose(0, 1).reshape(2 * I, K).contiguous()
    out = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_gemm_bf16_swiglu", x.data_ptr(), K, pairs.data_ptr(), K, out.data_ptr(), I, M,
              2 * I, K, kw, _lib.stream_handle(device))
    t = _tile(device, pairs)
    out_t = torch.full_like(out, float("nan"))
    _lib.call("dflash_gemm_bf16_swiglu_tiled", x.data_ptr(), K, t.data_ptr(), out_t.data_ptr(), I,
              M, 2 * I, K, kw, None, 0, _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert torch.equal(out_t, out)


def test_gemm_tiled_rejects_bad_arguments(device):
    lib = _lib.load()
    assert lib.dflash_weight_tile_bytes(40, 64) == 0          # N % 16
    assert lib.dflash_weight_tile_bf16(None, 64, None, 40, 64, None) == -2
    assert lib.dflash_gemm_bf16_tiled(None, 64, None, None, 64, 16, 40, 64, 1, 32, 4, None, 0,
                                      None) == -2
    assert lib.dflash_gemm_bf16_tiled(None, 64, None, None, 64, 16, 48, 64, 1, 48, 4, None, 0,
                                      None) == -3
