"""GPU parity of the residual add + RMSNorm folded into the projections
(dflash_gemm_bf16_tiled_residual_norm, dflash_gemm_bf16_tiled_normed,
dflash_gemm_bf16_swiglu_tiled_normed).

* Producer: with a zero residual, h is the projection r = bf16(x . w^T)
  itself, within one bf16 rounding of the fp32 torch product; with a real
  residual, h == bf16(resid + r) exactly (the same r: the kernel is
  deterministic); the capture copy equals h and nothing past the row is
  written; each tile's row sum of h^2 within 1e-6 of the fp64 sum of that h.
* Consumers: row_inv_out within 1e-6 of the fp64 1 / sqrt(sum / K + eps) of
  the given row sums, and the same bits whatever M (the summation order is
  fixed); the output bit-identical to the plain tiled GEMM of
  y = bf16((h * inv) * w) computed by torch from the same h, norm weight and
  the kernel's inv.
* The hybrid runner with fused norms against the add + RMSNorm launches is
  tested in test_gpu_hybrid.py.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib
from dflash_mlx.runtime import tile_weight

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _producer(device, x, wt, resid, M, N, K, cap_stride=None):
    h = resid.clone()
    sumsq = torch.full((N // 16, M), float("nan"), device=device)
    cap = None
    if cap_stride is not None:
        cap = torch.full((M, cap_stride), float("nan"), device=device).bfloat16()
    _lib.call("dflash_gemm_bf16_tiled_residual_norm", x.data_ptr(), K, wt.data_ptr(), M, N, K,
              h.data_ptr(), h.data_ptr(), _lib.ptr(cap), cap_stride or 0, sumsq.data_ptr(),
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    return h, sumsq, cap


@pytest.mark.parametrize("M,N,K", [(16, 2560, 4096), (16, 2560, 9216), (16, 2560, 2048),
                                   (37, 2576, 1024), (64, 1040, 640), (1, 160, 128), (5, 96, 64),
                                   (16, 2560, 1024), (16, 2560, 5120), (16, 2560, 6144)])
def test_residual_norm_producer(device, M, N, K):
    print(f"[fused norm producer] M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(M * 31 + N + K)
    x = torch.randn(M, K, generator=g, device=device).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16()
    resid = torch.randn(M, N, generator=g, device=device).bfloat16()
    wt = tile_weight(w)
    # zero residual: h is the projection itself
    r, _, _ = _producer(device, x, wt, torch.zeros_like(resid), M, N, K)
    ref = x.float() @ w.float().t()
    scale = ref.pow(2).mean().sqrt().item()
    assert ((r.float() - ref).abs() - (2 ** -8) * ref.abs()).max().item() <= 1e-3 * scale
    # the residual add, exactly
    h, sumsq, cap = _producer(device, x, wt, resid, M, N, K, cap_stride=N + 16)
    want = (resid.float() + r.float()).bfloat16()
    assert torch.equal(h, want)
    assert torch.equal(cap[:, :N], h)
    assert torch.isnan(cap[:, N:].float()).all()
    h64 = h.double().view(M, N // 16, 16)
    ss64 = (h64 * h64).sum(-1).t()  # [tiles, M]
    rel = ((sumsq.double() - ss64).abs() / ss64.clamp_min(1e-30)).max().item()
    assert rel <= 1e-6, rel


def _normed_inputs(device, M, K, tiles, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    h = torch.randn(M, K, generator=g, device=device).bfloat16()
    nw = (1.0 + 0.1 * torch.randn(K, generator=g, device=device)).bfloat16()
    sumsq = (K / tiles) * (0.5 + torch.rand(tiles, M, generator=g, device=device))
    return h, nw, sumsq


def _check_inv(inv, sumsq, K):
    inv64 = 1.0 / torch.sqrt(sumsq.double().sum(0) / K + EPS)
    assert ((inv.double() - inv64).abs() / inv64).max().item() <= 1e-6


@pytest.mark.parametrize("M,N,K,nsplit,rpw,tiles", [
    (16, 12352, 2560, 1, 64, 160), (16, 12352, 2560, 1, 32, 160), (16, 5120, 2560, 1, 32, 160),
    (37, 1008, 640, 1, 16, 40), (64, 800, 1024, 3, 32, 300), (3, 64, 128, 2, 64, 1)])
def test_normed_consumer_bit_identical(device, M, N, K, nsplit, rpw, tiles):
    print(f"[fused norm consumer] M={M} N={N} K={K} nsplit={nsplit} rpw={rpw} tiles={tiles}",
          flush=True)
    h, nw, sumsq = _normed_inputs(device, M, K, tiles, seed=N + K)
    w = (0.02 * torch.randn(N, K, generator=torch.Generator(device=device).manual_seed(M),
                            device=device)).bfloat16()
    wt = tile_weight(w)
    lib = _lib.load()
    st = _lib.stream_handle(device)
    used = int(lib.dflash_gemm_splits(K, nsplit))
    shape = (used, M, N) if nsplit > 1 else (M, N)
    dt = torch.float32 if nsplit > 1 else torch.bfloat16
    got = torch.full(shape, float("nan"), device=device).to(dt)
    inv = torch.full((M,), float("nan"), device=device)
    _lib.call("dflash_gemm_bf16_tiled_normed", h.data_ptr(), K, nw.data_ptr(), sumsq.data_ptr(),
              tiles, EPS, inv.data_ptr(), wt.data_ptr(), got.data_ptr(), N, M, N, K, nsplit, rpw, 4,
              None, 0, st)
    torch.cuda.synchronize()
    _check_inv(inv, sumsq, K)
    # one row alone: the same inverse RMS bits
    inv1 = torch.full((1,), float("nan"), device=device)
    got1 = torch.empty((used, 1, N) if nsplit > 1 else (1, N), device=device).to(dt)
    s1 = sumsq[:, :1].contiguous()
    _lib.call("dflash_gemm_bf16_tiled_normed", h.data_ptr(), K, nw.data_ptr(), s1.data_ptr(), tiles,
              EPS, inv1.data_ptr(), wt.data_ptr(), got1.data_ptr(), N, 1, N, K, nsplit, rpw, 4, None,
              0, st)
    # the plain GEMM of y formed by torch with the kernel's inv
    y = ((h.float() * inv[:, None]) * nw.float()).bfloat16()
    ref = torch.full(shape, float("nan"), device=device).to(dt)
    _lib.call("dflash_gemm_bf16_tiled", y.data_ptr(), K, wt.data_ptr(), ref.data_ptr(), N, M, N, K,
              nsplit, rpw, 4, None, 0, st)
    torch.cuda.synchronize()
    assert torch.equal(inv1, inv[:1])
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,I,K,tiles", [(16, 9216, 2560, 160), (37, 512, 640, 40), (1, 64, 64, 4)])
def test_normed_swiglu_bit_identical(device, M, I, K, tiles):
    print(f"[fused norm swiglu] M={M} I={I} K={K}", flush=True)
    h, nw, sumsq = _normed_inputs(device, M, K, tiles, seed=I + K)
    w = (0.02 * torch.randn(2 * I, K, generator=torch.Generator(device=device).manual_seed(I),
                            device=device)).bfloat16()
    wt = tile_weight(w)
    st = _lib.stream_handle(device)
    got = torch.full((M, I), float("nan"), device=device).bfloat16()
    inv = torch.full((M,), float("nan"), device=device)
    _lib.call("dflash_gemm_bf16_swiglu_tiled_normed", h.data_ptr(), K, nw.data_ptr(),
              sumsq.data_ptr(), tiles, EPS, inv.data_ptr(), wt.data_ptr(), got.data_ptr(), I, M,
              2 * I, K, 4, None, 0, st)
    torch.cuda.synchronize()
    _check_inv(inv, sumsq, K)
    y = ((h.float() * inv[:, None]) * nw.float()).bfloat16()
    ref = torch.full((M, I), float("nan"), device=device).bfloat16()
    _lib.call("dflash_gemm_bf16_swiglu_tiled", y.data_ptr(), K, wt.data_ptr(), ref.data_ptr(), I, M,
              2 * I, K, 4, None, 0, st)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_fused_norm_entry_points_reject_bad_arguments(device):
    lib = _lib.load()
    x = torch.zeros(16, 256, dtype=torch.bfloat16, device=device)
    wt = torch.zeros(256 * 256, dtype=torch.bfloat16, device=device)
    ss = torch.zeros(16, 16, device=device)
    st = _lib.stream_handle(device)
    # N not a multiple of 16
    assert lib.dflash_gemm_bf16_tiled_residual_norm(x.data_ptr(), 256, wt.data_ptr(), 16, 250, 256,
                                                    x.data_ptr(), x.data_ptr(), None, 0,
                                                    ss.data_ptr(), st) != 0
    # no row sums
    assert lib.dflash_gemm_bf16_tiled_residual_norm(x.data_ptr(), 256, wt.data_ptr(), 16, 256, 256,
                                                    x.data_ptr(), x.data_ptr(), None, 0, None,
                                                    st) != 0
    # k_waves other than 4 for the normed consumer
    assert lib.dflash_gemm_bf16_tiled_normed(x.data_ptr(), 256, x.data_ptr(), ss.data_ptr(), 16,
                                             EPS, None, wt.data_ptr(), x.data_ptr(), 256, 16, 256,
                                             256, 1, 32, 1, None, 0, st) != 0
    # K beyond the staged norm weight
    assert lib.dflash_gemm_bf16_tiled_normed(x.data_ptr(), 32768, x.data_ptr(), ss.data_ptr(), 16,
                                             EPS, None, wt.data_ptr(), x.data_ptr(), 256, 16, 256,
                                             32768, 1, 32, 4, None, 0, st) != 0
    # no row tiles
    assert lib.dflash_gemm_bf16_tiled_normed(x.data_ptr(), 256, x.data_ptr(), ss.data_ptr(), 0,
                                             EPS, None, wt.data_ptr(), x.data_ptr(), 256, 16, 256,
                                             256, 1, 32, 4, None, 0, st) != 0
