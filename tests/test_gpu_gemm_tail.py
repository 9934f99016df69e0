"""The tiled GEMMs' tail split (dflash_gemm_bf16_tiled, _swiglu_tiled,
_tiled_normed and _swiglu_tiled_normed with a workspace).

With the workspace, the row groups of a short last round run as single-wave
k-quarter units merged through the workspace in the workgroup's own k order,
so the output must be the same bits as the call without a workspace (itself
bit-identical to the row-major GEMM and within one bf16 rounding of fp32
torch, tests/test_gpu_gemm.py).  Shapes are chosen from the device's CU count
so that the split engages: the config-c4 gate|up (N = 18432: 576 groups, a
last round of 64 on 256 CUs), in_proj and q/k/v at 16 rows a wave, last
rounds from one group to a quarter of the CUs with and without whole rounds
before them, every wave width (16, 32, 64 rows), every M tile count (1..4),
and K of 2 k-steps (two of the four quarters empty).  The
workspace counters must be zero after every call, with stale partial sums
(NaN) in the workspace before the first, across calls of shrinking M, and
across graph replays.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib
from dflash_mlx.runtime import tile_weight

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _cus(device):
    return torch.cuda.get_device_properties(device).multi_processor_count


COUNT_BYTES = 1024  # the workspace's first 1 KB holds the row-group counters


def _workspace(device, stale=True):
    lib = _lib.load()
    ws = torch.zeros(int(lib.dflash_gemm_tail_workspace_bytes()), dtype=torch.uint8, device=device)
    if stale:  # partial sums left by nobody: NaN, counters zero
        ws[COUNT_BYTES:].view(torch.float32).fill_(float("nan"))
    return ws


def _counters_zero(ws):
    return bool((ws[:COUNT_BYTES] == 0).all().item())


def _pairs_tiled(device, I, K, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    w = (0.02 * torch.randn(2 * I, K, generator=g, device=device)).bfloat16()
    return tile_weight(w)


def _swiglu(device, x, wt, I, K, ws):
    M = x.shape[0]
    out = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)
    wsp, wsn = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    _lib.call("dflash_gemm_bf16_swiglu_tiled", x.data_ptr(), x.stride(0), wt.data_ptr(),
              out.data_ptr(), I, M, 2 * I, K, 4, wsp, wsn, _lib.stream_handle(device))
    return out


def _shapes(device):
    cus = _cus(device)
    groups_c4 = 18432 // 32
    out = []
    if groups_c4 // cus >= 1 and 0 < groups_c4 % cus <= min(cus // 4, 64):
        out.append((16, 9216, 2560))
    out += [(1, 16 * (cus + 1), 640), (37, 16 * (cus + 7), 1024), (64, 16 * (2 * cus + 3), 128),
            (20, 16 * (cus + min(cus // 4, 64)), 256)]
    return out


def test_tail_split_bit_identical(device):
    ws = _workspace(device)
    for M, I, K in _shapes(device):
        print(f"[gemm tail] M={M} I={I} K={K}", flush=True)
        g = torch.Generator(device=device).manual_seed(M * 7 + I)
        x = torch.randn(M, K, generator=g, device=device).bfloat16()
        wt = _pairs_tiled(device, I, K, seed=I + K)
        ref = _swiglu(device, x, wt, I, K, None)
        got = _swiglu(device, x, wt, I, K, ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, I, K)
        assert _counters_zero(ws)


def _plain_shapes(device):
    """(M, N, K, rows_per_wave): last rounds of one group to a quarter of the
    CUs, with and without whole rounds before them, every wave width, a
    partial last group; and shapes past the quarter (no split engages)."""
    cus = _cus(device)
    q = min(cus // 4, 64)
    return [(16, 12352, 2560, 16), (16, 5120, 2560, 16), (16, 12352, 2560, 32),
            (16, 5120, 2560, 32), (37, 16 * q, 512, 16), (64, 64 * (cus + q), 256, 64),
            (1, 32 * (2 * cus + 1), 128, 32), (20, 64 * q - 48, 640, 64)]


@pytest.mark.parametrize("normed", [False, True])
def test_tail_split_plain_bit_identical(device, normed):
    ws = _workspace(device)
    st = _lib.stream_handle(device)
    for M, N, K, rpw in _plain_shapes(device):
        print(f"[gemm tail plain] normed={normed} M={M} N={N} K={K} rpw={rpw}", flush=True)
        g = torch.Generator(device=device).manual_seed(M * 13 + N + rpw)
        x = torch.randn(M, K, generator=g, device=device).bfloat16()
        wt = tile_weight((0.02 * torch.randn(N, K, generator=g, device=device)).bfloat16())
        nw = (1.0 + 0.1 * torch.randn(K, generator=g, device=device)).bfloat16()
        sumsq = (K / 16) * (0.5 + torch.rand(16, M, generator=g, device=device))
        outs = []
        for w in (None, ws):
            out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=device)
            wsp, wsn = (w.data_ptr(), w.numel()) if w is not None else (None, 0)
            if normed:
                _lib.call("dflash_gemm_bf16_tiled_normed", x.data_ptr(), K, nw.data_ptr(),
                          sumsq.data_ptr(), 16, EPS, None, wt.data_ptr(), out.data_ptr(), N, M, N,
                          K, 1, rpw, 4, wsp, wsn, st)
            else:
                _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), K, wt.data_ptr(), out.data_ptr(),
                          N, M, N, K, 1, rpw, 4, wsp, wsn, st)
            outs.append(out)
        torch.cuda.synchronize()
        assert not torch.isnan(outs[0].float()).any()
        assert torch.equal(outs[1], outs[0]), (M, N, K, rpw)
        assert _counters_zero(ws)


def test_tail_split_repeated_calls_shrinking_m(device):
    cus = _cus(device)
    I, K = 16 * (cus + 9), 512
    wt = _pairs_tiled(device, I, K, seed=5)
    g = torch.Generator(device=device).manual_seed(11)
    x = torch.randn(64, K, generator=g, device=device).bfloat16()
    ws = _workspace(device)
    for M in (64, 64, 33, 16, 1):
        print(f"[gemm tail repeat] M={M} I={I} K={K}", flush=True)
        ref = _swiglu(device, x[:M], wt, I, K, None)
        got = _swiglu(device, x[:M], wt, I, K, ws)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), M
        assert _counters_zero(ws)


@pytest.mark.parametrize("M", [16, 37])
def test_tail_split_normed_bit_identical(device, M):
    cus = _cus(device)
    I, K, tiles = (9216, 2560, 160) if 0 < (18432 // 32) % cus <= cus // 4 else (16 * (cus + 5), 2560, 160)
    print(f"[gemm tail normed] M={M} I={I} K={K}", flush=True)
    g = torch.Generator(device=device).manual_seed(M + I)
    h = torch.randn(M, K, generator=g, device=device).bfloat16()
    nw = (1.0 + 0.1 * torch.randn(K, generator=g, device=device)).bfloat16()
    sumsq = (K / tiles) * (0.5 + torch.rand(tiles, M, generator=g, device=device))
    wt = _pairs_tiled(device, I, K, seed=I)
    st = _lib.stream_handle(device)
    ws = _workspace(device)
    outs = []
    for w in (None, ws):
        out = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)
        inv = torch.full((M,), float("nan"), device=device)
        wsp, wsn = (w.data_ptr(), w.numel()) if w is not None else (None, 0)
        _lib.call("dflash_gemm_bf16_swiglu_tiled_normed", h.data_ptr(), K, nw.data_ptr(),
                  sumsq.data_ptr(), tiles, EPS, inv.data_ptr(), wt.data_ptr(), out.data_ptr(), I, M,
                  2 * I, K, 4, wsp, wsn, st)
        outs.append((out, inv))
    torch.cuda.synchronize()
    assert torch.equal(outs[1][0], outs[0][0])
    assert torch.equal(outs[1][1], outs[0][1])
    assert _counters_zero(ws)


def test_tail_split_graph_replays(device):
    cus = _cus(device)
    I, K, M = 16 * (cus + 13), 768, 16
    wt = _pairs_tiled(device, I, K, seed=3)
    x = torch.randn(M, K, generator=torch.Generator(device=device).manual_seed(2),
                    device=device).bfloat16()
    ref = _swiglu(device, x, wt, I, K, None)
    ws = _workspace(device)
    out = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device=device)

    def work():
        _lib.call("dflash_gemm_bf16_swiglu_tiled", x.data_ptr(), K, wt.data_ptr(), out.data_ptr(),
                  I, M, 2 * I, K, 4, ws.data_ptr(), ws.numel(), _lib.stream_handle(device))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        work()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work()
    for replay in range(4):
        print(f"[gemm tail graph] replay {replay}", flush=True)
        out.fill_(float("nan"))
        _swiglu(device, x[:5], wt, I, K, ws)  # eager use of the same workspace in between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), replay
        assert _counters_zero(ws)


def test_tail_workspace_validation(device):
    lib = _lib.load()
    need = int(lib.dflash_gemm_tail_workspace_bytes())
    assert need >= COUNT_BYTES + 64 * 4 * 16 * 1024
    x = torch.zeros(16, 128, dtype=torch.bfloat16, device=device)
    wt = torch.zeros(64 * 128, dtype=torch.bfloat16, device=device)
    out = torch.zeros(16, 32, dtype=torch.bfloat16, device=device)
    ws = torch.zeros(need + 512, dtype=torch.uint8, device=device)
    st = _lib.stream_handle(device)
    f = lib.dflash_gemm_bf16_swiglu_tiled
    # too small
    assert f(x.data_ptr(), 128, wt.data_ptr(), out.data_ptr(), 32, 16, 64, 128, 4, ws.data_ptr(),
             need - 1, st) == -5
    # not 256-byte aligned
    assert f(x.data_ptr(), 128, wt.data_ptr(), out.data_ptr(), 32, 16, 64, 128, 4,
             ws.data_ptr() + 16, need, st) == -4
    # a good call on a shape without a short last round leaves the workspace alone
    assert f(x.data_ptr(), 128, wt.data_ptr(), out.data_ptr(), 32, 16, 64, 128, 4, ws.data_ptr(),
             need, st) == 0
    torch.cuda.synchronize()
    assert bool((ws == 0).all().item())
