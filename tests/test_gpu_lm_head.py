"""GPU parity of the fused greedy LM head (MFMA, no logits in HBM) against an
fp64 CPU computation of the logits.

The fused kernel accumulates bf16 products in fp32, so it is not bit-equal to
any particular GEMM; the contract checked here:
* where the fp64 top-1 margin exceeds MARGIN, the argmax is identical;
* everywhere, the chosen token's fp64 logit is within MARGIN of the maximum;
* with planted winners (large margins) the accept (matched, bonus) is exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import _lib, greedy_accept, lm_head_argmax, lm_head_greedy_accept, tile_weight

pytestmark = pytest.mark.gpu

MARGIN = 2e-3  # relative to the row's max |logit|


def _inputs(M, H, V, seed):
    gen = torch.Generator().manual_seed(seed)
    hidden = (torch.randn(M, H, generator=gen) / H ** 0.25).bfloat16()
    weight = (torch.randn(V, H, generator=gen) / H ** 0.25).bfloat16()
    return hidden, weight


def _fp64_logits(hidden, weight):
    return hidden.double().numpy() @ weight.double().numpy().T


def _check_rows(post, logits):
    ref = np.argmax(logits, axis=-1)
    for m in range(logits.shape[0]):
        row = logits[m]
        scale = max(np.max(np.abs(row)), 1e-30)
        top2 = np.partition(row, -2)[-2:]
        margin = (top2[1] - top2[0]) / scale
        got = int(post[m])
        assert row[got] >= row.max() - MARGIN * scale, f"row {m}: token {got} not near the max"
        if margin > MARGIN:
            assert got == int(ref[m]), f"row {m}: argmax {got} != {ref[m]} (margin {margin:.2e})"


@pytest.mark.parametrize("M,H,V", [(1, 64, 1000), (16, 2560, 20011), (17, 512, 4096),
                                   (33, 256, 3000), (64, 2560, 8192), (16, 192, 2000),
                                   (16, 320, 2000), (5, 448, 1000)])
def test_lm_head_argmax_matches_fp64(device, M, H, V):
    hidden, weight = _inputs(M, H, V, seed=M * 7 + V)
    print(f"[lm_head M={M} H={H} V={V}]", flush=True)
    post = lm_head_argmax(hidden.to(device), weight.to(device))
    torch.cuda.synchronize()
    assert tuple(post.shape) == (M,)
    _check_rows(post.cpu().numpy(), _fp64_logits(hidden, weight))


def test_planted_winners_exact_accept(device):
    """Each position's winner is planted with a large margin, so the fused
    accept must reproduce the draft comparison exactly."""
    B, N, H, V = 2, 16, 2560, 50000
    hidden, weight = _inputs(B * N, H, V, seed=3)
    gen = torch.Generator().manual_seed(4)
    targets = torch.randint(0, V, (B * N,), generator=gen)
    w = weight.clone()
    for m in range(B * N):
        w[targets[m]] = (hidden[m].float() * 4.0).bfloat16()
    accept = [5, 16]
    draft = targets.reshape(B, N).clone().to(torch.int32)
    for b, a in enumerate(accept):
        if a < N:
            draft[b, a] = (draft[b, a] + 1) % V
    post, matched, bonus = lm_head_greedy_accept(hidden.reshape(B, N, H).to(device), w.to(device),
                                                 draft.to(device))
    torch.cuda.synchronize()
    assert post.cpu().reshape(-1).tolist() == targets.tolist()
    assert matched.cpu().tolist() == accept
    assert bonus.cpu().tolist() == [int(targets[5]), -1]


def test_full_vocab_agrees_with_unfused_path(device):
    """Qwen3.5-4B shape (H=2560, V=151936, 16 rows): fused result vs fp32
    logits from torch (hipBLASLt) + the greedy accept kernel."""
    M, H, V = 16, 2560, 151936
    gen = torch.Generator(device=device).manual_seed(5)
    hidden = (torch.randn(M, H, generator=gen, device=device) / H ** 0.25).bfloat16()
    weight = (torch.randn(V, H, generator=gen, device=device) / H ** 0.25).bfloat16()
    post = lm_head_argmax(hidden, weight)
    logits = hidden.float() @ weight.float().t().contiguous()
    ref_post, _, _ = greedy_accept(logits[None], None)
    torch.cuda.synchronize()
    lg = logits.double().cpu().numpy()
    got, ref = post.cpu().numpy(), ref_post[0].cpu().numpy()
    for m in range(M):
        scale = np.max(np.abs(lg[m]))
        assert lg[m, got[m]] >= lg[m].max() - MARGIN * scale
        top2 = np.partition(lg[m], -2)[-2:]
        if (top2[1] - top2[0]) / scale > MARGIN:
            assert got[m] == ref[m]


def test_rejects_unsupported(device):
    h = torch.zeros(65, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(100, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.DFlashError):
        lm_head_argmax(h, w)
    with pytest.raises(_lib.DFlashError):
        lm_head_argmax(h[:4, :48].contiguous(), w[:, :48].contiguous())  # H % 64 != 0


@pytest.mark.parametrize("M,H,V", [(1, 64, 1008), (16, 2560, 20016), (17, 512, 4096),
                                   (33, 256, 3008), (64, 2560, 8192), (16, 192, 2000),
                                   (16, 320, 2000), (5, 448, 1008), (16, 1216, 2000)])
def test_tiled_head_matches_fp64(device, M, H, V):
    """The head over its fragment-tiled copy (tile_weight): same contract."""
    hidden, weight = _inputs(M, H, V, seed=M * 11 + V)
    print(f"[lm_head tiled M={M} H={H} V={V}]", flush=True)
    w = weight.to(device)
    post = lm_head_argmax(hidden.to(device), w, weight_tiled=tile_weight(w))
    torch.cuda.synchronize()
    assert tuple(post.shape) == (M,)
    _check_rows(post.cpu().numpy(), _fp64_logits(hidden, weight))


def test_tiled_head_planted_winners_and_row_major_agree(device):
    """Planted winners: the tiled and row-major heads give the exact accept;
    on random rows the two agree wherever the top-2 margin exceeds fp32
    rounding of the split contraction."""
    B, N, H, V = 2, 16, 2560, 50000
    hidden, weight = _inputs(B * N, H, V, seed=13)
    gen = torch.Generator().manual_seed(14)
    targets = torch.randint(0, V, (B * N,), generator=gen)
    w = weight.clone()
    for m in range(B * N):
        w[targets[m]] = (hidden[m].float() * 4.0).bfloat16()
    accept = [7, 16]
    draft = targets.reshape(B, N).clone().to(torch.int32)
    draft[0, 7] = (draft[0, 7] + 1) % V
    wd = w.to(device)
    wt = tile_weight(wd)
    post, matched, bonus = lm_head_greedy_accept(hidden.reshape(B, N, H).to(device), wd,
                                                 draft.to(device), weight_tiled=wt)
    torch.cuda.synchronize()
    assert post.cpu().reshape(-1).tolist() == targets.tolist()
    assert matched.cpu().tolist() == accept
    assert bonus.cpu().tolist() == [int(targets[7]), -1]
    h2, w2 = _inputs(B * N, H, V, seed=15)
    hd, wd2 = h2.to(device), w2.to(device)
    a = lm_head_argmax(hd, wd2)
    b = lm_head_argmax(hd, wd2, weight_tiled=tile_weight(wd2))
    torch.cuda.synchronize()
    lg = _fp64_logits(h2, w2)
    for m in range(B * N):
        scale = np.max(np.abs(lg[m]))
        top2 = np.partition(lg[m], -2)[-2:]
        if (top2[1] - top2[0]) / scale > 1e-5:
            assert int(a[m]) == int(b[m]), f"row {m}"


def test_tiled_head_rejects_unsupported(device):
    h = torch.zeros(4, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(100, 64, dtype=torch.bfloat16, device=device)      # V % 16 != 0
    with pytest.raises(ValueError):
        tile_weight(w)
    w112 = torch.zeros(112, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):                                     # buffer too small
        lm_head_argmax(h, w112, weight_tiled=torch.zeros(16, dtype=torch.bfloat16, device=device))
