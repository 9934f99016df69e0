"""GPU parity of the prompt-pass attention (dflash_attn_prefill).

Prompt row i of one sequence attends to cache positions 0 .. L0 + i, where
L0 is the cache length before the prompt and the prompt's own keys and
values sit at L0 .. L0 + P - 1 (dflash_attn_prep's layout: keys
[Hkv, Smax, D], values transposed [Hkv, D, Smax]); the output is multiplied
by sigmoid of the gate held in the projection rows.

* Against an fp32 CPU reference of the same bf16 inputs (softmax(scale q k^T)
  v * sigmoid(gate)): the kernel rounds the probabilities to bf16 before
  the P.V product and the output to bf16, so the bound is 1e-2 of the
  output's largest magnitude.
* Against the verify attention (dflash_attn_verify) run block by block over
  the same prompt (16 rows a call at cache length L0 + 16 b, the decode loop's
  schedule): the same bound (the two split the keys differently).
Cases: GQA 1, 2 and 4 query heads per kv head, prompts that are not whole
16-row blocks, empty and non-empty caches before the prompt, a prompt that
ends at the last cache position.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib

pytestmark = pytest.mark.gpu

D = 128


def _make(device, P, L0, Hq, Hkv, Smax, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(P, Hq, D, generator=g).bfloat16()
    keys = torch.randn(Hkv, L0 + P, D, generator=g).bfloat16()
    vals = torch.randn(Hkv, L0 + P, D, generator=g).bfloat16()
    stride = 2 * Hq * D + 64  # projection rows wider than the query|gate block
    gate_rows = torch.randn(P, stride, generator=g).bfloat16()
    kc = torch.zeros(Hkv, Smax, D, dtype=torch.bfloat16)
    vt = torch.zeros(Hkv, D, Smax, dtype=torch.bfloat16)
    kc[:, :L0 + P] = keys
    vt[:, :, :L0 + P] = vals.transpose(1, 2)
    return q, keys, vals, gate_rows, kc, vt


def _reference(q, keys, vals, gate_rows, L0, Hq, Hkv, scale):
    P = q.shape[0]
    rep = Hq // Hkv
    out = torch.empty(P, Hq * D)
    qf, kf, vf = q.float(), keys.float(), vals.float()
    for qh in range(Hq):
        h = qh // rep
        s = (qf[:, qh] @ kf[h].t()) * scale  # [P, L0 + P]
        pos = torch.arange(L0 + P)[None, :]
        s = s.masked_fill(pos > (L0 + torch.arange(P))[:, None], float("-inf"))
        o = torch.softmax(s, -1) @ vf[h]
        gt = gate_rows[:, qh * 2 * D + D: qh * 2 * D + 2 * D].float()
        out[:, qh * D:(qh + 1) * D] = o * torch.sigmoid(gt)
    return out


def _run_prefill(device, q, kc, vt, gate_rows, L0, P, Hq, Hkv, Smax, scale):
    qd, kd, vd, gd = (t.to(device) for t in (q, kc, vt, gate_rows))
    lens = torch.tensor([L0], dtype=torch.int32, device=device)
    out = torch.full((P, Hq * D), float("nan"), dtype=torch.bfloat16, device=device)
    _lib.call("dflash_attn_prefill", qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), lens.data_ptr(),
              gd.data_ptr(), gd.stride(0), out.data_ptr(), P, Hq, Hkv, D, Smax, scale,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("P,L0,Hq,Hkv,Smax", [
    (1, 0, 4, 4, 64), (16, 0, 16, 4, 64), (37, 5, 8, 4, 128), (300, 130, 16, 4, 512),
    (200, 0, 3, 1, 256), (64, 448, 16, 4, 512)])
def test_attn_prefill_matches_reference(device, P, L0, Hq, Hkv, Smax):
    print(f"[attn prefill] P={P} L0={L0} Hq={Hq} Hkv={Hkv} Smax={Smax}", flush=True)
    scale = D ** -0.5
    q, keys, vals, gate_rows, kc, vt = _make(device, P, L0, Hq, Hkv, Smax, seed=P + L0 + Hq)
    got = _run_prefill(device, q, kc, vt, gate_rows, L0, P, Hq, Hkv, Smax, scale)
    ref = _reference(q, keys, vals, gate_rows, L0, Hq, Hkv, scale)
    assert torch.isfinite(got.float()).all()
    err = (got.float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err


def test_attn_prefill_matches_blockwise_verify(device):
    """The prompt as one call against the decode schedule: the verify
    attention over 16-row blocks at growing cache lengths."""
    P, L0, Hq, Hkv, Smax = 100, 20, 16, 4, 256
    scale = D ** -0.5
    q, keys, vals, gate_rows, kc, vt = _make(device, P, L0, Hq, Hkv, Smax, seed=5)
    got = _run_prefill(device, q, kc, vt, gate_rows, L0, P, Hq, Hkv, Smax, scale)
    qd, kd, vd, gd = (t.to(device) for t in (q, kc, vt, gate_rows))
    lib = _lib.load()
    ws = torch.empty(int(lib.dflash_attn_verify_workspace_bytes(1, Hq, Hkv, Smax)),
                     dtype=torch.uint8, device=device)
    blk = torch.empty(P, Hq * D, dtype=torch.bfloat16, device=device)
    for b0 in range(0, P, 16):
        T = min(16, P - b0)
        lens = torch.tensor([L0 + b0], dtype=torch.int32, device=device)
        _lib.call("dflash_attn_verify", qd[b0:].data_ptr(), kd.data_ptr(), vd.data_ptr(),
                  lens.data_ptr(), gd[b0:].data_ptr(), gd.stride(0), blk[b0:].data_ptr(), 1, T,
                  Hq, Hkv, D, Smax, L0 + b0 + T, scale, ws.data_ptr(), ws.numel(),
                  _lib.stream_handle(device))
    torch.cuda.synchronize()
    err = (got.float() - blk.float().cpu()).abs().max().item()
    assert err <= 1e-2 * blk.float().abs().max().item(), err

