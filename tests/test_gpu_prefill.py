"""GPU parity of the chunked (WY / UT-transform) prefill kernel.

The chunked form sums in a different order from the token-by-token scan, so
the bar is the stated tolerance, not bit equality: bf16 ``out`` max-abs
<= 2e-2 and fp32 final state normwise relative error <= 1e-3
(max|x - ref| / max|ref|), against the CPU oracle (fp64 accumulation) at
small sizes and at the full config-3 size (B=1, T=8192, Hk=16, Hv=32,
Dk=Dv=128), and against the sequential GPU scan kernel.  Strided inputs
(views of one fused qkv buffer) must give bit-identical results to
contiguous copies.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import _lib, chunked_prefill_workspace_bytes, gated_delta_kernel, gated_delta_prefill
from dflash_mlx.workloads import CONFIGS, ScanConfig, make_scan_inputs

pytestmark = pytest.mark.gpu

OUT_ATOL = 2e-2
STATE_RTOL = 1e-3


def _rel(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def _np(x):
    return x.float().cpu().numpy()


def _dev(x, device):
    return {k: v.to(device) for k, v in x.items() if not k.startswith("_")}


def _cfg(base: ScanConfig, **kw) -> ScanConfig:
    return ScanConfig(**{**base.__dict__, **kw})


SMALL = [
    _cfg(CONFIGS[3], T=200, Hk=2, Hv=4, state_std=0.05),   # 3 chunks + 8 tokens, GQA
    _cfg(CONFIGS[3], B=2, T=64, Hk=2, Hv=2, state_std=0.05),  # one full chunk, B=2
    _cfg(CONFIGS[3], T=1, Hk=1, Hv=2, state_std=0.05),     # single token
    _cfg(CONFIGS[3], T=129, Hk=4, Hv=4),                   # zero state, 1 token past 2 chunks
    _cfg(CONFIGS[3], B=2, T=130, Hk=1, Hv=4, state_std=0.05),  # 4 value heads share Q / K^T
]


@pytest.mark.parametrize("cfg", SMALL, ids=lambda c: f"B{c.B}T{c.T}Hk{c.Hk}Hv{c.Hv}")
def test_prefill_matches_oracle_small(oracle, device, cfg):
    x = make_scan_inputs(cfg)
    d = _dev(x, device)
    print(f"[prefill small] {cfg}", flush=True)
    out, fin = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])
    torch.cuda.synchronize()
    ins = [_np(x[n]) for n in ("q", "k", "v", "g", "beta", "state")]
    o_ref, f_ref, _ = oracle.scan_c(*ins, acc64=True, with_tape=False)
    out_err = float(np.max(np.abs(_np(out) - o_ref)))
    fin_err = _rel(_np(fin), f_ref)
    print(f"  out max-abs {out_err:.3e}  final rel {fin_err:.3e}", flush=True)
    assert out_err <= OUT_ATOL
    assert fin_err <= STATE_RTOL


def test_prefill_config3_full_size(oracle, device):
    """Config 3 at full size against the oracle and the sequential GPU scan."""
    cfg = CONFIGS[3]
    x = make_scan_inputs(cfg)
    d = _dev(x, device)
    print(f"[prefill c3] {cfg.name} B={cfg.B} T={cfg.T}", flush=True)
    out, fin = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])
    out_s, fin_s = gated_delta_kernel(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])
    torch.cuda.synchronize()
    print("  GPU done; running the oracle", flush=True)
    ins = [_np(x[n]) for n in ("q", "k", "v", "g", "beta", "state")]
    o_ref, f_ref, _ = oracle.scan_c(*ins, acc64=True, with_tape=False)
    out_err = float(np.max(np.abs(_np(out) - o_ref)))
    fin_err = _rel(_np(fin), f_ref)
    seq_out_err = float(np.max(np.abs(_np(out) - _np(out_s))))
    seq_fin_err = _rel(_np(fin), _np(fin_s))
    print(f"  vs oracle: out max-abs {out_err:.3e} final rel {fin_err:.3e}; "
          f"vs sequential scan: out {seq_out_err:.3e} final {seq_fin_err:.3e}", flush=True)
    assert out_err <= OUT_ATOL and fin_err <= STATE_RTOL
    assert seq_out_err <= OUT_ATOL and seq_fin_err <= STATE_RTOL


def test_prefill_strided_views_bit_identical(device):
    """q, k, v as column views of one [B, T, 2HkDk + HvDv] buffer (the layout
    the conv prologue writes) give the same bits as contiguous copies."""
    cfg = _cfg(CONFIGS[3], T=150, Hk=2, Hv=4, state_std=0.05)
    x = make_scan_inputs(cfg)
    d = _dev(x, device)
    B, T, Hk, Hv, D = cfg.B, cfg.T, cfg.Hk, cfg.Hv, 128
    buf = torch.cat([d["q"].reshape(B, T, -1), d["k"].reshape(B, T, -1),
                     d["v"].reshape(B, T, -1)], dim=-1).contiguous()
    qv = buf[..., :Hk * D].view(B, T, Hk, D)
    kv = buf[..., Hk * D:2 * Hk * D].view(B, T, Hk, D)
    vv = buf[..., 2 * Hk * D:].view(B, T, Hv, D)
    assert not qv.is_contiguous()
    out_a, fin_a = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])
    out_b, fin_b = gated_delta_prefill(qv, kv, vv, d["g"], d["beta"], d["state"])
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
    assert torch.equal(fin_a, fin_b)


def test_prefill_reused_workspace_and_repeat(device):
    """A caller-owned workspace (dirty from a larger call) gives the same bits."""
    cfg = _cfg(CONFIGS[3], T=300, Hk=2, Hv=4, state_std=0.05)
    x = make_scan_inputs(cfg)
    d = _dev(x, device)
    need = chunked_prefill_workspace_bytes(cfg.B, 600, cfg.Hv)
    ws = torch.full((need,), 0x7F, dtype=torch.uint8, device=device)
    out_a, fin_a = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])
    out_b, fin_b = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"],
                                       workspace=ws)
    out_c, fin_c = gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"],
                                       workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.equal(out_a, out_c)
    assert torch.equal(fin_a, fin_b) and torch.equal(fin_a, fin_c)


def test_prefill_rejects_bad_arguments(device):
    cfg = _cfg(CONFIGS[3], T=64, Hk=1, Hv=2)
    d = _dev(make_scan_inputs(cfg), device)
    small = torch.empty(16, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError):
        gated_delta_prefill(d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"], workspace=small)
    c64 = _cfg(CONFIGS[0], T=64)
    d64 = _dev(make_scan_inputs(c64), device)
    with pytest.raises(ValueError):
        gated_delta_prefill(d64["q"], d64["k"], d64["v"], d64["g"], d64["beta"], d64["state"])
    # The C ABI itself rejects a short workspace before any launch.
    rc = _lib.load().dflash_gdn_chunked_prefill(
        d["q"].data_ptr(), d["k"].data_ptr(), d["v"].data_ptr(), d["g"].data_ptr(),
        d["beta"].data_ptr(), d["state"].data_ptr(), small.data_ptr(), None, 1, 64, 1, 2, 128,
        128, None, small.data_ptr(), 16, None)
    assert rc == -5  # DFLASH_ERR_WORKSPACE
