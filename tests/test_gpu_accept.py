"""GPU parity of the fused greedy accept (argmax + longest prefix + bonus):
bit-exact against the CPU oracle on every config and edge case."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import greedy_accept, sample_tokens
from dflash_mlx.workloads import CONFIGS, ScanConfig, make_accept_inputs

pytestmark = pytest.mark.gpu


def _check(oracle, logits_cpu, draft_cpu, device, dtype=torch.float32, label=""):
    lg = logits_cpu.to(dtype)
    post, matched, bonus = greedy_accept(lg.to(device), draft_cpu.to(device))
    torch.cuda.synchronize()
    ref_post, ref_m, ref_b = oracle.greedy_accept(lg.float().numpy(), draft_cpu.numpy())
    print(f"[accept {label}] matched {matched.cpu().tolist()[:8]}", flush=True)
    np.testing.assert_array_equal(post.cpu().numpy(), ref_post)
    np.testing.assert_array_equal(matched.cpu().numpy(), ref_m)
    np.testing.assert_array_equal(bonus.cpu().numpy(), ref_b)
    return matched.cpu().numpy()


def test_config0_known_answer(oracle, device):
    acc = make_accept_inputs(CONFIGS[0])
    m = _check(oracle, acc["logits"], acc["draft"], device, label="c0")
    assert m.tolist() == [7]


@pytest.mark.parametrize("cfg_id,B", [(1, 1), (2, 32)])
def test_benchmark_configs(oracle, device, cfg_id, B):
    cfg = ScanConfig(**{**CONFIGS[cfg_id].__dict__, "layers": 1})
    acc = make_accept_inputs(cfg, gen=torch.Generator().manual_seed(100 + cfg_id), B=B)
    m = _check(oracle, acc["logits"], acc["draft"], device, label=f"c{cfg_id}")
    np.testing.assert_array_equal(m, acc["accept"].numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_logits(oracle, device, dtype):
    cfg = ScanConfig(**{**CONFIGS[1].__dict__, "layers": 1})
    acc = make_accept_inputs(cfg, gen=torch.Generator().manual_seed(7), B=2)
    # Draft from the argmax of the rounded logits so the accept length is known.
    lg = acc["logits"].to(dtype)
    am = torch.from_numpy(oracle.argmax_rows(lg.float().numpy()))
    pos = torch.arange(cfg.T)[None]
    draft = torch.where(pos < acc["accept"][:, None], am, (am + 1) % cfg.V).to(torch.int32)
    m = _check(oracle, acc["logits"], draft, device, dtype=dtype, label=str(dtype))
    np.testing.assert_array_equal(m, acc["accept"].numpy())


def test_reference_wiring_block_minus_one(oracle, device):
    """runtime.py:145-147: draft = block[1:] (T-1 tokens) against T rows."""
    T, V = 16, 151936
    gen = torch.Generator().manual_seed(5)
    logits = torch.randn(1, T, V, generator=gen)
    post = logits[0].argmax(-1)
    for a in (0, 3, 15):
        block = [11] + [int(post[i]) if i < a else int((post[i] + 1) % V) for i in range(T - 1)]
        draft = torch.tensor([block[1:]], dtype=torch.int32)
        _, matched, bonus = greedy_accept(logits.to(device), draft.to(device), want_posterior=False)
        assert int(matched[0]) == a
        assert int(bonus[0]) == int(post[a])


def test_ties_nan_zero_and_odd_vocab(oracle, device):
    V = 1027  # not a multiple of 4: scalar tail / scalar path
    lg = torch.randn(2, 5, V, generator=torch.Generator().manual_seed(3))
    lg[0, 0, [10, 500, 1026]] = 9.0           # tie -> 10
    lg[0, 1, :] = -0.0
    lg[0, 1, 700] = 0.0                       # -0 == +0 -> 0
    lg[0, 2, [3, 800]] = float("nan")         # first NaN -> 3
    lg[1, 0, :] = float("-inf")               # all -inf -> 0
    lg[1, 1, 1026] = 50.0                     # max at the last index
    draft = torch.zeros(2, 5, dtype=torch.int32)
    _check(oracle, lg, draft, device, label="edge")
    # Strided rows: logits as a slice of a wider buffer (row stride V + 9).
    wide = torch.randn(2, 5, V + 9, generator=torch.Generator().manual_seed(4))
    view = wide.to(device)[..., :V]
    post, _, _ = greedy_accept(view, None)
    ref = oracle.argmax_rows(wide[..., :V].numpy())
    np.testing.assert_array_equal(post.cpu().numpy(), ref)


def test_sample_tokens_greedy(oracle, device):
    lg = torch.randn(3, 4, 5000, generator=torch.Generator().manual_seed(9))
    out = sample_tokens(lg.to(device), 0.0)
    assert tuple(out.shape) == (3, 4) and out.dtype == torch.int32
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.argmax_rows(lg.numpy()))


def test_full_match_has_no_bonus(device):
    lg = torch.randn(2, 4, 300, generator=torch.Generator().manual_seed(10)).to(device)
    post, _, _ = greedy_accept(lg, None)
    _, matched, bonus = greedy_accept(lg, post)
    assert matched.cpu().tolist() == [4, 4] and bonus.cpu().tolist() == [-1, -1]
