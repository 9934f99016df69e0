"""Host-side logic of the hot path: accept wiring, KV trim, cache layout and
the benchmark workloads (CPU only)."""
from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from dflash_mlx import KVCache, Qwen35TargetAdapter, longest_prefix_match, rewind_kv_caches
from dflash_mlx.workloads import CONFIGS, make_accept_inputs, make_scan_inputs


@settings(max_examples=200, deadline=None)
@given(st.lists(st.integers(0, 5), max_size=20), st.lists(st.integers(0, 5), max_size=20))
def test_longest_prefix_match_matches_oracle(a, b):
    from oracle import oracle as orc

    assert longest_prefix_match(a, b) == orc.longest_prefix_match(a, b)
    m = longest_prefix_match(a, b)
    assert a[:m] == b[:m]
    assert m == min(len(a), len(b)) or a[m] != b[m]


def test_public_names_follow_reference():
    """dflash_mlx/__init__.py:3-22 exports longest_prefix_match and
    sample_tokens; the hot-path ops keep the reference's names."""
    import dflash_mlx

    for name in ("longest_prefix_match", "sample_tokens", "advance_gated_delta_states",
                 "gated_delta_kernel", "rollback_linear_caches", "rewind_kv_caches",
                 "verify_block_parallel_replay"):
        assert name in dflash_mlx.__all__ and hasattr(dflash_mlx, name)


def test_kv_trim_is_offset_arithmetic():
    import torch

    c = KVCache()
    c.update_and_fetch(torch.zeros(1, 2, 20, 4), torch.zeros(1, 2, 20, 4))
    c.update_and_fetch(torch.ones(1, 2, 16, 4), torch.ones(1, 2, 16, 4))
    assert c.offset == 36
    accepted_inputs = 6
    rewind_kv_caches([c, object()], 16 - accepted_inputs)  # runtime.py:155
    assert c.offset == 26
    assert c.trim(100) == 26 and c.offset == 0


def test_make_cache_pattern_is_3_to_1():
    """custom_qwen35_model.py:818: layer i is linear unless (i+1) % 4 == 0."""
    cache = Qwen35TargetAdapter().make_cache(num_layers=32)
    kinds = ["kv" if isinstance(c, KVCache) else "ssm" for c in cache]
    assert kinds.count("ssm") == 24 and kinds.count("kv") == 8
    assert [i for i, k in enumerate(kinds) if k == "kv"] == [3, 7, 11, 15, 19, 23, 27, 31]


def test_scan_bytes_match_baseline_table():
    """Algorithmic bytes per scan launch, as tabulated for the benchmark."""
    assert CONFIGS[0].scan_bytes() == 1_212_928
    assert CONFIGS[1].scan_bytes() == 915_505_152
    assert CONFIGS[2].scan_bytes() == 1_220_673_536


def test_argmax_placement_follows_logit_size():
    """The fused step runs the accept's argmax inside the scan's launch only
    while the verify logits are small (c1: 9.7 MB) and a conv window exists;
    c2's 311 MB of logits get a launch of their own."""
    from dflash_mlx.step import ARGMAX_IN_SCAN_MAX_BYTES, StepShape
    from dflash_mlx.workloads import CONFIGS

    def shape(c, conv_dim=8192):
        return StepShape(L=c.layers, B=c.B, T=c.T, Hk=c.Hk, Hv=c.Hv, Dk=c.Dk, Dv=c.Dv, V=c.V,
                         conv_dim=conv_dim)

    assert shape(CONFIGS[0]).fuse_argmax() and shape(CONFIGS[1]).fuse_argmax()
    assert not shape(CONFIGS[2]).fuse_argmax()
    assert not shape(CONFIGS[1], conv_dim=0).fuse_argmax()
    edge = StepShape(L=1, B=1, T=1, Hk=1, Hv=1, Dk=1, Dv=1, V=ARGMAX_IN_SCAN_MAX_BYTES // 4,
                     conv_dim=1)
    assert edge.fuse_argmax()
    assert not StepShape(**{**edge.__dict__, "V": edge.V + 1}).fuse_argmax()


def test_single_launch_follows_window_size():
    """The whole fused step is one launch at c0 (48 KB of conv windows), two
    at c1 (1.2 MB: one workgroup would copy them slower than the scan runs)
    and three at c2 (logits too large for the scan's launch)."""
    from dflash_mlx.step import SINGLE_LAUNCH_MAX_CONV_BYTES, StepShape
    from dflash_mlx.workloads import CONFIGS

    def shape(c, **kw):
        return StepShape(**{**dict(L=c.layers, B=c.B, T=c.T, Hk=c.Hk, Hv=c.Hv, Dk=c.Dk, Dv=c.Dv,
                                   V=c.V, conv_dim=8192), **kw})

    assert shape(CONFIGS[0]).single_launch()
    assert not shape(CONFIGS[1]).single_launch()
    assert not shape(CONFIGS[2]).single_launch()
    assert not shape(CONFIGS[0], conv_dim=8190).single_launch()  # rows not 16-byte multiples
    assert not shape(CONFIGS[0], K1=5).single_launch()
    edge = shape(CONFIGS[0],
                 conv_dim=SINGLE_LAUNCH_MAX_CONV_BYTES // (2 * 3 * CONFIGS[0].layers) // 8 * 8)
    assert edge.single_launch()
    assert not StepShape(**{**edge.__dict__, "conv_dim": edge.conv_dim + 8}).single_launch()


def test_workload_inputs_follow_the_recipe():
    x = make_scan_inputs(CONFIGS[0])
    import torch

    assert x["q"].dtype == torch.bfloat16 and x["state"].abs().max() == 0
    norms = torch.linalg.vector_norm(x["k"].float(), dim=-1)
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-2)
    assert bool(((x["g"] > 0) & (x["g"] < 1)).all()) and bool(((x["beta"] > 0) & (x["beta"] < 1)).all())


@pytest.mark.parametrize("cfg_id", [0, 1])
def test_accept_inputs_have_the_drawn_accept_length(cfg_id):
    from oracle import oracle as orc

    cfg = CONFIGS[cfg_id]
    if cfg_id == 1:
        cfg = type(cfg)(**{**cfg.__dict__, "layers": 1, "state_std": 0.0})
    acc = make_accept_inputs(cfg)
    post, matched, _ = orc.greedy_accept(acc["logits"].numpy(), acc["draft"].numpy())
    np.testing.assert_array_equal(matched, acc["accept"].numpy())


def test_cache_lengths_are_checked_on_the_host():
    """The hybrid runner refuses cache lengths whose next block would fall
    outside the KV cache before any launch (dflash_attn_prep never writes
    there and flags such a sequence)."""
    import pytest
    from dflash_mlx.hybrid_model import check_cache_lengths

    assert check_cache_lengths([0, 4080], 2, 16, 4096).tolist() == [0, 4080]
    with pytest.raises(ValueError):
        check_cache_lengths([4081], 1, 16, 4096)  # 4081 + 16 > 4096
    with pytest.raises(ValueError):
        check_cache_lengths([-1, 3], 2, 16, 4096)
    with pytest.raises(ValueError):
        check_cache_lengths([1, 2, 3], 2, 16, 4096)


def test_prompt_splits_follow_the_measured_rule():
    """Split counts of the prompt pass's bf16 projections on 256 compute
    units: the largest count up to 4 whose 256 x 128 tile units still fit the
    device once; one launch when the 256 x 256 tiles fill it.  The values at
    the c4 widths are the counts measured fastest (in_proj N = 12352, q|k|v
    5120, gate|up pairs 18432)."""
    from dflash_mlx.prefill import MAX_SPLITS, prompt_splits

    want = {(12352, 128): 4, (12352, 256): 2, (12352, 512): 1, (12352, 1024): 1,
            (5120, 128): 4, (5120, 256): 4, (5120, 512): 3, (5120, 768): 2, (5120, 1024): 1,
            (18432, 128): 3, (18432, 256): 1, (18432, 4096): 1}
    for (N, P), s in want.items():
        assert prompt_splits(N, P, 256) == s, (N, P)
    for N in (16, 272, 2560, 5120, 12352, 18432):
        for P in (1, 17, 128, 300, 1000, 4096):
            s = prompt_splits(N, P, 256)
            assert 1 <= s <= MAX_SPLITS
            tiles = -(-N // 256) * -(-P // 128)
            assert s == 1 or tiles * s <= 256


def test_residual_splits_follow_the_measured_rule():
    """Split counts of the prompt pass's residual projections (N = 2560) on
    256 compute units: while the 256 x 128 tiles fill at most half the units,
    the largest count whose units fit once, at least 8 k-steps a split and at
    most 16 (the counts measured fastest or within 6 % of it); past that the
    cost model of whole rounds and partial traffic (its picks at 2048 and
    4096 rows are the counts measured fastest)."""
    from dflash_mlx.prefill import MAX_RESIDUAL_SPLITS, residual_splits

    want = {(128, 4096): 8, (256, 4096): 8, (512, 4096): 6, (1024, 4096): 3,
            (128, 2048): 4, (256, 2048): 4, (512, 2048): 4,
            (128, 9216): 16, (256, 9216): 12, (512, 9216): 6, (1024, 9216): 3,
            (2048, 2048): 3, (2048, 4096): 3, (2048, 9216): 3,
            (4096, 2048): 1, (4096, 4096): 3, (4096, 9216): 3, (8192, 9216): 3}
    for (P, K), s in want.items():
        assert residual_splits(2560, P, 256, K) == s, (P, K)
    for P in (1, 64, 128, 300, 1000, 3000, 8192):
        for K in (64, 512, 2048, 4096, 9216):
            s = residual_splits(2560, P, 256, K)
            assert 1 <= s <= MAX_RESIDUAL_SPLITS
