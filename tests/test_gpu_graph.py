"""The verify path under HIP graph capture (torch.cuda.CUDAGraph).

None of the kernels records a memset; all launch on the capturing stream.
Each captured graph is replayed several times with eager work and
synchronisations in between, and every replay is compared bit-exactly with
the same work run eagerly.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import greedy_accept
from dflash_mlx.gdn_layer import GatedDeltaConfig, GatedDeltaWeights, gdn_layer_verify
from dflash_mlx.step import StepShape, VerifyStepRunner
from dflash_mlx.workloads import (CONFIGS, ScanConfig, make_accept_inputs, make_scan_inputs,
                                  make_verify_block)

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    return graph, outs


def test_layer_verify_and_accept_graph_replays(device):
    cfg = GatedDeltaConfig()
    gen = torch.Generator().manual_seed(3)
    B, T = 1, 16
    C, Hv = cfg.conv_dim, cfg.linear_num_value_heads
    qkv = torch.randn(B, T, C, generator=gen).bfloat16().to(device)
    z = torch.randn(B, T, Hv * 128, generator=gen).bfloat16().to(device)
    a = torch.randn(B, T, Hv, generator=gen).bfloat16().to(device)
    b = torch.randn(B, T, Hv, generator=gen).bfloat16().to(device)
    conv_state = torch.randn(B, 3, C, generator=gen).bfloat16().to(device)
    state = (0.05 * torch.randn(B, Hv, 128, 128, generator=gen)).to(device)
    w = GatedDeltaWeights.random(cfg, device, gen)
    logits = torch.randn(B, T, 5000, generator=gen).to(device)
    draft = logits.argmax(-1).to(torch.int32)
    draft[0, 9] += 1

    def work():
        y, new_conv, final, tape, _ = gdn_layer_verify(qkv, z, a, b, conv_state, state, w, cfg)
        post, matched, bonus = greedy_accept(logits, draft)
        return y, new_conv, final, tape, post, matched, bonus

    eager = work()
    torch.cuda.synchronize()
    graph, outs = _capture(work)
    for replay in range(3):
        # unrelated eager work between replays
        junk = torch.randn(1 << 20, device=device).sum()
        work()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph replay {replay}] junk={float(junk):.3f}", flush=True)
        for got, want in zip(outs, eager):
            assert torch.equal(got, want), f"replay {replay} differs"
    assert int(outs[5][0]) == 9


@pytest.mark.parametrize("single_launch,argmax_in_scan,conv_in_launch", [
    (True, True, True), (True, True, False), (False, True, True), (False, False, True)])
def test_fused_step_runner_graph_replays(device, single_launch, argmax_in_scan, conv_in_launch):
    """Two fused steps captured as one graph (the keep counts alternate
    between two buffers), replayed against two eager steps each time."""
    cfg = ScanConfig(**{**CONFIGS[2].__dict__, "B": 2, "V": 3000})
    x = make_scan_inputs(cfg)
    acc = make_accept_inputs(cfg, gen=x["_gen"])
    shape = StepShape(L=1, B=2, T=16, Hk=16, Hv=32, Dk=128, Dv=128, V=3000, conv_dim=256)
    runners = []
    for _ in range(2):
        r = VerifyStepRunner(shape, device)
        r.single_launch, r.argmax_in_scan = single_launch, argmax_in_scan
        r.conv_in_launch = conv_in_launch
        for n in ("q", "k", "v", "g", "beta", "state"):
            getattr(r, n).copy_(x[n])
        r.logits.copy_(acc["logits"])
        r.block.copy_(make_verify_block(acc))
        for i, t in enumerate(r.conv_in + r.qkv):
            t.copy_(torch.randn(t.shape, generator=torch.Generator().manual_seed(i)).bfloat16())
        runners.append(r)
    eager, graphed = runners
    torch.cuda.synchronize()
    # The runner's own buffers are the graph's inputs and outputs.
    graphed.run_fused()  # eager first call (lazy per-device launch-shape queries)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.run_fused()
        graphed.run_fused()
    # Capture does not execute: reset the graphed runner's carried state (the
    # capture flipped the current keep buffer twice: back to the first).
    graphed.state.copy_(x["state"])
    graphed.keep.zero_()
    torch.cuda.synchronize()
    for step in range(4):
        eager.run_fused()
        eager.run_fused()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph step {step}] matched {graphed.matched.cpu().tolist()}", flush=True)
        assert torch.equal(graphed.matched, eager.matched)
        assert torch.equal(graphed.keep, eager.keep)
        assert torch.equal(graphed.tape, eager.tape)
        assert torch.equal(graphed.state, eager.state)
        assert torch.equal(graphed.out, eager.out)
        for a, b in zip(graphed.conv_out, eager.conv_out):
            assert torch.equal(a, b)
