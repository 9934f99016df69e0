"""dflash_greedy_accept_noalloc against dflash_greedy_accept, through the C ABI.

The allocation-free entry point keeps its argmax keys in a static device
array instead of a caller workspace; its outputs must be the workspace
entry point's, bit for bit.  Two calls in a row (the second smaller, so its
keys overwrite only part of what the first left in the shared array), a
bf16 call, a call on torch's current stream inside a HIP graph replayed
several times, and the refusal of a shape whose keys exceed the array.
"""
from __future__ import annotations

import pytest
import torch

from dflash_mlx import _lib

pytestmark = pytest.mark.gpu


def _inputs(B, N, V, seed, dtype=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, N, V, generator=gen).to(dtype)
    post = logits.float().argmax(-1).to(torch.int32)
    draft = post.clone()
    for b in range(B):  # sequence b agrees on its first b % (N + 1) tokens
        m = b % (N + 1)
        if m < N:
            draft[b, m] = (draft[b, m] + 1) % V
    return logits, draft


def _run(fn, logits, draft, device, stream=None):
    B, N, V = logits.shape
    lg, dr = logits.to(device), draft.to(device)
    post = torch.full((B, N), -7, dtype=torch.int32, device=device)
    matched = torch.full((B,), -7, dtype=torch.int32, device=device)
    bonus = torch.full((B,), -7, dtype=torch.int32, device=device)
    st = stream if stream is not None else _lib.stream_handle(device)
    args = (lg.data_ptr(), _lib.dtype_tag(lg.dtype), lg.stride(0), lg.stride(1), dr.data_ptr(),
            dr.stride(0), N, post.data_ptr(), matched.data_ptr(), bonus.data_ptr(), B, N, V)
    lib = _lib.load()
    if fn == "noalloc":
        _lib.call("dflash_greedy_accept_noalloc", *args, st)
    else:
        ws = torch.empty(max(int(lib.dflash_greedy_accept_workspace_bytes(B, N, V)), 8),
                         dtype=torch.uint8, device=device)
        _lib.call("dflash_greedy_accept", *args, ws.data_ptr(), ws.numel(), st)
    torch.cuda.synchronize()
    return post.cpu(), matched.cpu(), bonus.cpu()


@pytest.mark.parametrize("first,second", [((4, 16, 151936), (1, 16, 1024)),
                                          ((32, 16, 8192), (3, 5, 777))])
def test_noalloc_equals_workspace_entry_point_two_calls(device, first, second):
    for i, shape in enumerate((first, second)):
        print(f"[noalloc] call {i} shape {shape}", flush=True)
        logits, draft = _inputs(*shape, seed=11 + i)
        got = _run("noalloc", logits, draft, device)
        want = _run("workspace", logits, draft, device)
        for g, w in zip(got, want):
            assert torch.equal(g, w)
        assert torch.equal(got[1], torch.tensor([b % (shape[1] + 1) for b in range(shape[0])],
                                                dtype=torch.int32))


def test_noalloc_bf16_logits(device):
    logits, draft = _inputs(2, 16, 4099, seed=5, dtype=torch.bfloat16)
    got = _run("noalloc", logits, draft, device)
    want = _run("workspace", logits, draft, device)
    for g, w in zip(got, want):
        assert torch.equal(g, w)


def test_noalloc_in_a_graph_replays_like_eager(device):
    B, N, V = 2, 16, 32000
    lib = _lib.load()
    lg = torch.empty(B, N, V, device=device)
    dr = torch.empty(B, N, dtype=torch.int32, device=device)
    post = torch.empty(B, N, dtype=torch.int32, device=device)
    matched = torch.empty(B, dtype=torch.int32, device=device)
    bonus = torch.empty(B, dtype=torch.int32, device=device)
    logits, draft = _inputs(B, N, V, seed=1)
    lg.copy_(logits)
    dr.copy_(draft)
    _run("noalloc", logits, draft, device)  # the device's scratch address is resolved here
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        rc = lib.dflash_greedy_accept_noalloc(
            lg.data_ptr(), _lib.DFLASH_DTYPE_F32, lg.stride(0), lg.stride(1), dr.data_ptr(),
            dr.stride(0), N, post.data_ptr(), matched.data_ptr(), bonus.data_ptr(), B, N, V,
            s.cuda_stream)
    assert rc == 0
    for i in range(3):
        logits, draft = _inputs(B, N, V, seed=20 + i)
        lg.copy_(logits)
        dr.copy_(draft)
        junk = _run("noalloc", *_inputs(1, 3, 100, seed=90 + i), device)  # eager use between
        graph.replay()
        torch.cuda.synchronize()
        want = _run("workspace", logits, draft, device)
        print(f"[noalloc graph] replay {i} matched {matched.cpu().tolist()} junk {junk[1].tolist()}",
              flush=True)
        assert torch.equal(post.cpu(), want[0])
        assert torch.equal(matched.cpu(), want[1])
        assert torch.equal(bonus.cpu(), want[2])


def test_noalloc_refuses_shapes_beyond_its_array(device):
    """The size refusal on the device.  The buffers are real and as large as
    the shape says (2.1 GB of logits), so if the check ever stopped
    refusing, the call would compute into them rather than read past an
    allocation."""
    lib = _lib.load()
    assert int(lib.dflash_greedy_accept_noalloc_max_bytes()) == 1 << 20
    B, N, V = 8193, 16, 4096  # 131088 rows -> 1 MiB + 128 B of keys
    assert int(lib.dflash_greedy_accept_workspace_bytes(B, N, V)) > 1 << 20
    logits = torch.zeros(B * N * V, dtype=torch.float32, device=device)
    post = torch.full((B * N,), -7, dtype=torch.int32, device=device)
    rc = lib.dflash_greedy_accept_noalloc(logits.data_ptr(), _lib.DFLASH_DTYPE_F32, N * V, V, None,
                                          0, 0, post.data_ptr(), None, None, B, N, V,
                                          _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert rc == -5
    assert bool((post == -7).all())  # refused before any launch
    del logits
