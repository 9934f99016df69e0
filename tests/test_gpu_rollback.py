"""GPU parity of the cache rollback (tape gather + conv window), bit-exact
against the CPU oracle, and an end-to-end verify step through
verify_block_parallel_replay with a toy gated-delta target."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import (
    ArraysCache,
    KVCache,
    advance_gated_delta_states,
    conv_rollback,
    gated_delta_verify,
    make_rollback_record,
    rewind_kv_caches,
    rollback_linear_caches,
    tape_select,
    verify_block_parallel_replay,
)

pytestmark = pytest.mark.gpu


def test_tape_select_many_layers(oracle, device):
    """40 layers (more than one launch's pointer table), per-sequence a in 0..T."""
    gen = torch.Generator().manual_seed(1)
    L, T, B = 40, 16, 4
    tapes = [torch.randn(T, B, 2, 16, 64, generator=gen) for _ in range(L)]
    s0 = [torch.randn(B, 2, 16, 64, generator=gen) for _ in range(L)]
    acc = torch.tensor([0, 1, 9, 16], dtype=torch.int32)
    print("[tape_select L=40]", flush=True)
    out = tape_select([t.to(device) for t in tapes], [s.to(device) for s in s0], acc.to(device))
    for l in range(L):
        np.testing.assert_array_equal(out[l].cpu().numpy(),
                                      oracle.tape_select(tapes[l].numpy(), s0[l].numpy(), acc.numpy()))


def test_tape_select_in_place_and_scalar_path(oracle, device):
    gen = torch.Generator().manual_seed(2)
    T, B = 5, 3
    tape = torch.randn(T, B, 3, 5, 7, generator=gen)   # 105 floats per state: scalar path
    s0 = torch.randn(B, 3, 5, 7, generator=gen)
    acc = torch.tensor([2, 0, 5], dtype=torch.int32)
    st = s0.to(device)
    tape_select([tape.to(device)], [st], acc.to(device), states_out=[st])
    np.testing.assert_array_equal(st.cpu().numpy(), oracle.tape_select(tape.numpy(), s0.numpy(), acc.numpy()))


@pytest.mark.parametrize("dtype,C,T", [(torch.bfloat16, 8192, 16), (torch.float32, 8192, 16),
                                       (torch.bfloat16, 37, 16),
                                       (torch.bfloat16, 8192, 24)])  # T + K1 > 20: rows loaded after the count
def test_conv_rollback(oracle, device, dtype, C, T):
    gen = torch.Generator().manual_seed(3)
    L, B, K1 = 3, 2, 3
    conv = [torch.randn(B, K1, C, generator=gen).to(dtype) for _ in range(L)]
    qkv = [torch.randn(B, T, C, generator=gen).to(dtype) for _ in range(L)]
    for accs in ([0, T], [1, 2], [3, 7]):
        acc = torch.tensor(accs, dtype=torch.int32)
        print(f"[conv_rollback {dtype} C={C} a={accs}]", flush=True)
        out = conv_rollback([c.to(device) for c in conv], [q.to(device) for q in qkv], acc.to(device))
        for l in range(L):
            ref = oracle.conv_rollback(conv[l].float().numpy(), qkv[l].float().numpy(), accs)
            np.testing.assert_array_equal(out[l].float().cpu().numpy(), ref)
    # In place, qkv as a strided view of a wider projection output.
    wide = torch.randn(B, T, C + 16, generator=gen).to(dtype)
    cd = conv[0].to(device)
    conv_rollback([cd], [wide.to(device)[..., :C]], 5, conv_out=[cd])
    ref = oracle.conv_rollback(conv[0].float().numpy(), wide[..., :C].float().numpy(), [5, 5])
    np.testing.assert_array_equal(cd.float().cpu().numpy(), ref)


class ToyGatedDeltaTarget:
    """Minimal target for the verify orchestration: L gated-delta layers whose
    per-token inputs come from token-indexed tables (so a token's inputs never
    depend on the batch), and logits that make the greedy continuation of
    token x equal succ[x].  Follows the LoadedTargetModel facade used by
    verify_block_parallel_replay (dflash_mlx/adapters.py:755-823)."""

    def __init__(self, device, L=3, V=64, Hk=2, Hv=4, Dk=64, Dv=64, K1=3, seed=0):
        gen = torch.Generator().manual_seed(seed)
        self.device = device
        self.L, self.V, self.Hk, self.Hv, self.Dk, self.Dv, self.K1 = L, V, Hk, Hv, Dk, Dv, K1
        self.C = 2 * Hk * Dk + Hv * Dv
        unit = lambda x: x / x.norm(dim=-1, keepdim=True)
        self.q_tab = unit(torch.randn(L, V, Hk, Dk, generator=gen)).bfloat16().to(device)
        self.k_tab = unit(torch.randn(L, V, Hk, Dk, generator=gen)).bfloat16().to(device)
        self.v_tab = torch.randn(L, V, Hv, Dv, generator=gen).bfloat16().to(device)
        self.g_tab = torch.sigmoid(torch.randn(L, V, Hv, generator=gen) + 2).to(device)
        self.b_tab = torch.sigmoid(torch.randn(L, V, Hv, generator=gen)).to(device)
        self.qkv_tab = torch.randn(L, V, self.C, generator=gen).bfloat16().to(device)
        self.succ = torch.randperm(V, generator=gen)
        logit_tab = torch.randn(V, V, generator=gen)
        logit_tab[torch.arange(V), self.succ] = 100.0
        self.logit_tab = logit_tab.to(device)

    def make_cache(self):
        gen = torch.Generator().manual_seed(99)
        cache = []
        for l in range(self.L):
            c = ArraysCache(2)
            c[0] = torch.randn(1, self.K1, self.C, generator=gen).bfloat16().to(self.device)
            c[1] = (0.05 * torch.randn(1, self.Hv, self.Dv, self.Dk, generator=gen)).to(self.device)
            cache.append(c)
        cache.append(KVCache())
        return cache

    def layer_inputs(self, l, tokens):
        t = tokens.long()
        return (self.q_tab[l][t], self.k_tab[l][t], self.v_tab[l][t], self.g_tab[l][t],
                self.b_tab[l][t], self.qkv_tab[l][t])

    def forward_with_hidden_states(self, inputs, cache, layer_ids, return_rollback_records=False):
        records = {}
        for l in range(self.L):
            q, k, v, g, b, qkv = self.layer_inputs(l, inputs)
            s0, conv0 = cache[l][1], cache[l][0]
            out, fin, tape = gated_delta_verify(q, k, v, g, b, s0)
            cache[l][1] = fin
            cache[l][0] = torch.cat([conv0, qkv], dim=1)[:, -self.K1:]
            records[l] = make_rollback_record(conv0, s0, qkv, tape)
        kv = cache[self.L]
        T = inputs.shape[1]
        z = torch.zeros(1, 1, T, 4, device=self.device)
        kv.update_and_fetch(z, z)
        logits = self.logit_tab[inputs.long()]
        hidden = torch.zeros(1, T, 8, device=self.device)
        return (logits, hidden, records) if return_rollback_records else (logits, hidden)

    def rewind_kv_caches(self, cache, n):
        rewind_kv_caches(cache, n)

    def rollback_linear_caches(self, cache, records, accepted_inputs):
        rollback_linear_caches(cache, records, accepted_inputs)


@pytest.mark.parametrize("accept_len", [0, 4, 14, 15])
def test_verify_block_parallel_replay_end_to_end(oracle, device, accept_len):
    tgt = ToyGatedDeltaTarget(device)
    cache = tgt.make_cache()
    T = 16
    s_before = [cache[l][1].clone() for l in range(tgt.L)]
    c_before = [cache[l][0].clone() for l in range(tgt.L)]
    kv_before = cache[tgt.L].offset
    tok = 5
    block = [tok]
    for i in range(T - 1):
        nxt = int(tgt.succ[block[-1]])
        block.append(nxt if i < accept_len else (nxt + 1) % tgt.V)
    print(f"[verify e2e accept_len={accept_len}]", flush=True)
    accepted_inputs, bonus, hidden = verify_block_parallel_replay(
        tgt, cache, block, T, 0.0, [0])
    assert accepted_inputs == accept_len + 1
    assert bonus == int(tgt.succ[block[accepted_inputs - 1]])
    assert hidden.shape[1] == accepted_inputs
    assert cache[tgt.L].offset == kv_before + accepted_inputs
    toks = torch.tensor([block[:accepted_inputs]], dtype=torch.int32, device=device)
    for l in range(tgt.L):
        q, k, v, g, b, qkv = tgt.layer_inputs(l, toks)
        # The rolled-back state is bit-identical to replaying the accepted prefix.
        rep = advance_gated_delta_states(s_before[l], k, v, g, b)
        assert torch.equal(cache[l][1], rep)
        ref_conv = oracle.conv_rollback(c_before[l].float().cpu().numpy(),
                                        qkv.float().cpu().numpy(), [accepted_inputs])
        np.testing.assert_array_equal(cache[l][0].float().cpu().numpy(), ref_conv)


def test_device_side_accept_rollback_batched(oracle, device):
    """Batched serving: per-sequence accepted counts stay on the device and
    drive the state and conv gathers directly (no host sync)."""
    gen = torch.Generator().manual_seed(6)
    B, T, Hk, Hv, D, C, K1 = 4, 16, 2, 4, 64, 512, 3
    q = (torch.randn(B, T, Hk, D, generator=gen) / 8).bfloat16().to(device)
    k = torch.nn.functional.normalize(torch.randn(B, T, Hk, D, generator=gen), dim=-1).bfloat16().to(device)
    v = torch.randn(B, T, Hv, D, generator=gen).bfloat16().to(device)
    g = torch.rand(B, T, Hv, generator=gen).to(device)
    be = torch.rand(B, T, Hv, generator=gen).to(device)
    s0 = (0.05 * torch.randn(B, Hv, D, D, generator=gen)).to(device)
    conv0 = torch.randn(B, K1, C, generator=gen).bfloat16().to(device)
    qkv = torch.randn(B, T, C, generator=gen).bfloat16().to(device)
    _, fin, tape = gated_delta_verify(q, k, v, g, be, s0)
    cache = [ArraysCache(2)]
    cache[0][0], cache[0][1] = conv0, fin
    acc = torch.tensor([0, 3, 11, 16], dtype=torch.int32, device=device)
    rollback_linear_caches(cache, {0: make_rollback_record(conv0, s0, qkv, tape)}, acc)
    torch.cuda.synchronize()
    for b, a in enumerate([0, 3, 11, 16]):
        want = s0[b] if a == 0 else tape[a - 1, b]
        assert torch.equal(cache[0][1][b], want)
    ref_conv = oracle.conv_rollback(conv0.float().cpu().numpy(), qkv.float().cpu().numpy(), [0, 3, 11, 16])
    np.testing.assert_array_equal(cache[0][0].float().cpu().numpy(), ref_conv)


def _step_inputs(gen, Bt, T, Hk, Hv, D, device):
    q = torch.nn.functional.normalize(torch.randn(Bt, T, Hk, D, generator=gen), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(Bt, T, Hk, D, generator=gen), dim=-1).bfloat16()
    v = torch.randn(Bt, T, Hv, D, generator=gen).bfloat16()
    g = torch.exp(-torch.nn.functional.softplus(torch.randn(Bt, T, Hv, generator=gen)))
    be = torch.sigmoid(torch.randn(Bt, T, Hv, generator=gen))
    return [t.to(device) for t in (q, k, v, g, be)]


@pytest.mark.parametrize("in_place", [False, True])
def test_fused_rollback_scan_equals_gather_then_scan(device, in_place):
    """Three verify steps of 2 stacked layers x 3 sequences: the fused scan
    (state read from the previous tape at the device-side accepted count) gives
    bit-identical out and tape to tape_select followed by the plain scan."""
    from dflash_mlx import gated_delta_verify_rollback

    gen = torch.Generator().manual_seed(11)
    L, B, T, Hk, Hv, D = 2, 3, 16, 2, 4, 128
    Bt = L * B
    s0 = (0.05 * torch.randn(Bt, Hv, D, D, generator=gen)).to(device)
    accepts = [[0, 5, 16], [16, 1, 0], [7, 7, 2]]
    # explicit
    st_e = s0.clone()
    tape_e = torch.zeros(T, Bt, Hv, D, D, device=device)
    # fused
    st_f = s0.clone()
    tape_f = torch.zeros(T, Bt, Hv, D, D, device=device)
    acc_f = torch.zeros(B, dtype=torch.int32, device=device)
    for step, acc in enumerate(accepts):
        print(f"[fused step {step} in_place={in_place}]", flush=True)
        q, k, v, g, be = _step_inputs(gen, Bt, T, Hk, Hv, D, device)
        out_e, _, tape_new = gated_delta_verify(q, k, v, g, be, st_e)
        out_f, tape_out = gated_delta_verify_rollback(
            q, k, v, g, be, st_f, tape_f, acc_f, accepted_period=B,
            tape_out=tape_f if in_place else None)
        assert torch.equal(st_f, st_e), f"rolled-back state differs at step {step}"
        assert torch.equal(out_f, out_e) and torch.equal(tape_out, tape_new)
        tape_f = tape_out
        # rollback for the next step
        acc_t = torch.tensor(acc, dtype=torch.int32, device=device)
        st_e = tape_select([tape_new], [st_e], acc_t.repeat(L))[0]
        acc_f = acc_t
        tape_e = tape_new
    del tape_e


FORMS = {"single": (True, True, True), "single_conv_apart": (True, True, False),
         "argmax_in_scan": (False, True, True), "separate": (False, False, True)}


def _set_form(r, form):
    """single_launch, argmax_in_scan, conv_in_launch of a VerifyStepRunner by
    form name."""
    r.single_launch, r.argmax_in_scan, r.conv_in_launch = FORMS[form]


@pytest.mark.parametrize("form", list(FORMS))
def test_step_runner_fused_matches_explicit(device, form):
    """VerifyStepRunner: run_fused (rollback folded into the next scan) and run
    (explicit gather) leave the same rolled-back state and the same tape, with
    the whole fused step in one launch (the conv windows copied in it or in
    a launch of their own), the accept's argmax in the scan's launch, or in
    its own."""
    from dflash_mlx.step import StepShape, VerifyStepRunner
    from dflash_mlx.workloads import (CONFIGS, ScanConfig, make_accept_inputs, make_scan_inputs,
                                      make_verify_block)

    cfg = ScanConfig(**{**CONFIGS[2].__dict__, "B": 4, "V": 5000})
    x = make_scan_inputs(cfg)
    acc = make_accept_inputs(cfg, gen=x["_gen"])
    shape = StepShape(L=1, B=4, T=16, Hk=16, Hv=32, Dk=128, Dv=128, V=5000, conv_dim=512)
    runs = []
    for fused in (False, True):
        assert not VerifyStepRunner(shape, device).argmax_in_scan  # dependent schedule by default
        r = VerifyStepRunner(shape, device, overlap_accept=True)
        # 1.3 MB of logits and 32 KB of windows: with the logits given before
        # the scan, one launch
        assert r.argmax_in_scan and r.single_launch and r.conv_in_launch
        _set_form(r, form)
        for n in ("q", "k", "v", "g", "beta", "state"):
            getattr(r, n).copy_(x[n])
        r.logits.copy_(acc["logits"])
        r.block.copy_(make_verify_block(acc))
        for i, t in enumerate(r.conv_in + r.qkv):
            t.copy_(torch.randn(t.shape, generator=torch.Generator().manual_seed(i)).bfloat16())
        (r.run_fused if fused else r.run)()
        torch.cuda.synchronize()
        # drafts block[1:] against posterior rows 0..14 (the reference's wiring)
        matched = [min(a, 15) for a in acc["accept"].tolist()]
        assert r.matched.cpu().tolist() == matched
        assert r.keep.cpu().tolist() == [m + 1 for m in matched]
        runs.append(r)
    explicit, fused = runs
    for a, b in zip(explicit.conv_out, fused.conv_out):
        assert torch.equal(a, b)
    assert torch.equal(explicit.tape, fused.tape)
    assert torch.equal(explicit.out, fused.out)
    assert torch.equal(fused.rolled_back_state(), explicit.new_state)


@pytest.mark.parametrize("B,N,V,L,K1,C,offset,dtype", [
    (1, 16, 151936, 24, 3, 8192, 0, torch.float32),   # the c1 step: 24 layers, 16-byte units
    (3, 16, 3000, 2, 3, 100, 1, torch.bfloat16),      # ragged C (2-byte units), keep = matched + 1
    (2, 5, 1000, 40, 2, 64, 1, torch.float16),        # more layers than one launch holds
    (2, 24, 2000, 3, 3, 256, 1, torch.bfloat16),      # T + K1 > 20: window rows loaded after the count
])
def test_accept_conv_rollback_matches_two_calls(device, B, N, V, L, K1, C, offset, dtype):
    """dflash_greedy_accept_conv_rollback (finalize inside the window copy)
    gives the bits of dflash_greedy_accept then dflash_conv_rollback with
    accepted = matched + offset: posterior, matched, bonus and every window."""
    import ctypes

    from dflash_mlx import _lib, greedy_accept

    print(f"[accept+conv B={B} N={N} V={V} L={L} K1={K1} C={C} offset={offset} {dtype}]", flush=True)
    gen = torch.Generator().manual_seed(B * 131 + L)
    logits = torch.randn(B, N, V, generator=gen).to(dtype)
    am = logits.float().argmax(-1).to(torch.int32)
    accept = torch.randint(0, N + 1, (B,), generator=gen, dtype=torch.int32)
    pos = torch.arange(N, dtype=torch.int32)[None, :]
    draft = torch.where(pos < accept[:, None], am, (am + 1) % V).to(torch.int32)
    conv = [torch.randn(B, K1, C, generator=gen).bfloat16() for _ in range(L)]
    qkv = [torch.randn(B, N, C, generator=gen).bfloat16() for _ in range(L)]
    ld, dd = logits.to(device), draft.to(device)

    post_a, m_a, b_a = greedy_accept(ld, dd)
    conv_a = conv_rollback([c.to(device) for c in conv], [q.to(device) for q in qkv], m_a + offset)

    lib = _lib.load()
    ws = torch.empty(int(lib.dflash_greedy_accept_workspace_bytes(B, N, V)), dtype=torch.uint8,
                     device=device)
    post_b = torch.full((B, N), -7, dtype=torch.int32, device=device)
    m_b = torch.full((B,), -7, dtype=torch.int32, device=device)
    b_b = torch.full((B,), -7, dtype=torch.int32, device=device)
    keep = torch.full((B,), -7, dtype=torch.int32, device=device)
    cin = [c.to(device) for c in conv]
    qd = [q.to(device) for q in qkv]
    cout = [torch.empty_like(c) for c in cin]
    _lib.call("dflash_greedy_accept_conv_rollback", ld.data_ptr(), _lib.dtype_tag(dtype), N * V, V,
              dd.data_ptr(), N, N, post_b.data_ptr(), m_b.data_ptr(), b_b.data_ptr(), B, N, V,
              ws.data_ptr(), ws.numel(), _lib.ptr_array(cin), _lib.ptr_array(qd),
              _lib.ptr_array(cout), offset, keep.data_ptr(), L, N, K1, C, N * C, C, 2,
              _lib.stream_handle(device))
    torch.cuda.synchronize()
    assert m_b.cpu().tolist() == accept.tolist()
    assert keep.cpu().tolist() == [min(a + offset, N) for a in accept.tolist()]
    assert torch.equal(post_a, post_b) and torch.equal(m_a, m_b) and torch.equal(b_a, b_b)
    for l in range(L):
        assert torch.equal(conv_a[l], cout[l]), f"layer {l}"


@pytest.mark.parametrize("B,Hk,Hv,D,V,dtype", [
    (1, 4, 4, 64, 1024, torch.float32),     # c0 shapes
    (3, 16, 32, 128, 5000, torch.bfloat16),  # batched, GQA, bf16 logits
])
def test_scan_with_argmax_matches_separate_launches(device, B, Hk, Hv, D, V, dtype):
    """dflash_gdn_verify_scan_rollback_argmax + dflash_accept_keys_conv_rollback
    (the accept's argmax in the scan's launch) against
    dflash_gdn_verify_scan_rollback + dflash_greedy_accept_conv_rollback over
    two chained steps (the second starts from the first one's keep): out,
    tape, state, posterior, matched, bonus, keep and every conv window
    bit-identical."""
    from dflash_mlx import _lib

    T, L, K1, C = 16, 2, 3, 96
    print(f"[scan+argmax B={B} Hk={Hk} Hv={Hv} D={D} V={V} {dtype}]", flush=True)
    gen = torch.Generator().manual_seed(B * 7 + V)
    lib = _lib.load()
    st = _lib.stream_handle(device)
    steps = []
    for _ in range(2):
        q = torch.randn(B, T, Hk, D, generator=gen).bfloat16()
        k = torch.nn.functional.normalize(torch.randn(B, T, Hk, D, generator=gen), dim=-1).bfloat16()
        v = torch.randn(B, T, Hv, D, generator=gen).bfloat16()
        g = torch.sigmoid(torch.randn(B, T, Hv, generator=gen)) * 0.5 + 0.5
        beta = torch.sigmoid(torch.randn(B, T, Hv, generator=gen))
        logits = torch.randn(B, T, V, generator=gen).to(dtype)
        am = logits.float().argmax(-1).to(torch.int32)
        acc = torch.randint(0, T + 1, (B,), generator=gen, dtype=torch.int32)
        pos = torch.arange(T, dtype=torch.int32)[None, :]
        draft = torch.where(pos < acc[:, None], am, (am + 1) % V)
        block = torch.zeros(B, T, dtype=torch.int32)
        block[:, 1:] = draft[:, :-1]
        qkv = [torch.randn(B, T, C, generator=gen).bfloat16() for _ in range(L)]
        steps.append([t.to(device) for t in (q, k, v, g, beta, logits, block)] +
                     [[x.to(device) for x in qkv]])
    state0 = (0.05 * torch.randn(B, Hv, D, D, generator=gen)).to(device)
    conv0 = [torch.randn(B, K1, C, generator=gen).bfloat16().to(device) for _ in range(L)]
    results = []
    for joint in (True, False):
        state = state0.clone()
        tape = torch.zeros(T, B, Hv, D, D, device=device)
        keep = torch.zeros(B, dtype=torch.int32, device=device)
        conv = [c.clone() for c in conv0]
        ws = torch.empty(int(lib.dflash_greedy_accept_workspace_bytes(B, T, V)), dtype=torch.uint8,
                         device=device)
        got = []
        for q, k, v, g, beta, logits, block, qkv in steps:
            out = torch.empty(B, T, Hv, D, device=device).bfloat16()
            post = torch.full((B, T), -7, dtype=torch.int32, device=device)
            matched = torch.full((B,), -7, dtype=torch.int32, device=device)
            bonus = torch.full((B,), -7, dtype=torch.int32, device=device)
            scan = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                    state.data_ptr(), tape.data_ptr(), keep.data_ptr(), T, B, out.data_ptr(), None,
                    tape.data_ptr(), B, T, Hk, Hv, D, D, None)
            cv = (_lib.ptr_array(conv), _lib.ptr_array(qkv), _lib.ptr_array(conv), 1,
                  keep.data_ptr(), L, T, K1, C, T * C, C, 2)
            if joint:
                _lib.call("dflash_gdn_verify_scan_rollback_argmax", *scan, logits.data_ptr(),
                          _lib.dtype_tag(dtype), T * V, V, B, T, V, ws.data_ptr(), ws.numel(), st)
                _lib.call("dflash_accept_keys_conv_rollback", block.data_ptr() + 4, T, T - 1,
                          post.data_ptr(), matched.data_ptr(), bonus.data_ptr(), B, T, V,
                          ws.data_ptr(), ws.numel(), *cv, st)
            else:
                _lib.call("dflash_gdn_verify_scan_rollback", *scan, st)
                _lib.call("dflash_greedy_accept_conv_rollback", logits.data_ptr(),
                          _lib.dtype_tag(dtype), T * V, V, block.data_ptr() + 4, T, T - 1,
                          post.data_ptr(), matched.data_ptr(), bonus.data_ptr(), B, T, V,
                          ws.data_ptr(), ws.numel(), *cv, st)
            torch.cuda.synchronize()
            got += [out.clone(), tape.clone(), state.clone(), post.clone(), matched.clone(),
                    bonus.clone(), keep.clone()] + [c.clone() for c in conv]
        results.append(got)
    for a, b in zip(*results):
        assert torch.equal(a, b)


def _one_launch_inputs(L, B, T, V, C, Hk, Hv, K1, seed, device):
    g = torch.Generator().manual_seed(seed)
    Bt, D = L * B, 128
    x = dict(
        q=torch.randn(Bt, T, Hk, D, generator=g).bfloat16(),
        k=(torch.randn(Bt, T, Hk, D, generator=g) / D ** 0.5).bfloat16(),
        v=torch.randn(Bt, T, Hv, D, generator=g).bfloat16(),
        g=torch.rand(Bt, T, Hv, generator=g) * 0.5 + 0.5,
        beta=torch.rand(Bt, T, Hv, generator=g),
        state=0.05 * torch.randn(Bt, Hv, D, D, generator=g),
        logits=torch.randn(B, T, V, generator=g),
        conv=[torch.randn(B, K1, C, generator=g).bfloat16() for _ in range(L)],
        qkv=[torch.randn(B, T, C, generator=g).bfloat16() for _ in range(L)],
    )
    am = x["logits"].argmax(-1).to(torch.int32)
    accept = torch.randint(0, T, (B,), generator=g, dtype=torch.int32)
    block = torch.zeros(B, T, dtype=torch.int32)
    pos = torch.arange(T - 1, dtype=torch.int32)[None, :]
    block[:, 1:] = torch.where(pos < accept[:, None], am[:, :-1], (am[:, :-1] + 1) % V)
    x["block"] = block
    return {k: ([t.to(device) for t in v] if isinstance(v, list) else v.to(device))
            for k, v in x.items()}


@pytest.mark.parametrize("L,B,T,V,C,Hk,Hv,K1,bf16", [
    (3, 2, 16, 3000, 256, 2, 4, 3, False),
    (24, 1, 16, 20000, 8192, 2, 4, 3, False),  # c1's 24 layers of 8192-channel windows
    (2, 3, 5, 1000, 64, 1, 2, 2, True),        # short block, two window rows, bf16 logits
    (1, 1, 1, 512, 128, 1, 1, 3, True),        # one token
    (2, 2, 64, 700, 64, 1, 2, 3, False),       # 64 rows, the most one finisher holds
])
def test_single_launch_step_matches_two_launches(device, L, B, T, V, C, Hk, Hv, K1, bf16):
    """dflash_gdn_verify_step (scan + rollback load + argmax, the last argmax
    workgroup of each sequence finishing the accept and the conv windows)
    gives the bits of dflash_gdn_verify_scan_rollback_argmax then
    dflash_accept_keys_conv_rollback over two steps (the second rolling back
    to the first one's keep): out, tape, state, posterior, matched, bonus,
    keep and every window; the arrival counts are zero after each call."""
    from dflash_mlx import _lib

    print(f"[single-launch step L={L} B={B} T={T} V={V} C={C} Hk={Hk} Hv={Hv} K1={K1}]",
          flush=True)
    x = _one_launch_inputs(L, B, T, V, C, Hk, Hv, K1, seed=L * 7 + B + T, device=device)
    ltag = _lib.DFLASH_DTYPE_F32
    if bf16:
        x["logits"] = x["logits"].bfloat16()
        ltag = _lib.DFLASH_DTYPE_BF16
    lib = _lib.load()
    st = _lib.stream_handle(device)
    Bt, D, i32 = L * B, 128, torch.int32
    runs = []
    for single in (False, True):
        state = x["state"].clone()
        tape = torch.zeros(T, Bt, Hv, D, D, device=device)
        out = torch.empty(Bt, T, Hv, D, dtype=torch.bfloat16, device=device)
        post = torch.full((B, T), -7, dtype=i32, device=device)
        matched = torch.full((B,), -7, dtype=i32, device=device)
        bonus = torch.full((B,), -7, dtype=i32, device=device)
        keeps = [torch.zeros(B, dtype=i32, device=device) for _ in range(3)]
        couts = [torch.full_like(c, float("nan")) for c in x["conv"]]
        nws = (int(lib.dflash_gdn_verify_step_workspace_bytes(B, T, V)) if single
               else int(lib.dflash_greedy_accept_workspace_bytes(B, T, V)))
        ws = torch.zeros(nws, dtype=torch.uint8, device=device)
        cin, qkv, cout = (_lib.ptr_array(t) for t in (x["conv"], x["qkv"], couts))
        got = []
        for step in range(2):
            kin, kout = keeps[step], keeps[step + 1]
            scan = (x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(),
                    x["beta"].data_ptr(), state.data_ptr(), tape.data_ptr(), kin.data_ptr(), T, B,
                    out.data_ptr(), None, tape.data_ptr(), Bt, T, Hk, Hv, D, D, None,
                    x["logits"].data_ptr(), ltag, T * V, V, B, T, V)
            acc = (x["block"].data_ptr() + 4, T, T - 1, post.data_ptr(), matched.data_ptr(),
                   bonus.data_ptr())
            if single:
                _lib.call("dflash_gdn_verify_step", *scan, *acc, 1, kout.data_ptr(), cin, qkv,
                          cout, L, K1, C, T * C, C, ws.data_ptr(), ws.numel(), st)
            else:
                _lib.call("dflash_gdn_verify_scan_rollback_argmax", *scan, ws.data_ptr(),
                          ws.numel(), st)
                _lib.call("dflash_accept_keys_conv_rollback", *acc, B, T, V, ws.data_ptr(),
                          ws.numel(), cin, qkv, cout, 1, kout.data_ptr(), L, T, K1, C, T * C, C,
                          2, st)
            torch.cuda.synchronize()
            got.append([t.clone() for t in (out, tape, state, post, matched, bonus, kout, *couts)])
            if single:
                counts = ws[int(lib.dflash_gdn_verify_step_workspace_bytes(B, T, V)) - 4 * B:]
                assert bool((counts == 0).all().item()), step
        runs.append(got)
    for step in range(2):
        for i, (a, b) in enumerate(zip(runs[0][step], runs[1][step])):
            assert torch.equal(a, b), (step, i)
    keep = runs[1][0][6].cpu()
    assert bool(((keep >= 1) & (keep <= T)).all())


def test_single_launch_step_validation(device):
    from dflash_mlx import _lib

    lib = _lib.load()
    f = lib.dflash_gdn_verify_step
    B, T, V, L, C, Hv = 1, 16, 1000, 1, 256, 2
    x = _one_launch_inputs(L, B, T, V, C, 1, Hv, 3, seed=1, device=device)
    st = _lib.stream_handle(device)
    tape = torch.zeros(T, B, Hv, 128, 128, device=device)
    out = torch.empty(B, T, Hv, 128, dtype=torch.bfloat16, device=device)
    keep = torch.zeros(2, B, dtype=torch.int32, device=device)
    nws = int(lib.dflash_gdn_verify_step_workspace_bytes(B, T, V))
    ws = torch.zeros(nws + 512, dtype=torch.uint8, device=device)
    couts = [torch.empty_like(c) for c in x["conv"]]
    cin, qkv, cout = (_lib.ptr_array(t) for t in (x["conv"], x["qkv"], couts))

    def call(kout=keep[1], N=T, K1=3, conv_out=cout, wsp=ws.data_ptr(), wsn=nws, cv=cin):
        return f(x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(),
                 x["beta"].data_ptr(), x["state"].data_ptr(), tape.data_ptr(),
                 keep[0].data_ptr(), T, B, out.data_ptr(), None, tape.data_ptr(), B, T, 1, Hv,
                 128, 128, None, x["logits"].data_ptr(), _lib.DFLASH_DTYPE_F32, T * V, V, B, N, V,
                 x["block"].data_ptr() + 4, T, T - 1, None, None, None, 1, kout.data_ptr(),
                 cv, qkv, conv_out, L, K1, C, T * C, C, wsp, wsn, st)

    assert call(kout=keep[0]) == -2          # writes the count its scan reads
    assert call(N=65) == -3                  # more rows than the finisher holds
    assert call(K1=5) == -3                  # more window rows than it copies
    assert call(wsn=nws - 1) == -5           # workspace too small
    assert call(wsp=ws.data_ptr() + 16) == -4  # workspace not 256-byte aligned
    odd = [c[..., 1:] for c in x["conv"]]    # rows not 16-byte aligned: 2-byte units
    assert call(cv=_lib.ptr_array(odd)) == -4
    assert call() == 0
    torch.cuda.synchronize()
