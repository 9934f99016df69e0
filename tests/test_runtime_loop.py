"""The DFlash decode loop and its verify modes on the host (no GPU).

dflash_generate_stream (runtime.py:360-555 of the reference) is driven with a
deterministic recurrent fake target and a drafter that proposes the target's
own greedy continuation with mistakes planted at chosen block offsets.  The
fake target's state is a running hash of every token it has consumed, and
its KV length a token count, so a rollback or KV rewind that keeps the wrong
number of tokens changes every later token.  Checked, for all five verify
modes:

* the output equals plain greedy decoding of the fake target, token for
  token (the reference's exactness gate, ADDING_MODELS.md:76-137);
* the acceptance lengths are the planted ones (a mistake at block offset j
  accepts j inputs; a clean block accepts all of them);
* the drafter sees target hidden rows for exactly the accepted positions;
* the streamed events concatenate to the output; stop tokens and
  max_new_tokens cut the output where the reference cuts it.

The loop's device kernels (greedy accept, sampling) are replaced here by the
CPU oracle's greedy accept and argmax: this file tests the host logic only;
tests/test_gpu_generate.py runs the same loop on the GPU path.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import DFlashGenerator, LoadedTargetModel
from dflash_mlx import runtime as rt
from dflash_mlx.cache import ArraysCache, KVCache
from oracle import oracle as orc

V = 97
MOD = 1009


def _advance(h: int, tok: int) -> int:
    return (h * 31 + tok + 7) % MOD


def _next_token(h: int) -> int:
    return (h * 13 + 5) % V


def _one_hot(tokens, scale=10.0):
    x = torch.zeros(1, len(tokens), V)
    x[0, torch.arange(len(tokens)), torch.tensor(tokens)] = scale
    return x


class FakeModel:
    """Model object with the DFlash methods (forward_dflash, rollback,
    snapshot/restore, LM head); hidden state = the hash after each token."""

    device = "cpu"

    def __init__(self, eos_token_ids=()):
        self.eos_token_ids = set(eos_token_ids)
        self.forward_calls = 0

    def make_cache(self):
        lin = ArraysCache(2)
        lin[0] = torch.tensor(0)  # tokens consumed
        lin[1] = torch.tensor(0)  # hash state
        return [lin, KVCache()]

    def forward_dflash(self, inputs, cache, layer_ids, return_rollback_records=False):
        self.forward_calls += 1
        toks = [int(t) for t in torch.as_tensor(inputs).reshape(-1)]
        lin, kv = cache
        assert kv.offset == int(lin[0]), "KV length and linear state disagree"
        h0, n0 = int(lin[1]), int(lin[0])
        tape, h = [], h0
        for t in toks:
            h = _advance(h, t)
            tape.append(h)
        lin[0], lin[1] = torch.tensor(n0 + len(toks)), torch.tensor(h)
        kv.offset += len(toks)
        norm_hidden = _one_hot([_next_token(x) for x in tape])
        target_hidden = torch.tensor(tape, dtype=torch.float64).view(1, -1, 1).repeat(
            1, 1, len(layer_ids))
        if not return_rollback_records:
            return norm_hidden, target_hidden
        rec = {0: {"h0": h0, "n0": n0, "tape": tape}}
        return norm_hidden, target_hidden, rec

    def rollback_linear_caches(self, cache, records, accepted_inputs):
        r = records[0]
        a = int(accepted_inputs)
        cache[0][0] = torch.tensor(r["n0"] + a)
        cache[0][1] = torch.tensor(r["tape"][a - 1] if a >= 1 else r["h0"])

    def snapshot_linear_caches(self, cache):
        return {0: [cache[0][0].clone(), cache[0][1].clone()]}

    def restore_linear_caches(self, cache, snapshots):
        cache[0][0], cache[0][1] = snapshots[0]

    def embed_tokens(self, tokens):
        return _one_hot([int(t) for t in torch.as_tensor(tokens).reshape(-1)])

    def lm_head_logits(self, hidden):
        return hidden.float()

    def lm_head_argmax(self, hidden):
        return hidden.argmax(-1).to(torch.int32)


def greedy_reference(prompt, n):
    h = 0
    for t in prompt:
        h = _advance(h, t)
    out, hs = [], []
    for _ in range(n):
        tok = _next_token(h)
        out.append(tok)
        h = _advance(h, tok)
        hs.append(h)
    return out


class PlantedDrafter:
    """Proposes the greedy continuation, wrong at block offset plan[k] of
    its k-th block (None: every draft right).  Tracks its position from the
    number of target hidden rows it is given, as a real drafter's context
    grows."""

    mask_token_id = 0
    target_layer_ids = [1, 3]

    def __init__(self, full_ref, prompt_len, plan, block_size=16):
        self.full_ref, self.plan, self.block_size = full_ref, plan, block_size
        self.start = None
        self.prompt_len = prompt_len
        self.calls = 0
        self.hidden_rows: list[int] = []

    def make_cache(self):
        return [KVCache()]

    def __call__(self, noise_embedding, target_hidden, cache=None):
        rows = target_hidden.shape[1]
        assert target_hidden.shape[2] == len(self.target_layer_ids)
        self.hidden_rows.append(rows)
        self.start = self.prompt_len if self.start is None else self.start + rows
        s, bs = self.start, noise_embedding.shape[1]
        assert int(noise_embedding[0, 0].argmax()) == self.full_ref[s]
        wrong = self.plan[self.calls] if self.calls < len(self.plan) else None
        toks = [self.full_ref[s]]
        for i in range(1, bs):
            t = self.full_ref[s + i]
            toks.append((t + 1) % V if i == wrong else t)
        self.calls += 1
        return _one_hot(toks)


def expected_acceptance(plan, prompt_len, n_new, bs):
    start, acc, k = prompt_len, [], 0
    while start < prompt_len + n_new:
        j = plan[k] if k < len(plan) else None
        a = j if j else bs
        acc.append(a)
        start += a
        k += 1
    return acc


@pytest.fixture
def host_kernels(monkeypatch):
    """The loop's two device calls, as the CPU oracle."""

    def sample_tokens(logits, temperature):
        assert temperature < 1e-5
        return torch.from_numpy(orc.argmax_rows(logits.float().numpy())).to(torch.int32)

    def greedy_accept(logits, draft, want_posterior=True):
        post, matched, bonus = orc.greedy_accept(logits.float().numpy(), draft.numpy())
        return (torch.from_numpy(post) if want_posterior else None,
                torch.from_numpy(np.asarray(matched)), torch.from_numpy(np.asarray(bonus)))

    monkeypatch.setattr(rt, "sample_tokens", sample_tokens)
    monkeypatch.setattr(rt, "greedy_accept", greedy_accept)


PLAN = [3, None, 1, 15, 7, None, 2]


@pytest.mark.parametrize("mode", rt.VERIFY_MODES)
def test_decode_loop_reproduces_greedy(host_kernels, mode):
    prompt = [5, 17, 42, 8, 64, 23, 11]
    n_new, bs = 70, 16
    ref = greedy_reference(prompt, n_new + 2 * bs)
    full = prompt + ref
    model = FakeModel()
    drafter = PlantedDrafter(full, len(prompt), PLAN, bs)
    gen = DFlashGenerator(model, drafter)
    res = gen.generate_from_tokens(torch.tensor(prompt), max_new_tokens=n_new, verify_mode=mode,
                                   verify_chunk_size=4)
    assert res.output_tokens == full[:len(prompt) + n_new]
    assert res.generated_tokens == ref[:n_new]
    acc = expected_acceptance(PLAN, len(prompt), n_new, bs)
    assert res.metrics["acceptance_lengths"] == acc
    assert res.metrics["num_output_tokens"] == n_new
    assert drafter.hidden_rows == [len(prompt)] + acc[:-1]
    assert res.metrics["target_cache_summary"] == "0:ssm=() 1:kv=%d" % (len(prompt) + sum(acc))


def test_stream_events_concatenate_and_stop_tokens_cut(host_kernels):
    prompt = [3, 1, 4, 1, 5]
    n_new, bs = 60, 16
    ref = greedy_reference(prompt, n_new + 2 * bs)
    full = prompt + ref
    stop_at = 23  # a generated position inside a block
    stop_tok = ref[stop_at]
    first = ref.index(stop_tok)
    target = LoadedTargetModel(model=FakeModel(eos_token_ids={stop_tok}))
    events = list(DFlashGenerator(target, PlantedDrafter(full, len(prompt), PLAN, bs))
                  .stream_from_tokens(torch.tensor(prompt), max_new_tokens=n_new))
    assert events[-1].finished and events[-1].metrics is not None
    streamed = [t for e in events for t in e.token_ids]
    out = events[-1].output_tokens
    assert out == full[:len(prompt) + first + 1]
    assert streamed == out[len(prompt):]
    assert events[0].token_ids == [ref[0]]  # the prefill's token comes first
    assert all(e.generated_tokens == e.output_tokens[len(prompt):] for e in events)


@pytest.mark.parametrize("n_new", [1, 2, 17, 33])
def test_max_new_tokens_cuts_inside_a_block(host_kernels, n_new):
    prompt = [9, 9, 9]
    bs = 16
    ref = greedy_reference(prompt, n_new + 2 * bs)
    full = prompt + ref
    res = DFlashGenerator(FakeModel(), PlantedDrafter(full, len(prompt), [None] * 8, bs)) \
        .generate_from_tokens(torch.tensor(prompt), max_new_tokens=n_new)
    assert res.output_tokens == full[:len(prompt) + n_new]


def test_speculative_tokens_shrinks_the_block(host_kernels):
    prompt = [1, 2, 3]
    n_new = 20
    ref = greedy_reference(prompt, n_new + 40)
    full = prompt + ref
    drafter = PlantedDrafter(full, len(prompt), [None] * 20, 16)
    res = DFlashGenerator(FakeModel(), drafter).generate_from_tokens(
        torch.tensor(prompt), max_new_tokens=n_new, speculative_tokens=4)
    assert res.output_tokens == full[:len(prompt) + n_new]
    assert set(res.metrics["acceptance_lengths"]) == {4}
    assert res.metrics["speculative_tokens"] == 4


def test_greedy_argmax_mode_refuses_sampling(host_kernels):
    with pytest.raises(ValueError):
        rt.verify_block_parallel_greedy_argmax(None, [], [1, 2], 2, 0.5, [0])
    with pytest.raises(ValueError):
        list(rt.dflash_generate_stream(None, None, [1], 1, 0.0, set(), [0], None, "bogus", 4))


def test_planted_mistake_is_caught_by_the_loop_test(host_kernels, monkeypatch):
    """A rollback that keeps one token too many must break the greedy match
    (so the tests above would see such a bug)."""
    orig = FakeModel.rollback_linear_caches

    def off_by_one(self, cache, records, accepted_inputs):
        orig(self, cache, records, min(accepted_inputs + 1, len(records[0]["tape"])))
        cache[0][0] = torch.tensor(records[0]["n0"] + accepted_inputs)  # keep the KV check quiet

    monkeypatch.setattr(FakeModel, "rollback_linear_caches", off_by_one)
    prompt = [5, 17, 42]
    ref = greedy_reference(prompt, 80)
    try:
        res = DFlashGenerator(FakeModel(), PlantedDrafter(prompt + ref, 3, PLAN, 16)) \
            .generate_from_tokens(torch.tensor(prompt), max_new_tokens=40)
    except AssertionError:
        return  # the drafter saw a block that does not start on the greedy path
    assert res.output_tokens != (prompt + ref)[:43]
