"""DFlash generation through the reference's API on the MI355X hybrid target.

DFlashGenerator -> dflash_generate(_stream) -> LoadedTargetModel ->
HybridTargetModel -> HybridVerifyRunner -> libdflash_gfx950.so, on a small
hybrid model (3 gated-delta layers + 1 attention layer, vocab 1024 so the LM
head runs in its fragment-tiled form).

* Plain greedy decoding through the same facade (the prompt, then one token
  per forward) is pinned to the fp64 CPU oracle by teacher forcing: one
  oracle step over the whole generated sequence must choose each greedy
  token wherever its top-1 margin is clear, and agree on the hidden states
  the facade captures at layer_ids.
* Every verify mode of the decode loop then reproduces that greedy output
  token for token (the reference's exactness gate, ADDING_MODELS.md:76-137)
  with a drafter that proposes the greedy continuation with mistakes planted
  at known block offsets, so the acceptance lengths are known exactly; the
  drafter checks the target hidden rows it is handed against the greedy
  run's.
* Stop tokens cut the output; the KV and linear caches end at the accepted
  length.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from dflash_mlx import DFlashGenerator, LoadedTargetModel, sample_tokens
from dflash_mlx import runtime as rt
from dflash_mlx.gdn_layer import GatedDeltaConfig
from dflash_mlx.hybrid_model import HybridConfig, HybridWeights
from dflash_mlx.target import HybridTargetModel
from oracle import hybrid_oracle as ho

pytestmark = pytest.mark.gpu

CFG = HybridConfig(hidden_size=256, num_hidden_layers=4, intermediate_size=512, vocab_size=1024,
                   num_attention_heads=4, num_key_value_heads=1, head_dim=128,
                   linear=GatedDeltaConfig(linear_num_key_heads=2, linear_num_value_heads=4))
LAYER_IDS = [1, 3]
PROMPT_LEN, N_NEW, BS = 21, 56, 16
N_REF = N_NEW + BS  # greedy tokens computed: the last block may draft past N_NEW
PLAN = [3, None, 1, 15, 7, 2, None]


def _np(x):
    return x.float().cpu().numpy().astype(np.float64)


def _np_weights(w: HybridWeights):
    layers = []
    for lw in w.layers:
        d = {k: _np(v) for k, v in lw.items() if k != "gdn" and not k.startswith("w_gu_pairs")
             and not k.endswith("_tiled")}
        if "gdn" in lw:
            g = lw["gdn"]
            d.update(conv_w=_np(g.conv_weight), A_log=_np(g.A_log), dt_bias=_np(g.dt_bias),
                     norm_w=_np(g.norm_weight))
        layers.append(d)
    return dict(embed=_np(w.embed), final_norm=_np(w.final_norm), lm_head=_np(w.lm_head),
                layers=layers)


@pytest.fixture(scope="module")
def model(device):
    w = HybridWeights.random(CFG, device, seed=5, on_device=False)
    return HybridTargetModel(CFG, w, device, max_seq_len=256, block_size=BS)


def _plain_greedy(model, device, prompt, fused):
    """Plain greedy decode through the facade, one token per forward.  The
    choice is argmax over the bf16 logits of lm_head_logits (sample_tokens,
    as the reference's greedy on its bf16 logits) or, with fused, the fused
    LM-head kernel's argmax over fp32 logits (lm_head_argmax, what the
    parallel-greedy-argmax mode uses); bf16 rounding makes near ties differ.
    Returns (prompt, N_REF tokens, hidden rows [P + N_REF - 1, n * H])."""
    target = LoadedTargetModel(model=model)
    cache = target.make_cache()

    def step(tokens):
        norm, hid = model.forward_dflash(torch.tensor([tokens], dtype=torch.int32, device=device),
                                         cache, LAYER_IDS)
        last = norm[:, -1:]
        if fused:
            return int(target.lm_head_argmax(last)[0, 0]), hid[0]
        return int(sample_tokens(target.lm_head_logits(last), 0.0)[0, 0]), hid[0]

    tok, hid = step(prompt)
    toks, hiddens = [tok], [hid]
    for _ in range(N_REF - 1):
        tok, hid = step([toks[-1]])
        toks.append(tok)
        hiddens.append(hid)
    assert cache[3].offset == PROMPT_LEN + N_REF - 1
    return prompt, toks, torch.cat(hiddens)


PROMPT = torch.randint(0, CFG.vocab_size, (PROMPT_LEN,),
                       generator=torch.Generator().manual_seed(77)).tolist()


@pytest.fixture(scope="module")
def greedy(model, device):
    print("[generate] plain greedy, bf16 logits", flush=True)
    return _plain_greedy(model, device, PROMPT, fused=False)


@pytest.fixture(scope="module")
def greedy_fused(model, device):
    print("[generate] plain greedy, fused LM-head argmax", flush=True)
    return _plain_greedy(model, device, PROMPT, fused=True)


@pytest.mark.parametrize("fused", [False, True])
def test_plain_greedy_matches_the_oracle_by_teacher_forcing(model, greedy, greedy_fused, fused):
    prompt, toks, hidden = greedy_fused if fused else greedy
    lc = CFG.linear
    K1, C = lc.linear_conv_kernel_dim - 1, lc.conv_dim
    Hv, Dv, Dk = lc.linear_num_value_heads, lc.linear_value_head_dim, lc.linear_key_head_dim
    state = dict(lens=np.array([0]), conv=[np.zeros((1, K1, C))] * CFG.n_linear,
                 rec=[np.zeros((1, Hv, Dv, Dk))] * CFG.n_linear,
                 k=[np.zeros((1, CFG.num_key_value_heads, 0, CFG.head_dim))] * CFG.n_attention,
                 v=[np.zeros((1, CFG.num_key_value_heads, 0, CFG.head_dim))] * CFG.n_attention)
    seq = np.array([prompt + toks[:-1]])
    ref = ho.model_step(CFG, _np_weights(model.weights), state, seq, CFG.rms_norm_eps)
    rows = ref["logits"][0, PROMPT_LEN - 1:]
    scale = float(np.max(np.abs(rows)))
    clear = 0
    for j, tok in enumerate(toks):
        srt = np.sort(rows[j])
        if srt[-1] - srt[-2] > 2e-2 * scale:
            assert tok == int(np.argmax(rows[j])), j
            clear += 1
        else:  # a near tie: the chosen token is one of the top ones
            assert srt[-1] - rows[j][tok] <= 2e-2 * scale, j
    print(f"  greedy tokens equal to the oracle's on {clear} clear-margin rows of {N_REF}",
          flush=True)
    assert clear >= N_REF // 2
    ref_h = np.concatenate([ref["layer_hidden"][i][0] for i in LAYER_IDS], axis=-1)
    err = np.max(np.abs(_np(hidden) - ref_h)) / np.max(np.abs(ref_h))
    print(f"  captured hidden rel {err:.2e}", flush=True)
    assert err <= 3e-2


class PlantedDrafter:
    """The DFlash drafter interface (block_size, mask_token_id,
    target_layer_ids, make_cache, __call__) proposing the greedy
    continuation, wrong at block offset plan[k] of its k-th block.  Its draft
    hidden rows are rows of the LM head, whose logits peak at the row's own
    token by a wide margin at this width."""

    mask_token_id = 0
    target_layer_ids = LAYER_IDS
    block_size = BS

    def __init__(self, model, full, greedy_hidden, plan):
        self.model, self.full, self.hidden, self.plan = model, full, greedy_hidden, plan
        self.start = None
        self.calls = 0
        self.hidden_rows: list[int] = []
        self.hidden_bit_equal = True

    def make_cache(self):
        return []

    def __call__(self, noise_embedding, target_hidden, cache=None):
        rows = target_hidden.shape[1]
        prev = self.start
        self.start = PROMPT_LEN if prev is None else prev + rows
        lo = 0 if prev is None else prev
        want = self.hidden[lo:lo + rows]
        got = target_hidden[0]
        assert got.shape == want.shape
        self.hidden_bit_equal &= bool(torch.equal(got, want))
        err = float((got.float() - want.float()).abs().max() / want.float().abs().max())
        assert err <= 1e-2, err
        self.hidden_rows.append(rows)
        s = self.start
        assert torch.equal(noise_embedding[0, 0], self.model.weights.embed[self.full[s]])
        wrong = self.plan[self.calls] if self.calls < len(self.plan) else None
        toks = [self.full[s]]
        for i in range(1, noise_embedding.shape[1]):
            t = self.full[s + i]
            toks.append((t + 1) % CFG.vocab_size if i == wrong else t)
        self.calls += 1
        return (self.model.weights.lm_head[torch.tensor(toks, device=self.model.device)] * 8)[None]


def test_planted_drafts_are_what_the_lm_head_reads(model):
    w = model.weights.lm_head.float()
    assert torch.equal((w @ w.T).argmax(-1).cpu(), torch.arange(CFG.vocab_size))


def _expected_acceptance(plan):
    start, acc, k = PROMPT_LEN, [], 0
    while start < PROMPT_LEN + N_NEW:
        j = plan[k] if k < len(plan) else None
        acc.append(j if j else BS)
        start += acc[-1]
        k += 1
    return acc


@pytest.mark.parametrize("mode", rt.VERIFY_MODES)
def test_dflash_generate_reproduces_plain_greedy(model, greedy, greedy_fused, mode):
    prompt, toks, hidden = greedy_fused if mode == "parallel-greedy-argmax" else greedy
    drafter = PlantedDrafter(model, prompt + toks, hidden, PLAN)
    print(f"[generate] mode={mode}", flush=True)
    res = DFlashGenerator(model, drafter).generate_from_tokens(
        torch.tensor(prompt, dtype=torch.int32), max_new_tokens=N_NEW, verify_mode=mode,
        verify_chunk_size=4)
    print(f"  acceptance {res.metrics['acceptance_lengths']} hidden bit-equal "
          f"{drafter.hidden_bit_equal}", flush=True)
    assert res.generated_tokens == toks[:N_NEW]
    assert res.metrics["acceptance_lengths"] == _expected_acceptance(PLAN)
    acc = res.metrics["acceptance_lengths"]
    assert drafter.hidden_rows == [PROMPT_LEN] + acc[:-1]
    kv = PROMPT_LEN + sum(acc)
    assert f"3:kv={kv}" in res.metrics["target_cache_summary"]


def test_stop_token_and_cache_state(model, greedy, device):
    prompt, toks, hidden = greedy
    stop_tok = toks[30]
    first = toks.index(stop_tok)
    eos_model = HybridTargetModel(CFG, model.weights, device, max_seq_len=256, block_size=BS,
                                  eos_token_ids={stop_tok})
    drafter = PlantedDrafter(eos_model, prompt + toks, hidden, PLAN)
    events = list(DFlashGenerator(eos_model, drafter).stream_from_tokens(
        torch.tensor(prompt, dtype=torch.int32), max_new_tokens=N_NEW))
    out = events[-1].output_tokens
    assert out == prompt + toks[:first + 1]
    assert [t for e in events for t in e.token_ids] == toks[:first + 1]


def test_rollback_leaves_the_caches_of_the_accepted_prefix(model, greedy, device):
    """After one parallel-replay verify with a planted mistake, the facade's
    caches equal those of a run that fed only the accepted tokens: the next
    forward gives the same bits."""
    prompt, toks, _ = greedy
    target = LoadedTargetModel(model=model)
    dev_prompt = torch.tensor([prompt], dtype=torch.int32, device=device)
    block = [toks[0]] + toks[1:BS]
    block[6] = (block[6] + 1) % CFG.vocab_size  # drafts 1..5 right: accept 6 inputs
    a_cache = target.make_cache()
    target.forward_with_hidden_states(dev_prompt, a_cache, LAYER_IDS)
    acc, bonus, _ = rt.verify_block_parallel_replay(target, a_cache, block, BS, 0.0, LAYER_IDS)
    assert acc == 6 and bonus == toks[6]
    b_cache = target.make_cache()
    target.forward_with_hidden_states(dev_prompt, b_cache, LAYER_IDS)
    target.forward_with_hidden_states(torch.tensor([block[:acc]], dtype=torch.int32, device=device),
                                      b_cache, LAYER_IDS)
    nxt = torch.tensor([[bonus] + toks[7:7 + 4]], dtype=torch.int32, device=device)
    la, ha = target.forward_with_hidden_states(nxt, a_cache, LAYER_IDS)
    lb, hb = target.forward_with_hidden_states(nxt, b_cache, LAYER_IDS)
    assert torch.equal(la, lb) and torch.equal(ha, hb)
    assert target.cache_summary(a_cache) == target.cache_summary(b_cache)
