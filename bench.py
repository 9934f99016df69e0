#!/usr/bin/env python
"""Benchmark of the gated-delta verify hot path on one MI355X.

Workload (config c1): Qwen3.5-4B-shaped verify block, B=1, T=16, Hk=16, Hv=32,
Dk=Dv=128, for all 24 gated-delta layers (stacked as batch entries of one scan
launch), greedy accept over [16, 151936] fp32 logits with the reference's
wiring (drafts block[1:] against posterior rows 0..14, bonus from the row of
the first mismatch, accepted_inputs = matched + 1), and the cache rollback to
the accepted length (recurrent state + conv window, conv_dim 8192).

Two step forms are timed, both through the C ABI with preallocated buffers and
inputs resident in HBM:
  fused    (headline)  scan whose state load performs the previous step's
                       rollback (state read from the previous tape at the
                       device-side keep count) -> greedy accept + conv
                       rollback (argmax slices, then the accept's finalize
                       inside the window copy, which also writes the keep
                       count).  3 kernels, no host sync.  Timed eagerly with
                       HIP events between phases (the breakdown) and as K
                       replays of the step captured as one HIP graph (the
                       value: how the device-driven serving loop launches it).
  explicit             scan (+ final state) -> greedy accept + keep ->
                       tape gather of all 24 layers' states -> conv rollback.
                       Eager.
Each launch of the headline starts after the launch whose output it reads,
as in a decode, where the verify logits come out of the block's own scan.
Beside it, "synthetic_logits_step" times the overlapped forms (the accept's
argmax in the scan's launch), which only a benchmark with logits given
before the scan can schedule; it is labelled and never the value.
The c1 line also carries configs c0 (the reference's tiny CPU-runnable case)
and c2 (B = 32 serving batch) under "configs", each with its own roofline and
CPU baseline.  Prints one JSON line.

python bench.py [--steps K] [--warmup W] [--config 0|1|2] [--cpu-seconds S]
                [--no-configs] [--no-extras]
                [--only lm_head|layer|prefill|hybrid|gemm|prompt|decode]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "dflash-mlx_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "gated-delta verify tokens/s + HBM GB/s (% of peak), Qwen3.5-4B shape, T=16"
PEAK_HBM_GBPS = 8000.0
CONV_DIM = 8192  # 2*Hk*Dk + Hv*Dv at the Qwen3.5-4B shape


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2),
                    help="0: the reference's tiny CPU-runnable case (latency-bound); "
                         "1: the headline (default); 2: batched serving, B=32")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample of the headline config (0 disables it)")
    ap.add_argument("--cpu-seconds-other", type=float, default=4.0,
                    help="bounded CPU-baseline sample of each of c0 and c2")
    ap.add_argument("--no-configs", action="store_true",
                    help="measure only --config (by default the c1 headline also carries c0 "
                         "and c2 under 'configs')")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the measurements of the next-row kernels (fused LM head)")
    ap.add_argument("--only", choices=("lm_head", "layer", "prefill", "hybrid", "gemm", "prompt",
                                       "decode"),
                    default=None,
                    help="measure one next-row kernel alone and print its JSON (for profiling)")
    ap.add_argument("--probe", action="store_true",
                    help="for rocprofv3 --pmc runs: 3 explicit scans, 3 fused scans and 3 "
                         "calibration copies of 256 MiB, then exit without timing")
    return ap.parse_args()


PROBE_COPY_BYTES = 256 << 20


def probe(torch, fused, explicit) -> int:
    """Launch sequence for the HBM-traffic counters.  The calibration copy
    (torch's elementwise copy of a 256 MiB fp32 buffer) reads and writes
    exactly PROBE_COPY_BYTES, which scales FETCH_SIZE / WRITE_SIZE."""
    src = torch.ones(PROBE_COPY_BYTES // 4, device=fused.device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        explicit.scan()
    for _ in range(3):
        if fused.single_launch:
            fused.step_single()
        elif fused.argmax_in_scan:
            fused.scan_rolled_argmax()
        else:
            fused.scan_rolled()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] probe done: copy bytes {PROBE_COPY_BYTES}", file=sys.stderr, flush=True)
    return 0


def host_cores() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def traffic_from_profiles(workload: str):
    """HBM bytes per scan launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = ROOT / "profiles" / f"gdn_scan_{workload}_pmc.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", path.read_text())
    return int(m.group(1)) if m else None


def counter_from_profile(fname: str, key: str):
    """An integer `key: value` line of a committed profiles/ summary."""
    path = ROOT / "profiles" / fname
    if not path.exists():
        return None
    m = re.search(rf"^{key}:\s*([0-9]+)", path.read_text(), re.M)
    return int(m.group(1)) if m else None


def mfma_from_profiles(name: str):
    """Counter-measured MFMA busy fraction and executed TFLOP/s per kernel from
    a committed rocprofv3 --pmc summary (profiles/<name>_mfma_pmc.md)."""
    path = ROOT / "profiles" / f"{name}_mfma_pmc.md"
    if not path.exists():
        return None
    text = path.read_text()
    out = {}
    for key in ("mfma_busy_frac", "mfma_executed_tflops"):
        m = re.search(rf"^{key}:(.*)$", text, re.M)
        if m:
            out[key] = {k: float(v) for k, v in (kv.split("=") for kv in m.group(1).split())}
    out["source"] = f"profiles/{path.name}"
    return out


def time_steps(torch, K: int, phases):
    """Run K steps of `phases` [(name, fn)], HIP events between phases on the
    launch stream; returns wall ms/step and per-phase / whole-step GPU µs."""
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(K)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        e = ev[i]
        e[0].record()
        for j, (_, fn) in enumerate(phases):
            fn()
            e[j + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = {"ms_per_step": wall * 1e3 / K}
    for j, (name, _) in enumerate(phases):
        res[name] = sum(e[j].elapsed_time(e[j + 1]) for e in ev) * 1e3 / K
    res["gpu_step"] = sum(e[0].elapsed_time(e[-1]) for e in ev) * 1e3 / K
    return res


def measure_lm_head(torch, dev, M=16, H=2560, V=151936, n=50):
    """Fused greedy LM head + accept (MFMA, no logits) at the
    Qwen3.5-4B shape, over the row-major [V, H] weight and over its
    fragment-tiled copy (tile_weight, made once), vs the unfused path
    (hipBLASLt bf16 logits via a 2-D F.linear, then the greedy-accept
    kernel).  HBM-bound on the weight."""
    from dflash_mlx.runtime import greedy_accept, lm_head_greedy_accept, tile_weight

    gen = torch.Generator(device=dev).manual_seed(0)
    hidden = (torch.randn(M, H, generator=gen, device=dev) / H ** 0.25).to(torch.bfloat16)
    weight = (torch.randn(V, H, generator=gen, device=dev) / H ** 0.25).to(torch.bfloat16)
    draft = torch.zeros(1, M, dtype=torch.int32, device=dev)

    weight_tiled = tile_weight(weight)

    def fused():
        lm_head_greedy_accept(hidden[None], weight, draft, want_posterior=False)

    def fused_tiled():
        lm_head_greedy_accept(hidden[None], weight, draft, want_posterior=False,
                              weight_tiled=weight_tiled)

    def unfused():
        logits = torch.nn.functional.linear(hidden, weight)
        greedy_accept(logits[None], draft, want_posterior=False)

    out = {}
    for name, fn in (("fused", fused), ("fused_tiled", fused_tiled), ("unfused", unfused)):
        for _ in range(20):  # a few ms of work first: the first calls run at lower clocks
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = e0.elapsed_time(e1) * 1e3 / n
    del weight_tiled
    bytes_alg = 2 * V * H + 2 * M * H
    gbps = bytes_alg / (out["fused"] / 1e6) / 1e9
    gbps_t = bytes_alg / (out["fused_tiled"] / 1e6) / 1e9
    return {
        "shape": {"M": M, "H": H, "V": V},
        "fused_us": round(out["fused"], 2),
        "fused_tiled_us": round(out["fused_tiled"], 2),
        "unfused_us": round(out["unfused"], 2),
        "bytes_alg": bytes_alg,
        "fused_gbps": round(gbps, 1),
        "fused_frac": round(gbps / PEAK_HBM_GBPS, 4),
        "fused_tiled_gbps": round(gbps_t, 1),
        "fused_tiled_frac": round(gbps_t / PEAK_HBM_GBPS, 4),
        "note": "per call, back-to-back launches incl. Python dispatch (fused: 2 kernels over the "
                "row-major weight; fused_tiled: the same over its fragment-tiled copy; unfused: "
                "GEMM + 2 kernels)",
    }


PEAK_BF16_TFLOPS = 2500.0


def chunked_prefill_flops(T: int, heads: int, chunk: int = 64, D: int = 128) -> int:
    """Algorithmic flops of the chunked prefill (one multiply-add = 2), counted
    once per product of the chunk form regardless of how many bf16 passes the
    kernels spend on it: K K^T, Q K^T, W = T'K, U~ = T_b V (phase 1) and
    W S^T, Q S^T, P U, U^T K (phase 2) per (head, chunk), plus the triangular
    inverse (C^3 / 3)."""
    nc = -(-T // chunk)
    per = (2 * chunk * chunk * D * 2 + 2 * chunk * chunk * D * 2
           + 3 * chunk * D * D * 2 + chunk * chunk * D * 2 + chunk ** 3 // 3)
    return heads * nc * per


def measure_prefill(torch, dev, n=50):
    """Chunked (WY / UT-transform) prefill on MFMA at config c3 (B=1,
    T=8192, Hk=16, Hv=32, Dk=Dv=128, zero initial state) against the
    sequential scan kernel on the same inputs."""
    from dflash_mlx.gated_delta import (chunked_prefill_workspace_bytes, gated_delta_kernel,
                                        gated_delta_prefill)
    from dflash_mlx.workloads import CONFIGS, make_scan_inputs

    cfg = CONFIGS[3]
    x = make_scan_inputs(cfg)
    d = {k: v.to(dev) for k, v in x.items() if not k.startswith("_")}
    ws = torch.empty(chunked_prefill_workspace_bytes(cfg.B, cfg.T, cfg.Hv), dtype=torch.uint8,
                     device=dev)
    args = (d["q"], d["k"], d["v"], d["g"], d["beta"], d["state"])

    def timed(fn, reps, warm):
        # The warmup runs the GPU for a few milliseconds first: the first
        # ~5 ms of back-to-back calls run at lower clocks (measured ~350 us
        # per chunked call over the first ten against ~303 us after twenty).
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    chunked_us = timed(lambda: gated_delta_prefill(*args, workspace=ws), n, 20)
    seq_us = timed(lambda: gated_delta_kernel(*args), 3, 1)
    tokens = cfg.B * cfg.T
    flops = chunked_prefill_flops(cfg.T, cfg.B * cfg.Hv)
    hbm = (2 * tokens * (2 * cfg.Hk * cfg.Dk + 2 * cfg.Hv * cfg.Dv) + 8 * tokens * cfg.Hv
           + 2 * 4 * cfg.B * cfg.Hv * cfg.Dv * cfg.Dk)
    tflops = flops / (chunked_us / 1e6) / 1e12
    return {
        "workload": cfg.name,
        "shape": {"B": cfg.B, "T": cfg.T, "Hk": cfg.Hk, "Hv": cfg.Hv, "Dk": cfg.Dk, "Dv": cfg.Dv,
                  "chunk": 64},
        "chunked_us": round(chunked_us, 1),
        "sequential_us": round(seq_us, 1),
        "speedup_vs_sequential": round(seq_us / chunked_us, 2),
        "tokens_per_s": round(tokens / (chunked_us / 1e6), 1),
        "flops_alg": flops,
        "tflops": round(tflops, 2),
        "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "mfma_counters": mfma_from_profiles("chunked_prefill_c3-prefill-8k"),
        "hbm_bytes_alg": hbm,
        "hbm_frac": round(hbm / (chunked_us / 1e6) / 1e9 / PEAK_HBM_GBPS, 4),
        "traffic": counter_from_profile("chunked_prefill_c3-prefill-8k_traffic_pmc.md",
                                        "traffic_bytes_per_call"),
        "note": "per call incl. Python dispatch, 50 calls after 20 untimed; two kernels "
                "(chunk prep, chunk state); traffic: HBM bytes per call from FETCH_SIZE / "
                "WRITE_SIZE counters (the prep kernel's operand fragments round-trip through HBM)",
    }


def measure_gemm(torch, dev, reps=8, copies=4):
    """The c4 step's six verify-sized projection GEMMs alone (M = 16 block
    rows, fragment-tiled weights, the runner's launch plans), each timed over
    `copies` distinct weights in rotation so that, as in the step, no launch
    finds its weight in the 256 MB Infinity Cache."""
    from dflash_mlx import _lib
    from dflash_mlx.hybrid_model import HybridConfig, HybridVerifyRunner
    from dflash_mlx.runtime import tile_weight

    cfg = HybridConfig()
    lc, H, I, M = cfg.linear, cfg.hidden_size, cfg.intermediate_size, 16
    dims = {"w_in": (cfg.in_proj_rows, H), "w_out": (H, lc.value_dim),
            "w_qkv": (cfg.attn_proj_rows, H), "w_o": (H, cfg.num_attention_heads * cfg.head_dim),
            "w_gu": (2 * I, H), "w_down": (H, I)}
    lib = _lib.load()
    stream = _lib.stream_handle(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    x = (torch.randn(M, max(k for _, k in dims.values()), generator=gen, device=dev)
         ).to(torch.bfloat16)
    gws = torch.zeros(int(lib.dflash_gemm_tail_workspace_bytes()), dtype=torch.uint8, device=dev)
    res = {}
    for name, (N, K) in dims.items():
        ns, rpw, kw = HybridVerifyRunner.TILED_PLAN[name]
        ws = [tile_weight((0.02 * torch.randn(N, K, generator=gen, device=dev)).to(torch.bfloat16))
              for _ in range(copies)]
        splits = int(lib.dflash_gemm_splits(K, ns)) if ns > 1 else 0
        out = torch.empty(max(splits, 1) * M * N, dtype=torch.float32, device=dev)

        def call(w):
            if name == "w_gu":
                _lib.call("dflash_gemm_bf16_swiglu_tiled", x.data_ptr(), x.stride(0), w.data_ptr(),
                          out.data_ptr(), N // 2, M, N, K, kw, gws.data_ptr(), gws.numel(), stream)
            else:
                _lib.call("dflash_gemm_bf16_tiled", x.data_ptr(), x.stride(0), w.data_ptr(),
                          out.data_ptr(), 0 if splits else N, M, N, K, ns, rpw, kw, gws.data_ptr(),
                          gws.numel(), stream)

        for w in ws:
            call(w)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            for w in ws:
                call(w)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
        res[name] = {"N": N, "K": K, "plan": [ns, rpw, kw], "splits": splits, "us": round(us, 2),
                     "weight_gbps": round(2 * N * K / us / 1e3, 1)}
        del ws, out
    return {"M": M, "projections": res,
            "note": "per launch incl. dispatch; weights rotated over %d copies" % copies}


def measure_hybrid(torch, dev, steps=40):
    """Config c4: one verify step of the random-init Qwen3.5-4B-shaped hybrid
    target (32 layers 3:1, hidden 2560, 16/4 heads of 128, vocab 151936) on a
    4096-token cache: embed -> 32 layers -> final norm -> fused LM-head greedy
    accept -> commit (keep counts, KV lengths, conv windows; the recurrent
    states roll back inside the next step's scan).  Timed as a HIP graph of
    the whole step (no host sync inside), and eagerly for comparison."""
    from dflash_mlx.hybrid_model import HybridConfig, HybridVerifyRunner, HybridWeights

    cfg = HybridConfig()
    lc = cfg.linear
    B, T, L0, Smax = 1, 16, 4096, 4096 + 1024
    w = HybridWeights.random(cfg, dev, seed=0, on_device=True)
    gen = torch.Generator(device=dev).manual_seed(1)
    conv = [torch.randn(B, 3, lc.conv_dim, generator=gen, device=dev).bfloat16()
            for _ in range(cfg.n_linear)]
    rec = [0.05 * torch.randn(B, lc.linear_num_value_heads, lc.linear_value_head_dim,
                              lc.linear_key_head_dim, generator=gen, device=dev)
           for _ in range(cfg.n_linear)]
    kv = [torch.randn(B, cfg.num_key_value_heads, L0, cfg.head_dim, generator=gen,
                      device=dev).bfloat16() for _ in range(2 * cfg.n_attention)]
    run = HybridVerifyRunner(cfg, w, B, T, Smax, dev)
    run.set_state([L0], conv, rec, kv[0::2], kv[1::2])
    run.tokens.copy_(torch.randint(0, cfg.vocab_size, (B, T), generator=gen, device=dev,
                                   dtype=torch.int32))
    del conv, rec, kv

    def timed(fn, n):
        run.lens.fill_(L0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for _ in range(3):
        run.step()
    eager_ms = timed(run.step, 5)
    run.capture_step()
    for _ in range(3):
        run.replay()
    graph_ms = timed(run.replay, steps)
    wbytes = 2 * (w.lm_head.numel() + w.final_norm.numel() + B * T * cfg.hidden_size)
    for lw in w.layers:
        for k_, v_ in lw.items():
            # one copy of each weight is read: skip the regrouped gate|up and the
            # fragment-tiled copies the GEMMs stream in place of the originals
            if isinstance(v_, torch.Tensor) and k_ != "w_gu_pairs" and not k_.endswith("_tiled"):
                wbytes += 2 * v_.numel()
    tape_bytes = 4 * cfg.n_linear * (T + 1) * B * lc.linear_num_value_heads * \
        lc.linear_value_head_dim * lc.linear_key_head_dim
    kv_bytes = 2 * 2 * cfg.n_attention * B * cfg.num_key_value_heads * (L0 + T) * cfg.head_dim
    total = wbytes + tape_bytes + kv_bytes
    return {
        "workload": "c4-hybrid-qwen35-4b-verify",
        "shape": {"layers": cfg.num_hidden_layers, "linear_layers": cfg.n_linear,
                  "attention_layers": cfg.n_attention, "hidden": cfg.hidden_size,
                  "intermediate": cfg.intermediate_size, "vocab": cfg.vocab_size, "B": B, "T": T,
                  "kv_len": L0},
        "graph_step_ms": round(graph_ms, 4),
        "eager_step_ms": round(eager_ms, 4),
        "block_tokens_per_s": round(B * T / (graph_ms / 1e3), 1),
        "hbm_bytes_alg": total,
        "hbm_bytes_breakdown": {"weights": wbytes, "state_tape": tape_bytes, "kv_cache": kv_bytes},
        "hbm_frac": round(total / (graph_ms / 1e3) / 1e9 / PEAK_HBM_GBPS, 4),
        "reference_m4max_verify_ms": 56.7,
        "note": "random-init bf16 weights ~N(0,0.02), synthetic caches; reference figure: "
                "benchmarks/qwen35-results.md, 21.59 s verifier forward+logits over the "
                "~381 verify steps of a 2048-token decode on an M4 Max (other hardware)",
    }


def measure_prompt(torch, dev, P=4096, reps=3):
    """The drop-in's prompt pass at the config-c4 shape (the random-init
    Qwen3.5-4B-shaped target, 32 layers) over a P-token prompt from empty
    caches: HybridTargetModel.forward_dflash (the reference's prefill,
    runtime.py:384-390) through prefill.HybridPrefill.  Timed with HIP events
    around whole calls; then its parts alone on the same buffers (every
    projection on the prompt-sized MFMA GEMM, the 24 chunked gated-delta
    scans, the 8 prompt attentions), hipBLASLt on the same GEMM shapes
    (torch F.linear, row-major weights) for context, the all-row bf16 logits
    the reference's prefill also computes, and the same prompt through the
    verify runner 16 tokens at a time."""
    from dflash_mlx import _lib
    from dflash_mlx.hybrid_model import HybridConfig, HybridWeights
    from dflash_mlx.target import HybridTargetModel

    cfg = HybridConfig()
    lc = cfg.linear
    w = HybridWeights.random(cfg, dev, seed=0, on_device=True)
    toks = torch.randint(0, cfg.vocab_size, (1, P), generator=torch.Generator().manual_seed(3),
                         dtype=torch.int32).to(dev)
    layer_ids = [1, 15, 31]

    def setup(mode):
        model = HybridTargetModel(cfg, w, dev, max_seq_len=P + 64, block_size=16, prompt_pass=mode)
        return model, model.make_cache()

    def reset(model, cache):
        run = cache.runner
        for i in cache.attn_idx:
            cache[i].offset = 0
        run.keep.zero_()
        for st in run.state:
            st.zero_()
        run.conv_all.zero_()
        model._install(cache, run.state)

    def ev_time(fn, n=1):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    model, cache = setup("prefill")
    reset(model, cache)
    norm, _ = model.forward_dflash(toks, cache, layer_ids)  # buffers, tiled copies, first clocks
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        reset(model, cache)
        times.append(ev_time(lambda: model.forward_dflash(toks, cache, layer_ids)))
    prompt_ms = sorted(times)[len(times) // 2]

    # the parts alone, on the prompt pass's own buffers and weights
    pre, run = cache._prefill, cache.runner
    stream = _lib.stream_handle(dev)
    H, I = cfg.hidden_size, cfg.intermediate_size
    Hv, Dv, Hk, Dk = lc.linear_num_value_heads, lc.linear_value_head_dim, \
        lc.linear_num_key_heads, lc.linear_key_head_dim
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    gemms = []  # (name, x, x_stride, weight, out, out_stride, N, K, kind)
    for i in range(cfg.num_hidden_layers):
        t = pre.w[i]
        if cfg.is_linear(i):
            gemms.append(("w_in", pre.xn, H, t["w_in"], pre.proj, pre.in_stride, H, "plain"))
            gemms.append(("w_out", pre.gnorm, Hv * Dv, t["w_out"], None, H, Hv * Dv, "residual"))
        else:
            gemms.append(("w_qkv", pre.xn, H, t["w_qkv"], pre.aproj, cfg.attn_proj_rows, H,
                          "plain"))
            gemms.append(("w_o", pre.attn_out, Hq * D, t["w_o"], None, H, Hq * D, "residual"))
        gemms.append(("w_gu", pre.xn, H, t["w_gu_pairs"], pre.mlp_act, I, H, "swiglu"))
        gemms.append(("w_down", pre.mlp_act, I, t["w_down"], None, H, I, "residual"))

    def run_gemms():
        # as the prompt pass runs them (split-K where their tiles would
        # underfill the device: the residual projections' partials go to the
        # add + norm, the bf16 ones' through their reduce)
        for _, x, xs, (wt, n), out, os_, k, kind in gemms:
            if kind == "residual":
                pre._to_residual((wt, n), x.data_ptr(), k, P, stream)
            else:
                pre._bf16_proj((wt, n), x.data_ptr(), k, P, out.data_ptr(), os_,
                               kind == "swiglu", stream)

    gemm_flops = sum(2 * P * n * k for _, _, _, (_, n), _, _, k, _ in gemms)
    run_gemms()
    gemm_ms = ev_time(run_gemms, 2)
    C = lc.conv_dim
    import ctypes
    strides = (ctypes.c_int64 * 13)(P * C, C, Dk, P * C, C, Dk, P * C, C, Dv, P * Hv, Hv, P * Hv, Hv)
    act = pre.act.data_ptr()

    def run_chunked():
        for gi in range(cfg.n_linear):
            _lib.call("dflash_gdn_chunked_prefill", act, act + 2 * Hk * Dk, act + 4 * Hk * Dk,
                      pre.g.data_ptr(), pre.beta.data_ptr(), run.state[gi].data_ptr(),
                      pre.scan_out.data_ptr(), run.tape[gi][0].data_ptr(), 1, P, Hk, Hv, Dk, Dv,
                      strides, pre.chunk_ws.data_ptr(), pre.chunk_ws.numel(), stream)

    chunk_ms = ev_time(run_chunked, 2)
    run.lens.zero_()

    def run_attn():
        for ai in range(cfg.n_attention):
            _lib.call("dflash_attn_prefill", pre.q.data_ptr(), run.k_cache[ai].data_ptr(),
                      run.vt_cache[ai].data_ptr(), run.lens.data_ptr(), pre.aproj.data_ptr(),
                      cfg.attn_proj_rows, pre.attn_out.data_ptr(), P, Hq, Hkv, D, run.Smax,
                      float(D ** -0.5), stream)

    attn_ms = ev_time(run_attn, 2)
    attn_flops = cfg.n_attention * Hq * 2 * 2 * D * (P * (P + 1) // 2)

    # hipBLASLt on the same shapes (row-major weights), for context
    xs_ = {}
    lib_gemms = []
    for i, lw in enumerate(w.layers):
        names = (("w_in", H), ("w_out", Hv * Dv)) if cfg.is_linear(i) else (("w_qkv", H),
                                                                          ("w_o", Hq * D))
        for name, k in names + (("w_gu", H), ("w_down", I)):
            if k not in xs_:
                xs_[k] = torch.randn(P, k, device=dev).bfloat16()
            lib_gemms.append((xs_[k], lw[name]))

    def run_lib():
        for x, wt in lib_gemms:
            torch.nn.functional.linear(x, wt)

    run_lib()
    lib_ms = ev_time(run_lib, 2)
    del xs_, lib_gemms
    logits_ms = ev_time(lambda: model.lm_head_logits(norm), 2)
    del model, cache, pre, run
    torch.cuda.empty_cache()

    print("[bench] prompt pass: the same prompt through the verify runner, 16 tokens a time",
          file=sys.stderr, flush=True)
    bmodel, bcache = setup("blocks")
    reset(bmodel, bcache)
    bmodel.forward_dflash(toks[:, :64], bcache, layer_ids)
    reset(bmodel, bcache)
    block_ms = ev_time(lambda: bmodel.forward_dflash(toks, bcache, layer_ids))
    del bmodel, bcache
    torch.cuda.empty_cache()
    total_flops = gemm_flops + attn_flops
    gemm_tflops = gemm_flops / (gemm_ms / 1e3) / 1e12
    return {
        "workload": "c4-hybrid-qwen35-4b-prompt",
        "shape": {"layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size,
                  "intermediate": cfg.intermediate_size, "prompt_tokens": P, "B": 1},
        "prompt_ms": round(prompt_ms, 3),
        "prompt_tokens_per_s": round(P / (prompt_ms / 1e3), 1),
        "breakdown_ms": {"projection_gemms": round(gemm_ms, 3),
                         "chunked_gated_delta": round(chunk_ms, 3),
                         "prompt_attention": round(attn_ms, 3),
                         "other": round(prompt_ms - gemm_ms - chunk_ms - attn_ms, 3)},
        "roofline": {"kernel": "prefill_gemm_wide_kernel (dflash_gemm_bf16_tiled_prefill / _swiglu / _splitk; 256 x 256 tiles)",
                     "bound": "mfma", "flops": gemm_flops,
                     "achieved": round(gemm_tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / 2500.0, 4)},
        "pass_tflops": round(total_flops / (prompt_ms / 1e3) / 1e12, 1),
        "hipblaslt_same_gemms_ms": round(lib_ms, 3),
        "hipblaslt_tflops": round(gemm_flops / (lib_ms / 1e3) / 1e12, 1),
        "attention_tflops": round(attn_flops / (attn_ms / 1e3) / 1e12, 1),
        "all_row_logits_ms": round(logits_ms, 3),
        "block_path_ms": round(block_ms, 3),
        "speedup_vs_block_path": round(block_ms / prompt_ms, 2),
        "mfma_counters": mfma_from_profiles("prompt_pass_c4-prompt-4k"),
        "note": "random-init bf16 weights ~N(0,0.02); prompt_ms is forward_dflash from empty "
                "caches (no logits); all_row_logits_ms is the [P, 151936] bf16 LM head the "
                "reference's prefill also evaluates; hipBLASLt is context, not the product path",
    }


class _PlantedDrafter:
    """The DFlash drafter interface (block_size, mask_token_id,
    target_layer_ids, make_cache, __call__) proposing a known continuation
    with one wrong token at block offset plan[k % len(plan)] of its k-th
    block (None: none wrong), so a decode's acceptance lengths are fixed in
    advance.  Its draft hidden rows are LM-head rows scaled by 8, whose
    logits peak at the row's own token by a wide margin (w_i . w_i ~ 1 against
    |w_i . w_j| ~ 0.02 at the c4 shape)."""

    mask_token_id = 0
    block_size = 16

    def __init__(self, lm_head, continuation, prompt_len, plan, layer_ids):
        self.lm_head, self.full, self.plan = lm_head, continuation, plan
        self.target_layer_ids = layer_ids
        self.prompt_len, self.start, self.calls = prompt_len, None, 0

    def make_cache(self):
        return []

    def __call__(self, noise_embedding, target_hidden, cache=None):
        import torch

        rows = target_hidden.shape[1]
        self.start = self.prompt_len if self.start is None else self.start + rows
        wrong = self.plan[self.calls % len(self.plan)]
        s = self.start
        toks = [self.full[min(s + i, len(self.full) - 1)] for i in range(noise_embedding.shape[1])]
        if wrong is not None:
            toks[wrong] = (toks[wrong] + 1) % self.lm_head.shape[0]
        self.calls += 1
        return (self.lm_head[torch.tensor(toks, device=self.lm_head.device)] * 8)[None]


def measure_decode(torch, dev, P=256, N=192):
    """The drop-in decode step at the config-c4 shape: DFlashGenerator.
    generate_from_tokens (runtime.py:360-589 -> LoadedTargetModel ->
    HybridTargetModel) over a P-token prompt for N new tokens, with a drafter
    that proposes the target's own greedy continuation with planted
    mistakes (acceptance lengths known in advance), for the
    parallel-replay and parallel-greedy-argmax verify modes.  Reports wall
    time per verify step (host-synchronous, as the reference's loop) and the
    runtime's own profile split."""
    from dflash_mlx import DFlashGenerator, LoadedTargetModel, sample_tokens
    from dflash_mlx.hybrid_model import HybridConfig, HybridWeights
    from dflash_mlx.target import HybridTargetModel

    cfg = HybridConfig()
    w = HybridWeights.random(cfg, dev, seed=0, on_device=True)
    layer_ids = [1, 8, 15, 22, 29]
    model = HybridTargetModel(cfg, w, dev, max_seq_len=P + N + 64, block_size=16)
    target = LoadedTargetModel(model=model)
    prompt = torch.randint(0, cfg.vocab_size, (P,), generator=torch.Generator().manual_seed(5),
                           dtype=torch.int32)
    def greedy(fused):
        """The target's greedy continuation through the same facade, one token
        a forward: the first token from the prompt's bf16 logits (as the
        decode loop takes it), the rest from the bf16 logits or, as the
        parallel-greedy-argmax mode does, the fused LM-head argmax over fp32
        logits (near ties in bf16 resolve differently)."""
        cache = target.make_cache()
        norm, _ = model.forward_dflash(prompt[None].to(dev), cache, layer_ids)
        cont = prompt.tolist()
        for j in range(N + 16):
            if fused and j > 0:
                tok = int(target.lm_head_argmax(norm[:, -1:])[0, 0])
            else:
                tok = int(sample_tokens(target.lm_head_logits(norm[:, -1:]), 0.0)[0, 0])
            cont.append(tok)
            norm, _ = model.forward_dflash(torch.tensor([[tok]], dtype=torch.int32, device=dev),
                                           cache, layer_ids)
        return cont

    plan = [7, 5, 9, None, 6, 3, 11, 8]  # accepted inputs 7 5 9 16 6 3 11 8: mean 8.1
    out = {}
    for mode in ("parallel-replay", "parallel-greedy-argmax"):
        cont = greedy(mode == "parallel-greedy-argmax")
        for rep in range(2):  # the first run warms the graphs, buffers and clocks
            drafter = _PlantedDrafter(w.lm_head, cont, P, plan, layer_ids)
            gen = DFlashGenerator(target, drafter)
            res = gen.generate_from_tokens(prompt, max_new_tokens=N, verify_mode=mode,
                                           profile=True)
        m = res.metrics
        steps = len(m["acceptance_lengths"])
        prof = {k: round(v * 1e3 / steps, 3) for k, v in m["profile"].items()
                if k.endswith("_time_s")}
        agree = res.generated_tokens == cont[P:P + len(res.generated_tokens)]
        out[mode] = {"ms_per_verify_step": round(m["decode_time_s"] * 1e3 / steps, 3),
                     "steps": steps, "avg_acceptance_length": round(m["avg_acceptance_length"], 2),
                     "generation_tps": round(m["generation_tps"], 1),
                     "prefill_ms": round(m["prefill_time_s"] * 1e3, 2),
                     "ms_per_step_profile": prof, "tokens_equal_greedy": bool(agree)}
    return {"workload": "c4-hybrid-qwen35-4b-decode", "prompt_tokens": P, "new_tokens": N,
            "modes": out,
            "note": "host-synchronous decode loop through DFlashGenerator -> LoadedTargetModel "
                    "-> HybridTargetModel, one small device->host read per step as the "
                    "reference's mx.eval; the drafter network itself is not timed (planted "
                    "hidden rows); reference figure: ~57 ms a verify step on an M4 Max "
                    "(benchmarks/qwen35-results.md:23, other hardware)"}


def _graph_time_us(torch, fn, n=20):
    """Average replay time of a HIP graph capturing fn (µs)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / n


def measure_layer(torch, dev, L=24, B=1, T=16):
    """The gated-delta layer between its projections (prologue ->
    scan -> gated-norm epilogue) for L layers of the Qwen3.5-4B shape, each
    phase captured as one HIP graph of L launches, against the same prologue
    and epilogue written as torch op chains."""
    from dflash_mlx.gated_delta import gated_delta_verify
    from dflash_mlx.gdn_layer import (GatedDeltaConfig, GatedDeltaWeights, gated_rmsnorm,
                                      gdn_layer_verify, gdn_prologue)

    cfg = GatedDeltaConfig()
    gen = torch.Generator().manual_seed(0)
    C, K, Hk, Hv = cfg.conv_dim, cfg.linear_conv_kernel_dim, cfg.linear_num_key_heads, cfg.linear_num_value_heads
    Dk, Dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    layers = []
    for _ in range(L):
        layers.append(dict(
            qkv=torch.randn(B, T, C, generator=gen).bfloat16().to(dev),
            z=torch.randn(B, T, Hv * Dv, generator=gen).bfloat16().to(dev),
            a=torch.randn(B, T, Hv, generator=gen).bfloat16().to(dev),
            b=torch.randn(B, T, Hv, generator=gen).bfloat16().to(dev),
            conv=torch.randn(B, K - 1, C, generator=gen).bfloat16().to(dev),
            state=(0.05 * torch.randn(B, Hv, Dv, Dk, generator=gen)).to(dev),
            w=GatedDeltaWeights.random(cfg, dev, gen)))
    pro = [gdn_prologue(l["qkv"], l["conv"], l["a"], l["b"], l["w"], cfg) for l in layers]
    outs = [gated_delta_verify(*p[:5], l["state"])[0] for p, l in zip(pro, layers)]
    zs = [l["z"].reshape(B, T, Hv, Dv) for l in layers]

    def t_prologue():
        for l in layers:
            gdn_prologue(l["qkv"], l["conv"], l["a"], l["b"], l["w"], cfg)

    def t_scan():
        for p, l in zip(pro, layers):
            gated_delta_verify(*p[:5], l["state"])

    def t_epilogue():
        for o, z, l in zip(outs, zs, layers):
            gated_rmsnorm(o, z, l["w"].norm_weight, cfg.rms_norm_eps)

    def t_layer():
        for l in layers:
            gdn_layer_verify(l["qkv"], l["z"], l["a"], l["b"], l["conv"], l["state"], l["w"], cfg)

    F = torch.nn.functional

    def torch_prologue(l):
        x = torch.cat([l["conv"], l["qkv"]], dim=1).float()
        wc = l["w"].conv_weight.float()
        conv = sum(wc[:, j] * x[:, j:j + T] for j in range(K))
        act = F.silu(conv)
        q = act[..., :Hk * Dk].unflatten(-1, (Hk, Dk))
        k = act[..., Hk * Dk:2 * Hk * Dk].unflatten(-1, (Hk, Dk))
        v = act[..., 2 * Hk * Dk:].unflatten(-1, (Hv, Dv))
        q = (Dk ** -1.0) * q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6)
        k = (Dk ** -0.5) * k * torch.rsqrt(k.pow(2).mean(-1, keepdim=True) + 1e-6)
        g = torch.exp(-torch.exp(l["w"].A_log) * F.softplus(l["a"].float() + l["w"].dt_bias.float()))
        beta = torch.sigmoid(l["b"].float())
        return q.bfloat16(), k.bfloat16(), v.bfloat16(), g, beta, x[:, -(K - 1):].bfloat16()

    def torch_epilogue(o, z, w):
        of = o.float()
        y = of * torch.rsqrt(of.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float() * F.silu(z.float())
        return y.bfloat16()

    def t_torch_pe():
        for o, z, l in zip(outs, zs, layers):
            torch_prologue(l)
            torch_epilogue(o, z, l["w"].norm_weight)

    res = {name: _graph_time_us(torch, fn) for name, fn in (
        ("prologue", t_prologue), ("scan", t_scan), ("epilogue", t_epilogue),
        ("layer", t_layer), ("torch_prologue_epilogue", t_torch_pe))}
    return {
        "shape": {"layers": L, "B": B, "T": T, "Hk": Hk, "Hv": Hv, "Dk": Dk, "Dv": Dv, "conv_dim": C},
        "per_step_us": {k: round(v, 2) for k, v in res.items()},
        "per_layer_us": {k: round(v / L, 2) for k, v in res.items()},
        "note": f"each phase = one HIP graph of {L} per-layer launches; torch_prologue_epilogue "
                "= the same prologue + epilogue maths as torch op chains",
    }


def cpu_baseline(cfg, x, acc, block, conv, seconds: float):
    """The CPU oracle (C restatement, OpenMP over heads) running the same step
    on a bounded sample: whole steps repeated for ~`seconds`."""
    import numpy as np

    from oracle import oracle as orc

    cores = host_cores()
    ins = [x[n].float().numpy() for n in ("q", "k", "v", "g", "beta", "state")]
    logits = acc["logits"].numpy()
    drafts = block[:, 1:].numpy()
    conv_in, qkv = conv
    conv_in_np = [c.float().numpy() for c in conv_in]
    qkv_np = [q.float().numpy() for q in qkv]
    L, B = cfg.layers, cfg.B
    steps = 0
    t0 = time.perf_counter()
    while True:
        _, _, tape = orc.scan_c(*ins, threads=cores)
        _, matched, _ = orc.greedy_accept_c(logits, drafts)  # block[1:] vs posterior rows
        keep = np.asarray(matched) + 1                        # accepted_inputs
        orc.tape_select(tape, ins[5], np.tile(keep, L))
        for l in range(L):
            orc.conv_rollback(conv_in_np[l], qkv_np[l], keep)
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    tokens = steps * B * cfg.T
    return {
        "value": round(tokens / el, 2),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{steps} full steps of {cfg.name} (scan+tape over {L} layers, accept over "
                  f"[{B},{cfg.T},{cfg.V}] fp32, state gather + conv rollback to matched + 1) in "
                  f"{el:.1f} s; oracle/gdn_oracle.c fp32, OpenMP over heads",
    }


def graph_steps(torch, dev, run, K: int, warmup: int) -> dict:
    """K fused steps of a VerifyStepRunner as HIP graph replays.  The graph
    holds two steps: the keep counts alternate between two buffers (each
    step reads one and writes the other), so K steps are K // 2 replays,
    plus one eager step when K is odd (the same for the warmup).  The graph
    bakes in the keep buffers current at capture, so the odd eager warmup
    step runs before it: replays then always start from the buffer they
    were captured with (the odd timed step comes after them)."""
    K2 = K // 2
    if warmup % 2:
        run.run_fused()
    cap = torch.cuda.Stream(device=dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        run.run_fused()
        run.run_fused()
    torch.cuda.synchronize()
    for _ in range(warmup // 2):
        graph.replay()
    torch.cuda.synchronize()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    g0.record()
    for _ in range(K2):
        graph.replay()
    if K % 2:
        run.run_fused()
    g1.record()
    torch.cuda.synchronize()
    out = {"ms_per_step": (time.perf_counter() - t0) * 1e3 / K,
           "gpu_step": g0.elapsed_time(g1) * 1e3 / K}
    del graph
    return out


def measure_verify(torch, dev, cfg, steps: int, warmup: int, cpu_seconds: float,
                   probe_only: bool = False):
    """One config's verify step (scan + tape, greedy accept with the
    reference's wiring: drafts block[1:] against the posterior rows, keep =
    matched + 1; state and conv rollback to keep), fused and explicit forms.
    Returns the config's result dict (value, roofline, cpu_baseline, ...)."""
    from dflash_mlx.step import StepShape, VerifyStepRunner
    from dflash_mlx.workloads import ScanConfig, make_accept_inputs, make_scan_inputs, make_verify_block

    L, B, T = cfg.layers, cfg.B, cfg.T
    shape = StepShape(L=L, B=B, T=T, Hk=cfg.Hk, Hv=cfg.Hv, Dk=cfg.Dk, Dv=cfg.Dv,
                      V=cfg.V, conv_dim=CONV_DIM, K1=3)
    print(f"[bench] {cfg.name}: building inputs", file=sys.stderr, flush=True)
    x = make_scan_inputs(cfg)
    acc = make_accept_inputs(ScanConfig(**{**cfg.__dict__, "layers": 1}), gen=x["_gen"])
    block = make_verify_block(acc)
    gen = x["_gen"]
    conv_in = [torch.randn(B, 3, CONV_DIM, generator=gen).to(torch.bfloat16) for _ in range(L)]
    qkv = [torch.randn(B, T, CONV_DIM, generator=gen).to(torch.bfloat16) for _ in range(L)]

    runners = {}
    # "overlap": the fused step with the accept's argmax in the scan's launch
    # (and, with small windows, the whole step in one launch).  The verify
    # logits are synthetic inputs here; in a decode they come out of the
    # block's own scan, so that schedule exists only in this benchmark: it is
    # reported beside the headline, never as it.
    overlap_differs = shape.fuse_argmax()
    forms = ("fused", "explicit") + (("overlap",) if overlap_differs else ())
    for form in forms:
        run = VerifyStepRunner(shape, dev, overlap_accept=(form == "overlap"))
        for name in ("q", "k", "v", "g", "beta", "state"):
            getattr(run, name).copy_(x[name])
        run.logits.copy_(acc["logits"])
        run.block.copy_(block)
        for l in range(L):
            run.conv_in[l].copy_(conv_in[l])
            run.qkv[l].copy_(qkv[l])
        runners[form] = run
    torch.cuda.synchronize()

    fused, explicit = runners["fused"], runners["explicit"]
    overlap = runners.get("overlap")
    print(f"[bench] {cfg.name}: warmup {warmup}", file=sys.stderr, flush=True)
    for _ in range(max(warmup, 1)):
        fused.run_fused()
        explicit.run()
        if overlap is not None:
            overlap.run_fused()
    torch.cuda.synchronize()
    # The drafts agree with the argmax on exactly the drawn accept length
    # (capped at the T - 1 drafts a block holds).
    want = [min(a, T - 1) for a in acc["accept"].tolist()]
    for form, r in runners.items():
        if r.matched.cpu().tolist() != want or r.keep.cpu().tolist() != [m + 1 for m in want]:
            raise RuntimeError(f"{cfg.name} {form}: accept mismatch")
    keep = [m + 1 for m in want]
    if probe_only:
        return {"probe": probe(torch, fused, explicit)}

    K = steps
    print(f"[bench] {cfg.name}: timing {K} fused + {K} explicit steps", file=sys.stderr, flush=True)
    # The phases of run_fused(): with small logits the whole step is one
    # launch (the accept's argmax workgroups in the scan's launch, the last of
    # each sequence finishing the accept and the conv windows), otherwise the
    # argmax runs in a launch of its own after the scan.
    single = fused.single_launch
    in_scan = fused.argmax_in_scan
    lead = "step" if single else ("scan_argmax" if in_scan else "scan")
    if single:
        tf = time_steps(torch, K, [(lead, fused.step_launch)] + (
            [] if fused.conv_in_launch else [("conv_rollback", fused.conv_rollback)]))
    elif in_scan:
        tf = time_steps(torch, K, [(lead, fused.scan_rolled_argmax),
                                   ("accept_rollback", fused.accept_keys_conv_rollback)])
    else:
        tf = time_steps(torch, K, [(lead, fused.scan_rolled),
                                   ("accept_rollback", fused.accept_conv_rollback)])
    te = time_steps(torch, K, [("scan", explicit.scan), ("accept", explicit.accept),
                               ("rollback", explicit.rollback)])
    # The same fused step as the device-driven serving loop launches it: captured
    # once as a HIP graph (no host work inside), W replays untimed, then K replays
    # between synchronizes.  The eager per-phase timing above is the breakdown.
    print(f"[bench] {cfg.name}: timing {K} fused steps as graph replays of two",
          file=sys.stderr, flush=True)
    tg = graph_steps(torch, dev, fused, K, warmup)
    # Algorithmic HBM bytes.  Scan: bf16 q,k,v,out + fp32 g,beta + fp32 state
    # read + tape (T states per head).  The fused scan also writes the
    # rolled-back state for sequences that kept >= 1 token (every sequence:
    # keep = matched + 1); the explicit scan writes the final state instead.
    S_bytes = 4 * cfg.Hv * cfg.Dv * cfg.Dk
    io = 2 * L * B * T * (2 * cfg.Hk * cfg.Dk + 2 * cfg.Hv * cfg.Dv) + 8 * L * B * T * cfg.Hv
    n_wb = L * sum(1 for a in keep if a >= 1)
    scan_fused_bytes = io + S_bytes * (L * B * (1 + T) + n_wb)
    scan_expl_bytes = shape.scan_bytes()
    accept_bytes = shape.accept_bytes()
    conv_bytes = 2 * 2 * L * B * 3 * CONV_DIM
    gather_bytes = 2 * S_bytes * L * B
    tokens = B * T

    # The dominant launch: the scan + tape, with the accept's argmax workgroups
    # (which read the verify logits once) when they share its launch, and the
    # conv windows when the whole step is that launch.
    conv_inl = single and fused.conv_in_launch  # the conv windows copied in the step's launch
    launch_bytes = (scan_fused_bytes + (accept_bytes if in_scan else 0)
                    + (conv_bytes if conv_inl else 0))
    achieved = launch_bytes / (tf[lead] / 1e6) / 1e9
    roof = {
        "bound": "hbm",
        "kernel": ("gdn_scan_kernel<DK,R> + accept argmax workgroups finishing the accept"
                   + (" and the conv windows" if conv_inl else "") + " via dflash_gdn_verify_step")
                  if single else
                  ("gdn_scan_kernel<DK,R> + accept argmax workgroups via "
                   "dflash_gdn_verify_scan_rollback_argmax") if in_scan else
                  "gdn_scan_kernel<DK,R> via dflash_gdn_verify_scan_rollback",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBPS, 4),
        "traffic": traffic_from_profiles(cfg.name),
        "bytes_alg_per_launch": launch_bytes,
        "avg_launch_us": round(tf[lead], 2),
    }
    r2 = lambda d: {k: round(v, 2) for k, v in d.items() if k != "ms_per_step"}
    expl_scan_gbps = scan_expl_bytes / (te["scan"] / 1e6) / 1e9
    res = {
        "value": round(tokens / (tg["ms_per_step"] / 1e3), 1),
        "unit": "tokens/s",
        "ms_per_step": round(tg["ms_per_step"], 4),
        "config": {
            "workload": cfg.name, "B": B, "T": T, "Hk": cfg.Hk, "Hv": cfg.Hv,
            "Dk": cfg.Dk, "Dv": cfg.Dv, "layers": L, "vocab": cfg.V, "conv_dim": CONV_DIM,
            "accepted_inputs": keep,
            "io": "bf16 q/k/v/out, fp32 g/beta/state/tape, fp32 logits",
            "accept": "drafts block[1:] vs posterior rows 0..T-2, bonus = posterior[matched], "
                      "keep = matched + 1 (runtime.py:145-147)",
            "step": ("fused: scan+tape with the previous step's state rollback in its load, "
                     "the greedy accept's argmax slices as extra workgroups, the last of each "
                     "sequence's merging the keys and writing matched / bonus / keep"
                     + (" and copying the conv windows (1 launch)" if conv_inl else
                        " (1 launch) -> the conv-window copy (1 launch)")
                     + "; HIP graph of two steps (keep buffers alternate), replayed K // 2 times, one eager step more for odd K")
                    if single else
                    ("fused: scan+tape with the previous step's state rollback in its load, "
                     "with the greedy accept's argmax slices in the same launch -> the accept's "
                     "finalize inside the conv-window rollback copy, which also writes keep "
                     "(2 launches); HIP graph of two steps, replayed K // 2 times, one eager step more for odd K") if in_scan else
                    ("fused: scan+tape with the previous step's state rollback in its load -> "
                     "the greedy accept's argmax slices -> its finalize inside the conv-window "
                     "rollback copy, which also writes keep (3 launches, each after the one "
                     "whose output it reads, as in a decode where the logits come out of the "
                     "block's scan); HIP graph of two steps, replayed K // 2 times, one eager "
                     "step more for odd K"),
        },
        "roofline": roof,
        "graph_step_us": round(tg["gpu_step"], 2),
        "eager_step": {"value": round(tokens / (tf["ms_per_step"] / 1e3), 1),
                       "ms_per_step": round(tf["ms_per_step"], 4)},
        "breakdown_us": r2(tf),
        "step_hbm_gbps": round((scan_fused_bytes + accept_bytes + conv_bytes)
                               / (tf["gpu_step"] / 1e6) / 1e9, 1),
        "explicit_step": {
            "value": round(tokens / (te["ms_per_step"] / 1e3), 1),
            "ms_per_step": round(te["ms_per_step"], 4),
            "breakdown_us": r2(te),
            "scan_gbps": round(expl_scan_gbps, 1),
            "scan_frac": round(expl_scan_gbps / PEAK_HBM_GBPS, 4),
            "scan_bytes_alg": scan_expl_bytes,
            "step_hbm_gbps": round((scan_expl_bytes + accept_bytes + gather_bytes + conv_bytes)
                                   / (te["gpu_step"] / 1e6) / 1e9, 1),
        },
    }
    if overlap is not None:
        # Labelled apart from the headline: the argmax reads the synthetic
        # logits while the scan that would produce them in a decode still runs.
        print(f"[bench] {cfg.name}: timing {K} overlapped-accept steps (synthetic logits)",
              file=sys.stderr, flush=True)
        to = graph_steps(torch, dev, overlap, K, warmup)
        res["synthetic_logits_step"] = {
            "value": round(tokens / (to["ms_per_step"] / 1e3), 1),
            "ms_per_step": round(to["ms_per_step"], 4),
            "graph_step_us": round(to["gpu_step"], 2),
            "form": ("the whole step in one launch (dflash_gdn_verify_step)"
                     if overlap.single_launch else
                     "the accept's argmax in the scan's launch "
                     "(dflash_gdn_verify_scan_rollback_argmax) -> finalize inside the conv copy"),
            "note": "not a decode schedule: the accept reads logits given before the scan, "
                    "which in a decode come out of that scan through the later layers and "
                    "the LM head; not the headline",
        }
    del runners, fused, explicit, overlap
    torch.cuda.empty_cache()
    if cpu_seconds > 0:
        print(f"[bench] {cfg.name}: cpu baseline (~{cpu_seconds:.0f} s)", file=sys.stderr,
              flush=True)
        res["cpu_baseline"] = cpu_baseline(cfg, x, acc, block, (conv_in, qkv), cpu_seconds)
    else:
        res["cpu_baseline"] = None
    return res


def main() -> int:
    args = parse_args()
    if args.steps < 1 or args.warmup < 0:
        print("bench.py needs --steps >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); this build runs on a single MI355X and the verify scan "
              "would shard across GPUs by (sequence, head) with no communication", file=sys.stderr)
        return 2

    import torch

    if args.only is not None:
        dev = torch.device("cuda", 0)
        fn = {"lm_head": measure_lm_head, "layer": measure_layer, "prefill": measure_prefill,
              "hybrid": measure_hybrid, "gemm": measure_gemm, "prompt": measure_prompt,
              "decode": measure_decode}
        print(json.dumps({args.only: fn[args.only](torch, dev)}), flush=True)
        return 0

    from dflash_mlx.workloads import CONFIGS

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    if args.probe:
        return measure_verify(torch, dev, cfg, args.steps, args.warmup, 0, probe_only=True)["probe"]
    head = measure_verify(torch, dev, cfg, args.steps, args.warmup, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": head.pop("value"),
        "unit": head.pop("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": head.pop("config"),
        "roofline": head.pop("roofline"),
        "cpu_baseline": head.pop("cpu_baseline"),
    }
    line.update(head)
    if not args.no_configs and args.config == 1:
        line["configs"] = {}
        for ci in (0, 2):
            c = CONFIGS[ci]
            line["configs"][c.name] = measure_verify(torch, dev, c, args.steps, args.warmup,
                                                     args.cpu_seconds_other)
    if not args.no_extras:
        print("[bench] next rows: fused LM head", file=sys.stderr, flush=True)
        line["next_rows"] = {"lm_head_greedy_accept": measure_lm_head(torch, dev)}
        print("[bench] next rows: gated-delta layer prologue/epilogue", file=sys.stderr, flush=True)
        line["next_rows"]["gdn_layer"] = measure_layer(torch, dev)
        print("[bench] next rows: chunked prefill (config c3)", file=sys.stderr, flush=True)
        line["next_rows"]["chunked_prefill"] = measure_prefill(torch, dev)
        print("[bench] next rows: hybrid verify step (config c4)", file=sys.stderr, flush=True)
        line["next_rows"]["hybrid_verify_step"] = measure_hybrid(torch, dev)
        print("[bench] next rows: prompt pass (config c4 shape, 4096 tokens)", file=sys.stderr,
              flush=True)
        line["next_rows"]["prompt_pass"] = measure_prompt(torch, dev)
        print("[bench] next rows: decode through DFlashGenerator (config c4 shape)",
              file=sys.stderr, flush=True)
        line["next_rows"]["decode_step"] = measure_decode(torch, dev)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
