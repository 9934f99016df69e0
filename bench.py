#!/usr/bin/env python
"""Benchmark of the gated-delta verify hot path on one MI355X.

One step = one verify pass over the Qwen3.5-4B-shaped block (B=1, T=16,
Hk=16, Hv=32, Dk=Dv=128) for all 24 gated-delta layers:
  scan with out + final state + per-token tape (one launch, layers stacked)
  -> fused greedy accept over [16, 151936] fp32 logits
  -> rollback: tape gather of all 24 layers' states + conv-window rebuild
     (conv_dim 8192, kernel 4), driven by the device-side accepted count.
Inputs are resident in HBM before timing; the step runs through the C ABI
with preallocated buffers.  Prints one JSON line (see DESIGN.md for fields).

python bench.py [--steps K] [--warmup W] [--config 1|2] [--cpu-seconds S]
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
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1, choices=(1, 2))
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample (0 disables it)")
    return ap.parse_args()


def host_cores() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def traffic_from_profiles(workload: str):
    """HBM bytes per scan launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration)."""
    path = ROOT / "profiles" / f"gdn_verify_scan_{workload}_pmc.md"
    if not path.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", path.read_text())
    return int(m.group(1)) if m else None


def cpu_baseline(cfg, x, acc, conv, seconds: float):
    """The CPU oracle (C restatement, OpenMP over heads) running the same step
    on a bounded sample: whole 24-layer steps repeated for ~`seconds`."""
    import numpy as np

    from oracle import oracle as orc

    cores = host_cores()
    ins = [x[n].float().numpy() for n in ("q", "k", "v", "g", "beta", "state")]
    logits = acc["logits"].numpy()
    draft = acc["draft"].numpy()
    conv_in, qkv = conv
    conv_in_np = [c.float().numpy() for c in conv_in]
    qkv_np = [q.float().numpy() for q in qkv]
    L, B = cfg.layers, cfg.B
    steps = 0
    t0 = time.perf_counter()
    while True:
        _, _, tape = orc.scan_c(*ins, threads=cores)
        _, matched, _ = orc.greedy_accept_c(logits, draft)
        a = np.tile(matched, L)
        orc.tape_select(tape, ins[5], a)
        for l in range(L):
            orc.conv_rollback(conv_in_np[l], qkv_np[l], matched)
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
                  f"[{B},{cfg.T},{cfg.V}] fp32, tape + conv rollback) in {el:.1f} s; "
                  "oracle/gdn_oracle.c fp32, OpenMP over heads",
    }


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the verify scan shards with no communication, see DESIGN.md", file=sys.stderr)
        return 2

    import torch

    from dflash_mlx.step import StepShape, VerifyStepRunner
    from dflash_mlx.workloads import CONFIGS, ScanConfig, make_accept_inputs, make_scan_inputs

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    cfg = CONFIGS[args.config]
    L = cfg.layers
    shape = StepShape(L=L, B=cfg.B, T=cfg.T, Hk=cfg.Hk, Hv=cfg.Hv, Dk=cfg.Dk, Dv=cfg.Dv,
                      V=cfg.V, conv_dim=CONV_DIM, K1=3)
    print(f"[bench] {cfg.name}: building inputs", file=sys.stderr, flush=True)
    x = make_scan_inputs(cfg)
    acc_cfg = ScanConfig(**{**cfg.__dict__, "layers": 1})
    acc = make_accept_inputs(acc_cfg, gen=x["_gen"])
    gen = x["_gen"]
    conv_in = [torch.randn(cfg.B, 3, CONV_DIM, generator=gen).to(torch.bfloat16) for _ in range(L)]
    qkv = [torch.randn(cfg.B, cfg.T, CONV_DIM, generator=gen).to(torch.bfloat16) for _ in range(L)]

    run = VerifyStepRunner(shape, dev)
    for name in ("q", "k", "v", "g", "beta", "state"):
        getattr(run, name).copy_(x[name])
    run.logits.copy_(acc["logits"])
    run.draft.copy_(acc["draft"])
    for l in range(L):
        run.conv_in[l].copy_(conv_in[l])
        run.qkv[l].copy_(qkv[l])
    torch.cuda.synchronize()

    print(f"[bench] warmup {args.warmup}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        run.run()
    torch.cuda.synchronize()
    # The accept result is checked once: the draft agrees with the argmax on
    # exactly the drawn accept length.
    if run.matched.cpu().tolist() != acc["accept"].tolist():
        print("[bench] accept mismatch", file=sys.stderr)
        return 1

    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(K)]
    print(f"[bench] timing {K} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        e = ev[i]
        e[0].record()
        run.scan()
        e[1].record()
        run.accept()
        e[2].record()
        run.rollback()
        e[3].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    scan_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    accept_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K
    roll_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / K
    gpu_step_ms = sum(e[0].elapsed_time(e[3]) for e in ev) / K
    ms_per_step = wall * 1e3 / K
    tokens = cfg.B * cfg.T
    value = tokens / (ms_per_step / 1e3)

    scan_bytes = shape.scan_bytes()
    step_bytes = scan_bytes + shape.accept_bytes() + shape.rollback_bytes()
    achieved = scan_bytes / (scan_ms / 1e3) / 1e9
    roof = {
        "bound": "hbm",
        "kernel": "gdn_scan_kernel (dflash_gdn_verify_scan)",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBPS, 4),
        "traffic": traffic_from_profiles(cfg.name),
        "bytes_alg_per_launch": scan_bytes,
        "avg_launch_us": round(scan_ms * 1e3, 2),
    }

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": cfg.name, "B": cfg.B, "T": cfg.T, "Hk": cfg.Hk, "Hv": cfg.Hv,
            "Dk": cfg.Dk, "Dv": cfg.Dv, "layers": L, "vocab": cfg.V, "conv_dim": CONV_DIM,
            "io": "bf16 q/k/v/out, fp32 g/beta/state/tape, fp32 logits",
            "step": "scan+tape (1 launch) -> greedy accept (2) -> tape gather (1) + conv rollback (1)",
        },
        "roofline": roof,
        "breakdown_us": {
            "scan": round(scan_ms * 1e3, 2), "accept": round(accept_ms * 1e3, 2),
            "rollback": round(roll_ms * 1e3, 2), "gpu_step": round(gpu_step_ms * 1e3, 2),
        },
        "step_hbm_gbps": round(step_bytes / (gpu_step_ms / 1e3) / 1e9, 1),
        "scan_tokens_per_s": round(tokens / (scan_ms / 1e3), 1),
    }
    if args.cpu_seconds > 0:
        print(f"[bench] cpu baseline (~{args.cpu_seconds:.0f} s)", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(cfg, x, acc, (conv_in, qkv), args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
