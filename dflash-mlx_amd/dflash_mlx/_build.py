"""Build libdflash_gfx950.so from csrc/ with hipcc (cross-compiles without a GPU).

Usage: python -m dflash_mlx._build   (or call build_library()).
The library is written next to this file so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT_DIR = PKG_DIR.parent  # dflash-mlx_amd/
CSRC_DIR = ROOT_DIR / "csrc"
INCLUDE_DIR = ROOT_DIR.parent / "include"
LIB_NAME = "libdflash_gfx950.so"
LIB_PATH = PKG_DIR / LIB_NAME

SOURCES = ["gdn_scan.hip", "gdn_layer_ops.hip", "gdn_chunked.hip", "greedy_accept.hip", "lm_head_argmax.hip",
           "rollback.hip", "model_ops.hip", "skinny_gemm.hip", "prefill_gemm.hip", "abi.cpp"]
HEADERS = ["device_common.h", "host_common.h", "accept_common.h"]

# -packed-fp32-ops off: v_pk_{add,mul,fma}_f32 have given silent wrong results
# on these machines, so the compiler must not form them from scalar code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return path


def build_library(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    build_dir = ROOT_DIR / "_build"
    build_dir.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    procs = []
    for src in SOURCES:
        obj = build_dir / (src.rsplit(".", 1)[0] + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmd = [cc, *HIPCC_FLAGS, *lang, "-I", str(INCLUDE_DIR), "-I", str(CSRC_DIR),
               "-c", str(CSRC_DIR / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _drain(procs, verbose)
    _drain(procs, verbose)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _drain(procs, verbose):
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
        if p.returncode != 0:
            failed.append((src, "\n".join(lines)))
        elif verbose and any(ln.strip() for ln in lines):
            print("\n".join(lines), flush=True)
    procs.clear()
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(f"[{s}]\n{t}" for s, t in failed))


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
