"""Shared pytest setup: import paths, the `gpu` marker and device fixtures."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "dflash-mlx_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as orc

    if not orc.LIB_PATH.exists():
        orc.build(force=False)
    return orc


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from dflash_mlx import _lib

    _lib.load()  # raises if the HIP library is missing: no silent fallback
    return torch.device("cuda", 0)


def pytest_report_header(config):
    return f"dflash-mlx_amd tests; ROCR_VISIBLE_DEVICES={os.environ.get('ROCR_VISIBLE_DEVICES')}"
