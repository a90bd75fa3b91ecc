"""Shared pytest setup: import paths, the `gpu` marker, common fixtures."""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "tiktok-techjam-2026_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libtjk.so")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible ROCm GPU")
    from tjkernels import _lib
    _lib.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda", 0)
