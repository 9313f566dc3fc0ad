"""Shared pytest setup: the `gpu` marker, import paths and helpers.

CPU tests (`-m "not gpu"`) cover the oracle against the reference's known
answers, the host logic and the C ABI's exports. GPU tests (`-m gpu`) are the
parity tests proper: they call the HIP library through the C ABI and compare
with the oracle on the same seeded inputs.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "sota-papers-lab_amd"
for p in (ROOT, PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle

    pyoracle.lib()
    return pyoracle


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch


def to_device16(torch, a: np.ndarray, dtype: int):
    """uint16 codes -> torch bf16/fp16 device tensor of the same shape."""
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16))
    t = t.view(torch.bfloat16 if dtype == 0 else torch.float16)
    return t.cuda()


def from_device16(t) -> np.ndarray:
    import torch

    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
