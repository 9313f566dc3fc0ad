"""GPU parity through the C++ host API (include/spl_sage.hpp): runs
tests/cpp/bin/gpu_parity, the reference's gpu_prologue_matches_reference and
gpu_attention_matches_float_reference (tests.rs:606-700) restated in C++ with
the C oracle as checker: workspace buffers bit-exact, outputs within the
north-star gate of the reference arithmetic and the reference's f64 gate. It
also runs the reference's caller, the VGGT trunk's sage scheduler (sched.rs),
restated in include/spl_sage_sched.hpp, on the shipped `ours+sage` schedule."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "gpu_parity"


def test_cpp_gpu_parity():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
