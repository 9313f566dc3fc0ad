"""GPU parity through the C++ host API (include/spl_sage.hpp): runs
tests/cpp/bin/gpu_parity, the reference's gpu_prologue_matches_reference and
gpu_attention_matches_float_reference (tests.rs:606-700) restated in C++ with
the C oracle as checker: workspace buffers bit-exact, outputs within the
north-star gate of the reference arithmetic and the reference's f64 gate. It
also runs the reference's caller, the VGGT trunk's sage scheduler (sched.rs),
restated in include/spl_sage_sched.hpp, on the shipped `ours+sage` schedule.
The same program runs again under AddressSanitizer and UndefinedBehaviorSanitizer
on its host code and the library's host API (tests/cpp/bin/san; the device
code is the product's, uninstrumented)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "gpu_parity"
SAN_BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "san" / "gpu_parity"


def test_cpp_gpu_parity():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


def test_cpp_gpu_parity_under_sanitizers():
    """Host-side ASan + UBSan over the whole GPU path of the C++ API: workspace
    creation, prepare, attend, the QKV prologue and the caller's scheduler.
    Leak detection is off here: the HIP runtime keeps process-lifetime
    allocations that are not this library's."""
    assert SAN_BIN.exists(), f"{SAN_BIN} is not built; run `python __graft_entry__.py` (build)"
    env = {**os.environ, "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}
    r = subprocess.run([str(SAN_BIN)], capture_output=True, text=True, timeout=110, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
    assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, r.stderr
