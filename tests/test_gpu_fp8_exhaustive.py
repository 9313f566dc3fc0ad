"""The prologue's device E4M3 encoder (sage_device.hpp, e4m3_pair: the
hardware converter with a clamp and a NaN patch) equals the C oracle's
encoder (the reference's cvt.rn.satfinite semantics, reference.rs:40-70) on
all 2^32 f32 inputs: runs tests/cpp/bin/fp8_exhaustive."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "fp8_exhaustive"


def test_device_e4m3_encoder_is_exhaustively_the_oracle():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 of 256 chunks differ" in r.stdout
