"""The prologue's device encoders equal the C oracle's on all 2^32 f32
inputs: the E4M3 encoder (sage_device.hpp e4m3_pair: the hardware converter
with a clamp and a NaN patch) against the reference's cvt.rn.satfinite
semantics (reference.rs:40-70), and the INT8 encoder (s8_code: v_rndne_f32,
v_cvt_i32_f32, an integer clamp) against sg_s8 (sage_common.cu:95-99: round to
nearest even, clamp to +-127, NaN to 0), and the QK-norm's rstd (rsqrt_rn2: a
short square root and reciprocal on most of the range) against the oracle's
correctly rounded 1 / sqrt. Runs tests/cpp/bin/codec_exhaustive."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "codec_exhaustive"


def test_device_encoders_are_exhaustively_the_oracle():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=200)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "e4m3: 0 of 256 chunks differ" in r.stdout and "s8: 0 of 256 chunks differ" in r.stdout
    assert "rstd: 0 of 256 chunks differ" in r.stdout
