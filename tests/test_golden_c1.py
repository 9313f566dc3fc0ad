"""The committed golden fixture of benchmark configuration C1 (B1 H2 N256 D64
fp16, seed 1; tests/golden/c1.npz, written by tests/golden/make_c1.py).

The reference keeps no golden vectors for this path and cannot run here, so
the fixture holds this repository's oracle outputs, frozen: the generator's
inputs, the prologue's codes, scales and statistics, the quantised attention's
fp16 output and the f64 attention. The CPU tests check that the oracle still
reproduces every array bit for bit and that the frozen values satisfy what the
mathematics fixes (a code of magnitude 127 in every quantisation group with a
nonzero range, outputs inside the convex hull of the V rows, the reference's
gate against f64, tests.rs:699); the GPU test runs the HIP path on the
fixture's inputs and checks its codes bit for bit and its output at the north
star's gate (cos >= 0.999, max-abs <= 2e-2) against the frozen output.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

FIXTURE = Path(__file__).resolve().parent / "golden" / "c1.npz"
CODES = ("q8", "q_scale", "k8", "k_scale", "v8", "stats")


@pytest.fixture(scope="module")
def gold():
    with np.load(FIXTURE) as d:  # allow_pickle stays False
        return {k: d[k] for k in d.files}


def _bits(a: np.ndarray) -> np.ndarray:
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_generator_reproduces_the_inputs(oracle, gold):
    p, g = oracle.config(1)
    q, k, v = oracle.generate(p, g)
    for name, got in (("q", q), ("k", k), ("v", v)):
        assert np.array_equal(got, gold[name]), name


def test_prologue_reproduces_the_codes(oracle, gold):
    p, _ = oracle.config(1)
    pro = oracle.prologue(p, gold["q"], gold["k"], gold["v"])
    for name in CODES:
        assert np.array_equal(_bits(pro[name]), _bits(gold[name])), name


def test_emulator_and_f64_attention_reproduce_the_outputs(oracle, gold):
    p, _ = oracle.config(1)
    pro = {name: gold[name] for name in CODES}
    _, out16 = oracle.sage_emulate(p, pro, out_dtype=oracle.F16)
    assert np.array_equal(out16, gold["out16"])
    f64 = oracle.attention_f64(p, gold["q"], gold["k"], gold["v"])
    assert np.array_equal(_bits(f64), _bits(gold["out_f64"]))


def test_every_group_reaches_code_127(oracle, gold):
    """A Q group of 16 rows and a K block of 64 keys with a nonzero range hold
    a code of magnitude 127 (the group's amax maps to 127, sage_quant.cu:85-127,
    259-316), and none exceeds it; every V channel's extreme maps to +-448."""
    q8 = gold["q8"].reshape(1, 2, 16, 16, 64).astype(np.int32)
    assert np.all(np.abs(q8).max(axis=(3, 4)) == 127) and np.all(gold["q_scale"] > 0)
    k8 = gold["k8"].reshape(1, 2, 4, 64, 64).astype(np.int32)
    assert np.all(np.abs(k8).max(axis=(3, 4)) == 127) and np.all(gold["k_scale"] > 0)
    v = np.abs(oracle.e4m3_decode(gold["v8"]))
    assert np.all(v.max(axis=2) == 448.0)


def test_outputs_lie_in_the_hull_of_v_and_meet_the_gate(oracle, gold):
    """Softmax weights are convex, so each output channel lies between the
    smallest and largest V value of its head (the f64 output exactly, the fp16
    output within its rounding); the quantised output meets the reference's gate
    against f64 (cos > 0.999, rel_l2 < 0.04, tests.rs:699)."""
    v = oracle.decode16(gold["v"], oracle.F16).transpose(0, 2, 1, 3)  # [B,H,T,D]
    lo, hi = v.min(axis=2, keepdims=True), v.max(axis=2, keepdims=True)
    f64 = gold["out_f64"]
    assert np.all(f64 >= lo - 1e-6) and np.all(f64 <= hi + 1e-6)
    out = oracle.decode16(gold["out16"], oracle.F16)
    assert np.all(out >= lo - 2e-2) and np.all(out <= hi + 2e-2)
    e = oracle.errors(out, f64)
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


@pytest.mark.gpu
def test_hip_path_matches_the_fixture(torch_gpu, oracle, gold):
    from sage_gpu_helpers import run

    p, _ = oracle.config(1)
    ws, o = run(torch_gpu, p, gold["q"], gold["k"], gold["v"])
    for name in CODES:
        assert np.array_equal(_bits(ws[name]), _bits(gold[name])), name
    got = oracle.decode16(o, oracle.F16).transpose(0, 2, 1, 3)  # [B,T,H,D] -> [B,H,T,D]
    want = oracle.decode16(gold["out16"], oracle.F16)
    e = oracle.errors(got, want)
    assert e["cos"] >= 0.999 and e["max_abs"] <= 2e-2, e
    ef = oracle.errors(got, gold["out_f64"])
    assert ef["cos"] > 0.999 and ef["rel_l2"] < 0.04, ef
