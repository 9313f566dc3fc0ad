"""Pins the oracle's PvAccum::F16 mode on the CPU (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/mod.rs:170-185, cuda/sage_attn.cu:326-344): the f16
rounding of its block accumulator against numpy's float16, the reference's
prologue checks for the mode (V within +-2.25, tests.rs:633-648) and its
attention gate (tests.rs:655-700, the F16 cases), and that the 2.25 range is
what keeps a block's f16 partial finite."""
from __future__ import annotations

import numpy as np
import pytest

from prologue_invariants import check_prologue

SMALL_LAYOUT = (3, 5, 7, 10, 1)  # tests.rs:596-605
SMALL_TOKENS = 3 * (5 + 7 * 10)


def test_round_f16_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    xs = [0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, -70000.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
          2.0 ** -14, 2.0 ** -14 - 2.0 ** -25]
    xs += list(rng.standard_normal(2000) * 10.0 ** rng.uniform(-8, 5, 2000))
    # Exact ties between neighbouring f16 values, normal and subnormal, both signs.
    h = rng.integers(1, 0x7BFF, 2000).astype(np.uint16).view(np.float16).astype(np.float64)
    up = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    xs += list((h + up) / 2) + list(-(h + up) / 2)
    for x in xs:
        with np.errstate(over="ignore"):
            want = float(np.float64(x).astype(np.float16))
        got = oracle.round_f16(x)
        assert got == want or (np.isinf(got) and np.isinf(want) and np.sign(got) == np.sign(want)), (x, got, want)


@pytest.mark.parametrize("d", [64, 128])
def test_pv16_prologue_passes_reference_checks(oracle, d):
    """tests.rs:633-648: the F16 prologue passes check_prologue, every V code
    decodes within +-2.25, and the V scale is positive."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, pv16=True)
    q, k, v = oracle.reference_synthetic(p, 11)
    pro = oracle.prologue(p, q, k, v)
    dec = lambda x: oracle.decode16(x, 0)
    check_prologue(p, dec(q), dec(k), dec(v), pro)
    vmax = np.abs(oracle.e4m3_decode(pro["v8"])).max()
    assert vmax <= 2.25
    assert np.all(pro["stats"][:, :, 2] > 0)
    # The range is the mode's only prologue change: V scales are the F32 mode's times 448 / 2.25.
    ref = oracle.prologue(oracle.Problem(2, 3, SMALL_TOKENS, d), q, k, v)
    assert np.array_equal(pro["k8"], ref["k8"]) and np.array_equal(pro["q8"], ref["q8"])
    assert np.allclose(pro["stats"][:, :, 2], ref["stats"][:, :, 2] * (448 / 2.25), rtol=1e-6)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("merge", [1, 2])
def test_pv16_emulation_meets_reference_gate(oracle, d, merge):
    """tests.rs:655-700 for PvAccum::F16: cos > 0.999 and rel_l2 < 0.04 against f64."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, merge=merge, layout=SMALL_LAYOUT, pv16=True)
    q, k, v = oracle.reference_synthetic(p, 5)
    pro = oracle.prologue(p, q, k, v)
    emu, _ = oracle.sage_emulate(p, pro)
    e = oracle.errors(emu, oracle.attention_f64(p, q, k, v))
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


def test_pv16_accumulator_rounds_to_f16(oracle):
    """The f16 partials move the output by about f16's step, no more: the
    emulation with and without the rounding on the same F16 prologue."""
    p = oracle.Problem(1, 2, 700, 128, pv16=True)
    q, k, v = oracle.generate(p, oracle.GenSpec(seed=6))
    pro = oracle.prologue(p, q, k, v)
    a, _ = oracle.sage_emulate(p, pro)
    exact = oracle.Problem(1, 2, 700, 128)  # same tensors, fp32 partials
    b, _ = oracle.sage_emulate(exact, pro)
    diff = np.abs(a - b).max()
    assert 0 < diff < 2.0 ** -9 * np.abs(b).max() * 4


def test_pv16_needs_the_small_v_range(oracle):
    """A planted mistake: f16 partials over V quantised to +-448 (the F32
    mode's range) overflow f16 and the output is no longer finite."""
    p16 = oracle.Problem(1, 1, 256, 64, pv16=True)
    q, k, v = oracle.generate(p16, oracle.GenSpec(seed=2))
    wide = oracle.prologue(oracle.Problem(1, 1, 256, 64), q, k, v)
    bad, _ = oracle.sage_emulate(p16, wide)
    assert not np.isfinite(bad).all()
    good, _ = oracle.sage_emulate(p16, oracle.prologue(p16, q, k, v))
    assert np.isfinite(good).all()
