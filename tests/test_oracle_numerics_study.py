"""The CPU study behind the attention kernel's choice of softmax numerics.

The north star gates the output against the reference's own output at
cosine >= 0.999 and max-abs <= 2e-2. The attention kernel is VALU-bound, and
each cheaper softmax below would cut VALU work (the fp32 row sum, the fp32
exps, or the 64-accumulator rescale); the question is whether any of them
still meets that gate. This test reruns the study on the CPU: for each
benchmark configuration C2-C5 at full size it draws 64 query rows of every
(batch, head), emulates the reference's arithmetic (sage_attn.cu:264-330,
restated in oracle_sage_emulate) and each alternative
(oracle_sage_emulate_numerics, pinned by test_oracle_numerics.py), and
compares them. The table it checks is the one the design notes quote;
the pass/fail pattern is the decision: every alternative fails the max-abs
gate at C3 and C5 (and the power-of-two max at C4 as well), so the kernel
keeps the reference's numerics.

The alternatives are about as accurate as the reference's own arithmetic
(checked against f64 attention, reference.rs:148-184): they fail the gate
because it is absolute and C3's x20 outlier channels and C5's x10 tokens make
outputs of magnitude 3.6 and 42.5, where a different rounding of the P grid
moves single elements by more than 2e-2.
"""
from __future__ import annotations

import numpy as np
import pytest

COS_MIN, MAX_ABS = 0.999, 2e-2
ROWS_PER_HEAD, ROW_SEED, THREADS = 64, 7, 8

MODES = {
    "l_from_p8": dict(l_from_p8=True),
    "exp_f16": dict(exp_f16=True),
    "exp_f16+l_from_p8": dict(exp_f16=True, l_from_p8=True),
    "pow2": dict(pow2_max=True),
    "pow2+l_from_p8": dict(pow2_max=True, l_from_p8=True),
    "tau2+l_from_p8": dict(tau=2.0, l_from_p8=True),
    "tau4+l_from_p8": dict(tau=4.0, l_from_p8=True),
}

# (cosine, max-abs) of each mode against the reference's numerics on the
# sampled rows, and the reference's own (cosine, rel_l2, max-abs) against f64.
TABLE = {
    2: {"l_from_p8": (1.000000, 0.0002), "exp_f16": (0.999985, 0.0016), "exp_f16+l_from_p8": (0.999985, 0.0016),
        "pow2": (0.999341, 0.0048), "pow2+l_from_p8": (0.999341, 0.0048), "tau2+l_from_p8": (0.999537, 0.0047),
        "tau4+l_from_p8": (0.999387, 0.0050)},
    3: {"l_from_p8": (0.999993, 0.0338), "exp_f16": (0.999998, 0.0633), "exp_f16+l_from_p8": (0.999991, 0.0597),
        "pow2": (0.999617, 0.1496), "pow2+l_from_p8": (0.999839, 0.0908), "tau2+l_from_p8": (0.999943, 0.0679),
        "tau4+l_from_p8": (0.999909, 0.0682)},
    4: {"l_from_p8": (0.999995, 0.0085), "exp_f16": (0.999991, 0.0047), "exp_f16+l_from_p8": (0.999986, 0.0085),
        "pow2": (0.999376, 0.0803), "pow2+l_from_p8": (0.999437, 0.0454), "tau2+l_from_p8": (0.999718, 0.0142),
        "tau4+l_from_p8": (0.999666, 0.0142)},
    5: {"l_from_p8": (0.999992, 0.4493), "exp_f16": (1.000000, 0.7369), "exp_f16+l_from_p8": (0.999992, 0.7390),
        "pow2": (0.999634, 1.9170), "pow2+l_from_p8": (0.999951, 1.1597), "tau2+l_from_p8": (0.999979, 0.9638),
        "tau4+l_from_p8": (0.999946, 2.5241)},
}
REF_VS_F64 = {2: (0.999220, 0.03950, 0.0065), 3: (0.995488, 0.09498, 0.4901),
              4: (0.999310, 0.03717, 0.0781), 5: (0.992886, 0.11928, 17.8434)}

# The decision: the modes that fail the north-star gate, per configuration.
FAILS = {
    2: set(),
    3: set(MODES),
    4: {"pow2", "pow2+l_from_p8"},
    5: set(MODES),
}

_cache: dict = {}


def _study(oracle, c: int) -> dict:
    if c in _cache:
        return _cache[c]
    p, g = oracle.config(c)
    q, k, v = oracle.generate(p, g)
    pro = oracle.prologue(p, q, k, v, threads=THREADS)
    rng = np.random.default_rng(ROW_SEED)
    rows = np.sort(np.stack([rng.choice(p.tokens, ROWS_PER_HEAD, replace=False)
                             for _ in range(p.batch * p.heads)]), axis=1).astype(np.int32)
    od = oracle.BF16 if p.dtype == oracle.BF16 else oracle.F16
    ref, _ = oracle.sage_emulate(p, pro, rows=rows, out_dtype=od, threads=THREADS)
    f64 = oracle.attention_f64(p, q, k, v, rows=rows, threads=THREADS)
    res = {"ref_f64": oracle.errors(ref, f64), "modes": {}}
    for name, m in MODES.items():
        out, _ = oracle.sage_emulate(p, pro, rows=rows, out_dtype=od, threads=THREADS,
                                     numerics=oracle.Numerics(**m))
        res["modes"][name] = (oracle.errors(out, ref), oracle.errors(out, f64))
    _cache[c] = res
    return res


def _passes(e: dict) -> bool:
    return e["cos"] >= COS_MIN and e["max_abs"] <= MAX_ABS


@pytest.mark.parametrize("c", [2, 3, 4, 5])
def test_numerics_study_table_and_gate(oracle, c):
    """Each mode's (cos, max-abs) against the reference's numerics equals the
    quoted table to its printed digits, and the modes that fail the gate are
    exactly FAILS[c]."""
    res = _study(oracle, c)
    failing = set()
    for name, (e, _) in res["modes"].items():
        cos, mx = TABLE[c][name]
        assert abs(e["cos"] - cos) <= 1.5e-6, (c, name, e["cos"], cos)
        assert abs(e["max_abs"] - mx) <= 1.5e-4 * max(1.0, mx), (c, name, e["max_abs"], mx)
        if not _passes(e):
            failing.add(name)
    assert failing == FAILS[c], (c, sorted(failing))


@pytest.mark.parametrize("c", [2, 3, 4, 5])
def test_alternatives_are_about_as_accurate_as_the_reference(oracle, c):
    """Against f64 attention, every alternative's cosine is within 4e-4 of the
    reference arithmetic's, and its relative L2 error within 3% (12% for the
    power-of-two max, whose P grid sits up to one octave below 448): the gate
    failures above are not a loss of accuracy but a different rounding."""
    res = _study(oracle, c)
    r = res["ref_f64"]
    cos, rl2, mx = REF_VS_F64[c]
    assert abs(r["cos"] - cos) <= 1.5e-6 and abs(r["rel_l2"] - rl2) <= 1.5e-5
    assert abs(r["max_abs"] - mx) <= 1.5e-4 * max(1.0, mx)
    for name, (_, ef) in res["modes"].items():
        assert abs(ef["cos"] - r["cos"]) <= 4e-4, (c, name, ef["cos"], r["cos"])
        bound = 1.12 if name.startswith("pow2") else 1.03
        assert ef["rel_l2"] <= r["rel_l2"] * bound, (c, name, ef["rel_l2"], r["rel_l2"])
