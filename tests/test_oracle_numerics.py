"""Pins the oracle's per-(batch, head) row selection and its alternative
softmax numerics (oracle_sage_emulate_numerics), which judge on the CPU
whether a cheaper softmax than the reference's could meet the north-star
gate. The alternatives must be right for that judgement to stand, so each is
checked against closed forms: a query that sees one key gets that key's
value exactly when numerator and denominator share the E4M3 P, and a query
that sees two keys gets the weighted mean that the mode's weights fix."""
from __future__ import annotations

import numpy as np
import pytest

MODES = {
    "ref": None,
    "l_from_p8": dict(l_from_p8=True),
    "pow2": dict(pow2_max=True),
    "pow2+l_from_p8": dict(pow2_max=True, l_from_p8=True),
    "tau2+l_from_p8": dict(tau=2.0, l_from_p8=True),
    "exp_f16": dict(exp_f16=True),
}


def _problem(oracle, causal=True, tokens=200, heads=3, batch=2, d=64, seed=5):
    p = oracle.Problem(batch, heads, tokens, d, causal=causal)
    q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=2.0, seed=seed))
    return p, q, k, v, oracle.prologue(p, q, k, v)


def test_per_head_rows_match_shared_rows(oracle):
    """Rows given per (b, h) select, for each (b, h), the same outputs as those
    rows given to every (b, h): emulator (every mode) and f64 attention."""
    p, q, k, v, pro = _problem(oracle)
    rng = np.random.default_rng(0)
    bh = p.batch * p.heads
    rows = np.sort(np.stack([rng.choice(p.tokens, 7, replace=False) for _ in range(bh)]), axis=1).astype(np.int32)
    for mode in MODES.values():
        nv = None if mode is None else oracle.Numerics(**mode)
        per, _ = oracle.sage_emulate(p, pro, rows=rows, numerics=nv)
        for i in range(bh):
            shared, _ = oracle.sage_emulate(p, pro, rows=rows[i], numerics=nv)
            assert np.array_equal(per[i // p.heads, i % p.heads], shared[i // p.heads, i % p.heads])
    per = oracle.attention_f64(p, q, k, v, rows=rows)
    for i in range(bh):
        shared = oracle.attention_f64(p, q, k, v, rows=rows[i])
        assert np.array_equal(per[i // p.heads, i % p.heads], shared[i // p.heads, i % p.heads])


def test_default_numerics_are_the_references(oracle):
    """Numerics() with every field at its default is the reference's arithmetic, bit for bit."""
    p, _, _, _, pro = _problem(oracle, causal=False)
    a, _ = oracle.sage_emulate(p, pro)
    b, _ = oracle.sage_emulate(p, pro, numerics=oracle.Numerics())
    assert np.array_equal(a, b)


@pytest.mark.parametrize("mode", ["l_from_p8", "pow2+l_from_p8", "tau2+l_from_p8"])
def test_single_key_row_returns_that_value(oracle, mode):
    """Causal query 0 sees key 0 only. When l sums the E4M3 P, the weight cancels
    exactly: out = decoded v8[0] * v_scale + v_mean, whatever the P grid."""
    p, _, _, _, pro = _problem(oracle)
    out, _ = oracle.sage_emulate(p, pro, rows=np.array([0], np.int32), numerics=oracle.Numerics(**MODES[mode]))
    for b in range(p.batch):
        for h in range(p.heads):
            v8 = oracle.e4m3_decode(pro["v8"][b, h, 0]).astype(np.float64)
            st = pro["stats"][b, h].astype(np.float64)
            want = v8 * st[2] + st[1]
            assert np.allclose(out[b, h, 0], want, rtol=0, atol=1e-6 * (1 + np.abs(want).max())), (b, h)


def test_single_key_row_under_a_shifted_grid_keeps_the_rounding(oracle):
    """With l from the unrounded P, the one-key row carries e4m3(P)/P: 1 for the
    reference (P = 448 up to the exp2 argument's last bits; exact logits, since
    the fast logit's 1.5 * 2^23 offset rounds the argument by up to its ulp) and
    for tau = 2 (P = 112), not 1 in general for the power-of-two max
    (P = 448 * 2^(m - ceil m), E4M3 steps of 1/8 to 1/16)."""
    p, _, _, _, pro = _problem(oracle)
    row = np.array([0], np.int32)
    run = lambda nv: oracle.sage_emulate(p, pro, rows=row, fast_exp=False, numerics=nv)[0]
    exact = run(oracle.Numerics(l_from_p8=True))
    assert np.allclose(run(None), exact, rtol=1e-5, atol=1e-5)
    assert not np.allclose(run(oracle.Numerics(pow2_max=True)), exact, rtol=1e-3, atol=1e-3)
    assert np.allclose(run(oracle.Numerics(tau=2.0)), exact, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("mode", list(MODES))
def test_two_key_rows_closed_form(oracle, mode):
    """Causal query 1 sees keys 0 and 1 of the first block. From the int32
    scores S = q8 . k8 and x = S * qs * ks (log2 units): m = max x (reference),
    ceil(max x) (pow2), max x + tau (tau); P_j = 448 * 2^(x_j - m), optionally
    rounded to f16; l = P0 + P1 or e4m3(P0) + e4m3(P1); out = sum e4m3(P_j) v_j / l,
    dequantised. Computed here in float64 from the codes, against the
    emulator's fp32 result."""
    p, _, _, _, pro = _problem(oracle, d=128)
    cfg = MODES[mode] or {}
    out, _ = oracle.sage_emulate(p, pro, rows=np.array([1], np.int32), fast_exp=False,
                                 numerics=None if not cfg else oracle.Numerics(**cfg))
    for b in range(p.batch):
        for h in range(p.heads):
            q8 = pro["q8"][b, h, 1].astype(np.int64)
            k8 = pro["k8"][b, h, :2].astype(np.int64)
            s = k8 @ q8
            sc = np.float64(np.float32(pro["q_scale"][b, h, 0] * pro["k_scale"][b, h, 0]))
            x = s * sc
            m = x.max()
            if cfg.get("pow2_max"):
                m = np.ceil(m)
            m += cfg.get("tau", 0.0)
            pw = 448.0 * np.exp2(x - m)
            if cfg.get("exp_f16"):
                pw = pw.astype(np.float16).astype(np.float64)
            p8 = oracle.e4m3_decode(oracle.e4m3_encode(pw.astype(np.float32))).astype(np.float64)
            l = p8.sum() if cfg.get("l_from_p8") else pw.sum()
            v8 = oracle.e4m3_decode(pro["v8"][b, h, :2]).astype(np.float64)
            st = pro["stats"][b, h].astype(np.float64)
            want = (p8 @ v8) / l * st[2] + st[1]
            assert np.allclose(out[b, h, 0], want, rtol=1e-5, atol=1e-5), (mode, b, h, np.abs(out[b, h, 0] - want).max())
