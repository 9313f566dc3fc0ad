"""Pins the oracle's attention emulator (oracle_sage_emulate, both logit
modes of sage_attn.cu) on the CPU against what the mathematics fixes: the
textbook f64 attention, equal weights for equal scores, causal and padding
masks that ignore the keys they hide, and the size of the fast-logit shift."""
from __future__ import annotations

import numpy as np
import pytest


def _c1(oracle, seed=3, **kw):
    p, g = oracle.config(1, seed=seed)
    for k, v in kw.items():
        setattr(p, k, v)
    q, k, v = oracle.generate(p, g)
    return p, q, k, v, oracle.prologue(p, q, k, v)


@pytest.mark.parametrize("fast", [True, False])
@pytest.mark.parametrize("causal", [False, True])
def test_emulator_tracks_textbook_attention(oracle, fast, causal):
    """tests.rs:691-720 gate (cos > 0.999, rel_l2 < 0.04) of the quantised
    algorithm against f64 softmax attention of the same 16-bit inputs."""
    p, q, k, v, pro = _c1(oracle, causal=causal)
    emu, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=fast)
    ref = oracle.attention_f64(p, q, k, v)
    e = oracle.errors(emu, ref)
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


@pytest.mark.parametrize("fast", [True, False])
def test_equal_scores_give_equal_weights(oracle, fast):
    """All-zero Q codes make every score 0: each output channel is the mean of
    its V codes, decoded, times v_scale, plus v_mean, up to one common factor
    448 / p (p the fp32 weight before E4M3 rounding) that is 1 within the
    logit rounding of the mode. One key block (the fast mode's logit shift
    is per block), V smoothing off (code means far from zero)."""
    p, q, k, v, pro = _c1(oracle, smooth_v=False, tokens=64)
    pro = dict(pro)
    pro["q8"] = np.zeros_like(pro["q8"])
    emu, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=fast)
    n = p.tokens
    v8 = oracle.e4m3_decode(pro["v8"][:, :, :n]).astype(np.float64)  # [B, HK, N, D]
    mean = v8.mean(axis=2)                                            # [B, HK, D]
    vmean = pro["stats"][:, :, 1].astype(np.float64)
    vscale = pro["stats"][:, :, 2].astype(np.float64)
    got = (emu.astype(np.float64) - vmean[:, :, None, :]) / vscale[:, :, None, :]
    ok = np.abs(mean) > 1.0                                           # [B, HK, D]
    ratio = got / mean[:, :, None, :]                                 # [B, H, N, D]
    assert ok.sum() > 10
    r = np.where(ok[:, :, None, :], ratio, np.nan)
    tol = 2e-3 if fast else 1e-5
    assert np.nanmax(np.abs(r - 1)) < tol, np.nanmax(np.abs(r - 1))
    # one factor per row (its weights are all equal): across a row's channels
    # the ratio moves only by the fp32 rounding of the output arithmetic
    spread = np.nanmax(r, axis=-1) - np.nanmin(r, axis=-1)
    assert spread.max() < 1e-5, spread.max()


@pytest.mark.parametrize("fast", [True, False])
def test_causal_rows_ignore_future_keys(oracle, fast):
    """Causal row i must not see keys j > i: scrambling later K/V codes leaves
    it unchanged, and row 0 (one key) is that key's V, dequantised."""
    p, q, k, v, pro = _c1(oracle, causal=True)
    rows = np.array([0, 5, 63, 64, 130], np.int32)
    a, _ = oracle.sage_emulate(p, pro, rows=rows, out_dtype=p.dtype, fast_exp=fast)
    rng = np.random.default_rng(0)
    for i_idx, i in enumerate(rows):
        pro2 = {kk: vv.copy() for kk, vv in pro.items()}
        pro2["k8"][:, :, i + 1:] = rng.integers(-127, 128, pro2["k8"][:, :, i + 1:].shape, dtype=np.int8)
        pro2["v8"][:, :, i + 1:] = rng.integers(0, 0x7e, pro2["v8"][:, :, i + 1:].shape).astype(np.uint8)
        b, _ = oracle.sage_emulate(p, pro2, rows=rows[i_idx:i_idx + 1], out_dtype=p.dtype, fast_exp=fast)
        assert np.array_equal(a[:, :, i_idx], b[:, :, 0]), i
    v0 = oracle.e4m3_decode(pro["v8"][:, :, 0]).astype(np.float64)
    want = v0 * pro["stats"][:, :, 2] + pro["stats"][:, :, 1]
    np.testing.assert_allclose(a[:, :, 0], want, rtol=3e-3, atol=1e-5)


@pytest.mark.parametrize("fast", [True, False])
def test_padding_keys_are_ignored(oracle, fast):
    """Keys in [N, tk_pad) are padding: their codes never reach the output."""
    p, g = oracle.config(1, seed=4)
    p.tokens = 200  # tk_pad = 256
    q, k, v = oracle.generate(p, g)
    pro = oracle.prologue(p, q, k, v)
    a, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=fast)
    pro2 = {kk: vv.copy() for kk, vv in pro.items()}
    pro2["k8"][:, :, 200:] = 127
    pro2["v8"][:, :, 200:] = 0x7e
    b, _ = oracle.sage_emulate(p, pro2, out_dtype=p.dtype, fast_exp=fast)
    assert np.array_equal(a, b)


def test_fast_logits_equal_exact_ones_at_tiny_scale(oracle):
    """With q_scale * k_scale tiny, 1.5 * 2^23 * sc is small and the bias
    round trip (add in the accumulator, subtract in the FMA) is exact to fp32
    rounding of the logits: both modes agree to ~1e-6."""
    p, q, k, v, pro = _c1(oracle)
    pro = dict(pro)
    pro["q_scale"] = (pro["q_scale"] * np.float32(2.0 ** -14)).astype(np.float32)
    a, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=True)
    b, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=False)
    scale = np.abs(b).max()
    assert np.abs(a - b).max() <= 1e-5 * scale


def test_fast_logit_shift_is_small_at_baseline_scale(oracle):
    """At the baseline config's scales the fast mode moves each (row, block)
    logit by at most ulp(1.5 * 2^23 * sc): outputs stay within 1e-4 cosine
    distance of the exact mode, and not bit-identical (the shift is real)."""
    p, q, k, v, pro = _c1(oracle)
    a, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=True)
    b, _ = oracle.sage_emulate(p, pro, out_dtype=p.dtype, fast_exp=False)
    e = oracle.errors(a, b)
    assert e["cos"] > 1 - 1e-4, e
    sc_max = float(pro["q_scale"].max() * pro["k_scale"].max())
    ulp = np.spacing(np.float32(12582912.0 * sc_max))
    # a common factor 2^(shift) per block moves out by at most |out| * (2^(2 ulp) - 1) + E4M3 tie flips
    assert e["max_abs"] <= float(np.abs(b).max()) * (2.0 ** (2 * ulp) - 1) + 0.05, (e, ulp)


def test_f64_attention_closed_forms(oracle):
    """Textbook attention: constant V rows give that constant for every query
    (the weights sum to 1), and a causal row 0 sees only key 0."""
    p, g = oracle.config(1, seed=5)
    q, k, v = oracle.generate(p, g)
    c = oracle.encode16(np.array([1.75], np.float32), p.dtype)[0]
    vc = np.full_like(v, c)
    out = oracle.attention_f64(p, q, k, vc)
    np.testing.assert_allclose(out, 1.75, rtol=1e-6)
    p.causal = True
    out = oracle.attention_f64(p, q, k, v, rows=np.array([0], np.int32))
    v0 = oracle.decode16(v[:, 0], p.dtype)  # [B, HK, D]
    np.testing.assert_allclose(out[:, :, 0], v0, rtol=1e-6, atol=1e-7)
