"""Pins the oracle's codecs and RNG.

Known answers from the reference's own tests (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/tests.rs:24-83), the published splitmix64 vector,
and exhaustive or dense comparisons with independent exact methods (nearest
representable value by exact float64 distance; numpy's IEEE float16).
"""
from __future__ import annotations

import numpy as np
import pytest


def _f32(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


# ---------------------------------------------------------------- e4m3

def test_e4m3_codes_round_trip(oracle):
    """tests.rs:24-37."""
    codes = np.arange(256, dtype=np.uint8)
    vals = oracle.e4m3_decode(codes)
    for b in range(256):
        if b & 0x7F == 0x7F:
            assert np.isnan(vals[b])
            continue
        assert oracle.e4m3_encode(vals[b:b + 1])[0] == b, f"code {b:#04x} = {vals[b]}"
    assert vals[0x7E] == 448.0
    assert vals[0x01] == 2.0 ** -9
    assert vals[0x38] == 1.0


def test_e4m3_rounds_to_nearest_even_and_saturates(oracle):
    """tests.rs:39-55."""
    enc = lambda x: int(oracle.e4m3_encode(np.array([x], np.float32))[0])
    dec = lambda b: float(oracle.e4m3_decode(np.array([b], np.uint8))[0])
    assert dec(enc(1.0625)) == 1.0
    assert dec(enc(1.1875)) == 1.25
    assert dec(enc(-3.3)) == -3.25
    assert enc(1000.0) == 0x7E
    assert enc(-1000.0) == 0xFE
    assert enc(2.0 ** -10) == 0
    assert dec(enc(3.0 * 2.0 ** -10)) == 2.0 ** -8
    assert dec(enc(15.9)) == 16.0
    assert enc(float("nan")) == 0x7F
    assert enc(float("inf")) == 0x7E and enc(float("-inf")) == 0xFE


def _e4m3_exact(x: np.ndarray) -> np.ndarray:
    """Independent RNE-satfinite: nearest finite E4M3 value by exact float64
    distance after clamping to +-448, ties to the even code."""
    codes = np.arange(0, 0x7F, dtype=np.int64)  # non-negative finite codes 0x00..0x7e
    e = (codes >> 3) & 0xF
    m = codes & 7
    vals = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * np.exp2(e - 7.0))
    a = np.minimum(np.abs(x.astype(np.float64)), 448.0)
    i = np.clip(np.searchsorted(vals, a), 1, len(vals) - 1)
    lo, hi = vals[i - 1], vals[i]
    dlo, dhi = a - lo, hi - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (codes[i] % 2 == 0))
    c = np.where(pick_hi, codes[i], codes[i - 1])
    c = np.where(a < vals[0] + 1e-300, 0, c)  # exact zero
    sign = np.signbit(x).astype(np.int64) << 7
    return (c | sign).astype(np.uint8)


def test_e4m3_encode_matches_exact_rounding_densely(oracle):
    # every 241st positive float32 pattern up to inf, both signs, plus all exact ties
    bits = np.arange(0, 0x7F800000, 241, dtype=np.uint64).astype(np.uint32)
    x = _f32(bits)
    x = np.concatenate([x, -x])
    vals = oracle.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    ties = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, ties, -ties, vals.astype(np.float32)])
    got = oracle.e4m3_encode(x)
    want = _e4m3_exact(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]


# ---------------------------------------------------------------- bf16 / fp16

def test_bf16_rounds_to_nearest_even(oracle):
    """tests.rs:57-66."""
    enc = lambda x: int(oracle.encode16(np.array([x], np.float32), 0)[0])
    dec = lambda b: float(oracle.decode16(np.array([b], np.uint16), 0)[0])
    assert enc(1.0) == 0x3F80
    assert dec(enc(1.0 + 1.0 / 256.0)) == 1.0
    assert dec(enc(1.0 + 3.0 / 256.0)) == 1.0 + 4.0 / 256.0
    assert dec(enc(-2.5)) == -2.5


def test_bf16_encode_matches_exact_rounding_densely(oracle):
    bits = np.arange(0, 0x7F7F0000, 4099, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([_f32(bits), -_f32(bits)])
    got = oracle.encode16(x, 0)
    # independent: the two bf16 neighbours by exact float64 distance, ties to even
    t = (x.view(np.uint32) & 0xFFFF0000).astype(np.uint32)
    lo = t.view(np.float32).astype(np.float64)
    up = (t + 0x10000).astype(np.uint32).view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dup = np.abs(xd - lo), np.abs(up - xd)
    even_lo = ((t >> 16) & 1) == 0
    pick_up = (dup < dlo) | ((dup == dlo) & ~even_lo)
    want = np.where(pick_up, (t >> 16) + 1, t >> 16).astype(np.uint16)
    assert np.array_equal(got, want)
    dec = oracle.decode16(np.arange(65536, dtype=np.uint16), 0)
    assert np.array_equal(dec.view(np.uint32), np.arange(65536, dtype=np.uint32) << 16)


def test_f16_codecs_match_ieee_binary16(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    got = oracle.decode16(codes, 1)
    want = codes.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(50),
        (rng.standard_normal(200000) * 1e-5).astype(np.float32),
        np.array([65504, 65519.9, 65520, 1e6, -1e6, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0], np.float32),
    ])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.encode16(x, 1), want)


def test_s8_rounds_half_even_and_clamps(oracle):
    s8 = oracle.lib().oracle_s8
    cases = {0.5: 0, 1.5: 2, 2.5: 2, -0.5: 0, -1.5: -2, 126.5: 126, 127.4: 127, 127.6: 127, 300.0: 127,
             -300.0: -127, 0.49999997: 0}
    for x, want in cases.items():
        assert s8(x) == want, x


def test_v_permutation_matches_the_p_fragment(oracle):
    """tests.rs:68-83 (the reference's NVIDIA-fragment permutation)."""
    seen = [False] * 16
    for t in range(4):
        for e, key in enumerate([2 * t, 2 * t + 1, 8 + 2 * t, 9 + 2 * t]):
            assert oracle.lib().oracle_vpos_ref(key) == 4 * t + e
            seen[oracle.lib().oracle_vpos_ref(key)] = True
    assert all(seen)


# ---------------------------------------------------------------- RNG

def test_splitmix64_published_vector(oracle):
    r = oracle.Rng(1234567)
    assert [r.next_u64() for _ in range(5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431, 16408922859458223821]


def test_uniform_and_normal_follow_box_muller(oracle):
    r1, r2 = oracle.Rng(42), oracle.Rng(42)
    u = r1.uniform()
    assert u == (r2.next_u64() >> 11) / float(1 << 53)
    r = oracle.Rng(9)
    z = np.array([r.normal() for _ in range(100000)])
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    r1, r2 = oracle.Rng(5), oracle.Rng(5)
    u1, u2 = r2.uniform(), r2.uniform()
    want = np.float32(np.sqrt(-2.0 * np.log(max(u1, 1e-300))) * np.cos(2 * np.pi * u2))
    assert abs(r1.normal() - want) <= 1e-6 * max(1.0, abs(want))
