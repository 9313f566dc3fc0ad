"""Pins the oracle's fused QK LayerNorm (QkNorm) on the CPU: the fp32
LayerNorm of the prologue against the reference's own f64 layer_norm
(sezer-muhammed/sota-papers-lab, platform/spl-nn/src/sage/reference.rs:109-118)
on random, offset, eps-dominated and constant rows, with the bound shown to
reject plausible mistakes; then the reference's prologue checks
(tests.rs:606-631) and attention gate (tests.rs:673-700) on plans with the
norm, the parameters drawn as tests.rs:422-435 (ln_params) draws them."""
from __future__ import annotations

import numpy as np
import pytest

from prologue_invariants import check_prologue, layer_norm_rows

EPS = 1e-5
U = 2.0 ** -24


def ln_params(oracle, d: int, seed: int) -> np.ndarray:
    """tests.rs:422-435: weights 1 + 0.5 N(0,1), biases 0.8 N(0,1), in f32."""
    rng = oracle.Rng(seed)
    out = []
    for part in range(4):
        for _ in range(d):
            x = np.float32(rng.normal())
            out.append(np.float32(1.0) + np.float32(0.5) * x if part % 2 == 0 else np.float32(0.8) * x)
    return np.array(out, np.float32)


def row_kinds(d: int, rng) -> dict:
    return {
        "random": rng.standard_normal((64, d)) * 3 + 1,
        "offset": rng.standard_normal((64, d)) * 0.5 + 50,  # mean >> spread: the two-pass variance matters
        "eps_dominated": rng.standard_normal((64, d)) * 1e-4 + 0.3,  # variance << eps
        "large": rng.standard_normal((64, d)) * 300,
    }


def ln_bound(x: np.ndarray, w: np.ndarray, b: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """Eight f32 units of the row's conditioning: |w| (1 + |mean| / std) for
    the normalised value, plus |b| and |y| for the affine step."""
    x64 = x.astype(np.float64)
    m = x64.mean(-1, keepdims=True)
    sd = np.sqrt(((x64 - m) ** 2).mean(-1, keepdims=True) + EPS)
    return 8 * U * (np.abs(w) * (1 + np.abs(m) / sd) + np.abs(b) + np.abs(ref))


@pytest.mark.parametrize("d", [64, 128])
def test_layernorm_matches_reference_f64(oracle, d):
    lnp = ln_params(oracle, d, 3).reshape(4, d)
    rng = np.random.default_rng(d)
    for name, x in row_kinds(d, rng).items():
        x = x.astype(np.float32)
        for w, b in ((lnp[0], lnp[1]), (lnp[2], lnp[3])):
            got = oracle.layernorm(x, w, b, EPS)
            ref = layer_norm_rows(x, w, b, EPS)
            assert np.all(np.abs(got - ref) <= ln_bound(x, w, b, ref)), name
            # The oracle's f64 restatement is the reference's to the last f32 rounding.
            f64 = oracle.layernorm(x, w, b, EPS, f64=True)
            assert np.all(np.abs(f64 - ref) <= U * np.abs(ref) + 1e-30), name


@pytest.mark.parametrize("d", [64, 128])
def test_layernorm_bound_rejects_plausible_mistakes(oracle, d):
    """Each plausible slip, computed in f64 from the same rows, leaves the
    bound the oracle meets above."""
    lnp = ln_params(oracle, d, 3).reshape(4, d)
    w, b = lnp[0], lnp[1]
    rng = np.random.default_rng(7)
    kinds = row_kinds(d, rng)
    x = np.concatenate([kinds["random"], kinds["eps_dominated"]]).astype(np.float32)
    x64 = x.astype(np.float64)
    m = x64.mean(-1, keepdims=True)
    var = ((x64 - m) ** 2).mean(-1, keepdims=True)
    ref = layer_norm_rows(x, w, b, EPS)
    bound = ln_bound(x, w, b, ref)
    mistakes = {
        "unbiased variance": (x64 - m) / np.sqrt(var * d / (d - 1) + EPS) * w + b,
        "eps dropped": (x64 - m) / np.sqrt(var + 1e-30) * w + b,
        "eps outside the root": (x64 - m) / (np.sqrt(var) + EPS) * w + b,
        "weight and bias swapped": (x64 - m) / np.sqrt(var + EPS) * b + w,
        "K parameters": (x64 - m) / np.sqrt(var + EPS) * lnp[2] + lnp[3],
    }
    for name, y in mistakes.items():
        assert np.any(np.abs(y - ref) > bound), name
    assert np.all(np.abs(oracle.layernorm(x, w, b, EPS) - ref) <= bound)


def test_layernorm_closed_forms(oracle):
    d = 128
    lnp = ln_params(oracle, d, 5).reshape(4, d)
    w, b = lnp[0], lnp[1]
    # A constant row normalises to 0: the output is the bias, exactly.
    x = np.full((3, d), 2.75, np.float32)
    assert np.array_equal(oracle.layernorm(x, w, b, EPS), np.broadcast_to(b, x.shape))
    # Two values +-a: mean 0, variance a^2, rstd = 1/sqrt(a^2 + eps).
    a = np.float32(3.0)
    x = np.tile(np.array([a, -a], np.float32), d // 2)[None]
    one = np.ones(d, np.float32)
    zero = np.zeros(d, np.float32)
    got = oracle.layernorm(x, one, zero, EPS)
    rstd = np.float32(1.0) / np.sqrt(np.float32(a * a) + np.float32(EPS))
    assert np.array_equal(got[0], (x[0] * rstd).astype(np.float32))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("merge", [1, 4])
def test_prologue_with_qk_norm_passes_reference_checks(oracle, d, merge):
    """tests.rs:606-631 with the norm: (Dense, ln) and (Pool stride 4, ln), data
    seed 11, ln_params(d, 3), batch 2, 3 heads, the small frame layout."""
    lay = (3, 5, 7, 10, 1)
    tokens = lay[0] * (lay[1] + lay[2] * lay[3])
    p = oracle.Problem(2, 3, tokens, d, merge=merge, layout=lay, ln=ln_params(oracle, d, 3))
    q, k, v = oracle.reference_synthetic(p, 11)
    pro = oracle.prologue(p, q, k, v)
    dec = lambda x: oracle.decode16(x, 0)
    check_prologue(p, dec(q), dec(k), dec(v), pro)


def test_prologue_with_qk_norm_fails_checks_without_it(oracle):
    """The checks see the norm: the plain prologue fails them against normalised inputs."""
    d = 64
    p = oracle.Problem(1, 2, 200, d, ln=ln_params(oracle, d, 3))
    plain = oracle.Problem(1, 2, 200, d)
    q, k, v = oracle.reference_synthetic(p, 11)
    dec = lambda x: oracle.decode16(x, 0)
    with pytest.raises(AssertionError):
        check_prologue(p, dec(q), dec(k), dec(v), oracle.prologue(plain, q, k, v))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("merge", [1, 4])
def test_emulation_with_qk_norm_meets_reference_gate(oracle, d, merge):
    """tests.rs:673-700 with the norm: data seed 5, ln_params(d, 9), cos > 0.999
    and rel_l2 < 0.04 against the f64 reference with the same merge and norm."""
    lay = (3, 5, 7, 10, 1)
    tokens = lay[0] * (lay[1] + lay[2] * lay[3])
    p = oracle.Problem(2, 3, tokens, d, merge=merge, layout=lay, ln=ln_params(oracle, d, 9))
    q, k, v = oracle.reference_synthetic(p, 5)
    pro = oracle.prologue(p, q, k, v)
    emu, _ = oracle.sage_emulate(p, pro)
    ref = oracle.attention_f64(p, q, k, v)
    e = oracle.errors(emu, ref)
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e
    # A prologue that skips the norm misses the gate (rel_l2 < 0.04) by far.
    plain = oracle.Problem(2, 3, tokens, d, merge=merge, layout=lay)
    bad, _ = oracle.sage_emulate(plain, oracle.prologue(plain, q, k, v))
    assert oracle.errors(bad, ref)["rel_l2"] > 0.15


def test_f64_attention_with_qk_norm_equals_numpy(oracle):
    """The oracle's f64 attention under the norm against numpy float64 softmax
    attention of layer_norm_rows inputs (grouped-query: 4 Q heads, 2 KV heads)."""
    d, T, H, HK = 64, 96, 4, 2
    lnp = ln_params(oracle, d, 9)
    p = oracle.Problem(1, H, T, d, kv_heads=HK, ln=lnp)
    q, k, v = oracle.generate(p, oracle.GenSpec(seed=4))
    got = oracle.attention_f64(p, q, k, v)
    ln = lnp.reshape(4, d)
    qf = layer_norm_rows(oracle.decode16(q, 0), ln[0], ln[1], EPS).astype(np.float64)
    kf = layer_norm_rows(oracle.decode16(k, 0), ln[2], ln[3], EPS).astype(np.float64)
    vf = oracle.decode16(v, 0).astype(np.float64)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    for h in range(H):
        s = qf[0, :, h] @ kf[0, :, h // 2].T * scale
        w = np.exp(s - s.max(-1, keepdims=True))
        o = (w / w.sum(-1, keepdims=True)) @ vf[0, :, h // 2]
        assert np.allclose(got[0, h], o, atol=2e-6, rtol=1e-5), h
