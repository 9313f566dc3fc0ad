"""Pins the oracle's QKV prologue (oracle/qkv_oracle.c), the upstream step whose
bf16 Q, K and V the sage prologue reads (sezer-muhammed/sota-papers-lab,
platform/spl-nn/cuda/qkv.cu, src/qkv.rs): the reference's own table and
rotation tests (qkv.rs:374-451), its kernel-vs-CPU gate (tests.rs:447-570:
rel_rms <= 3e-3 and max_abs <= 0.06 against the f64 reference) on the VGGT
layout, and closed forms: no options is the identity, zero angles rotate
nothing, V is never normalised or rotated. The same gate is shown to reject
a flipped rotation sign, a variance without its mean, and the Q parameters
on K."""
from __future__ import annotations

import math

import numpy as np
import pytest

GRID_H, GRID_W, SPECIAL = 21, 32, 17  # 512 x 336 at 16 px: 689-token frames (tests.rs:451)


def _err(got, want):
    """testkit.rs Err: max_abs, rms, rel_rms (rms over the rms of want)."""
    g, w = np.asarray(got, np.float64).ravel(), np.asarray(want, np.float64).ravel()
    d = g - w
    rms = math.sqrt(float((d * d).mean()))
    return {"max_abs": float(np.abs(d).max()), "rms": rms, "rel_rms": rms / math.sqrt(float((w * w).mean()))}


def _gate(e):
    return e["rel_rms"] <= 3e-3 and e["max_abs"] <= 0.06


def test_layouts_pair_the_right_channels(oracle):
    """qkv.rs:378-393, plus the head-dim-128 extension."""
    O = oracle
    assert [O.rope_pair(O.ROPE_VGGT, 64, d) for d in (0, 16, 15)] == [0, 0, 15]
    assert [O.rope_pair(O.ROPE_VGGT, 64, d) for d in (32, 48, 63)] == [16, 16, 31]
    assert [O.rope_pair(O.ROPE_DINOV3, 64, d) for d in (0, 32, 31, 63)] == [0, 0, 31, 31]
    for D in (64, 128):
        for lay in (O.ROPE_VGGT, O.ROPE_DINOV3):
            h = O.rope_half(lay, D)
            assert h == (D // 4 if lay == O.ROPE_VGGT else D // 2)
            pairs = [O.rope_pair(lay, D, c) for c in range(D)]
            assert all(pairs[c] == pairs[c ^ h] for c in range(D))
            assert sorted(set(pairs)) == list(range(D // 2))


def test_vggt_table_matches_its_formula(oracle):
    """qkv.rs:396-410: 2 special tokens, a 3 x 4 grid."""
    t = oracle.rope_table(oracle.ROPE_VGGT, 64, 3, 4, 2, 100.0)
    assert t.shape == (14, 32, 2)
    assert tuple(t[1, 5]) == (1.0, 0.0)
    a = 2.0 * 100.0 ** (-3.0 / 16.0)  # token 9 = patch (1, 3): positions (2, 4)
    assert abs(t[9, 3, 0] - math.cos(a)) < 1e-7 and abs(t[9, 3, 1] - math.sin(a)) < 1e-7
    a = 4.0 * 100.0 ** (-5.0 / 16.0)
    assert abs(t[9, 16 + 5, 1] - math.sin(a)) < 1e-7


def test_dinov3_table_matches_its_formula(oracle):
    """qkv.rs:413-421."""
    t = oracle.rope_table(oracle.ROPE_DINOV3, 64, 2, 2, 1, 100.0)
    a = 2.0 * math.pi * -0.5  # patch (0, 1): coords (-0.5, 0.5)
    assert abs(t[2, 0, 1] - math.sin(a)) < 1e-7
    a = 2.0 * math.pi * 0.5 / 100.0 ** (2.0 / 16.0)
    assert abs(t[2, 18, 0] - math.cos(a)) < 1e-7


def _y(rng, s, scale=1.0):
    import sys
    from oracle import pyoracle as O

    y = rng.standard_normal((s.batch, s.tokens, s.row_stride())).astype(np.float32) * scale
    return O.encode16(y, 0)


def _spec(oracle, rng, D=64, heads=4, kv_heads=0, norm=0, rope=None, scaled=False, frames=2, batch=1):
    O = oracle
    tokens = frames * (SPECIAL + GRID_H * GRID_W)
    s = O.QkvSpec(batch, tokens, heads, D, kv_heads=kv_heads)
    s.ld = s.width + 8
    if scaled:
        s.tok = (0.5 + rng.random(batch * tokens)).astype(np.float32)
        s.chan = (0.5 + rng.random(s.width)).astype(np.float32)
    s.bias = O.encode16((0.2 * rng.standard_normal(s.width)).astype(np.float32), 0)
    if norm:
        s.norm = norm
        w = np.stack([1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
                      1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)]).astype(np.float32)
        s.norm_w = w
    if rope is not None:
        s.rope = O.rope_table(rope, D, GRID_H, GRID_W, SPECIAL, 100.0)
        s.rope_layout = rope
    return s


CASES = [  # tests.rs:457-462, plus head dim 128 and grouped heads (extensions)
    (64, 16, 0, "vggt", 1, False),
    (64, 16, 0, "dinov3", 2, True),
    (64, 6, 0, "vggt", 0, True),
    (64, 3, 0, None, 1, False),
    (128, 4, 2, "vggt", 1, True),
    (128, 4, 0, "dinov3", 2, False),
]


@pytest.mark.parametrize("D,heads,kv,rope,norm,scaled", CASES)
def test_kernel_arithmetic_meets_the_references_gate(oracle, D, heads, kv, rope, norm, scaled):
    """tests.rs:447-570 (gpu_qkv_prologue_matches_cpu): the fp32 restatement's
    bf16 outputs against the f64 reference, rel_rms <= 3e-3 and max_abs <= 0.06."""
    O = oracle
    rng = np.random.default_rng(5 + D + heads)
    lay = {None: None, "vggt": O.ROPE_VGGT, "dinov3": O.ROPE_DINOV3}[rope]
    s = _spec(O, rng, D, heads, kv, norm, lay, scaled, frames=2 if D == 64 else 1)
    y = _y(rng, s)
    got = O.qkv_prologue(s, y)
    want = O.qkv_reference_f64(s, y)
    for name, g, w in zip("qkv", got, want):
        e = _err(O.decode16(g, 0), w)
        print(f"D{D} H{heads} {rope} norm {norm} scaled {scaled} {name}: {e}")
        assert _gate(e), (name, e)


def test_no_options_is_the_identity(oracle):
    """No scales, bias, norm or rope: Q, K and V are the projection's bf16 values."""
    O = oracle
    rng = np.random.default_rng(1)
    s = O.QkvSpec(2, 50, 3, 64, kv_heads=1)
    s.ld = s.width + 16
    y = _y(rng, s)
    q, k, v = O.qkv_prologue(s, y)
    D = 64
    assert np.array_equal(q, y[:, :, :3 * D].reshape(2, 50, 3, D))
    assert np.array_equal(k, y[:, :, 3 * D:4 * D].reshape(2, 50, 1, D))
    assert np.array_equal(v, y[:, :, 4 * D:5 * D].reshape(2, 50, 1, D))


@pytest.mark.parametrize("D", [64, 128])
def test_rotation_preserves_pair_norms_and_spares_special_tokens(oracle, D):
    """qkv.rs:424-450: V is never rotated; every rotation pair keeps its norm
    (f64, and the fp32 restatement within bf16 rounding); special tokens (angle
    0) come out exactly as without RoPE."""
    O = oracle
    rng = np.random.default_rng(D)
    s = O.QkvSpec(1, 3, 2, D)
    y = _y(rng, s)
    base = O.qkv_reference_f64(s, y)
    s.rope = O.rope_table(O.ROPE_VGGT, D, 1, 2, 1, 100.0)
    s.rope_layout = O.ROPE_VGGT
    rot = O.qkv_reference_f64(s, y)
    assert np.array_equal(base[2], rot[2])
    h = O.rope_half(O.ROPE_VGGT, D)
    for a, b in ((base[0], rot[0]), (base[1], rot[1])):
        for d in range(D):
            if d & h:
                continue
            n0 = a[..., d].astype(np.float64) ** 2 + a[..., d + h].astype(np.float64) ** 2
            n1 = b[..., d].astype(np.float64) ** 2 + b[..., d + h].astype(np.float64) ** 2
            assert np.all(np.abs(n0 - n1) <= 1e-6 * np.maximum(n0, 1.0))
    assert np.array_equal(base[0][:, 0], rot[0][:, 0])
    # the fp32 restatement: token 0 bit-identical to the unrotated one, norms within bf16 steps
    q_plain = O.qkv_prologue(O.QkvSpec(1, 3, 2, D), y)[0]
    q_rot = O.qkv_prologue(s, y)[0]
    assert np.array_equal(q_plain[:, 0], q_rot[:, 0])
    a, b = O.decode16(q_plain, 0).astype(np.float64), O.decode16(q_rot, 0).astype(np.float64)
    for d in range(D):
        if not d & h:
            n0 = a[..., d] ** 2 + a[..., d + h] ** 2
            n1 = b[..., d] ** 2 + b[..., d + h] ** 2
            assert np.all(np.abs(n0 - n1) <= 2 * 2.0 ** -7 * np.maximum(n0, 1e-3))


def test_v_is_scaled_but_never_normalised(oracle):
    """QK-norm and RoPE act on q and k only (qkv.cu:84,105): V equals the
    no-norm, no-rope V bit for bit."""
    O = oracle
    rng = np.random.default_rng(3)
    s = _spec(O, rng, 64, 4, 0, O.NORM_LAYER, O.ROPE_DINOV3, True, frames=1)
    y = _y(rng, s)
    v = O.qkv_prologue(s, y)[2]
    s.norm, s.rope = 0, None
    assert np.array_equal(v, O.qkv_prologue(s, y)[2])


def test_the_gate_rejects_plausible_slips(oracle):
    """The fp32 restatement fails the reference gate against f64 references
    carrying a flipped rotation sign, a variance taken without its mean, or the
    Q norm parameters applied to K."""
    O = oracle
    rng = np.random.default_rng(9)
    s = _spec(O, rng, 64, 4, 0, O.NORM_LAYER, O.ROPE_VGGT, False, frames=1)
    y = _y(rng, s)
    q, k, _ = O.qkv_prologue(s, y)
    qf, kf = O.decode16(q, 0), O.decode16(k, 0)
    # flipped sign: rotate by -angle (sin negated)
    s2 = _spec(O, np.random.default_rng(9), 64, 4, 0, O.NORM_LAYER, O.ROPE_VGGT, False, frames=1)
    s2.rope = s2.rope.copy()
    s2.rope[..., 1] *= -1
    assert not _gate(_err(qf, O.qkv_reference_f64(s2, y)[0]))
    # RMS statistics where LayerNorm is asked (variance without its mean)
    s3 = _spec(O, np.random.default_rng(9), 64, 4, 0, O.NORM_RMS, O.ROPE_VGGT, False, frames=1)
    s3.norm_w = s.norm_w
    assert not _gate(_err(qf, O.qkv_reference_f64(s3, y)[0]))
    # the Q parameters on K
    s4 = _spec(O, np.random.default_rng(9), 64, 4, 0, O.NORM_LAYER, O.ROPE_VGGT, False, frames=1)
    w = s.norm_w.copy()
    w[2:] = w[:2]
    s4.norm_w = w
    assert not _gate(_err(kf, O.qkv_reference_f64(s4, y)[1]))


def test_v_in_fp16_meets_the_references_gate(oracle):
    """tests.rs:536-560: V written in fp16 (VFormat::F16) against the f64
    reference, rel_rms <= 5e-4 and max_abs <= 4e-3; Q and K stay bf16."""
    O = oracle
    rng = np.random.default_rng(11)
    s = _spec(O, rng, 64, 16, 0, O.NORM_LAYER, O.ROPE_VGGT, False, frames=2)
    y = _y(rng, s)
    q16, k16, v16 = O.qkv_prologue(s, y)
    s.v_f16 = True
    q, k, v = O.qkv_prologue(s, y)
    assert np.array_equal(q, q16) and np.array_equal(k, k16)
    e = _err(O.decode16(v, 1), O.qkv_reference_f64(s, y)[2])
    assert e["rel_rms"] <= 5e-4 and e["max_abs"] <= 4e-3, e
    assert not np.array_equal(v, v16)
