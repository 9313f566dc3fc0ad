"""Pins the oracle's KV merging (KvMerge::Pool) on the CPU: the reference's own
known answers for the pooled-key geometry (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/tests.rs:85-232), the log-count bias table against a
60-digit evaluation, the prologue's tolerance checks on merged plans
(tests.rs:476-594) and the merged == dense identity of attention on uniform
cells."""
from __future__ import annotations

from decimal import Decimal, getcontext

import numpy as np
import pytest

from prologue_invariants import check_prologue


def vggt_layout(frames: int, dense_frames: int = 0):
    """tests.rs:85-93: 17 special tokens and a 21 x 32 patch grid (689 tokens a frame)."""
    return (frames, 17, 21, 32, dense_frames)


def small_layout():
    """tests.rs:596-605: 3 frames, 5 special, a 7 x 10 grid, the first frame dense."""
    return (3, 5, 7, 10, 1)


def merged(oracle, stride, layout, heads=1, d=64, batch=1, **kw):
    frames, special, gh, gw, _ = layout
    return oracle.Problem(batch, heads, frames * (special + gh * gw), d, merge=stride, layout=layout, **kw)


def test_dense_first_frame_keeps_its_keys(oracle):
    """tests.rs:96-133."""
    p = merged(oracle, 4, vggt_layout(3, dense_frames=1))
    assert p.tk == 689 + 2 * 65
    for j in range(689):
        assert p.members(j) == [j]
    for j in range(689, 689 + 17):
        assert p.members(j) == [j]
    assert p.members(689 + 17) == [706, 707, 708, 709, 738, 739, 740, 741, 770, 771, 772, 773, 802, 803, 804, 805]
    seen = np.zeros(3 * 689, np.int64)
    for j in range(p.tk):
        for t in p.members(j):
            seen[t] += 1
    assert (seen == 1).all()


def test_vggt_merge_geometry(oracle):
    """tests.rs:136-173."""
    lay = vggt_layout(200)
    m2, m4 = merged(oracle, 2, lay, heads=16), merged(oracle, 4, lay, heads=16)
    assert m2.tk == 200 * (17 + 11 * 16)
    assert m4.tk == 200 * (17 + 6 * 8)
    for p, per in ((m2, 17 + 11 * 16), (m4, 17 + 6 * 8)):
        hit = np.zeros(689, np.int64)
        for j in range(per, 2 * per):
            for t in p.members(j):
                hit[t - 689] += 1
        assert (hit == 1).all()
        assert p.members(per + 3) == [689 + 3]
    assert len(m4.members(17)) == 16
    assert len(m4.members(17 + 5 * 8)) == 4  # row 20 only
    assert len(m2.members(17 + 10 * 16)) == 2


def test_log2_count_table_is_correctly_rounded(oracle):
    getcontext().prec = 60
    for n in range(1, 17):
        exact = Decimal(n).ln() / Decimal(2).ln()
        got = oracle.log2_count(n)
        f = np.float32(got)
        up, dn = np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))
        err = abs(Decimal(float(f)) - exact)
        assert err <= abs(Decimal(float(up)) - exact) and err <= abs(Decimal(float(dn)) - exact), n
        assert abs(got - float(np.log2(np.float32(n)))) <= float(np.spacing(f)), n  # numpy's f32 log2: within 1 ulp


@pytest.mark.parametrize("stride", [2, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_merged_prologue_passes_reference_checks(oracle, stride, d):
    """check_prologue (tests.rs:476-594) on merged plans, small_layout as gpu_prologue_matches_reference uses."""
    p = merged(oracle, stride, small_layout(), heads=2, d=d)
    q, k, v = oracle.reference_synthetic(p, 5)
    pro = oracle.prologue(p, q, k, v)
    dec = lambda x: oracle.decode16(x, 0)
    check_prologue(p, dec(q), dec(k), dec(v), pro)


def test_merged_prologue_of_single_members_equals_dense(oracle):
    """Dense frames and special tokens are one-member keys: their codes equal
    the dense plan's bit for bit (a full-cell key differs only by pooling)."""
    lay = (2, 5, 4, 4, 1)  # frame 0 dense (21 tokens), frame 1: 5 special + 2x2 cells of 4
    p = merged(oracle, 2, lay, heads=1, d=64)
    dense = oracle.Problem(1, 1, p.tokens, 64)
    q, k, v = oracle.generate(dense, oracle.GenSpec(seed=9))
    pm, pd = oracle.prologue(p, q, k, v), oracle.prologue(dense, q, k, v)
    assert np.array_equal(pm["stats"], pd["stats"])  # statistics run over every token
    assert np.array_equal(pm["q8"], pd["q8"]) and np.array_equal(pm["q_scale"], pd["q_scale"])
    vd = pd["v8"][0, 0, :26]
    vm = pm["v8"][0, 0, :26]
    assert np.array_equal(vm, vd)  # V codes need no block scale: single-member keys match exactly
    # A full 2 x 2 cell: the pooled value is the f32 mean of its members, up to the e4m3 step.
    cell = p.members(26)
    assert len(cell) == 4
    st = pm["stats"][0, 0]
    vf = oracle.decode16(v[0, :, 0], 0)
    pooled = (((np.float32(0) + vf[cell[0]]) + vf[cell[1]] + vf[cell[2]]) + vf[cell[3]]) * np.float32(0.25)
    got = oracle.e4m3_decode(pm["v8"][0, 0, 26]) * st[2] + st[1]
    assert np.all(np.abs(got - pooled) <= np.abs(pooled - st[1]) / 16 + st[2] * 2.0 ** -8 + 1e-6)


@pytest.mark.parametrize("stride", [2, 4])
def test_merged_attention_equals_dense_on_uniform_cells(oracle, stride):
    """tests.rs:193-232: when every pooled cell holds identical keys and values,
    attention over the pooled keys with the +log(count) bias is dense attention."""
    lay = (2, 3, 5, 7, 0)
    p = merged(oracle, stride, lay, heads=1, d=16, softmax_scale=0.25)
    dense = oracle.Problem(1, 1, p.tokens, 16, softmax_scale=0.25)
    rng = np.random.default_rng(7)
    cell_k = rng.standard_normal((p.tk, 16)).astype(np.float32)
    cell_v = rng.standard_normal((p.tk, 16)).astype(np.float32)
    k = np.zeros((1, p.tokens, 1, 16), np.float32)
    v = np.zeros_like(k)
    for j in range(p.tk):
        for t in p.members(j):
            k[0, t, 0] = cell_k[j]
            v[0, t, 0] = cell_v[j]
    q = (2.0 * rng.standard_normal((1, p.tokens, 1, 16))).astype(np.float32)
    enc = lambda x: oracle.encode16(x, 0)
    q16, k16, v16 = enc(q), enc(k), enc(v)
    out_d = oracle.attention_f64(dense, q16, k16, v16)
    out_m = oracle.attention_f64(p, q16, k16, v16)
    e = oracle.errors(out_m, out_d)
    assert e["max_abs"] < 1e-5, e


@pytest.mark.parametrize("stride", [2, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_merged_emulation_meets_the_reference_gate(oracle, stride, d):
    """The merged kernel's arithmetic against f64 merged attention: the reference's
    gate for gpu_attention_matches_float_reference (tests.rs:691-700)."""
    p = merged(oracle, stride, small_layout(), heads=2, d=d)
    q, k, v = oracle.reference_synthetic(p, 3)
    pro = oracle.prologue(p, q, k, v)
    emu, _ = oracle.sage_emulate(p, pro)
    ref = oracle.attention_f64(p, q, k, v)
    e = oracle.errors(emu, ref)
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


def test_merged_emulation_logit_modes_agree(oracle):
    """fast_exp (1.5*2^23-biased scores, the bias folded into the offset) and
    exact scores give the same output to rounding."""
    p = merged(oracle, 2, small_layout(), heads=1, d=64)
    q, k, v = oracle.reference_synthetic(p, 4)
    pro = oracle.prologue(p, q, k, v)
    a, _ = oracle.sage_emulate(p, pro, fast_exp=True)
    b, _ = oracle.sage_emulate(p, pro, fast_exp=False)
    e = oracle.errors(a, b)
    assert e["cos"] > 0.99999 and e["max_abs"] < 2e-2, e


def test_merged_bias_shifts_weight_to_pooled_keys(oracle):
    """A planted mistake: dropping the log-count bias (every kbias 0) must move the
    emulated output far off the f64 merged reference. With Q = 0 all logits
    are equal, so the weights are the member counts: the one special token of
    each frame (V = 4) weighs 1/65, not 1/5."""
    p = merged(oracle, 4, (2, 1, 8, 8, 0), heads=1, d=64)
    q, k, v = oracle.reference_synthetic(p, 6)
    q = oracle.encode16(np.zeros(q.shape, np.float32), 0)
    vf = oracle.decode16(v, 0)
    vf[:, [0, 65]] = 4.0
    v = oracle.encode16(vf, 0)
    pro = oracle.prologue(p, q, k, v)
    ref = oracle.attention_f64(p, q, k, v)
    good, _ = oracle.sage_emulate(p, pro)
    bad_pro = dict(pro)
    bad_pro["kbias"] = np.where(np.isfinite(pro["kbias"]), 0.0, -np.inf).astype(np.float32)
    bad, _ = oracle.sage_emulate(p, bad_pro)
    assert oracle.errors(good, ref)["rel_l2"] < 0.04
    assert oracle.errors(bad, ref)["rel_l2"] > 0.3
