"""Pins the oracle's prologue restatement on the CPU: the reference's own
tolerance checks (tests.rs:476-594) and closed forms that a dropped term, a
wrong sign or a transposed operand would break."""
from __future__ import annotations

import numpy as np
import pytest

from prologue_invariants import check_prologue


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("smooth", [True, False])
def test_oracle_passes_reference_prologue_checks(oracle, d, smooth):
    p = oracle.Problem(2, 3, 225, d, smooth_k=smooth, smooth_v=smooth)
    q, k, v = oracle.reference_synthetic(p, 11)
    pro = oracle.prologue(p, q, k, v)
    dec = lambda x: oracle.decode16(x, 0)
    check_prologue(p, dec(q), dec(k), dec(v), pro, smooth)


@pytest.mark.parametrize("cfg", [1])
def test_oracle_passes_checks_on_baseline_config(oracle, cfg):
    p, g = oracle.config(cfg, seed=3)
    q, k, v = oracle.generate(p, g)
    pro = oracle.prologue(p, q, k, v)
    dec = lambda x: oracle.decode16(x, p.dtype)
    check_prologue(p, dec(q), dec(k), dec(v), pro)


def test_gqa_prologue_quantises_each_kv_head_once(oracle):
    """Grouped-query: K/V statistics and codes per KV head equal those of the
    same KV head in a plain problem; Q is per query head."""
    p = oracle.Problem(1, 8, 300, 64, kv_heads=2)
    q, k, v = oracle.generate(p, oracle.GenSpec(seed=2))
    pro = oracle.prologue(p, q, k, v)
    for g in range(2):
        sub = oracle.Problem(1, 1, 300, 64)
        one = oracle.prologue(sub, q[:, :, 4 * g:4 * g + 1].copy(), k[:, :, g:g + 1].copy(), v[:, :, g:g + 1].copy())
        for n in ("k8", "k_scale", "v8", "stats"):
            assert np.array_equal(pro[n][:, g], one[n][:, 0]), n
        assert np.array_equal(pro["q8"][:, 4 * g], one["q8"][:, 0])


def test_constant_k_channel_gives_zero_codes_and_exact_mean(oracle):
    p = oracle.Problem(1, 2, 300, 128)
    q, k, v = oracle.generate(p, oracle.GenSpec(seed=4))
    c = oracle.encode16(np.array([3.25], np.float32), 0)[0]
    k[..., 9] = c
    v[..., 10] = c
    pro = oracle.prologue(p, q, k, v)
    assert (pro["k8"][..., :300, 9] == 0).all()
    assert (pro["stats"][:, :, 0, 9] == np.float32(3.25)).all()
    assert (pro["v8"][..., :300, 10] == 0).all()
    assert (pro["stats"][:, :, 1, 10] == np.float32(3.25)).all() and (pro["stats"][:, :, 2, 10] == 1.0).all()


def test_group_amax_element_gets_code_127_and_v_extremes_map_to_448(oracle):
    p = oracle.Problem(1, 1, 64, 64, smooth_v=False)
    q, k, v = oracle.generate(p, oracle.GenSpec(seed=5))
    x = oracle.encode16(np.array([-9.0, 7.0], np.float32), 0)
    q[0, 3, 0, 17] = x[0]  # the amax of 16-row group 0 (negative)
    v[0, 5, 0, 2] = x[0]   # V channel 2's minimum, mean 0 without smoothing
    pro = oracle.prologue(p, q, k, v)
    assert pro["q8"][0, 0, 3, 17] == -127
    assert pro["q_scale"][0, 0, 0] == np.float32(np.float32(9.0) * np.float32(1 / 127) * p.q_mul())
    assert pro["v8"][0, 0, 5, 2] == 0xFE  # -448
    assert pro["stats"][0, 0, 2, 2] == np.float32(9.0) / np.float32(448.0)


def test_stats_follow_the_reference_fold_order(oracle):
    """The K/V channel sums follow the reference's fp32 order (slot partials,
    warp butterfly, warp fold, even/odd tile fold). An independent numpy
    restatement must agree bit for bit; a plain sequential sum must not
    (so the order is actually exercised)."""
    for d in (64, 128):
        p = oracle.Problem(1, 1, 1000, d)
        q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=5.0, seed=6))
        pro = oracle.prologue(p, q, k, v)
        kf = oracle.decode16(k, 0)[0, :, 0]  # [T, D]
        T, CH = p.tokens, d // 8
        TPI, NI = 256 // CH, 128 // (256 // CH)
        qt = -(-T // 128)
        f = np.float32
        tiles = []
        for t in range(qt):
            P = np.zeros((TPI, d), np.float32)
            for s in range(TPI):
                acc = np.zeros(d, np.float32)
                for i in range(NI):
                    tok = t * 128 + s + TPI * i
                    if tok < T:
                        acc = (acc + kf[tok]).astype(f)
                P[s] = acc
            spw = 32 // CH
            W = [(P[2 * w] + P[2 * w + 1]).astype(f) if spw == 2 else
                 ((P[4 * w] + P[4 * w + 1]).astype(f) + (P[4 * w + 2] + P[4 * w + 3]).astype(f)).astype(f)
                 for w in range(8)]
            r = W[0]
            for w in range(1, 8):
                r = (r + W[w]).astype(f)
            tiles.append(r)
        r0 = np.zeros(d, f)
        r1 = np.zeros(d, f)
        for t in range(0, qt - 1, 2):
            r0 = (r0 + tiles[t]).astype(f)
            r1 = (r1 + tiles[t + 1]).astype(f)
        if qt % 2:
            r0 = (r0 + tiles[qt - 1]).astype(f)
        mean = ((r0 + r1).astype(f) / f(T)).astype(f)
        assert np.array_equal(pro["stats"][0, 0, 0].view(np.uint32), mean.view(np.uint32))
        seq = np.zeros(d, f)
        for tok in range(T):
            seq = (seq + kf[tok]).astype(f)
        assert not np.array_equal((seq / f(T)).astype(f), mean), "order-insensitive data"
