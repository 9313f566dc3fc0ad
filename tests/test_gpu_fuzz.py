"""Seeded random problems on the GPU, through the C ABI: every option of the
path drawn together (head dim, batch, grouped heads, ragged lengths, bf16 or
fp16 inputs and output, causal masking, KV merging over random frame
layouts, QK LayerNorm, PvAccum::F16, smoothing off, custom softmax scales,
strided Q/K/V layouts). Each case: the prologue bit-exact against the oracle
and the attention within the north-star gate of the reference arithmetic
(cos >= 0.999; max-abs 2e-2 plus half an output rounding step) and no
further from f64 than that arithmetic."""
from __future__ import annotations

import numpy as np
import pytest

from sage_gpu_helpers import assert_prologue_equal, gather_rows, run, sample_rows
from test_gpu_parity import COS_MIN, COS_SLACK, MAX_ABS as ABS_MAX, REL_L2_SLACK

pytestmark = pytest.mark.gpu

CASES = 32


def _case(oracle, i: int):
    rng = np.random.default_rng(1000 + i)
    d = int(rng.choice([64, 128]))
    b = int(rng.integers(1, 3))
    heads = int(rng.integers(1, 7))
    divisors = [x for x in range(1, heads + 1) if heads % x == 0]
    kv_heads = int(rng.choice(divisors))
    dtype = int(rng.integers(0, 2))
    merge = int(rng.choice([1, 1, 1, 2, 4]))
    kw = {}
    if merge > 1:
        frames = int(rng.integers(1, 4))
        layout = (frames, int(rng.integers(0, 7)), int(rng.integers(2, 10)), int(rng.integers(2, 12)),
                  int(rng.integers(0, frames + 1)))
        tokens = frames * (layout[1] + layout[2] * layout[3])
        kw.update(merge=merge, layout=layout)
        causal = False
    else:
        tokens = int(rng.integers(1, 701))
        causal = bool(rng.random() < 0.3)
    if rng.random() < 0.3:
        lnp = np.concatenate([1 + 0.5 * rng.standard_normal(d), 0.8 * rng.standard_normal(d),
                              1 + 0.5 * rng.standard_normal(d), 0.8 * rng.standard_normal(d)]).astype(np.float32)
        kw["ln"] = lnp
    smooth = bool(rng.random() < 0.8)
    scale = None if rng.random() < 0.6 else float(rng.uniform(0.05, 0.3))
    p = oracle.Problem(b, heads, tokens, d, kv_heads=kv_heads if kv_heads != heads else 0, dtype=dtype,
                       causal=causal, smooth_k=smooth, smooth_v=smooth, softmax_scale=scale,
                       pv16=bool(rng.random() < 0.25), **kw)
    gen = oracle.GenSpec(k_off_std=float(rng.uniform(0, 3)), outlier_channels=int(rng.integers(0, 3)),
                         outlier_scale=float(rng.uniform(1, 10)), token_frac=float(rng.choice([0.0, 0.02])),
                         token_scale=float(rng.uniform(1, 5)), seed=int(rng.integers(1, 1 << 30)))
    layouts = ["bthd", "bhtd"] + (["packed"] if kv_heads == heads else [])
    q_layout = str(rng.choice(layouts))
    out_dtype = int(rng.integers(0, 2))
    return p, gen, q_layout, out_dtype


def _check(oracle, p, want, o, rows, q, k, v, out_dtype, label):
    """The north-star gate against the emulated reference arithmetic, per
    element against its fp32 output: |ours - emu| <= 2e-2 plus half a step of
    the output type (2^-8 |emu| for bf16, 2^-11 |emu| for fp16) -- scaled
    tokens make outputs large enough that one rounding step of bf16 exceeds
    2e-2 -- and cos >= 0.999; and no further from f64 than the emulation."""
    emu, emu16 = oracle.sage_emulate(p, want, rows=rows, out_dtype=out_dtype)
    ours = oracle.decode16(gather_rows(o, rows), out_dtype)
    exact = oracle.attention_f64(p, q, k, v, rows=rows)
    e = oracle.errors(ours, emu)
    e64 = oracle.errors(ours, exact)
    emu64 = oracle.errors(oracle.decode16(emu16, out_dtype), exact)
    print(f"{label}: vs reference arithmetic {e}; vs f64 {e64}; reference arithmetic vs f64 {emu64}")
    assert np.isfinite(ours).all()
    half_step = 2.0 ** (-8 if out_dtype == 0 else -11)
    assert np.all(np.abs(ours - emu) <= ABS_MAX + half_step * np.abs(emu)), e
    assert e["cos"] >= COS_MIN, e
    assert e64["cos"] >= emu64["cos"] - COS_SLACK, (e64, emu64)
    assert e64["rel_l2"] <= emu64["rel_l2"] * 1.02 + REL_L2_SLACK, (e64, emu64)


@pytest.mark.parametrize("i", range(CASES))
def test_random_problem(oracle, torch_gpu, i):
    p, gen, q_layout, out_dtype = _case(oracle, i)
    print(f"case {i}: B{p.batch} H{p.heads}/{p.hk} N{p.tokens} D{p.head_dim} dtype {p.dtype} out {out_dtype} "
          f"causal {p.causal} merge {p.merge} {p.layout if p.merge > 1 else ''} ln {p.ln is not None} "
          f"pv16 {p.pv16} smooth {p.smooth_k} scale {p.softmax_scale} layout {q_layout}", flush=True)
    q, k, v = oracle.generate(p, gen)
    pro, o = run(torch_gpu, p, q, k, v, out_dtype=out_dtype, q_layout=q_layout)
    want = oracle.prologue(p, q, k, v)
    assert_prologue_equal(pro, want)
    _check(oracle, p, want, o, sample_rows(p.tokens, 256, seed=i), q, k, v, out_dtype, f"case {i}")
