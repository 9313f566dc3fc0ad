"""The fused QK LayerNorm (QkNorm, sezer-muhammed/sota-papers-lab
platform/spl-nn/src/sage/mod.rs:337-344, cuda/sage_quant.cu:34-52) on the GPU,
through the C ABI: the prologue with the norm (codes, scales and statistics of
the normalised Q and K rows) bit-exact against the oracle, the reference's own
prologue checks on it, and the attention gated at cosine >= 0.999 and max-abs
<= 2e-2 against the oracle's emulation and by the reference's gate against f64
attention of the normalised rows (tests.rs:606-700, the ln cases)."""
from __future__ import annotations

import numpy as np
import pytest

from prologue_invariants import check_prologue
from sage_gpu_helpers import assert_prologue_equal, gather_rows, run, sample_rows
from test_gpu_parity import _check_attention
from test_oracle_qknorm import ln_params

pytestmark = pytest.mark.gpu

SMALL_LAYOUT = (3, 5, 7, 10, 1)  # tests.rs:596-605
SMALL_TOKENS = 3 * (5 + 7 * 10)

# name: (batch, heads, tokens, d, Problem kwargs)
CASES = {
    "d64": (1, 2, 1000, 64, {}),
    "d128": (1, 2, 1000, 128, {}),
    "d128_f16_ragged": (2, 2, 333, 128, {"dtype": 1}),
    "d64_gqa": (1, 4, 700, 64, {"kv_heads": 2}),
    "d128_nosmooth": (1, 2, 517, 128, {"smooth_k": False, "smooth_v": False}),
    "d64_eps1e-3": (1, 2, 400, 64, {"ln_eps": 1e-3}),
    "d128_merge4": (1, 2, SMALL_TOKENS, 128, {"merge": 4, "layout": SMALL_LAYOUT}),
    "d64_merge2": (1, 3, SMALL_TOKENS, 64, {"merge": 2, "layout": SMALL_LAYOUT}),
}


@pytest.mark.parametrize("name", list(CASES))
def test_qk_norm_prologue_and_attention(oracle, torch_gpu, name):
    b, h, t, d, kw = CASES[name]
    p = oracle.Problem(b, h, t, d, ln=ln_params(oracle, d, 3), **kw)
    q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=2.0, seed=41))
    pro, o = run(torch_gpu, p, q, k, v)
    want = oracle.prologue(p, q, k, v)
    assert_prologue_equal(pro, want)
    dec = lambda x: oracle.decode16(x, p.dtype)
    check_prologue(p, dec(q), dec(k), dec(v), pro, smooth=p.smooth_k)
    rows = sample_rows(p.tokens, 384, seed=5)
    _check_attention(oracle, p, want, o, rows, q, k, v, name)


@pytest.mark.parametrize("merge", [1, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_qk_norm_reference_gate(oracle, torch_gpu, merge, d):
    """gpu_attention_matches_float_reference (tests.rs:655-700), the ln cases:
    batch 2, 3 heads, data seed 5, ln_params(d, 9); cos > 0.999 and rel_l2 < 0.04
    against f64 attention of the normalised (and pooled) rows."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, merge=merge, layout=SMALL_LAYOUT, ln=ln_params(oracle, d, 9))
    q, k, v = oracle.reference_synthetic(p, 5)
    _, o = run(torch_gpu, p, q, k, v, want_ws=False)
    ours = oracle.decode16(gather_rows(o, np.arange(p.tokens)), 0)
    e = oracle.errors(ours, oracle.attention_f64(p, q, k, v))
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


def test_qk_norm_params_are_validated(oracle, torch_gpu):
    """mod.rs:701-709: fewer than 4 * head_dim floats is an error; so is a
    parameter tensor that is not contiguous float32."""
    import spl_sage as S

    sa = S.SageAttention(None, 64)
    ws = sa.workspace(S.Shape(1, 1, 128))
    x = torch_gpu.zeros((1, 128, 1, 64), dtype=torch_gpu.bfloat16, device="cuda")
    short = torch_gpu.ones(4 * 64 - 1, dtype=torch_gpu.float32, device="cuda")
    with pytest.raises(S.SageError) as err:
        sa.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x), S.Options(qk_norm=S.QkNorm(short)))
    assert err.value.status == 1 and "QK-norm params" in str(err.value)
    half = torch_gpu.ones(4 * 64, dtype=torch_gpu.float16, device="cuda")
    with pytest.raises(S.SageError):
        sa.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x), S.Options(qk_norm=S.QkNorm(half)))
