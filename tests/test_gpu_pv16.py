"""PvAccum::F16 on the GPU, through the C ABI (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/mod.rs:170-185): the prologue of the mode (V scaled to
+-2.25) bit-exact against the oracle and passing the reference's checks for it
(tests.rs:633-648); the attention, which keeps fp32 block partials on gfx950,
gated at cosine >= 0.999 and max-abs <= 2e-2 against the oracle's emulation of
the reference's f16 partials, and by the reference's gate against f64
(tests.rs:655-700, the F16 cases)."""
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

CASES = {
    "d64": (1, 2, 1000, 64, {}),
    "d128": (2, 2, 777, 128, {}),
    "d128_causal_gqa": (1, 4, 600, 128, {"kv_heads": 2, "causal": True}),
    "d64_merge4_ln": (1, 2, SMALL_TOKENS, 64, {"merge": 4, "layout": SMALL_LAYOUT, "ln": "ln"}),
}


@pytest.mark.parametrize("name", list(CASES))
def test_pv16_prologue_and_attention(oracle, torch_gpu, name):
    b, h, t, d, kw = CASES[name]
    kw = dict(kw)
    if kw.get("ln") == "ln":
        kw["ln"] = ln_params(oracle, d, 3)
    p = oracle.Problem(b, h, t, d, pv16=True, **kw)
    q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=2.0, seed=43))
    pro, o = run(torch_gpu, p, q, k, v)
    want = oracle.prologue(p, q, k, v)
    assert_prologue_equal(pro, want)
    dec = lambda x: oracle.decode16(x, p.dtype)
    check_prologue(p, dec(q), dec(k), dec(v), pro)
    assert np.abs(oracle.e4m3_decode(pro["v8"])).max() <= 2.25
    rows = sample_rows(p.tokens, 384, seed=5)
    _check_attention(oracle, p, want, o, rows, q, k, v, name)


@pytest.mark.parametrize("d", [64, 128])
def test_pv16_reference_gate(oracle, torch_gpu, d):
    """tests.rs:655-700 for (d, PvAccum::F16), Dense: batch 2, 3 heads, data seed 5."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, pv16=True)
    q, k, v = oracle.reference_synthetic(p, 5)
    _, o = run(torch_gpu, p, q, k, v, want_ws=False)
    ours = oracle.decode16(gather_rows(o, np.arange(p.tokens)), 0)
    e = oracle.errors(ours, oracle.attention_f64(p, q, k, v))
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e
