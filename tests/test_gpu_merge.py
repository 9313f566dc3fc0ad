"""KV merging (KvMerge::Pool) on the GPU, through the C ABI: the pooled
prologue (codes, scales, statistics and the log-count bias) bit-exact against
the oracle, and the merged attention (the reference's sg_attn_merge,
sezer-muhammed/sota-papers-lab platform/spl-nn/cuda/sage_attn.cu:238-246) gated
at cosine >= 0.999 and max-abs <= 2e-2 against the oracle's emulation of it,
and no further from f64 merged attention than that emulation (the reference's
gpu_prologue_matches_reference / gpu_attention_matches_float_reference cases,
tests.rs:609-700, on its small_layout)."""
from __future__ import annotations

import numpy as np
import pytest

from sage_gpu_helpers import assert_prologue_equal, gather_rows, run, sample_rows
from test_gpu_parity import _check_attention

pytestmark = pytest.mark.gpu

SMALL_LAYOUT = (3, 5, 7, 10, 1)  # tests.rs:596-605: 3 frames, 5 special, 7 x 10 grid, first frame dense
VGGT_LAYOUT = (4, 17, 21, 32, 1)  # VGGT-Omega's 689-token frames (tests.rs:85-93), reference frame dense


def _merged(oracle, stride, layout, heads, d, **kw):
    frames, special, gh, gw, _ = layout
    return oracle.Problem(1, heads, frames * (special + gh * gw), d, merge=stride, layout=layout, **kw)


CASES = {
    "small_s2_d64": (2, SMALL_LAYOUT, 2, 64, {}),
    "small_s4_d128": (4, SMALL_LAYOUT, 2, 128, {}),
    "small_s2_d128_f16": (2, SMALL_LAYOUT, 3, 128, {"dtype": 1}),
    "vggt_s2_d64": (2, VGGT_LAYOUT, 2, 64, {}),
    "vggt_s4_d128_gqa": (4, VGGT_LAYOUT, 4, 128, {"kv_heads": 2}),
    "vggt_s4_d64_nosmooth": (4, VGGT_LAYOUT, 2, 64, {"smooth_k": False, "smooth_v": False}),
}


@pytest.mark.parametrize("name", list(CASES))
def test_merged_prologue_and_attention(oracle, torch_gpu, name):
    stride, layout, heads, d, kw = CASES[name]
    p = _merged(oracle, stride, layout, heads, d, **kw)
    q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=2.0, seed=31))
    pro, o = run(torch_gpu, p, q, k, v)
    want = oracle.prologue(p, q, k, v)
    assert_prologue_equal(pro, want)
    rows = sample_rows(p.tokens, 384, seed=5)
    _check_attention(oracle, p, want, o, rows, q, k, v, name)


@pytest.mark.parametrize("stride", [2, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_merged_reference_gate(oracle, torch_gpu, stride, d):
    """gpu_attention_matches_float_reference (tests.rs:655-700) on the reference's
    clustered data: cos > 0.999 and rel_l2 < 0.04 against f64 merged attention."""
    p = _merged(oracle, stride, SMALL_LAYOUT, 2, d)
    q, k, v = oracle.reference_synthetic(p, 17)
    _, o = run(torch_gpu, p, q, k, v, want_ws=False)
    ours = oracle.decode16(gather_rows(o, np.arange(p.tokens)), 0)
    e = oracle.errors(ours, oracle.attention_f64(p, q, k, v))
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


def test_causal_over_merged_keys_is_refused(oracle, torch_gpu):
    import spl_sage as S

    p = _merged(oracle, 2, SMALL_LAYOUT, 1, 64)
    sa = S.SageAttention(None, 64)
    ws = sa.workspace(S.Shape(1, 1, p.tokens), S.KvMerge.Pool(2, S.FrameLayout(*SMALL_LAYOUT)))
    x = torch_gpu.zeros((1, p.tokens, 1, 64), dtype=torch_gpu.bfloat16, device="cuda")
    with pytest.raises(S.SageError) as err:
        sa.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x), S.Options(causal=True))
    assert err.value.status == 2 and "merged keys" in str(err.value)


@pytest.mark.parametrize("stride", [2, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_merged_attention_equals_dense_on_uniform_cells(oracle, torch_gpu, stride, d):
    """merged_attention_equals_dense_on_uniform_cells (tests.rs:193-232) through
    the GPU path: when every pooled cell holds identical keys and values,
    attention over the pooled keys with the log2-count bias is attention over
    all keys. Both runs quantise, and their 64-key blocks (hence their K scales
    and the running maxima their P grids follow) differ, so the two agree to
    the algorithm's own quantisation error rather than bit for bit: on the
    CPU emulator they differ by cos 0.9998 and max-abs up to 0.33 at outputs of
    3.7, each at cos 0.9994 against f64. Here: cos >= 0.999 and rel_l2 < 0.04
    between them, and each within the reference's gate against f64 dense
    attention (cos > 0.999, rel_l2 < 0.04, tests.rs:699)."""
    lay = (3, 5, 7, 10, 0)
    p = _merged(oracle, stride, lay, 2, d, softmax_scale=0.25)
    dense = oracle.Problem(1, 2, p.tokens, d, softmax_scale=0.25)
    rng = np.random.default_rng(7 + stride)
    cell_k = rng.standard_normal((2, p.tk, d)).astype(np.float32)
    cell_v = rng.standard_normal((2, p.tk, d)).astype(np.float32)
    k = np.zeros((1, p.tokens, 2, d), np.float32)
    v = np.zeros_like(k)
    for j in range(p.tk):
        for t in p.members(j):
            k[0, t] = cell_k[:, j]
            v[0, t] = cell_v[:, j]
    q = (2.0 * rng.standard_normal((1, p.tokens, 2, d))).astype(np.float32)
    q16, k16, v16 = (oracle.encode16(x, 0) for x in (q, k, v))
    _, om = run(torch_gpu, p, q16, k16, v16, want_ws=False)
    _, od = run(torch_gpu, dense, q16, k16, v16, want_ws=False)
    rows = np.arange(p.tokens)
    merged_out = oracle.decode16(gather_rows(om, rows), 0)
    dense_out = oracle.decode16(gather_rows(od, rows), 0)
    e = oracle.errors(merged_out, dense_out)
    assert e["cos"] >= 0.999 and e["rel_l2"] < 0.04, e
    exact = oracle.attention_f64(dense, q16, k16, v16)
    for out in (merged_out, dense_out):
        e64 = oracle.errors(out, exact)
        assert e64["cos"] > 0.999 and e64["rel_l2"] < 0.04, e64
