"""The reference's dense GPU tests (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/tests.rs:597-729), ported to the HIP path on the
reference's own test data (Data::synthetic, tests.rs:300-329), with the
reference's gates. Their KV-merge, QK LayerNorm and FP16 P.V variants are
ported in test_gpu_merge.py, test_gpu_qknorm.py and test_gpu_pv16.py."""
from __future__ import annotations

import numpy as np
import pytest

from prologue_invariants import check_prologue
from sage_gpu_helpers import assert_prologue_equal, gather_rows, run

pytestmark = pytest.mark.gpu

SMALL_TOKENS = 3 * (5 + 7 * 10)  # small_layout(): 3 frames of 5 special + 7x10 patches (tests.rs:586-595)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("smooth", [True, False])
def test_gpu_prologue_matches_reference(oracle, torch_gpu, d, smooth):
    """tests.rs:597-651: the reference's tolerance checks, plus bit-exactness."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, smooth_k=smooth, smooth_v=smooth)
    q, k, v = oracle.reference_synthetic(p, 11)
    pro, _ = run(torch_gpu, p, q, k, v)
    dec = lambda x: oracle.decode16(x, 0)
    check_prologue(p, dec(q), dec(k), dec(v), pro, smooth)
    assert_prologue_equal(pro, oracle.prologue(p, q, k, v))


def test_gpu_attention_has_no_spill(torch_gpu):
    """tests.rs:667-669: the attention kernel must not spill."""
    import spl_sage as S

    for d in (64, 128):
        regs, spill = S.SageAttention(None, d).attn_resources()
        print(f"d {d}: {regs} VGPRs, {spill} scratch bytes")
        assert spill == 0, f"the attention kernel spills at head dim {d}"


# Per kernel: the VGPR limit of the waves a SIMD it is built for (512 VGPRs a
# lane per SIMD, allocated in blocks of 8): 128 for four waves, 168 for three,
# 256 for two (the merged head-dim-128 kernel).
KERNEL_VGPR_LIMITS = {(64, "dense"): 128, (64, "causal"): 128, (64, "merged"): 128,
                      (128, "dense"): 168, (128, "causal"): 168, (128, "merged"): 256}


@pytest.mark.parametrize("d,kernel", sorted(KERNEL_VGPR_LIMITS))
def test_gpu_every_attention_kernel_fits(torch_gpu, d, kernel):
    """Every attention kernel (dense, causal, merged; both head dims) is free of
    spills and keeps the waves a SIMD it is built for."""
    import spl_sage as S

    regs, spill, lds = S.SageAttention(None, d).attn_kernel_resources(kernel)
    print(f"d {d} {kernel}: {regs} VGPRs, {spill} scratch bytes, {lds} LDS bytes")
    assert spill == 0, f"the {kernel} attention kernel spills at head dim {d}"
    assert regs <= KERNEL_VGPR_LIMITS[(d, kernel)], (d, kernel, regs)


def test_gpu_attention_keeps_its_occupancy(torch_gpu):
    """This build's occupancy (no reference counterpart): a SIMD holds 512
    VGPRs a lane, so head dim 128 must stay within 168 (three waves a SIMD) and
    head dim 64 within 128 (four waves). A change that crosses either limit
    loses a wave per SIMD without failing any numerical test."""
    import spl_sage as S

    for d, limit in ((64, 128), (128, 168)):
        regs, _ = S.SageAttention(None, d).attn_resources()
        assert regs <= limit, f"head dim {d}: {regs} VGPRs > {limit}"


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("smooth", [True, False])
def test_gpu_attention_matches_float_reference(oracle, torch_gpu, d, smooth):
    """tests.rs:653-702: cos > 0.999 and rel_l2 < 0.04 against f64 attention."""
    p = oracle.Problem(2, 3, SMALL_TOKENS, d, smooth_k=smooth, smooth_v=smooth)
    q, k, v = oracle.reference_synthetic(p, 5)
    _, o = run(torch_gpu, p, q, k, v, want_ws=False)
    rows = np.arange(p.tokens, dtype=np.int32)
    e = oracle.errors(oracle.decode16(gather_rows(o, rows), 0), oracle.attention_f64(p, q, k, v))
    print(f"d {d} smooth {smooth}: {e}")
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e


def test_gpu_long_sequence_single_head(oracle, torch_gpu):
    """tests.rs:704-729: T = 3001, ragged Q and K tails, many key blocks."""
    p = oracle.Problem(1, 2, 3001, 64)
    q, k, v = oracle.reference_synthetic(p, 21)
    _, o = run(torch_gpu, p, q, k, v, want_ws=False)
    rows = np.arange(p.tokens, dtype=np.int32)
    e = oracle.errors(oracle.decode16(gather_rows(o, rows), 0), oracle.attention_f64(p, q, k, v))
    print(f"T 3001: {e}")
    assert e["cos"] > 0.999 and e["rel_l2"] < 0.04, e
