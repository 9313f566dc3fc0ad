"""sage_forward_noalloc (no counterpart in the reference; for callers that
cannot allocate device memory): called through the C ABI, its output must
equal sage_forward's (the existing entry point, with its own workspace) bit
for bit, on consecutive calls that share the library's scratch array, the
second one smaller; a shape whose buffers exceed the array is refused before
any launch."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_device16, to_device16

pytestmark = pytest.mark.gpu


def _tensors(torch, oracle, p, seed):
    q, k, v = oracle.generate(p, oracle.GenSpec(k_off_std=2.0, seed=seed))
    return tuple(to_device16(torch, x, p.dtype) for x in (q, k, v))


def _both(torch, S, sa, p, qkv, merge=None):
    """(noalloc output, forward output) as uint16 arrays."""
    km = merge if merge is not None else S.KvMerge.Dense
    shape = S.Shape(p.batch, p.heads, p.tokens, p.kv_heads)
    q, k, v = qkv
    tdt = torch.bfloat16 if p.dtype == 0 else torch.float16
    o_na = torch.full((p.batch, p.tokens, p.heads, p.head_dim), float("nan"), dtype=tdt, device="cuda")
    o_ws = torch.empty_like(o_na)
    opts = S.Options(causal=p.causal)
    sa.forward_noalloc(shape, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(o_na), opts, km)
    ws = sa.workspace(shape, km)
    sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(o_ws), opts)
    torch.cuda.synchronize()
    return from_device16(o_na), from_device16(o_ws)


@pytest.mark.parametrize("d", [64, 128])
def test_noalloc_equals_forward_on_consecutive_calls(oracle, torch_gpu, d):
    import spl_sage as S

    torch = torch_gpu
    sa = S.SageAttention(None, d)
    big = oracle.Problem(2, 8, 1500, d, kv_heads=4, causal=True)
    small = oracle.Problem(1, 3, 200, d, dtype=1)
    for p, seed in ((big, 1), (small, 2)):
        print(f"d {d}: B{p.batch} H{p.heads}/{p.hk} N{p.tokens} causal {p.causal} dtype {p.dtype}", flush=True)
        got, want = _both(torch, S, sa, p, _tensors(torch, oracle, p, seed))
        assert np.array_equal(got, want), (d, p)


def test_noalloc_merged_plan(oracle, torch_gpu):
    import spl_sage as S

    torch = torch_gpu
    layout = (3, 5, 7, 10, 1)
    p = oracle.Problem(1, 4, 3 * 75, 64, merge=4, layout=layout)
    sa = S.SageAttention(None, 64)
    got, want = _both(torch, S, sa, p, _tensors(torch, oracle, p, 3), S.KvMerge.Pool(4, S.FrameLayout(*layout)))
    assert np.array_equal(got, want)


def test_noalloc_refuses_shapes_beyond_its_scratch(torch_gpu):
    """C3's shape (B1 H32 N16384 D128) needs ~205 MB, more than the 128 MiB
    array: refused with SAGE_ERR_INVALID and a message naming the limit, and
    the output is left untouched."""
    import spl_sage as S

    torch = torch_gpu
    sa = S.SageAttention(None, 128)
    n = 16384
    x = torch.zeros((1, n, 32, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.full_like(x, 7.0)
    with pytest.raises(S.SageError, match="maximum of 134217728"):
        sa.forward_noalloc(S.Shape(1, 32, n), S.Tensor(x), S.Tensor(x), S.Tensor(x), S.TensorMut(out))
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
