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


_CAPTURE_CHILD = r'''
import sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch
import spl_sage as S

torch.cuda.set_device(0)
B, H, N, D = 2, 4, 700, 128
shape = S.Shape(B, H, N)
rng = np.random.default_rng(5)
def rnd():
    return torch.from_numpy(rng.standard_normal((B, N, H, D)).astype(np.float32)).cuda().to(torch.bfloat16)
q, k, v = rnd(), rnd(), rnd()
stream = torch.cuda.Stream()
sa = S.SageAttention(stream, D)  # resolves the no-allocation scratch on this device
out_g = torch.empty_like(q)
out_e = torch.empty_like(q)
ws = sa.workspace(shape)
with torch.cuda.stream(stream):  # the kernels' first launches, outside any capture
    sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out_e))
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=stream):  # this process's first sage_forward_noalloc call
    sa.forward_noalloc(shape, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out_g))
torch.cuda.synchronize()
for rep in range(4):
    q.copy_(rnd()); k.copy_(rnd()); v.copy_(rnd())
    torch.cuda.synchronize()
    out_g.fill_(0)
    graph.replay()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out_e))
    torch.cuda.synchronize()
    a = out_g.view(torch.int16).cpu().numpy()
    b = out_e.view(torch.int16).cpu().numpy()
    if not np.array_equal(a, b):
        print(f"replay {rep}: {int((a != b).sum())} outputs differ from sage_forward", flush=True)
        sys.exit(1)
print("CAPTURE_OK", flush=True)
'''


def test_first_noalloc_call_under_graph_capture(torch_gpu, tmp_path):
    """A fresh process's first sage_forward_noalloc call, captured in a HIP
    graph: the scratch address was resolved by sage_new, so the call only
    launches kernels; every replay (new inputs between them) equals
    sage_forward bit for bit."""
    import subprocess
    import sys

    from conftest import PKG, ROOT

    script = tmp_path / "capture_noalloc.py"
    script.write_text(_CAPTURE_CHILD)
    r = subprocess.run([sys.executable, "-u", str(script), str(ROOT), str(PKG)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
