"""prepare and attend inside a HIP graph: the path allocates nothing and never
synchronises, so a caller can capture it (the reference's engine captures
the VGGT trunk, sezer-muhammed/sota-papers-lab apps/image-to-3d/src/vggt/
graph.rs, sched.rs:120-121). A captured forward is replayed several times,
with eager work and synchronisations between the replays and new inputs
copied into the captured buffers, and every replay must equal an eager
forward on the same inputs bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_device16, to_device16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,merge", [(128, 1), (64, 4)])
def test_captured_forward_replays_like_eager(oracle, torch_gpu, d, merge):
    import spl_sage as S

    torch = torch_gpu
    layout = (3, 5, 7, 10, 1)
    tokens = 3 * 75 if merge > 1 else 700
    p = oracle.Problem(2, 4, tokens, d, kv_heads=2 if merge == 1 else 0, merge=merge, layout=layout)
    stream = torch.cuda.Stream()
    sa = S.SageAttention(stream, d)
    km = S.KvMerge.Pool(merge, S.FrameLayout(*layout)) if merge > 1 else S.KvMerge.Dense
    ws_graph = sa.workspace(S.Shape(p.batch, p.heads, p.tokens, p.kv_heads), km)
    ws_eager = sa.workspace(S.Shape(p.batch, p.heads, p.tokens, p.kv_heads), km)
    inputs = [oracle.generate(p, oracle.GenSpec(seed=70 + i)) for i in range(3)]
    q, k, v = (to_device16(torch, x, p.dtype) for x in inputs[0])
    out = torch.empty((p.batch, p.tokens, p.heads, d), dtype=torch.bfloat16, device="cuda")
    out_eager = torch.empty_like(out)
    torch.cuda.synchronize()

    def fwd(ws, o):
        sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(o))

    with torch.cuda.stream(stream):
        fwd(ws_graph, out)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fwd(ws_graph, out)
    torch.cuda.synchronize()

    for rep in range(6):
        qi, ki, vi = inputs[rep % 3]
        q.copy_(to_device16(torch, qi, p.dtype))
        k.copy_(to_device16(torch, ki, p.dtype))
        v.copy_(to_device16(torch, vi, p.dtype))
        torch.cuda.synchronize()
        out.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            fwd(ws_eager, out_eager)  # eager work between the replays
        torch.cuda.synchronize()
        got, want = from_device16(out), from_device16(out_eager)
        assert np.array_equal(got, want), f"replay {rep} differs from eager"
        # And the eager forward itself is the oracle's prologue + gated attention.
        if rep < 3:
            pro = oracle.prologue(p, qi, ki, vi)
            rows = np.arange(0, p.tokens, 7, dtype=np.int32)
            _, emu16 = oracle.sage_emulate(p, pro, rows=rows, out_dtype=p.dtype)
            ours = oracle.decode16(np.ascontiguousarray(want[:, rows].transpose(0, 2, 1, 3)), p.dtype)
            e = oracle.errors(ours, oracle.decode16(emu16, p.dtype))
            assert e["cos"] >= 0.999 and e["max_abs"] <= 2e-2, e
