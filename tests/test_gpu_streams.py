"""Two SageAttention contexts on two streams at once (the reference's engine is
Send + Sync and enqueues on its own stream without synchronising, mod.rs:509-510,
tests.rs:17-22): every launch goes to the context's stream and no state is
shared, so forwards interleaved on two streams, with no synchronisation between
them, equal the same forwards run one after the other, bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_device16, to_device16

pytestmark = pytest.mark.gpu


def test_two_streams_interleaved_equal_sequential(oracle, torch_gpu):
    import spl_sage as S

    torch = torch_gpu
    P, G = oracle.Problem, oracle.GenSpec
    problems = [(P(1, 4, 1500, 128, causal=True), G(k_off_std=2.0, seed=31)),
                (P(2, 3, 777, 64, dtype=1), G(k_off_std=3.0, seed=32))]
    inputs = []
    for p, g in problems:
        q, k, v = oracle.generate(p, g)
        dev = [to_device16(torch, a, p.dtype) for a in (q, k, v)]
        inputs.append((p, dev))
    torch.cuda.synchronize()

    def forward(stream, p, dev, reps):
        sa = S.SageAttention(stream, p.head_dim)
        ws = sa.workspace(S.Shape(p.batch, p.heads, p.tokens))
        out = torch.empty((p.batch, p.tokens, p.heads, p.head_dim),
                          dtype=torch.float16 if p.dtype else torch.bfloat16, device="cuda")
        for _ in range(reps):
            sa.forward(ws, *(S.Tensor(x) for x in dev), S.TensorMut(out), S.Options(causal=p.causal))
        return sa, ws, out

    # one after the other on the default stream
    want = []
    for p, dev in inputs:
        _, _, out = forward(None, p, dev, 1)
        torch.cuda.synchronize()
        want.append(from_device16(out))

    # interleaved on two side streams (default priority), repeated so that they overlap
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    keep = []
    for rep in range(3):
        for (p, dev), st in zip(inputs, streams):
            keep.append(forward(st, p, dev, 4))
    torch.cuda.synchronize()
    for i, (_, _, out) in enumerate(keep):
        got = from_device16(out)
        assert np.array_equal(got, want[i % 2]), (i, int((got != want[i % 2]).sum()))
