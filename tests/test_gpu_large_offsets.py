"""Element offsets past 2^31: 4200 heads of N = 4096, D = 128 in one
[B][T][H][D] bf16 tensor, 2.2e9 elements a tensor. The late tokens' input and
output offsets, and the late heads' code, scale and statistics offsets in the
workspace, lie beyond 2^31 elements, so this is the case that a 32-bit index
anywhere on the path (prologue, fold, code pass, attention, epilogue) would
break. Heads 0, 2100 and 4199 (the largest offsets) are checked against the
oracle run on those heads alone: codes, scales and statistics bit for bit
(reference.rs:8-70, sage_quant.cu:59-319), and the output at the north star's
gate against the emulated attention (sage_attn.cu:262-344) on the first, last
and random query rows of every head checked. About 32 GB of device memory.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_device16
from sage_gpu_helpers import assert_prologue_equal, sample_rows, v8_logical

pytestmark = pytest.mark.gpu

B, T, H, D = 1, 4096, 4200, 128
CHECK_HEADS = (0, 2100, 4199)


def test_offsets_past_2_31_elements(torch_gpu, oracle):
    torch = torch_gpu
    import spl_sage as S

    assert B * T * H * D > 2 ** 31 and (T - 1) * H * D > 2 ** 31
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn((B, T, H, D), generator=g, device="cuda", dtype=torch.bfloat16)
    k = torch.randn((B, T, H, D), generator=g, device="cuda", dtype=torch.bfloat16)
    k += (2.0 * torch.randn((H, D), generator=g, device="cuda")).to(torch.bfloat16)
    v = torch.randn((B, T, H, D), generator=g, device="cuda", dtype=torch.bfloat16)
    out = torch.empty_like(q)

    sa = S.SageAttention(None, D)
    ws = sa.workspace(S.Shape(B, H, T))
    plan = ws.plan()
    sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out), S.Options())
    torch.cuda.synchronize()

    def head16(t, h):
        return from_device16(t[:, :, h:h + 1, :].contiguous())  # [B,T,1,D] uint16

    q8 = ws.tensor("q8").view(B, H, plan.tq_pad, D)
    q_scale = ws.tensor("q_scale").view(B, H, plan.tq_pad // 16)
    k8 = ws.tensor("k8").view(B, H, plan.tk_pad, D)
    k_scale = ws.tensor("k_scale").view(B, H, plan.tk_pad // 64)
    v8 = ws.tensor("v8").view(B, H, plan.tk_pad * D)
    stats = ws.tensor("stats").view(B, H, 4, D)
    p = oracle.Problem(B, 1, T, D, dtype=oracle.BF16)
    rows = sample_rows(T, 256, seed=3)
    for h in CHECK_HEADS:
        qh, kh, vh = head16(q, h), head16(k, h), head16(v, h)
        want = oracle.prologue(p, qh, kh, vh)
        got = {
            "q8": q8[:, h:h + 1].cpu().numpy(),
            "q_scale": q_scale[:, h:h + 1].cpu().numpy(),
            "k8": k8[:, h:h + 1].cpu().numpy(),
            "k_scale": k_scale[:, h:h + 1].cpu().numpy(),
            "v8": v8_logical(v8[:, h:h + 1].cpu().numpy(), B, 1, plan.tk_pad, D),
            "stats": stats[:, h:h + 1].cpu().numpy(),
        }
        assert_prologue_equal(got, want)
        ref, _ = oracle.sage_emulate(p, want, rows=rows, out_dtype=oracle.BF16)
        o = oracle.decode16(head16(out, h)[:, rows], oracle.BF16).transpose(0, 2, 1, 3)  # [B,1,R,D]
        e = oracle.errors(o, ref)
        assert e["cos"] >= 0.999 and e["max_abs"] <= 2e-2, (h, e)
