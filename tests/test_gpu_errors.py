"""Argument errors of the C ABI on a GPU context, through spl_sage: each bad
call is refused before any launch with the reference's text
(sezer-muhammed/sota-papers-lab, platform/spl-nn/src/sage/mod.rs:251-259,
587-589, 681-709, 841-852) and status, and a refused call leaves the
workspace usable. Only valid launches run on the GPU."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture
def ctx(torch_gpu):
    import spl_sage as S

    torch = torch_gpu
    sa = S.SageAttention(None, 64)
    ws = sa.workspace(S.Shape(1, 2, 256))
    x = torch.zeros((1, 256, 2, 64), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(x)
    return S, torch, sa, ws, x, out


def _status(err):
    return err.value.status


def test_head_dim_is_64_or_128(ctx):
    S = ctx[0]
    with pytest.raises(S.SageError, match="sage attention supports head dim 64 or 128, got 96") as e:
        S.SageAttention(None, 96)
    assert _status(e) == 1


def test_workspace_sizes_do_not_wrap(ctx):
    """A plan whose every count fits i32 can still need more than 2^64 bytes of
    codes (here 2^31 - 32768 heads of 2^30 padded queries at head dim 64): the
    workspace is refused before any allocation, not sized by a wrapped product."""
    S = ctx[0]
    sa = ctx[2]
    with pytest.raises(S.SageError, match="sage workspace for .* is too large to address") as e:
        sa.workspace(S.Shape(32768, 65535, 2**30))
    assert _status(e) == 1


def test_attend_before_prepare(ctx):
    S, torch, sa, ws, x, out = ctx
    with pytest.raises(S.SageError, match="sage workspace has not been prepared") as e:
        sa.attend(ws, S.TensorMut(out))
    assert _status(e) == 4


def test_workspace_head_dim_must_match(ctx):
    S, torch, sa, ws, x, out = ctx
    sa128 = S.SageAttention(None, 128)
    with pytest.raises(S.SageError, match="workspace was made for head dim 64, kernels are 128"):
        sa128.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x))


def test_tensor_extent_and_strides(ctx):
    S, torch, sa, ws, x, out = ctx
    # A tensor's extent is counted from its first element to the end of its storage.
    short = torch.zeros(x.numel() - 8, dtype=x.dtype, device="cuda")
    with pytest.raises(S.SageError, match="Q holds 32760 elements, its shape and strides need 32768"):
        sa.prepare(ws, S.Tensor(short, S.Strides.bthd(256, 2, 64)), S.Tensor(x), S.Tensor(x))
    with pytest.raises(S.SageError, match="K strides must be multiples of 8 elements"):
        sa.prepare(ws, S.Tensor(x), S.Tensor(x, S.Strides(256 * 128, 128, 68)), S.Tensor(x))
    big = torch.zeros(x.numel() + 8, dtype=x.dtype, device="cuda")
    with pytest.raises(S.SageError, match="V must start at a 16-byte aligned device address"):
        sa.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(big[1:], S.Strides.bthd(256, 2, 64)))


def test_element_types(ctx):
    S, torch, sa, ws, x, out = ctx
    h = x.to(torch.float16)
    with pytest.raises(S.SageError, match="Q, K and V must share one element type"):
        sa.prepare(ws, S.Tensor(x), S.Tensor(h), S.Tensor(x))
    with pytest.raises(S.SageError, match="sage tensors are bf16 or fp16"):
        sa.prepare(ws, S.Tensor(x.float()), S.Tensor(x), S.Tensor(x))


def test_output_extent(ctx):
    S, torch, sa, ws, x, out = ctx
    sa.prepare(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x))
    small = torch.empty(1000, dtype=out.dtype, device="cuda")
    with pytest.raises(S.SageError, match="output holds 1000 elements, its shape and strides need 32768"):
        sa.attend(ws, S.TensorMut(small, S.Strides.bthd(256, 2, 64)))


def test_refused_call_leaves_workspace_usable(ctx):
    """After refused calls, a valid prepare + attend still runs: zero inputs give
    zero outputs (uniform weights over zero values)."""
    S, torch, sa, ws, x, out = ctx
    with pytest.raises(S.SageError):
        sa.prepare(ws, S.Tensor(x), S.Tensor(x.to(torch.float16)), S.Tensor(x))
    out.fill_(1.0)
    sa.forward(ws, S.Tensor(x), S.Tensor(x), S.Tensor(x), S.TensorMut(out))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
