"""spl_sage.qkv -- the QKV prologue behind the reference's API.

Python mirror of `spl_nn::qkv` (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/qkv.rs): RopeLayout, RopeTable, NormKind, QkNorm, Rope,
QkvIn, VFormat, QkvOut and QkvPrologue, with the same argument meanings and
error messages, over the C ABI in include/sage_hip.h. The fused form,
SageAttention.prepare_qkv / forward_qkv, feeds the sage workspace straight
from the projection (no counterpart in the reference). Head dim 64 is the
reference's (HEAD_DIM); 128 is an extension. Device buffers are torch tensors.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import SageError, TensorMut, _abi, _check, _elems_from
from ._abi import lib

HEAD_DIM = 64
PAIRS = HEAD_DIM // 2


class RopeLayout(enum.IntEnum):
    """qkv.rs:33-58: Vggt rotates pairs (i, i + D/4) inside each half of the
    head; Dinov3 pairs (i, i + D/2)."""

    Vggt = 0
    Dinov3 = 1

    def half(self, head_dim: int = HEAD_DIM) -> int:
        return head_dim // 4 if self == RopeLayout.Vggt else head_dim // 2

    def pair(self, d: int, head_dim: int = HEAD_DIM) -> int:
        h = self.half(head_dim)
        return (d // (2 * h)) * h + d % h


@dataclass
class RopeTable:
    """qkv.rs:60-136: cos/sin per (token in frame, pair), float32
    [frame_len][head_dim/2][2] on the host."""

    layout: RopeLayout
    frame_len: int
    cos_sin: np.ndarray

    @staticmethod
    def _build(layout, grid_h, grid_w, special, base, head_dim) -> "RopeTable":
        n = special + grid_h * grid_w
        out = np.empty((n, head_dim // 2, 2), np.float32)
        _check(lib().sage_rope_table(int(layout), head_dim, grid_h, grid_w, special, float(base),
                                     out.ctypes.data, out.size))
        return RopeTable(RopeLayout(layout), n, out)

    @staticmethod
    def vggt(grid_h: int, grid_w: int, special: int, base: float, head_dim: int = HEAD_DIM) -> "RopeTable":
        return RopeTable._build(RopeLayout.Vggt, grid_h, grid_w, special, base, head_dim)

    @staticmethod
    def dinov3(grid_h: int, grid_w: int, special: int, base: float, head_dim: int = HEAD_DIM) -> "RopeTable":
        return RopeTable._build(RopeLayout.Dinov3, grid_h, grid_w, special, base, head_dim)

    @staticmethod
    def from_angles(layout: RopeLayout, frame_len: int, angle, head_dim: int = HEAD_DIM) -> "RopeTable":
        """qkv.rs:67-85: angle(token, pair) in radians, f64 cos/sin rounded to f32."""
        import math

        cs = np.empty((frame_len, head_dim // 2, 2), np.float32)
        for t in range(frame_len):
            for p in range(head_dim // 2):
                a = angle(t, p)
                cs[t, p] = (math.cos(a), math.sin(a))
        return RopeTable(RopeLayout(layout), frame_len, cs)

    def upload(self, device="cuda"):
        import torch

        return torch.from_numpy(np.ascontiguousarray(self.cos_sin).reshape(-1)).to(device)


class NormKind(enum.IntEnum):
    """qkv.rs:138-143."""

    LayerNorm = 1
    Rms = 2


@dataclass
class QkNorm:
    """qkv.rs:145-156: float32 [head_dim] device tensors shared across heads;
    the biases are read by LayerNorm only."""

    kind: NormKind
    q_weight: object
    k_weight: object
    q_bias: object = None
    k_bias: object = None
    eps: float = 1e-6

    def _c(self) -> _abi.sage_qkv_norm:
        ts = [t for t in (self.q_weight, self.q_bias, self.k_weight, self.k_bias) if t is not None]
        n = min(_floats(t) for t in ts)
        ptr = lambda t: None if t is None else _f32_ptr(t)
        return _abi.sage_qkv_norm(int(self.kind), ptr(self.q_weight), ptr(self.q_bias), ptr(self.k_weight),
                                  ptr(self.k_bias), n, float(self.eps))


@dataclass
class Rope:
    """qkv.rs:158-163: an uploaded RopeTable and its layout."""

    table: object
    layout: RopeLayout
    frame_len: int

    def _c(self) -> _abi.sage_qkv_rope:
        return _abi.sage_qkv_rope(_f32_ptr(self.table), _floats(self.table), int(self.layout), self.frame_len)


@dataclass
class QkvIn:
    """qkv.rs:165-177 with a batch dimension: y is a bf16 device tensor of
    token rows `ld` elements apart (q | k | v), batch items `batch_stride`
    apart (0: tokens * ld); tok ([batch * tokens]), chan and bias
    ([(heads + 2 kv_heads) * D], bias bf16) are optional device tensors."""

    y: object
    ld: int
    tok: object = None
    chan: object = None
    bias: object = None
    batch_stride: int = 0

    def _c(self) -> _abi.sage_qkv_in:
        import torch

        if self.y.dtype != torch.bfloat16:
            raise SageError(1, f"qkv y must be bf16, got {self.y.dtype}")
        if self.bias is not None and self.bias.dtype != torch.bfloat16:
            raise SageError(1, f"qkv bias must be bf16, got {self.bias.dtype}")
        opt = lambda t: (None, 0) if t is None else (t.data_ptr(), _elems_from(t))
        tok, chan, bias = opt(self.tok), opt(self.chan), opt(self.bias)
        if self.tok is not None:
            _f32_ptr(self.tok)
        if self.chan is not None:
            _f32_ptr(self.chan)
        return _abi.sage_qkv_in(self.y.data_ptr(), _elems_from(self.y), self.ld, self.batch_stride, tok[0], tok[1],
                                chan[0], chan[1], bias[0], bias[1])


class VFormat(enum.IntEnum):
    """qkv.rs:179-186."""

    Bf16 = 0
    F16 = 1


@dataclass
class QkvOut:
    """qkv.rs:188-196: Q, K and V outputs as TensorMut views (the reference's
    [heads][tokens][64] is Strides.bhtd); V's dtype is its VFormat."""

    q: TensorMut
    k: TensorMut
    v: TensorMut


class QkvPrologue:
    """qkv.rs:226-306 on a SageAttention context's stream and head dim."""

    def __init__(self, sa):
        self._sa = sa

    def run(self, input: QkvIn, tokens: int, heads: int, norm: Optional[QkNorm], rope: Optional[Rope], out: QkvOut,
            batch: int = 1, kv_heads: int = 0) -> None:
        from . import Shape

        shape = Shape(batch, heads, tokens, kv_heads)
        n = None if norm is None else C.byref(norm._c())
        r = None if rope is None else C.byref(rope._c())
        _check(lib().sage_qkv_prologue(self._sa._h, C.byref(shape._c()), C.byref(input._c()), n, r,
                                       C.byref(out.q._c()), C.byref(out.k._c()), C.byref(out.v._c())))


def _floats(t) -> int:
    return _elems_from(t)


def _f32_ptr(t) -> int:
    import torch

    if t.dtype != torch.float32:
        raise SageError(1, f"expected a float32 device tensor, got {t.dtype}")
    return t.data_ptr()


def prepare_qkv(sa, ws, input: QkvIn, norm: Optional[QkNorm] = None, rope: Optional[Rope] = None,
                opts=None) -> None:
    """sage_prepare_qkv: the workspace's codes straight from the projection."""
    from . import Options

    o = (opts or Options())._c()
    n = None if norm is None else C.byref(norm._c())
    r = None if rope is None else C.byref(rope._c())
    _check(lib().sage_prepare_qkv(sa._h, ws._h, C.byref(input._c()), n, r, C.byref(o)))


def forward_qkv(sa, ws, input: QkvIn, out: TensorMut, norm: Optional[QkNorm] = None, rope: Optional[Rope] = None,
                opts=None) -> None:
    """sage_forward_qkv: prepare_qkv, then attend."""
    from . import Options

    o = (opts or Options())._c()
    n = None if norm is None else C.byref(norm._c())
    r = None if rope is None else C.byref(rope._c())
    _check(lib().sage_forward_qkv(sa._h, ws._h, C.byref(input._c()), n, r, C.byref(out._c()), C.byref(o)))
