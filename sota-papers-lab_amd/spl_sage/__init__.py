"""spl_sage -- the gfx950 SageAttention2 forward path behind the reference's API.

Python mirror of `spl_nn::sage` (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/mod.rs): the same types (Tile, Config, PvAccum,
Strides, Shape, FrameLayout, KvMerge, Options, Plan, Workspace, Tensor,
TensorMut, SageAttention), the same argument meanings and the same error
messages, over the C ABI in include/sage_hip.h (libsage_hip.so). Every call
goes to the HIP library; there is no CPU fallback. Device buffers are torch
tensors (PyTorch supplies HBM allocations and the stream).
"""
from __future__ import annotations

import ctypes as C
import enum
import math
from dataclasses import dataclass, field
from typing import Optional

from . import _abi
from ._abi import lib

QGROUP = 16
QTILE = 128
KBLOCK = 64
FP8_MAX = 448.0
PV16_V_RANGE = 2.25

BF16 = 0
F16 = 1


class SageError(RuntimeError):
    """An `Err` of the reference API; `status` is the C ABI's sage_status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _check(status: int) -> None:
    if status != 0:
        raise SageError(status, lib().sage_last_error().decode())


# ------------------------------------------------------------------ config


@dataclass(frozen=True)
class Tile:
    """mod.rs:116-168: the reference's CTA shape (warps, 16-row m-tiles,
    K/V ring stages), validated as the reference validates it. It picks the
    workgroup layout, never the results: warps = 8 (dense and causal
    attention) runs eight waves a workgroup (score waves and output waves),
    every other tile four waves that each do a whole block."""

    warps: int
    m_tiles: int
    stages: int

    def rows(self) -> int:
        return 16 * self.m_tiles * self.warps

    def validate(self) -> None:
        _check(lib().sage_tile_validate(C.byref(self._c())))

    def _c(self) -> _abi.sage_tile:
        return _abi.sage_tile(self.warps, self.m_tiles, self.stages)

    @staticmethod
    def for_head_dim(head_dim: int) -> "Tile":
        return Config.for_head_dim(head_dim).tile


NOALLOC_MAX_BYTES = 128 << 20  # SAGE_NOALLOC_MAX_BYTES

Tile.DEFAULT = Tile(4, 2, 3)  # mod.rs:128-132
Tile.D128 = Tile(4, 1, 3)  # mod.rs:136-140


class PvAccum(enum.IntEnum):
    """mod.rs:170-181."""

    F32 = 0
    F16 = 1


@dataclass(frozen=True)
class Config:
    """mod.rs:187-201."""

    tile: Tile
    pv_accum: PvAccum = PvAccum.F32

    @staticmethod
    def for_head_dim(head_dim: int) -> "Config":
        c = lib().sage_config_for_head_dim(head_dim)
        return Config(Tile(c.tile.warps, c.tile.m_tiles, c.tile.stages), PvAccum(c.pv_accum))

    def _c(self) -> _abi.sage_config:
        return _abi.sage_config(self.tile._c(), int(self.pv_accum))


# ------------------------------------------------------------------ shapes


@dataclass(frozen=True)
class Strides:
    """Element strides of a [batch][token][head][dim] tensor (mod.rs:203-260)."""

    batch: int
    token: int
    head: int

    @staticmethod
    def bthd(tokens: int, heads: int, head_dim: int) -> "Strides":
        return Strides(tokens * heads * head_dim, heads * head_dim, head_dim)

    @staticmethod
    def bhtd(tokens: int, heads: int, head_dim: int) -> "Strides":
        return Strides(heads * tokens * head_dim, head_dim, tokens * head_dim)

    @staticmethod
    def packed_qkv(tokens: int, heads: int, head_dim: int) -> "Strides":
        return Strides(tokens * 3 * heads * head_dim, 3 * heads * head_dim, head_dim)

    def _c(self) -> _abi.sage_strides:
        return _abi.sage_strides(self.batch, self.token, self.head)

    def extent(self, shape: "Shape", head_dim: int, heads: Optional[int] = None) -> int:
        h = shape.heads if heads is None else heads
        return lib().sage_strides_extent(C.byref(self._c()), shape.batch, shape.tokens, h, head_dim)

    def check(self, what: str) -> None:
        _check(lib().sage_strides_check(C.byref(self._c()), what.encode()))


@dataclass(frozen=True)
class Shape:
    """mod.rs:262-268; kv_heads (0 = heads) is the grouped-query extension."""

    batch: int
    heads: int
    tokens: int
    kv_heads: int = 0

    def _c(self) -> _abi.sage_shape:
        return _abi.sage_shape(self.batch, self.heads, self.tokens, self.kv_heads)


@dataclass(frozen=True)
class FrameLayout:
    """mod.rs:270-300."""

    frames: int
    special: int
    grid_h: int
    grid_w: int
    dense_frames: int = 0

    def tokens_per_frame(self) -> int:
        return self.special + self.grid_h * self.grid_w

    def merged_per_frame(self, stride: int) -> int:
        return self.special + -(-self.grid_h // stride) * -(-self.grid_w // stride)

    def merged_keys(self, stride: int) -> int:
        d = min(self.dense_frames, self.frames)
        return d * self.tokens_per_frame() + (self.frames - d) * self.merged_per_frame(stride)

    def _c(self) -> _abi.sage_frame_layout:
        return _abi.sage_frame_layout(self.frames, self.special, self.grid_h, self.grid_w, self.dense_frames)


@dataclass(frozen=True)
class KvMerge:
    """mod.rs:302-311: `KvMerge.Dense` or `KvMerge.Pool(stride, layout)`."""

    stride: int = 1
    layout: Optional[FrameLayout] = None

    @staticmethod
    def Pool(stride: int, layout: FrameLayout) -> "KvMerge":
        return KvMerge(stride, layout)

    def is_dense(self) -> bool:
        return self.stride == 1

    def _c(self) -> _abi.sage_kv_merge:
        lay = self.layout._c() if self.layout is not None else _abi.sage_frame_layout()
        return _abi.sage_kv_merge(self.stride, lay)


KvMerge.Dense = KvMerge(1, None)


@dataclass
class QkNorm:
    """mod.rs:337-344: the per-head LayerNorm of Q and K fused into the
    prologue. `params` is a contiguous float32 device tensor holding
    [q weight, q bias, k weight, k bias], head_dim floats each."""

    params: object  # torch tensor of 4 * head_dim floats
    eps: float = 1e-5

    def _ptr(self) -> int:
        import torch

        p = self.params
        if p.dtype != torch.float32 or not p.is_contiguous():
            raise SageError(1, f"QK-norm params must be contiguous float32, got {p.dtype}")
        return p.data_ptr()


@dataclass
class Options:
    """mod.rs:313-335; `causal` is an extension."""

    softmax_scale: Optional[float] = None
    smooth_k: bool = True
    smooth_v: bool = True
    qk_norm: Optional[QkNorm] = None
    causal: bool = False

    def _c(self) -> _abi.sage_options:
        o = _abi.sage_options()
        o.softmax_scale = 0.0 if self.softmax_scale is None else float(self.softmax_scale)
        o.has_softmax_scale = 0 if self.softmax_scale is None else 1
        o.smooth_k = int(self.smooth_k)
        o.smooth_v = int(self.smooth_v)
        if self.qk_norm is not None:
            p = self.qk_norm.params
            o.qk_norm_params = self.qk_norm._ptr()
            o.qk_norm_len = p.numel()
            o.qk_norm_eps = self.qk_norm.eps
        o.causal = int(self.causal)
        return o


@dataclass(frozen=True)
class Plan:
    """mod.rs:391-454: sizes that follow from a Shape and a KvMerge."""

    shape: Shape
    merge: KvMerge
    tq_pad: int
    tk: int
    tk_pad: int

    @staticmethod
    def new(shape: Shape, merge: KvMerge = KvMerge.Dense) -> "Plan":
        out = _abi.sage_plan()
        _check(lib().sage_plan_new(C.byref(shape._c()), C.byref(merge._c()), C.byref(out)))
        return Plan._from_c(out, shape, merge)

    @staticmethod
    def _from_c(p: _abi.sage_plan, shape: Shape, merge: KvMerge) -> "Plan":
        return Plan(shape, merge, p.tq_pad, p.tk, p.tk_pad)

    def _c(self) -> _abi.sage_plan:
        p = _abi.sage_plan()
        lib().sage_plan_new(C.byref(self.shape._c()), C.byref(self.merge._c()), C.byref(p))
        return p

    def key_ratio(self) -> float:
        return self.tk / self.shape.tokens

    def q_tiles(self) -> int:
        return self.tq_pad // QTILE

    def kblocks(self) -> int:
        return self.tk_pad // KBLOCK

    def kv_heads(self) -> int:
        return self.shape.kv_heads or self.shape.heads


def flops(plan: Plan, head_dim: int, causal: bool = False) -> float:
    """mod.rs:903-910 (causal counts the pairs j <= i)."""
    return lib().sage_flops(C.byref(plan._c()), head_dim, int(causal))


def check_device(ordinal: int = 0) -> None:
    """mod.rs:552-566, for gfx950."""
    _check(lib().sage_check_device(ordinal))


def v8_position(k: int) -> int:
    """Byte of key k (0..63) within each channel row of a v8 block."""
    return lib().sage_v8_position(k)


# ------------------------------------------------------------------ tensors


def _dtype_code(t) -> int:
    import torch

    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float16:
        return F16
    raise SageError(1, f"sage tensors are bf16 or fp16, got {t.dtype}")


def _elems_from(t) -> int:
    """Elements from the view's first element to the end of its storage."""
    es = t.element_size()
    return t.untyped_storage().nbytes() // es - t.storage_offset()


@dataclass
class Tensor:
    """A 16-bit input: a device tensor (any view) plus its Strides (mod.rs:497-501)."""

    data: object
    strides: Optional[Strides] = None

    def _c(self) -> _abi.sage_tensor:
        t = self.data
        st = self.strides or Strides(t.stride(0), t.stride(1), t.stride(2))
        return _abi.sage_tensor(t.data_ptr(), _elems_from(t), st._c(), _dtype_code(t))


@dataclass
class TensorMut:
    """The 16-bit output (mod.rs:503-507)."""

    data: object
    strides: Optional[Strides] = None

    def _c(self) -> _abi.sage_tensor_mut:
        t = self.data
        st = self.strides or Strides(t.stride(0), t.stride(1), t.stride(2))
        return _abi.sage_tensor_mut(t.data_ptr(), _elems_from(t), st._c(), _dtype_code(t))


# ------------------------------------------------------------------ engine


class Workspace:
    """Device buffers of one Plan (mod.rs:456-495), owned by the library."""

    _names = {
        "q8": ("int8", "q8_len"),
        "q_scale": ("float32", "q_scale_len"),
        "k8": ("int8", "k8_len"),
        "k_scale": ("float32", "k_scale_len"),
        "v8": ("uint8", "v8_len"),
        "stats": ("float32", "stats_len"),
        "kbias": ("float32", "kbias_len"),
    }

    def __init__(self, handle: int, plan: Plan, head_dim: int):
        self._h = handle
        self._plan = plan
        self.head_dim = head_dim
        # Bound now: at interpreter exit the module's globals may be gone before __del__ runs.
        self._destroy = lib().sage_workspace_destroy

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        destroy = getattr(self, "_destroy", None)
        if h and destroy is not None:
            destroy(h)

    def plan(self) -> Plan:
        return self._plan

    def bytes(self) -> int:
        return lib().sage_workspace_bytes(self._h)

    def buffers(self) -> _abi.sage_ws_buffers:
        b = _abi.sage_ws_buffers()
        _check(lib().sage_workspace_buffers(self._h, C.byref(b)))
        return b

    def tensor(self, name: str):
        """A device copy (torch tensor) of one buffer: q8, q_scale, k8, k_scale,
        v8, stats or kbias, in the layouts include/sage_hip.h documents. The copy
        is ordered on torch's current stream."""
        import torch

        dt, ln = self._names[name]
        b = self.buffers()
        return _device_copy(getattr(b, name), getattr(b, ln), getattr(torch, dt))

    def __getattr__(self, name):
        if name in Workspace._names:
            return self.tensor(name)
        raise AttributeError(name)


_hip = None


def _device_copy(ptr: int, n: int, dtype):
    """torch tensor holding a copy of n elements of device memory at ptr."""
    import torch

    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpyAsync.restype = C.c_int
        _hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    t = torch.empty(n, dtype=dtype, device="cuda")
    if n:
        err = _hip.hipMemcpyAsync(t.data_ptr(), ptr, n * t.element_size(), 3,  # hipMemcpyDeviceToDevice
                                  torch.cuda.current_stream().cuda_stream)
        if err != 0:
            raise SageError(3, f"copy workspace buffer: hip error {err}")
    return t


def _stream_handle(stream) -> int:
    if stream is None:
        return 0
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


class SageAttention:
    """Kernels for one head dim and Config on one stream (mod.rs:509-901).
    Every call enqueues work and returns without synchronising."""

    def __init__(self, stream, head_dim: int, config: Optional[Config] = None):
        h = C.c_void_p()
        cfg = C.byref(config._c()) if config is not None else None
        _check(lib().sage_new(_stream_handle(stream), head_dim, cfg, C.byref(h)))
        self._h = h.value
        self._stream = stream
        self._destroy = lib().sage_destroy

    @classmethod
    def new(cls, stream, head_dim: int) -> "SageAttention":
        return cls(stream, head_dim)

    @classmethod
    def with_config(cls, stream, head_dim: int, config: Config) -> "SageAttention":
        return cls(stream, head_dim, config)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        destroy = getattr(self, "_destroy", None)
        if h and destroy is not None:
            destroy(h)

    def head_dim(self) -> int:
        return lib().sage_head_dim(self._h)

    def config(self) -> Config:
        c = lib().sage_get_config(self._h)
        return Config(Tile(c.tile.warps, c.tile.m_tiles, c.tile.stages), PvAccum(c.pv_accum))

    def stream(self):
        return self._stream

    def attn_resources(self) -> tuple:
        """(VGPRs per lane, scratch bytes per lane) of the attention kernel."""
        r, s, l = C.c_int32(), C.c_int32(), C.c_int32()
        _check(lib().sage_attn_resources(self._h, C.byref(r), C.byref(s), C.byref(l)))
        return r.value, s.value

    KERNELS = {"dense": 0, "causal": 1, "merged": 2}

    def attn_kernel_resources(self, kernel: str) -> tuple:
        """(VGPRs per lane, scratch bytes per lane, static LDS bytes) of the
        dense, causal or merged attention kernel (an extension)."""
        r, s, l = C.c_int32(), C.c_int32(), C.c_int32()
        _check(lib().sage_attn_kernel_resources(self._h, self.KERNELS[kernel], C.byref(r), C.byref(s),
                                                C.byref(l)))
        return r.value, s.value, l.value

    def workspace(self, shape: Shape, merge: KvMerge = KvMerge.Dense) -> Workspace:
        h = C.c_void_p()
        _check(lib().sage_workspace_new(self._h, C.byref(shape._c()), C.byref(merge._c()), C.byref(h)))
        p = _abi.sage_plan()
        _check(lib().sage_workspace_plan(h.value, C.byref(p)))
        return Workspace(h.value, Plan._from_c(p, shape, merge), self.head_dim())

    def prepare(self, ws: Workspace, q: Tensor, k: Tensor, v: Tensor, opts: Optional[Options] = None) -> None:
        o = (opts or Options())._c()
        _check(lib().sage_prepare(self._h, ws._h, C.byref(q._c()), C.byref(k._c()), C.byref(v._c()), C.byref(o)))

    def attend(self, ws: Workspace, out: TensorMut) -> None:
        _check(lib().sage_attend(self._h, ws._h, C.byref(out._c())))

    def forward(self, ws: Workspace, q: Tensor, k: Tensor, v: Tensor, out: TensorMut,
                opts: Optional[Options] = None) -> None:
        self.prepare(ws, q, k, v, opts)
        self.attend(ws, out)

    def prepare_qkv(self, ws: Workspace, input, norm=None, rope=None, opts: Optional[Options] = None) -> None:
        """prepare fed straight from the fused QKV projection (spl_sage.qkv)."""
        from . import qkv

        qkv.prepare_qkv(self, ws, input, norm, rope, opts)

    def forward_qkv(self, ws: Workspace, input, out: TensorMut, norm=None, rope=None,
                    opts: Optional[Options] = None) -> None:
        from . import qkv

        qkv.forward_qkv(self, ws, input, out, norm, rope, opts)

    def forward_noalloc(self, shape: Shape, q: Tensor, k: Tensor, v: Tensor, out: TensorMut,
                        opts: Optional[Options] = None, merge: KvMerge = KvMerge.Dense) -> None:
        """forward without a workspace (sage_forward_noalloc): the buffers come
        from the library's fixed per-GPU scratch array (NOALLOC_MAX_BYTES); no
        device memory is allocated. Calls that can overlap on one GPU race."""
        o = (opts or Options())._c()
        _check(lib().sage_forward_noalloc(self._h, C.byref(shape._c()), C.byref(merge._c()), C.byref(q._c()),
                                          C.byref(k._c()), C.byref(v._c()), C.byref(out._c()), C.byref(o)))

    def peak(self, which: int, iters: int = 2048) -> float:
        """Measured dense TOPS of one MFMA shape (0 INT8, 1 FP8, 2 BF16)."""
        t = C.c_double()
        _check(lib().sage_peak(self._h, which, iters, C.byref(t)))
        return t.value


__all__ = [
    "QGROUP", "QTILE", "KBLOCK", "FP8_MAX", "PV16_V_RANGE", "BF16", "F16", "SageError", "Tile", "PvAccum",
    "Config", "Strides", "Shape", "FrameLayout", "KvMerge", "QkNorm", "Options", "Plan", "flops",
    "check_device", "v8_position", "Tensor", "TensorMut", "Workspace", "SageAttention",
]
