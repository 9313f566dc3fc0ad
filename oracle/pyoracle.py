"""numpy front end of the C oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
as the checker. The product (spl_sage / libsage_hip.so) never imports it.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import subprocess
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

BF16, F16 = 0, 1
QGROUP, QTILE, KBLOCK = 16, 128, 64
LOG2E_F32 = np.float32(1.4426950408889634)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


class _Problem(C.Structure):
    _fields_ = [
        ("batch", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("tokens", C.c_int), ("head_dim", C.c_int),
        ("dtype", C.c_int),
        ("q_sb", C.c_longlong), ("q_st", C.c_longlong), ("q_sh", C.c_longlong),
        ("k_sb", C.c_longlong), ("k_st", C.c_longlong), ("k_sh", C.c_longlong),
        ("v_sb", C.c_longlong), ("v_st", C.c_longlong), ("v_sh", C.c_longlong),
        ("q_mul", C.c_float), ("smooth_k", C.c_int), ("smooth_v", C.c_int), ("v_range", C.c_float),
        ("merge", C.c_int), ("frames", C.c_int), ("special", C.c_int), ("grid_h", C.c_int), ("grid_w", C.c_int),
        ("dense_frames", C.c_int), ("ln", C.c_void_p), ("ln_eps", C.c_float), ("pv16", C.c_int),
    ]


class _GenSpec(C.Structure):
    _fields_ = [
        ("batch", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("tokens", C.c_int), ("head_dim", C.c_int),
        ("dtype", C.c_int), ("k_off_std", C.c_float), ("outlier_channels", C.c_int), ("outlier_scale", C.c_float),
        ("token_frac", C.c_float), ("token_scale", C.c_float), ("seed", C.c_uint64),
    ]


class _Numerics(C.Structure):
    _fields_ = [("l_from_p8", C.c_int), ("pow2_max", C.c_int), ("tau", C.c_float), ("exp_f16", C.c_int)]


@dataclass(frozen=True)
class Numerics:
    """Alternative softmax numerics (all defaults = the reference's): l from
    the E4M3-rounded P; the running max rounded up to an integer in log2
    units (power-of-two rescales); headroom tau before the max moves; p
    rounded to f16."""

    l_from_p8: bool = False
    pow2_max: bool = False
    tau: float = 0.0
    exp_f16: bool = False

    def _c(self) -> _Numerics:
        return _Numerics(int(self.l_from_p8), int(self.pow2_max), float(self.tau), int(self.exp_f16))


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        l = C.CDLL(os.fspath(LIB))
        vp = C.c_void_p
        l.oracle_bf16_to_f32.restype = C.c_float
        l.oracle_bf16_to_f32.argtypes = [C.c_uint16]
        l.oracle_f32_to_bf16.restype = C.c_uint16
        l.oracle_f32_to_bf16.argtypes = [C.c_float]
        l.oracle_f16_to_f32.restype = C.c_float
        l.oracle_f16_to_f32.argtypes = [C.c_uint16]
        l.oracle_f32_to_f16.restype = C.c_uint16
        l.oracle_f32_to_f16.argtypes = [C.c_float]
        l.oracle_e4m3_to_f32.restype = C.c_float
        l.oracle_e4m3_to_f32.argtypes = [C.c_uint8]
        l.oracle_f32_to_e4m3.restype = C.c_uint8
        l.oracle_f32_to_e4m3.argtypes = [C.c_float]
        l.oracle_s8.restype = C.c_int
        l.oracle_s8.argtypes = [C.c_float]
        l.oracle_vpos_ref.restype = C.c_int
        l.oracle_vpos_ref.argtypes = [C.c_int]
        for n in ("oracle_decode16", "oracle_encode16"):
            getattr(l, n).argtypes = [vp, vp, C.c_size_t, C.c_int]
        l.oracle_e4m3_encode.argtypes = [vp, vp, C.c_size_t]
        l.oracle_e4m3_decode.argtypes = [vp, vp, C.c_size_t]
        l.oracle_rng_next.restype = C.c_uint64
        l.oracle_rng_next.argtypes = [C.POINTER(C.c_uint64)]
        l.oracle_rng_uniform.restype = C.c_double
        l.oracle_rng_uniform.argtypes = [C.POINTER(C.c_uint64)]
        l.oracle_rng_normal.restype = C.c_float
        l.oracle_rng_normal.argtypes = [C.POINTER(C.c_uint64)]
        l.oracle_generate.argtypes = [C.POINTER(_GenSpec), vp, vp, vp]
        l.oracle_reference_synthetic.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64, vp, vp, vp]
        l.oracle_prologue.restype = C.c_int
        l.oracle_prologue.argtypes = [C.POINTER(_Problem), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int]
        l.oracle_merged_keys.restype = C.c_int
        l.oracle_merged_keys.argtypes = [C.POINTER(_Problem)]
        l.oracle_members.restype = C.c_int
        l.oracle_members.argtypes = [C.POINTER(_Problem), C.c_int, vp]
        l.oracle_log2_count.restype = C.c_float
        l.oracle_round_f16.restype = C.c_double
        l.oracle_round_f16.argtypes = [C.c_double]
        l.oracle_layernorm.argtypes = [vp, vp, C.c_int, vp, vp, C.c_float]
        l.oracle_layernorm_f64.argtypes = [vp, vp, C.c_int, vp, vp, C.c_float]
        l.oracle_log2_count.argtypes = [C.c_int]
        l.oracle_attention_f64.argtypes = [C.POINTER(_Problem), C.c_int, C.c_float, vp, vp, vp, vp, C.c_int, vp, C.c_int]
        l.oracle_sage_emulate.argtypes = [C.POINTER(_Problem), C.c_int, vp, vp, vp, vp, vp, vp, vp, vp, C.c_int, vp,
                                          vp, C.c_int, C.c_int, C.c_int]
        l.oracle_sage_emulate_numerics.argtypes = [C.POINTER(_Problem), C.c_int, vp, vp, vp, vp, vp, vp, vp, vp,
                                                   C.c_int, C.c_int, vp, vp, C.c_int, C.c_int,
                                                   C.POINTER(_Numerics), C.c_int]
        l.oracle_attention_f64_rows.argtypes = [C.POINTER(_Problem), C.c_int, C.c_float, vp, vp, vp, vp, C.c_int,
                                                C.c_int, vp, C.c_int]
        l.oracle_errors.argtypes = [vp, vp, C.c_size_t, vp]
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------------ codecs

def decode16(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().oracle_decode16(_p(x), _p(out), x.size, dtype)
    return out


def encode16(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_encode16(_p(x), _p(out), x.size, dtype)
    return out


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().oracle_e4m3_encode(_p(x), _p(out), x.size)
    return out


def e4m3_decode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint8)
    out = np.empty(x.shape, np.float32)
    lib().oracle_e4m3_decode(_p(x), _p(out), x.size)
    return out


class Rng:
    """splitmix64 (reference.rs:227-254)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def next_u64(self) -> int:
        return lib().oracle_rng_next(C.byref(self.state))

    def uniform(self) -> float:
        return lib().oracle_rng_uniform(C.byref(self.state))

    def normal(self) -> float:
        return lib().oracle_rng_normal(C.byref(self.state))


# ------------------------------------------------------------------ problems

@dataclass
class Problem:
    """One attention problem, inputs in [b][t][h][d] layout (bthd) unless strides given."""

    batch: int
    heads: int
    tokens: int
    head_dim: int
    kv_heads: int = 0
    dtype: int = BF16
    causal: bool = False
    smooth_k: bool = True
    smooth_v: bool = True
    softmax_scale: float | None = None
    strides: dict = field(default_factory=dict)  # optional {"q": (sb, st, sh), "k": ..., "v": ...}
    # KV merging (KvMerge::Pool): stride 1 = dense; layout = (frames, special, grid_h, grid_w, dense_frames)
    merge: int = 1
    layout: tuple = (1, 0, 0, 0, 0)
    # QK LayerNorm (QkNorm): None, or [4 * head_dim] float32 (q weight, q bias, k weight, k bias)
    ln: np.ndarray | None = field(default=None, compare=False)
    ln_eps: float = 1e-5
    # PvAccum::F16: V scaled to +-2.25 (PV16_V_RANGE) and f16 block partials in the emulator
    pv16: bool = False

    def __post_init__(self):
        if self.ln is not None:
            self.ln = np.ascontiguousarray(self.ln, dtype=np.float32).reshape(-1)
            assert self.ln.size >= 4 * self.head_dim

    @property
    def hk(self) -> int:
        return self.kv_heads or self.heads

    @property
    def tq_pad(self) -> int:
        return -(-self.tokens // QTILE) * QTILE

    @property
    def tk(self) -> int:
        """Keys after merging (FrameLayout::merged_keys, mod.rs:293-299)."""
        return lib().oracle_merged_keys(C.byref(self._c()))

    @property
    def tk_pad(self) -> int:
        return -(-self.tk // KBLOCK) * KBLOCK

    def members(self, j: int) -> list:
        """Tokens merged key j pools, in member order (reference.rs:79-109)."""
        buf = (C.c_int * 16)()
        n = lib().oracle_members(C.byref(self._c()), j, C.cast(buf, C.c_void_p))
        return list(buf[:n])

    def scale(self) -> np.float32:
        if self.softmax_scale is not None:
            return np.float32(self.softmax_scale)
        return np.float32(1.0) / np.sqrt(np.float32(self.head_dim))

    def q_mul(self) -> np.float32:
        return np.float32(self.scale() * LOG2E_F32)

    def _c(self) -> _Problem:
        d, t = self.head_dim, self.tokens
        def dflt(h):
            return (t * h * d, h * d, d)
        q = self.strides.get("q", dflt(self.heads))
        k = self.strides.get("k", dflt(self.hk))
        v = self.strides.get("v", dflt(self.hk))
        return _Problem(self.batch, self.heads, self.hk, t, d, self.dtype, *q, *k, *v, float(self.q_mul()),
                        int(self.smooth_k), int(self.smooth_v), 2.25 if self.pv16 else 448.0, int(self.merge),
                        *self.layout, None if self.ln is None else self.ln.ctypes.data, float(self.ln_eps),
                        int(self.pv16))


@dataclass
class GenSpec:
    k_off_std: float = 2.0
    outlier_channels: int = 0
    outlier_scale: float = 1.0
    token_frac: float = 0.0
    token_scale: float = 1.0
    seed: int = 1


def generate(p: Problem, g: GenSpec):
    """Seeded synthetic Q, K, V (uint16 codes of p.dtype), shapes [B,T,H,D] / [B,T,HKV,D]."""
    q = np.empty((p.batch, p.tokens, p.heads, p.head_dim), np.uint16)
    k = np.empty((p.batch, p.tokens, p.hk, p.head_dim), np.uint16)
    v = np.empty_like(k)
    s = _GenSpec(p.batch, p.heads, p.hk, p.tokens, p.head_dim, p.dtype, g.k_off_std, g.outlier_channels,
                 g.outlier_scale, g.token_frac, g.token_scale, g.seed)
    lib().oracle_generate(C.byref(s), _p(q), _p(k), _p(v))
    return q, k, v


def reference_synthetic(p: Problem, seed: int):
    """The reference tests' clustered bf16 activations (tests.rs:300-329), [B,T,H,D]."""
    assert p.dtype == BF16 and p.hk == p.heads
    shape = (p.batch, p.tokens, p.heads, p.head_dim)
    q, k, v = (np.empty(shape, np.uint16) for _ in range(3))
    lib().oracle_reference_synthetic(p.batch, p.tokens, p.heads, p.head_dim, seed, _p(q), _p(k), _p(v))
    return q, k, v


def prologue(p: Problem, q: np.ndarray, k: np.ndarray, v: np.ndarray, threads: int = 0) -> dict:
    """Bit-exact restatement of the reference prologue; logical layouts."""
    B, H, HK, D = p.batch, p.heads, p.hk, p.head_dim
    out = {
        "q8": np.zeros((B, H, p.tq_pad, D), np.int8),
        "q_scale": np.zeros((B, H, p.tq_pad // QGROUP), np.float32),
        "k8": np.zeros((B, HK, p.tk_pad, D), np.int8),
        "k_scale": np.zeros((B, HK, p.tk_pad // KBLOCK), np.float32),
        "v8": np.zeros((B, HK, p.tk_pad, D), np.uint8),
        "stats": np.zeros((B, HK, 4, D), np.float32),
        "kbias": np.zeros((p.tk_pad,), np.float32),
    }
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    r = lib().oracle_prologue(C.byref(p._c()), _p(q), _p(k), _p(v), _p(out["q8"]), _p(out["q_scale"]),
                              _p(out["k8"]), _p(out["k_scale"]), _p(out["v8"]), _p(out["stats"]), _p(out["kbias"]),
                              threads)
    if r != 0:
        raise ValueError("oracle prologue: unsupported head dim")
    return out


def _rows(rows, p: Problem):
    """rows: None (all), a 1-D array shared by every (b, h), or a
    [B*H, R] array of per-(b, h) rows. Returns (array or None, R, stride)."""
    if rows is None:
        return None, p.tokens, 0
    r = np.ascontiguousarray(rows, dtype=np.int32)
    assert r.min() >= 0 and r.max() < p.tokens
    if r.ndim == 2:
        assert r.shape[0] == p.batch * p.heads
        return r, r.shape[1], r.shape[1]
    return r, len(r), 0


def attention_f64(p: Problem, q, k, v, rows=None, threads: int = 0) -> np.ndarray:
    """f64 softmax attention (reference.rs:148-184), [B, H, R, D] float32."""
    r, R, rs = _rows(rows, p)
    out = np.empty((p.batch, p.heads, R, p.head_dim), np.float32)
    q, k, v = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, k, v))
    lib().oracle_attention_f64_rows(C.byref(p._c()), int(p.causal), float(p.scale()), _p(q), _p(k), _p(v),
                                    None if r is None else _p(r), R, rs, _p(out), threads)
    return out


def sage_emulate(p: Problem, pro: dict, rows=None, out_dtype: int = BF16, threads: int = 0, fast_exp: bool = True,
                 numerics: Numerics | None = None):
    """The reference's quantised attention arithmetic on `pro`; returns
    (float32 [B,H,R,D] before 16-bit rounding, uint16 codes of out_dtype).
    fast_exp=True is the reference's default logit arithmetic (SG_FAST_EXP=1,
    sage_attn.cu:59-61); False converts the scores exactly (SG_FAST_EXP=0).
    `numerics` selects an alternative softmax (None = the reference's)."""
    r, R, rs = _rows(rows, p)
    out = np.empty((p.batch, p.heads, R, p.head_dim), np.float32)
    o16 = np.empty(out.shape, np.uint16)
    kb = np.ascontiguousarray(pro.get("kbias", np.zeros(p.tk_pad, np.float32)), dtype=np.float32)
    nv = None if numerics is None else C.byref(numerics._c())
    lib().oracle_sage_emulate_numerics(C.byref(p._c()), int(p.causal), _p(pro["q8"]), _p(pro["q_scale"]),
                                       _p(pro["k8"]), _p(pro["k_scale"]), _p(pro["v8"]), _p(pro["stats"]), _p(kb),
                                       None if r is None else _p(r), R, rs, _p(out), _p(o16), out_dtype,
                                       int(bool(fast_exp)), nv, threads)
    return out, o16


def layernorm(x: np.ndarray, ln_w: np.ndarray, ln_b: np.ndarray, eps: float = 1e-5, f64: bool = False) -> np.ndarray:
    """Row-wise LayerNorm of x [..., D]: the prologue kernels' fp32 arithmetic
    (sage_quant.cu:34-52, correctly rounded reciprocal square root), or with
    f64=True the reference's CPU layer_norm (reference.rs:109-118)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(ln_w, dtype=np.float32)
    b = np.ascontiguousarray(ln_b, dtype=np.float32)
    D = x.shape[-1]
    out = np.empty_like(x)
    fn = lib().oracle_layernorm_f64 if f64 else lib().oracle_layernorm
    xr, orow = x.reshape(-1, D), out.reshape(-1, D)
    for i in range(xr.shape[0]):
        fn(xr[i].ctypes.data, orow[i].ctypes.data, D, _p(w), _p(b), C.c_float(eps))
    return out


def round_f16(x: float) -> float:
    """x rounded to the nearest f16 value (the PvAccum::F16 accumulator), as a float."""
    return lib().oracle_round_f16(float(x))


def log2_count(n: int) -> float:
    """The KV-merge bias of a key pooling n tokens: log2(n) rounded to f32."""
    return float(np.float32(lib().oracle_log2_count(n)))


def errors(ours: np.ndarray, ref: np.ndarray) -> dict:
    """reference.rs:186-225: cos, rel_l1, rel_l2, max_abs, ref_max."""
    a = np.ascontiguousarray(ours, dtype=np.float32).ravel()
    b = np.ascontiguousarray(ref, dtype=np.float32).ravel()
    assert a.size == b.size
    o = np.zeros(5, np.float64)
    lib().oracle_errors(_p(a), _p(b), a.size, _p(o))
    return dict(cos=o[0], rel_l1=o[1], rel_l2=o[2], max_abs=o[3], ref_max=o[4])


# The five benchmark configurations C1-C5, as (Problem, GenSpec).
def config(n: int, seed: int = 1):
    if n == 1:
        return Problem(1, 2, 256, 64, dtype=F16), GenSpec(k_off_std=2.0, seed=seed)
    if n == 2:
        return Problem(2, 32, 4096, 128, dtype=BF16), GenSpec(k_off_std=2.0, seed=seed)
    if n == 3:
        return (Problem(1, 32, 16384, 128, dtype=F16, causal=True),
                GenSpec(k_off_std=2.0, outlier_channels=4, outlier_scale=20.0, seed=seed))
    if n == 4:
        return (Problem(1, 32, 8192, 128, kv_heads=8, dtype=BF16, causal=True, softmax_scale=1 / math.sqrt(128)),
                GenSpec(k_off_std=2.0, seed=seed))
    if n == 5:
        return (Problem(1, 48, 17776, 64, dtype=F16),
                GenSpec(k_off_std=3.0, token_frac=0.02, token_scale=10.0, seed=seed))
    raise ValueError(n)


# ------------------------------------------------------------------ QKV prologue (qkv.cu, qkv.rs)

NORM_NONE, NORM_LAYER, NORM_RMS = 0, 1, 2
ROPE_VGGT, ROPE_DINOV3 = 0, 1


class _Qkv(C.Structure):
    _fields_ = [
        ("batch", C.c_int), ("tokens", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("head_dim", C.c_int),
        ("ld", C.c_longlong), ("batch_stride", C.c_longlong),
        ("tok", C.c_void_p), ("chan", C.c_void_p), ("bias", C.c_void_p),
        ("norm", C.c_int), ("q_w", C.c_void_p), ("q_b", C.c_void_p), ("k_w", C.c_void_p), ("k_b", C.c_void_p),
        ("eps", C.c_float), ("rope", C.c_void_p), ("rope_layout", C.c_int), ("frame_len", C.c_int),
        ("v_f16", C.c_int),
    ]


@dataclass
class QkvSpec:
    """The fused QKV projection's layout and the qkv_prologue options
    (qkv.cu:9-31): y is bf16 [batch][tokens][ld], q | k | v of heads*D,
    kv_heads*D, kv_heads*D channels. Arrays are numpy; None is off. norm_w is
    [4][D] float32 (q weight, q bias, k weight, k bias); rope is float32
    [frame_len][D/2][2] (cos, sin)."""

    batch: int
    tokens: int
    heads: int
    head_dim: int
    kv_heads: int = 0
    ld: int = 0
    tok: np.ndarray | None = field(default=None, compare=False)
    chan: np.ndarray | None = field(default=None, compare=False)
    bias: np.ndarray | None = field(default=None, compare=False)  # uint16 bf16 codes
    norm: int = NORM_NONE
    norm_w: np.ndarray | None = field(default=None, compare=False)
    eps: float = 1e-6
    rope: np.ndarray | None = field(default=None, compare=False)
    rope_layout: int = ROPE_VGGT
    v_f16: bool = False  # V as f16 codes (VFormat::F16)

    @property
    def hk(self) -> int:
        return self.kv_heads or self.heads

    @property
    def width(self) -> int:
        return (self.heads + 2 * self.hk) * self.head_dim

    def row_stride(self) -> int:
        return self.ld or self.width

    def _c(self) -> _Qkv:
        D = self.head_dim
        keep = []

        def ptr(a, dt):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dt)
            keep.append(a)
            return a.ctypes.data

        w = None if self.norm_w is None else np.ascontiguousarray(self.norm_w, np.float32).reshape(4, D)
        if w is not None:
            keep.append(w)
        rope = None if self.rope is None else np.ascontiguousarray(self.rope, np.float32)
        if rope is not None:
            keep.append(rope)
        c = _Qkv(self.batch, self.tokens, self.heads, self.hk, D, self.row_stride(),
                 self.tokens * self.row_stride(), ptr(self.tok, np.float32), ptr(self.chan, np.float32),
                 ptr(self.bias, np.uint16), int(self.norm),
                 None if w is None else w[0].ctypes.data, None if w is None else w[1].ctypes.data,
                 None if w is None else w[2].ctypes.data, None if w is None else w[3].ctypes.data,
                 float(self.eps), None if rope is None else rope.ctypes.data, int(self.rope_layout),
                 0 if rope is None else rope.shape[0], int(self.v_f16))
        c._keep = keep
        return c


def _qkv_lib():
    l = lib()
    if not getattr(l, "_qkv_ready", False):
        vp = C.c_void_p
        l.oracle_rope_table.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, vp]
        l.oracle_rope_half.restype = C.c_int
        l.oracle_rope_half.argtypes = [C.c_int, C.c_int]
        l.oracle_rope_pair.restype = C.c_int
        l.oracle_rope_pair.argtypes = [C.c_int, C.c_int, C.c_int]
        l.oracle_qkv_prologue.argtypes = [C.POINTER(_Qkv), vp, vp, vp, vp]
        l.oracle_qkv_reference_f64.argtypes = [C.POINTER(_Qkv), vp, vp, vp, vp]
        l._qkv_ready = True
    return l


def rope_table(layout: int, head_dim: int, grid_h: int, grid_w: int, special: int, base: float = 100.0):
    """RopeTable::vggt / ::dinov3 (qkv.rs:87-136): float32 [frame_len][D/2][2]."""
    n = special + grid_h * grid_w
    out = np.empty((n, head_dim // 2, 2), np.float32)
    _qkv_lib().oracle_rope_table(layout, head_dim, grid_h, grid_w, special, float(base), _p(out))
    return out


def rope_pair(layout: int, head_dim: int, d: int) -> int:
    return _qkv_lib().oracle_rope_pair(layout, head_dim, d)


def rope_half(layout: int, head_dim: int) -> int:
    return _qkv_lib().oracle_rope_half(layout, head_dim)


def _qkv_out(s: QkvSpec, dtype):
    D = s.head_dim
    return (np.empty((s.batch, s.tokens, s.heads, D), dtype), np.empty((s.batch, s.tokens, s.hk, D), dtype),
            np.empty((s.batch, s.tokens, s.hk, D), dtype))


def qkv_prologue(s: QkvSpec, y: np.ndarray):
    """qkv_prologue's fp32 arithmetic (qkv.cu:37-133): bf16 codes Q [B,T,H,D],
    K and V [B,T,HKV,D] from y (uint16 bf16 codes [B,T,ld])."""
    y = np.ascontiguousarray(y, dtype=np.uint16)
    assert y.shape == (s.batch, s.tokens, s.row_stride())
    q, k, v = _qkv_out(s, np.uint16)
    c = s._c()
    _qkv_lib().oracle_qkv_prologue(C.byref(c), _p(y), _p(q), _p(k), _p(v))
    return q, k, v


def qkv_reference_f64(s: QkvSpec, y: np.ndarray):
    """qkv::reference (qkv.rs:310-372): the f64 CPU reference, as float32."""
    y = np.ascontiguousarray(y, dtype=np.uint16)
    assert y.shape == (s.batch, s.tokens, s.row_stride())
    q, k, v = _qkv_out(s, np.float32)
    c = s._c()
    _qkv_lib().oracle_qkv_reference_f64(C.byref(c), _p(y), _p(q), _p(k), _p(v))
    return q, k, v
