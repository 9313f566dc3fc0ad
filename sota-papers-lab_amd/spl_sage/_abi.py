"""ctypes declarations of include/sage_hip.h (the C ABI of libsage_hip.so)."""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsage_hip.so"

u64 = C.c_uint64
i32 = C.c_int32
u32 = C.c_uint32


class sage_tile(C.Structure):
    _fields_ = [("warps", u32), ("m_tiles", u32), ("stages", u32)]


class sage_config(C.Structure):
    _fields_ = [("tile", sage_tile), ("pv_accum", i32)]


class sage_shape(C.Structure):
    _fields_ = [("batch", u64), ("heads", u64), ("tokens", u64), ("kv_heads", u64)]


class sage_frame_layout(C.Structure):
    _fields_ = [("frames", u64), ("special", u64), ("grid_h", u64), ("grid_w", u64), ("dense_frames", u64)]


class sage_kv_merge(C.Structure):
    _fields_ = [("stride", u32), ("layout", sage_frame_layout)]


class sage_plan(C.Structure):
    _fields_ = [("shape", sage_shape), ("merge", sage_kv_merge), ("tq_pad", u64), ("tk", u64), ("tk_pad", u64)]


class sage_strides(C.Structure):
    _fields_ = [("batch", u64), ("token", u64), ("head", u64)]


class sage_tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("len", u64), ("strides", sage_strides), ("dtype", i32)]


class sage_tensor_mut(C.Structure):
    _fields_ = [("data", C.c_void_p), ("len", u64), ("strides", sage_strides), ("dtype", i32)]


class sage_options(C.Structure):
    _fields_ = [
        ("softmax_scale", C.c_float),
        ("has_softmax_scale", i32),
        ("smooth_k", i32),
        ("smooth_v", i32),
        ("qk_norm_params", C.c_void_p),
        ("qk_norm_len", u64),
        ("qk_norm_eps", C.c_float),
        ("causal", i32),
    ]


class sage_ws_buffers(C.Structure):
    _fields_ = [
        ("q8", C.c_void_p),
        ("q_scale", C.c_void_p),
        ("k8", C.c_void_p),
        ("k_scale", C.c_void_p),
        ("v8", C.c_void_p),
        ("stats", C.c_void_p),
        ("kbias", C.c_void_p),
        ("q8_len", u64),
        ("q_scale_len", u64),
        ("k8_len", u64),
        ("k_scale_len", u64),
        ("v8_len", u64),
        ("stats_len", u64),
        ("kbias_len", u64),
    ]


class sage_qkv_in(C.Structure):
    _fields_ = [
        ("y", C.c_void_p), ("y_len", u64), ("ld", u64), ("batch_stride", u64),
        ("tok", C.c_void_p), ("tok_len", u64), ("chan", C.c_void_p), ("chan_len", u64),
        ("bias", C.c_void_p), ("bias_len", u64),
    ]


class sage_qkv_norm(C.Structure):
    _fields_ = [
        ("kind", i32), ("q_weight", C.c_void_p), ("q_bias", C.c_void_p), ("k_weight", C.c_void_p),
        ("k_bias", C.c_void_p), ("len", u64), ("eps", C.c_float),
    ]


class sage_qkv_rope(C.Structure):
    _fields_ = [("table", C.c_void_p), ("table_len", u64), ("layout", i32), ("frame_len", u64)]


P = C.POINTER
# name -> (restype, argtypes); every symbol include/sage_hip.h declares.
SIGNATURES = {
    "sage_last_error": (C.c_char_p, []),
    "sage_plan_new": (i32, [P(sage_shape), P(sage_kv_merge), P(sage_plan)]),
    "sage_flops": (C.c_double, [P(sage_plan), u64, i32]),
    "sage_strides_check": (i32, [P(sage_strides), C.c_char_p]),
    "sage_strides_extent": (u64, [P(sage_strides), u64, u64, u64, u64]),
    "sage_tile_validate": (i32, [P(sage_tile)]),
    "sage_config_for_head_dim": (sage_config, [u64]),
    "sage_check_device": (i32, [C.c_int]),
    "sage_new": (i32, [C.c_void_p, u64, P(sage_config), P(C.c_void_p)]),
    "sage_destroy": (None, [C.c_void_p]),
    "sage_head_dim": (u64, [C.c_void_p]),
    "sage_get_config": (sage_config, [C.c_void_p]),
    "sage_stream": (C.c_void_p, [C.c_void_p]),
    "sage_attn_resources": (i32, [C.c_void_p, P(i32), P(i32), P(i32)]),
    "sage_attn_kernel_resources": (i32, [C.c_void_p, i32, P(i32), P(i32), P(i32)]),
    "sage_workspace_new": (i32, [C.c_void_p, P(sage_shape), P(sage_kv_merge), P(C.c_void_p)]),
    "sage_workspace_destroy": (None, [C.c_void_p]),
    "sage_workspace_bytes": (u64, [C.c_void_p]),
    "sage_workspace_plan": (i32, [C.c_void_p, P(sage_plan)]),
    "sage_workspace_buffers": (i32, [C.c_void_p, P(sage_ws_buffers)]),
    "sage_prepare": (i32, [C.c_void_p, C.c_void_p, P(sage_tensor), P(sage_tensor), P(sage_tensor), P(sage_options)]),
    "sage_attend": (i32, [C.c_void_p, C.c_void_p, P(sage_tensor_mut)]),
    "sage_forward": (
        i32,
        [C.c_void_p, C.c_void_p, P(sage_tensor), P(sage_tensor), P(sage_tensor), P(sage_tensor_mut), P(sage_options)],
    ),
    "sage_forward_noalloc": (
        i32,
        [C.c_void_p, P(sage_shape), P(sage_kv_merge), P(sage_tensor), P(sage_tensor), P(sage_tensor),
         P(sage_tensor_mut), P(sage_options)],
    ),
    "sage_rope_table": (i32, [i32, u64, u64, u64, u64, C.c_double, C.c_void_p, u64]),
    "sage_qkv_prologue": (
        i32,
        [C.c_void_p, P(sage_shape), P(sage_qkv_in), P(sage_qkv_norm), P(sage_qkv_rope), P(sage_tensor_mut),
         P(sage_tensor_mut), P(sage_tensor_mut)],
    ),
    "sage_prepare_qkv": (
        i32, [C.c_void_p, C.c_void_p, P(sage_qkv_in), P(sage_qkv_norm), P(sage_qkv_rope), P(sage_options)],
    ),
    "sage_forward_qkv": (
        i32,
        [C.c_void_p, C.c_void_p, P(sage_qkv_in), P(sage_qkv_norm), P(sage_qkv_rope), P(sage_tensor_mut),
         P(sage_options)],
    ),
    "sage_v8_position": (i32, [i32]),
    "sage_peak": (i32, [C.c_void_p, i32, i32, P(C.c_double)]),
}

_lib = None


def lib() -> C.CDLL:
    """Loads libsage_hip.so (built by sota-papers-lab_amd/build.py). Raises
    if it is missing: there is no fallback path."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OSError(
                f"{LIB_PATH} is not built; run `python sota-papers-lab_amd/build.py` "
                "(or __graft_entry__.build())"
            )
        l = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib
