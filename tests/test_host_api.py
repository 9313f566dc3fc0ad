"""Host side of the C ABI on the CPU (no GPU compute): the library loads and
exports every function include/sage_hip.h declares, the ctypes mirror has
the C struct layouts, and the plan / stride / tile / flops logic passes the
reference's own known-answer tests (tests.rs:135-283) and error texts."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sage_hip.h"


@pytest.fixture(scope="module")
def S():
    import spl_sage

    return spl_sage


def _header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*[A-Za-z_][\w \*]*?\b(sage_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_function(S):
    from spl_sage import _abi

    names = _header_functions()
    assert len(names) >= 20, names
    lib = C.CDLL(str(_abi.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python mirror binds each of them with a signature
    assert sorted(_abi.SIGNATURES) == names


def test_ctypes_structs_match_the_c_layout(S, tmp_path):
    """sizeof / offsetof of every ABI struct, compiled from the header with gcc,
    equal the ctypes mirror's (the role of geom_matches_the_cuda_struct,
    tests.rs:234-243, at this boundary)."""
    from spl_sage import _abi

    structs = {
        "sage_tile": ["warps", "m_tiles", "stages"],
        "sage_config": ["tile", "pv_accum"],
        "sage_shape": ["batch", "heads", "tokens", "kv_heads"],
        "sage_frame_layout": ["frames", "special", "grid_h", "grid_w", "dense_frames"],
        "sage_kv_merge": ["stride", "layout"],
        "sage_plan": ["shape", "merge", "tq_pad", "tk", "tk_pad"],
        "sage_strides": ["batch", "token", "head"],
        "sage_tensor": ["data", "len", "strides", "dtype"],
        "sage_tensor_mut": ["data", "len", "strides", "dtype"],
        "sage_options": ["softmax_scale", "has_softmax_scale", "smooth_k", "smooth_v", "qk_norm_params",
                         "qk_norm_len", "qk_norm_eps", "causal"],
        "sage_ws_buffers": ["q8", "q_scale", "k8", "k_scale", "v8", "stats", "kbias", "q8_len", "q_scale_len",
                            "k8_len", "k_scale_len", "v8_len", "stats_len", "kbias_len"],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for s, fields in structs.items():
        lines.append(f'printf("{s} %zu\\n", sizeof({s}));')
        for f in fields:
            lines.append(f'printf("{s}.{f} %zu\\n", offsetof({s}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-o", str(exe), str(src)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                 text=True).stdout.splitlines())
    for s, fields in structs.items():
        cls = getattr(_abi, s)
        assert int(got[s]) == C.sizeof(cls), s
        for f in fields:
            assert int(got[f"{s}.{f}"]) == getattr(cls, f).offset, f"{s}.{f}"


def test_vggt_dense_geometry(S):
    """tests.rs:137-148: 200 frames x 689 tokens."""
    plan = S.Plan.new(S.Shape(1, 16, 200 * 689))
    assert (plan.tq_pad, plan.tk, plan.tk_pad) == (137856, 137800, 137856)


def _vggt_layout(S, frames: int, dense_frames: int = 0):
    return S.FrameLayout(frames, 17, 21, 32, dense_frames)


def test_vggt_merge_key_counts(S):
    """tests.rs:149-152 and :96-110: merged key counts of the pooled layouts."""
    layout = _vggt_layout(S, 200)
    assert layout.tokens_per_frame() == 689
    shape = S.Shape(1, 16, 200 * 689)
    assert S.Plan.new(shape, S.KvMerge.Pool(2, layout)).tk == 200 * (17 + 11 * 16)
    assert S.Plan.new(shape, S.KvMerge.Pool(4, layout)).tk == 200 * (17 + 6 * 8)
    dense1 = _vggt_layout(S, 3, dense_frames=1)
    assert S.Plan.new(S.Shape(1, 1, 3 * 689), S.KvMerge.Pool(4, dense1)).tk == 689 + 2 * 65


def test_plan_rejects_bad_layouts(S):
    """tests.rs:175-190, with the reference's error texts."""
    layout = _vggt_layout(S, 2)
    with pytest.raises(S.SageError, match="frame layout"):
        S.Plan.new(S.Shape(1, 2, 1000), S.KvMerge.Pool(2, layout))
    shape = S.Shape(1, 2, 2 * 689)
    with pytest.raises(S.SageError, match="KV merge stride must be 2 or 4, got 3"):
        S.Plan.new(shape, S.KvMerge.Pool(3, layout))
    S.Plan.new(shape, S.KvMerge.Pool(4, layout))
    with pytest.raises(S.SageError, match="empty attention shape"):
        S.Plan.new(S.Shape(1, 2, 0))


def test_plan_range_checks(S):
    """mod.rs:406-439: an empty patch grid, and every count the kernels index
    with i32 (padded queries, padded keys, batch x heads) refused with the
    reference's texts."""
    with pytest.raises(S.SageError, match="KV merge needs a patch grid"):
        S.Plan.new(S.Shape(1, 1, 10), S.KvMerge.Pool(2, S.FrameLayout(2, 5, 0, 4, 0)))
    with pytest.raises(S.SageError, match="padded queries = 2147483648 does not fit in i32"):
        S.Plan.new(S.Shape(1, 1, 2**31 - 5))
    with pytest.raises(S.SageError, match="batch .* heads = 2147483648 does not fit in i32"):
        S.Plan.new(S.Shape(2**16, 2**15, 128))
    # Sizes whose padding or product would wrap 64 bits are refused, not wrapped.
    with pytest.raises(S.SageError, match="padded queries"):
        S.Plan.new(S.Shape(1, 1, 2**64 - 1))
    with pytest.raises(S.SageError, match="batch .* heads"):
        S.Plan.new(S.Shape(2**40, 2**30, 128))
    # A frame layout whose token count wraps 64 bits is refused: 2 frames of
    # 2^63 + 1 tokens would otherwise wrap to the sequence's 2 tokens.
    with pytest.raises(S.SageError, match="covers more than 2\\^64 tokens, the sequence has 2"):
        S.Plan.new(S.Shape(1, 1, 2), S.KvMerge.Pool(2, S.FrameLayout(2, 1, 1, 2**63, 0)))
    with pytest.raises(S.SageError, match="covers more than 2\\^64 tokens"):
        S.Plan.new(S.Shape(1, 1, 2), S.KvMerge.Pool(2, S.FrameLayout(1, 0, 2**32, 2**32, 0)))
    # The largest sizes that fit are accepted.
    p = S.Plan.new(S.Shape(1, 1, 2**31 - 128))
    assert p.tq_pad == 2**31 - 128 and p.tk_pad == 2**31 - 128
    S.Plan.new(S.Shape(2**16, 2**15 - 1, 128))


def test_extent_does_not_wrap(S):
    """Strides whose extent would wrap 64 bits report the largest extent, so a
    view with them can never pass the length check."""
    shape = S.Shape(1, 1, 5)
    assert S.Strides(8, 2**62, 8).extent(shape, 64) == 2**64 - 1
    assert S.Strides(8, 2**61, 8).extent(shape, 64) == 4 * 2**61 + 64


def test_plan_padding_and_tails(S):
    """mod.rs:431-434: tq_pad to 128, tk_pad to 64; the C5 tail shape."""
    p = S.Plan.new(S.Shape(1, 48, 17776))
    assert (p.tq_pad, p.tk, p.tk_pad) == (17792, 17776, 17792)
    assert p.q_tiles() == 139 and p.kblocks() == 278
    p = S.Plan.new(S.Shape(2, 32, 4096))
    assert (p.tq_pad, p.tk_pad) == (4096, 4096)


def test_plan_rejects_bad_grouped_heads(S):
    with pytest.raises(S.SageError):
        S.Plan.new(S.Shape(1, 32, 128, kv_heads=5))
    assert S.Plan.new(S.Shape(1, 32, 128, kv_heads=8)).kv_heads() == 8


def test_strides_cover_the_tensor(S):
    """tests.rs:245-261."""
    shape = S.Shape(2, 3, 5)
    d = 64
    assert S.Strides.bthd(5, 3, d).extent(shape, d) == 2 * 5 * 3 * d
    assert S.Strides.bhtd(5, 3, d).extent(shape, d) == 2 * 3 * 5 * d
    assert S.Strides.packed_qkv(5, 3, d).extent(shape, d) + 2 * 3 * d == 2 * 5 * 3 * 3 * d
    with pytest.raises(S.SageError, match="x strides must be multiples of 8 elements"):
        S.Strides.bthd(5, 3, 60).check("x")


def test_flops_counts_the_metric(S):
    """mod.rs:905-910 (4 B H Tq Tk D); causal counts the visible half, 2 B H D N (N + 1)."""
    c2 = S.Plan.new(S.Shape(2, 32, 4096))
    assert S.flops(c2, 128) == 4.0 * 2 * 32 * 4096 * 4096 * 128
    assert abs(S.flops(c2, 128) - 5.498e11) / 5.498e11 < 1e-3
    c3 = S.Plan.new(S.Shape(1, 32, 16384))
    assert S.flops(c3, 128, causal=True) == 2.0 * 32 * 128 * 16384 * 16385
    c1 = S.Plan.new(S.Shape(1, 2, 256))
    assert S.flops(c1, 64) == 4.0 * 2 * 256 * 256 * 64  # 3.36e7


def test_v8_position_is_the_operand_permutation(S):
    """Every key of a 64-key block has one byte in its V^T row, and key k sits
    where lane-half g = (k >> 2) & 1, register (k >> 5) * 4 + ((k >> 3) & 3),
    byte k & 3 of the FP8 B operand puts it."""
    pos = [S.v8_position(k) for k in range(64)]
    assert sorted(pos) == list(range(64))
    for k in range(64):
        g, reg, byte = (k >> 2) & 1, (k >> 5) * 4 + ((k >> 3) & 3), k & 3
        assert pos[k] == 32 * g + 4 * reg + byte


def _reference_tile_ok(w: int, m: int, st: int) -> bool:
    """Tile::validate (mod.rs:158-167), restated."""
    return w in (2, 4, 8) and m in (1, 2, 4) and 2 <= st <= 6 and 128 % (16 * m * w) == 0


def test_tile_menu_and_errors(S):
    """mod.rs:116-168: exactly the tiles the reference accepts validate; every
    other tile is refused with the reference's message, which names it."""
    accepted = 0
    for w in range(0, 10):
        for m in range(0, 6):
            for st in range(0, 8):
                t = S.Tile(w, m, st)
                if _reference_tile_ok(w, m, st):
                    t.validate()
                    accepted += 1
                else:
                    with pytest.raises(S.SageError, match=r"unsupported sage tile Tile \{ warps: %d, m_tiles: %d, "
                                       r"stages: %d \}" % (w, m, st)):
                        t.validate()
    # (2,1), (2,2), (2,4), (4,1), (4,2), (8,1) with stages 2..6
    assert accepted == 6 * 5
    for t in (S.Tile(4, 4, 3), S.Tile(8, 2, 3), S.Tile(8, 1, 7), S.Tile(4, 1, 1), S.Tile(3, 1, 2)):
        with pytest.raises(S.SageError, match="unsupported sage tile"):
            t.validate()


def test_default_tiles_are_the_references(S):
    """Tile::DEFAULT {4,2,3} and Tile::D128 {4,1,3} (mod.rs:128-147); Config::for_head_dim
    picks D128 above head dim 64 (mod.rs:141-147, 194-200) with PvAccum::F32."""
    assert S.Tile.DEFAULT == S.Tile(4, 2, 3) and S.Tile.D128 == S.Tile(4, 1, 3)
    assert S.Config.for_head_dim(64) == S.Config(S.Tile(4, 2, 3), S.PvAccum.F32)
    assert S.Config.for_head_dim(128) == S.Config(S.Tile(4, 1, 3), S.PvAccum.F32)
    assert S.Tile.for_head_dim(64) == S.Tile.DEFAULT and S.Tile.for_head_dim(128) == S.Tile.D128
    assert S.Tile.DEFAULT.rows() == 128 and S.Tile.D128.rows() == 64


def test_device_gate_without_a_gpu(S):
    """check_device reports, without a GPU, a device error rather than crashing."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(S.SageError):
        S.check_device(0)


@pytest.mark.parametrize("d", [64, 128])
def test_rope_tables_match_the_oracle(S, oracle, d):
    """RopeTable::vggt / ::dinov3 (qkv.rs:87-136) built by the library equal the
    oracle's restatement, which the reference's own table tests pin; too small
    an output buffer is refused with the reference's buffer message."""
    import numpy as np

    from spl_sage import qkv as Q

    for layout in (Q.RopeLayout.Vggt, Q.RopeLayout.Dinov3):
        t = Q.RopeTable._build(layout, 21, 32, 17, 100.0, d)
        assert t.frame_len == 17 + 21 * 32
        assert np.array_equal(t.cos_sin, oracle.rope_table(int(layout), d, 21, 32, 17, 100.0))
    out = np.empty(10, np.float32)
    with pytest.raises(S.SageError, match="RoPE table: buffer holds 10 elements, needs"):
        _check = S._check
        _check(S.lib().sage_rope_table(0, d, 2, 2, 1, 100.0, out.ctypes.data, out.size))
