"""The attention kernel's two workgroup layouts, and the padding keys of a
partial last key block.

Tile { warps: 8 } (mod.rs:116-168) selects the eight-wave layout: four score
waves run QK^T and the online softmax, four output waves run the rescale and
P.V one key block behind them. Its arithmetic is the four-wave kernel's
operation for operation, so its outputs must be bit-identical, including
over ragged tails, causal diagonals, grouped heads and the benchmark
configurations' value distributions (C5's 17776 keys end in a 48-key block).

Keys past the sequence in the last 64-key block must have no influence at
all (sage_attn.cu:275-281 masks them to -inf, so P = 0): after prepare, the
padding rows of the INT8 K codes are overwritten with +127 and the padding
keys' FP8 V codes with 448, and the output must not change by one bit.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import from_device16, to_device16

pytestmark = pytest.mark.gpu

# (label, Problem kwargs, GenSpec kwargs)
CASES = [
    ("d128_bf16_n1000", dict(batch=2, heads=4, tokens=1000, head_dim=128), dict(k_off_std=2.0, seed=41)),
    ("d128_causal_outliers", dict(batch=1, heads=4, tokens=700, head_dim=128, dtype=1, causal=True),
     dict(k_off_std=2.0, outlier_channels=4, outlier_scale=20.0, seed=42)),
    ("d128_causal_gqa_xcd", dict(batch=2, heads=8, tokens=700, head_dim=128, kv_heads=4, causal=True),
     dict(k_off_std=2.0, seed=43)),
    ("d128_n65", dict(batch=1, heads=2, tokens=65, head_dim=128), dict(seed=44)),
    ("d64_c5_tail", dict(batch=1, heads=2, tokens=17776, head_dim=64, dtype=1),
     dict(k_off_std=3.0, token_frac=0.02, token_scale=10.0, seed=45)),
    ("d64_causal_gqa", dict(batch=1, heads=6, tokens=333, head_dim=64, kv_heads=3, causal=True),
     dict(k_off_std=1.0, seed=46)),
    ("d64_n1", dict(batch=1, heads=2, tokens=1, head_dim=64), dict(seed=47)),
]


def _problem(oracle, kw, gk):
    return oracle.Problem(**kw), oracle.GenSpec(**gk)


def _forward(torch, p, q, k, v, tile=None, poison=False):
    """prepare + attend through the C ABI; with poison, the padding keys' codes
    are overwritten between the two. Returns the uint16 output."""
    import spl_sage as S

    D = p.head_dim
    config = S.Config(tile, S.PvAccum.F32) if tile is not None else None
    sa = S.SageAttention(None, D, config)
    ws = sa.workspace(S.Shape(p.batch, p.heads, p.tokens, p.kv_heads))
    qt, kt, vt = (S.Tensor(to_device16(torch, x, p.dtype)) for x in (q, k, v))
    out = torch.empty((p.batch, p.tokens, p.heads, D), dtype=torch.bfloat16 if p.dtype == 0 else torch.float16,
                      device="cuda")
    opts = S.Options(causal=p.causal)
    sa.prepare(ws, qt, kt, vt, opts)
    torch.cuda.synchronize()
    if poison:
        _poison_padding(ws, p)
    sa.attend(ws, S.TensorMut(out))
    torch.cuda.synchronize()
    return from_device16(out)


_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        _HIP = C.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.restype = C.c_int
        _HIP.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return _HIP


def _poison_padding(ws, p) -> None:
    """INT8 K codes of keys tk .. tk_pad - 1 := +127; their FP8 V codes := 448
    (0x7E, E4M3's largest finite), at their v8 positions."""
    import spl_sage as S

    plan, b = ws.plan(), ws.buffers()
    tk, tkp, D, G = plan.tk, plan.tk_pad, p.head_dim, p.batch * p.hk
    assert tkp > tk
    hip = _hip()
    krows = np.full((tkp - tk) * D, 127, np.int8)
    pos = np.array([S.v8_position(j) for j in range(tk % 64, 64)])
    nblk = tkp // 64
    blk = np.empty((D, 64), np.uint8)
    for g in range(G):
        assert hip.hipMemcpy(b.k8 + (g * tkp + tk) * D, krows.ctypes.data, krows.nbytes, 1) == 0
        base = b.v8 + (g * nblk + nblk - 1) * D * 64
        assert hip.hipMemcpy(blk.ctypes.data, base, blk.nbytes, 2) == 0
        blk[:, pos] = 0x7E
        assert hip.hipMemcpy(base, blk.ctypes.data, blk.nbytes, 1) == 0


@pytest.mark.parametrize("label,kw,gk", CASES, ids=[c[0] for c in CASES])
def test_eight_wave_layout_is_bit_identical(oracle, torch_gpu, label, kw, gk):
    import spl_sage as S

    p, g = _problem(oracle, kw, gk)
    q, k, v = oracle.generate(p, g)
    base = _forward(torch_gpu, p, q, k, v)
    for tile in (S.Tile(8, 1, 3), S.Tile(8, 1, 4)):
        o = _forward(torch_gpu, p, q, k, v, tile=tile)
        diff = int((o != base).sum())
        assert diff == 0, f"{label}: {diff} of {o.size} outputs differ under {tile}"


@pytest.mark.parametrize("warps", [4, 8])
@pytest.mark.parametrize("label,kw,gk", [c for c in CASES if c[1]["tokens"] % 64], ids=[c[0] for c in CASES
                                                                                       if c[1]["tokens"] % 64])
def test_padding_keys_have_no_influence(oracle, torch_gpu, label, kw, gk, warps):
    import spl_sage as S

    p, g = _problem(oracle, kw, gk)
    q, k, v = oracle.generate(p, g)
    tile = S.Tile(warps, 1, 3)
    clean = _forward(torch_gpu, p, q, k, v, tile=tile)
    dirty = _forward(torch_gpu, p, q, k, v, tile=tile, poison=True)
    diff = int((clean != dirty).sum())
    assert diff == 0, f"{label} warps={warps}: {diff} of {clean.size} outputs moved when padding codes changed"


def test_merged_padding_keys_have_no_influence(oracle, torch_gpu):
    """KV-merged plans carry a -inf logit bias past tk instead of a mask
    (sage_attn.cu:238-246): the same poison leaves the output unchanged."""
    import spl_sage as S

    layout = S.FrameLayout(3, 17, 21, 32, 0)
    T, H, D = 3 * layout.tokens_per_frame(), 2, 64
    rng = np.random.default_rng(48)
    mk = lambda s: (torch_gpu.from_numpy((rng.standard_normal((1, T, H, D)) * s).astype(np.float32))
                    .to("cuda").to(torch_gpu.bfloat16))
    q, k, v = mk(1.0), mk(1.5), mk(1.0)
    sa = S.SageAttention(None, D)
    ws = sa.workspace(S.Shape(1, H, T), S.KvMerge.Pool(4, layout))
    plan = ws.plan()
    assert plan.tk_pad > plan.tk
    outs = []
    for poison in (False, True):
        out = torch_gpu.empty((1, T, H, D), dtype=torch_gpu.bfloat16, device="cuda")
        sa.prepare(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), S.Options())
        torch_gpu.cuda.synchronize()
        if poison:
            class _P:  # the fields _poison_padding reads
                head_dim, batch, hk = D, 1, H
            _poison_padding(ws, _P)
        sa.attend(ws, S.TensorMut(out))
        torch_gpu.cuda.synchronize()
        outs.append(from_device16(out))
    assert np.array_equal(outs[0], outs[1])
