"""Helpers for the GPU parity tests: run the HIP path through the C ABI
(spl_sage) on oracle-generated inputs and bring results back to numpy in the
oracle's logical layouts."""
from __future__ import annotations

import numpy as np

from conftest import from_device16, to_device16


def v8_logical(raw: np.ndarray, b: int, g: int, tk_pad: int, d: int) -> np.ndarray:
    """[b][g][blk][D][64 positions] -> [b][g][tk_pad][D] with keys in order."""
    import spl_sage

    perm = np.array([spl_sage.v8_position(k) for k in range(64)])
    x = raw.reshape(b, g, tk_pad // 64, d, 64)[..., perm]  # [..., D, key]
    return np.ascontiguousarray(x.transpose(0, 1, 2, 4, 3)).reshape(b, g, tk_pad, d)


def run(torch, p, q, k, v, out_dtype=None, q_layout="bthd", out_layout="bthd", want_ws=True, tile=None):
    """Runs prepare + attend on the GPU. q, k, v are uint16 [B,T,H,D] codes.
    `tile` (an spl_sage.Tile, default Config::for_head_dim's) configures the
    context. Returns (dict of workspace buffers in logical layouts, uint16
    output [B,T,H,D])."""
    import spl_sage as S

    B, T, H, HK, D = p.batch, p.tokens, p.heads, p.hk, p.head_dim
    config = None
    if p.pv16 or tile is not None:
        config = S.Config(tile if tile is not None else S.Config.for_head_dim(D).tile,
                          S.PvAccum.F16 if p.pv16 else S.PvAccum.F32)
    sa = S.SageAttention(None, D, config)
    merge = S.KvMerge.Dense
    if p.merge > 1:
        merge = S.KvMerge.Pool(p.merge, S.FrameLayout(*p.layout))
    ws = sa.workspace(S.Shape(B, H, T, p.kv_heads), merge)
    od = p.dtype if out_dtype is None else out_dtype
    tdt = torch.bfloat16 if od == 0 else torch.float16
    if q_layout == "packed" and H == HK:
        packed = np.stack([q, k, v], axis=2)  # [B,T,3,H,D]
        buf = to_device16(torch, packed, p.dtype).reshape(-1)
        st = S.Strides.packed_qkv(T, H, D)
        qt, kt, vt = (S.Tensor(buf[i * H * D:], st) for i in range(3))
    elif q_layout == "bhtd":
        qd = to_device16(torch, np.ascontiguousarray(q.transpose(0, 2, 1, 3)), p.dtype)
        kd = to_device16(torch, np.ascontiguousarray(k.transpose(0, 2, 1, 3)), p.dtype)
        vd = to_device16(torch, np.ascontiguousarray(v.transpose(0, 2, 1, 3)), p.dtype)
        qt, kt, vt = (S.Tensor(x, S.Strides.bhtd(T, h, D)) for x, h in ((qd, H), (kd, HK), (vd, HK)))
    else:
        qt, kt, vt = (S.Tensor(to_device16(torch, x, p.dtype)) for x in (q, k, v))
    if out_layout == "bhtd":
        out = torch.empty((B, H, T, D), dtype=tdt, device="cuda")
        om = S.TensorMut(out, S.Strides.bhtd(T, H, D))
    else:
        out = torch.empty((B, T, H, D), dtype=tdt, device="cuda")
        om = S.TensorMut(out)
    qk_norm = None
    if p.ln is not None:
        qk_norm = S.QkNorm(torch.from_numpy(p.ln.copy()).to("cuda"), float(p.ln_eps))
    opts = S.Options(softmax_scale=p.softmax_scale, smooth_k=p.smooth_k, smooth_v=p.smooth_v, causal=p.causal,
                     qk_norm=qk_norm)
    sa.forward(ws, qt, kt, vt, om, opts)
    torch.cuda.synchronize()
    o = from_device16(out)
    if out_layout == "bhtd":
        o = np.ascontiguousarray(o.transpose(0, 2, 1, 3))
    return (read_workspace(ws, p) if want_ws else None), o


def read_workspace(ws, p) -> dict:
    """A prepared workspace's codes, scales and statistics in the oracle's
    logical layouts."""
    B, H, HK, D = p.batch, p.heads, p.hk, p.head_dim
    plan = ws.plan()
    get = lambda n: ws.tensor(n).cpu().numpy()
    pro = {
        "q8": get("q8").reshape(B, H, plan.tq_pad, D),
        "q_scale": get("q_scale").reshape(B, H, plan.tq_pad // 16),
        "k8": get("k8").reshape(B, HK, plan.tk_pad, D),
        "k_scale": get("k_scale").reshape(B, HK, plan.tk_pad // 64),
        "v8": v8_logical(get("v8"), B, HK, plan.tk_pad, D),
        "stats": get("stats").reshape(B, HK, 4, D),
    }
    if p.merge > 1:
        pro["kbias"] = get("kbias").reshape(plan.tk_pad)
    return pro


def assert_prologue_equal(got: dict, want: dict) -> None:
    names = ("q8", "q_scale", "k8", "k_scale", "v8", "stats") + (("kbias",) if "kbias" in got else ())
    for name in names:
        a, b = got[name], want[name]
        assert a.shape == b.shape, (name, a.shape, b.shape)
        if a.dtype == np.float32:
            same = a.view(np.uint32) == b.view(np.uint32)
        else:
            same = a == b
        if not same.all():
            idx = np.argwhere(~same)[:5]
            raise AssertionError(
                f"{name}: {int((~same).sum())} of {a.size} differ; first {[(tuple(i), a[tuple(i)], b[tuple(i)]) for i in idx]}")


def sample_rows(n: int, count: int, seed: int = 0) -> np.ndarray:
    """First, last and random query rows (sorted, unique)."""
    if n <= count:
        return np.arange(n, dtype=np.int32)
    rng = np.random.default_rng(seed)
    r = set(rng.choice(n, size=count - 4, replace=False).tolist()) | {0, 1, n - 2, n - 1}
    return np.array(sorted(r), dtype=np.int32)


def tile_rows(n: int, heads_total: int, per_tile: int = 1, seed: int = 0) -> np.ndarray:
    """[heads_total, R] query rows: for every (batch, head) slot, `per_tile`
    distinct random rows inside each 128-query tile (the attention kernel's
    workgroup), drawn independently per slot, so every workgroup of every
    head is compared. R = tiles * per_tile (tiles holding fewer rows than
    per_tile give all of theirs, padded by repeats)."""
    rng = np.random.default_rng(seed)
    tiles = -(-n // 128)
    out = np.empty((heads_total, tiles * per_tile), np.int32)
    for bh in range(heads_total):
        for t in range(tiles):
            lo, hi = 128 * t, min(n, 128 * t + 128)
            pick = rng.choice(hi - lo, size=per_tile, replace=(hi - lo) < per_tile)
            out[bh, t * per_tile:(t + 1) * per_tile] = np.sort(lo + pick)
    return out


def gather_rows(o: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """[B,T,H,D] -> [B,H,R,D] for the given rows: a 1-D array shared by every
    (batch, head), or a [B*H, R] array of per-(batch, head) rows."""
    if rows.ndim == 1:
        return np.ascontiguousarray(o[:, rows].transpose(0, 2, 1, 3))
    B, _, H, D = o.shape
    r = rows.reshape(B, H, -1)
    b = np.arange(B)[:, None, None]
    h = np.arange(H)[None, :, None]
    return np.ascontiguousarray(o[b, r, h])
