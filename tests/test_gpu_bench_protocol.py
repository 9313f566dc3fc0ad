"""The reference benchmark's file protocol (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/tests.rs:796-1022 and torch_ref.py:1-30), through
`bench.py --gpu-bench`: a run directory's meta.txt and bf16 [T][H][D] q.bin,
k.bin, v.bin in; out_<mode>.bin and out_<mode>_pv16.bin for dense, merge2 and
merge4 written back, equal bit for bit to the library's own forward on the
same inputs; one JSON line a (config, mode) with the reference's keys in
$SAGE_OUT/bench_d<D>_f<frames>.json."""
from __future__ import annotations

import argparse
import json

import numpy as np
import pytest

from conftest import from_device16

pytestmark = pytest.mark.gpu

KEYS = {"tile", "variant", "pv_accum", "regs", "spill", "mode", "frames", "heads", "head_dim", "tokens", "keys",
        "prep_ms", "attn_ms", "attn_best_ms", "attn_tops", "dense_equiv_tops", "workspace_mb"}


def test_run_directory_round_trip(torch_gpu, tmp_path, monkeypatch):
    import bench
    import spl_sage as S

    torch = torch_gpu
    frames, heads, d, special, gh, gw = 3, 2, 64, 17, 21, 32
    T = frames * (special + gh * gw)
    run = tmp_path / "run"
    run.mkdir()
    (run / "meta.txt").write_text(f"frames={frames}\nheads={heads}\nhead_dim={d}\nspecial={special}\n"
                                  f"grid_h={gh}\ngrid_w={gw}\nsource=test\n")
    rng = np.random.default_rng(5)
    qkv = []
    for name in ("q", "k", "v"):
        x = rng.standard_normal((T, heads, d)).astype(np.float32)
        if name == "k":
            x += 2.0 * rng.standard_normal((heads, d)).astype(np.float32)
        b = (x.view(np.uint32) + 0x7FFF + ((x.view(np.uint32) >> 16) & 1)) >> 16  # round to nearest even bf16
        b = b.astype("<u2")
        b.tofile(run / f"{name}.bin")
        qkv.append(b)
    out_dir = tmp_path / "out"
    monkeypatch.setenv("SAGE_RUN", str(run))
    monkeypatch.setenv("SAGE_OUT", str(out_dir))
    monkeypatch.delenv("SAGE_TILES", raising=False)
    args = argparse.Namespace(frames=200, heads=16, head_dim=64, tiles="base")
    assert bench.gpu_bench(args, torch, S) == 0

    report = json.loads((out_dir / f"bench_d{d}_f{frames}.json").read_text())
    assert set(report["peaks_tops"]) == {"sg_peak_s8", "sg_peak_e4m3_f32", "sg_peak_bf16_f32"}
    runs = report["runs"]
    assert [(r["pv_accum"], r["mode"]) for r in runs] == [
        (pv, m) for pv in ("f32", "f16") for m in ("dense", "merge2", "merge4")]
    for r in runs:
        assert set(r) == KEYS and r["tokens"] == T and r["spill"] == 0, r

    # Each written output equals the library's forward on the same inputs.
    dev = [torch.from_numpy(a.view(np.int16).reshape(1, T, heads, d)).cuda().view(torch.bfloat16) for a in qkv]
    layout = S.FrameLayout(frames, special, gh, gw, 0)
    for pv, suffix in ((S.PvAccum.F32, ""), (S.PvAccum.F16, "_pv16")):
        sa = S.SageAttention(None, d, S.Config(S.Config.for_head_dim(d).tile, pv))
        for mode, merge in (("dense", S.KvMerge.Dense), ("merge2", S.KvMerge.Pool(2, layout)),
                            ("merge4", S.KvMerge.Pool(4, layout))):
            ws = sa.workspace(S.Shape(1, heads, T), merge)
            out = torch.empty((1, T, heads, d), dtype=torch.bfloat16, device="cuda")
            sa.forward(ws, *(S.Tensor(x) for x in dev), S.TensorMut(out))
            torch.cuda.synchronize()
            got = np.fromfile(run / f"out_{mode}{suffix}.bin", dtype="<u2").reshape(1, T, heads, d)
            assert np.array_equal(got, from_device16(out)), (mode, suffix)
