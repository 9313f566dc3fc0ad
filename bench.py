"""Benchmark of the gfx950 SageAttention2 forward path (headline metric:
"attention TOPS @ B2 H32 N4096 D128; % of INT8/FP8 MFMA peak").

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu]

A step is one forward pass of the hot path -- prepare (K smoothing, INT8 Q/K,
FP8 V) then attend (INT8 QK^T, online softmax, FP8 P.V) -- over one batch of
synthetic inputs already resident in HBM. `value` is whole-step throughput in
TOPS (4*B*H*N^2*D algorithmic ops per step, the reference's `flops`,
mod.rs:905-910); `attention` reports the attention kernel alone, like the
reference's attn_tops (tests.rs:968-971). One GPU only. Before the W warm-up
steps, untimed steps bring the warm-up to SETTLE steps in all, so that the
timed steps run at the sustained shader clock (clock_settle_steps).

    python bench.py --vggt [--frames 200] [--merge 1|2|4] [--pv16] [--qk-norm]

prints, instead of the headline line, the reference's own gpu_bench workload
(tests.rs:817-990: VGGT-Omega global attention, B1 H16 D64, 689-token frames)
in the chosen mode. `--qkv` puts the upstream QKV prologue in front of the
chosen configuration and times the reference's two steps against the fused
prepare_qkv. `--only attend|prepare|copy` times one kernel group (for the
profiler).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sota-papers-lab_amd"))

VENDOR_PEAK_TOPS = 5000.0   # MI355X dense INT8 (POPS) and FP8 (PFLOPS) MFMA, x1000
VENDOR_HBM_GBS = 8000.0
SETTLE = 100  # untimed steps before the timed region (the clock ramps over ~60 launches)

# Benchmark configurations C1-C5 as (B, H, HKV, N, D, dtype, causal, k_off_std, outlier_ch, outlier_scale, tok_frac, tok_scale)
CONFIGS = {
    1: (1, 2, 2, 256, 64, "f16", False, 2.0, 0, 1.0, 0.0, 1.0),
    2: (2, 32, 32, 4096, 128, "bf16", False, 2.0, 0, 1.0, 0.0, 1.0),
    3: (1, 32, 32, 16384, 128, "f16", True, 2.0, 4, 20.0, 0.0, 1.0),
    4: (1, 32, 8, 8192, 128, "bf16", True, 2.0, 0, 1.0, 0.0, 1.0),
    5: (1, 48, 48, 17776, 64, "f16", False, 3.0, 0, 1.0, 0.02, 10.0),
}
NAMES = {
    1: "C1 non-causal B1 H2 N256 D64 fp16",
    2: "C2 non-causal B2 H32 N4096 D128 bf16",
    3: "C3 causal B1 H32 N16384 D128 fp16, 4 K outlier channels x20",
    4: "C4 causal GQA B1 Hq32/Hkv8 N8192 D128 bf16",
    5: "C5 non-causal B1 H48 N17776 D64 fp16, 2% tokens x10",
}


def synthetic(torch, cfg: int, seed: int = 0):
    """Q, V ~ N(0,1); K ~ N(0,1) * s + off[h][c] (off ~ N(0, k_off_std)), as the
    configurations describe; generated on the GPU, layout [B][N][H][D]."""
    B, H, HK, N, D, dt, _, koff, och, osc, tfrac, tsc = CONFIGS[cfg]
    g = torch.Generator(device="cuda").manual_seed(seed)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    q = torch.randn((B, N, H, D), generator=g, device="cuda")
    k = torch.randn((B, N, HK, D), generator=g, device="cuda")
    v = torch.randn((B, N, HK, D), generator=g, device="cuda")
    if och:
        scale = torch.ones((HK, D), device="cuda")
        for h in range(HK):
            scale[h, torch.randperm(D, generator=g, device="cuda")[:och]] = osc
        k = k * scale
    k = k + koff * torch.randn((HK, D), generator=g, device="cuda")
    if tfrac:
        t = (torch.rand((B, N, 1, 1), generator=g, device="cuda") < tfrac).float() * (tsc - 1) + 1
        q, k, v = q * t, k * t, v * t
    return q.to(tdt), k.to(tdt), v.to(tdt)


def time_events(torch, stream, fn, reps: int) -> float:
    """Average ms per call of fn over `reps` back-to-back calls, HIP events on `stream`."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def time_median(torch, stream, fn, reps: int):
    """(median, minimum, mean) ms of `reps` individually event-timed calls of fn
    after one untimed call, HIP events on `stream` around each call: the
    reference bench's time_ms (tests.rs:733-748), which reports the median."""
    fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        fn()
        b.record(stream)
    evs[-1][1].synchronize()
    t = sorted(a.elapsed_time(b) for a, b in evs)
    return t[len(t) // 2], t[0], sum(t) / len(t)


def measured_traffic(cfg: int):
    """HBM bytes per attention launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary for this config (copy-calibrated), or None."""
    import re

    f = ROOT / "profiles" / f"sage_attn_c{cfg}_hbm_traffic.md"
    if not f.exists():
        return None
    m = re.search(rf"traffic_bytes_per_launch sage_attn C{cfg} = ([0-9.eE+]+)", f.read_text())
    return (float(m.group(1)), str(f.relative_to(ROOT))) if m else None


def _grow_rows(run, n: int, start: int, budget_s: float):
    """Times run(rows) on linspace row samples of growing size (x2) until one
    takes budget_s or all n rows are in; returns (rows, seconds)."""
    import numpy as np

    r = start
    while True:
        rows = np.unique(np.linspace(0, n - 1, min(r, n)).astype(np.int32))
        t0 = time.perf_counter()
        run(rows)
        dt = time.perf_counter() - t0
        if dt >= budget_s or len(rows) >= n:
            return rows, dt
        r *= 2


def cpu_baseline(q, k, v, cfg: int, budget_s: float = 3.0) -> dict:
    """The reference's CPU path timed on the host cores: its f64 softmax
    attention (reference.rs:148-184, restated in C as oracle_attention_f64)
    over a bounded sample of query rows of every (batch, head), single-threaded
    (as the reference runs it) and on `threads` OpenMP threads (the box's CPU
    share). Reported in TOPS of the sampled work, counted as the metric counts
    it (4 * D per visible (query, key) pair). The oracle's restatement of the
    quantised arithmetic (prologue + sage emulator) is reported beside it."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import pyoracle as O

    B, H, HK, N, D, dt, causal, *_ = CONFIGS[cfg]
    nproc = os.cpu_count() or 1
    threads = min(16, nproc)
    to16 = lambda t: t.cpu().contiguous().view(__import__("torch").int16).numpy().view(np.uint16)
    qh, kh, vh = to16(q), to16(k), to16(v)
    p = O.Problem(B, H, N, D, kv_heads=HK if HK != H else 0, dtype=0 if dt == "bf16" else 1, causal=causal)

    def ops_of(rows):
        keys = (rows.astype(np.float64) + 1).sum() if causal else float(N) * len(rows)
        return 4.0 * B * H * keys * D

    rows_m, t_m = _grow_rows(lambda r: O.attention_f64(p, qh, kh, vh, rows=r, threads=threads), N, 8, budget_s)
    rows_1, t_1 = _grow_rows(lambda r: O.attention_f64(p, qh, kh, vh, rows=r, threads=1), N, 1, budget_s)
    t0 = time.perf_counter()
    pro = O.prologue(p, qh, kh, vh, threads=threads)
    t_pro = time.perf_counter() - t0
    rows_e, t_e = _grow_rows(lambda r: O.sage_emulate(p, pro, rows=r, out_dtype=p.dtype, threads=threads), N, 8,
                             budget_s)
    tops = lambda rows, t: ops_of(rows) / t / 1e12
    return {
        "value": round(tops(rows_m, t_m), 5), "unit": "TOPS", "cores": threads, "kind": "port",
        "nproc": nproc,
        "single_thread": {"value": round(tops(rows_1, t_1), 5), "unit": "TOPS", "threads": 1,
                          "sample": f"{len(rows_1)} query rows x {B * H} (batch, head) in {t_1:.2f} s"},
        "quantised_emulator": {"value": round(tops(rows_e, t_e), 5), "unit": "TOPS", "threads": threads,
                               "sample": f"{len(rows_e)} query rows x {B * H} (batch, head) in {t_e:.2f} s; "
                                         f"its full prologue took {t_pro:.2f} s"},
        "sample": f"the reference's CPU path, f64 softmax attention (reference.rs:148-184, restated in "
                  f"oracle/sage_oracle.c), {len(rows_m)} evenly spaced query rows x {B * H} (batch, head) of the "
                  f"bench workload = {ops_of(rows_m):.3g} ops in {t_m:.2f} s on {threads} OpenMP threads "
                  f"({nproc} cores visible); the time includes decoding K and V to f32",
    }


def vggt_bench(args, torch, S) -> int:
    """The reference's gpu_bench (tests.rs:817-990): VGGT-Omega's global
    attention at 512x336, B1, `heads` heads of `head_dim` (16 and 64 by
    default, SAGE_HEADS / SAGE_D as the reference reads them), `frames` frames
    of 689 tokens (SAGE_FRAMES), dense or KV-merged (stride 2 or 4, every frame
    merged as in vggt_layout), with the PvAccum and QK-norm options. With
    --tiles all (SAGE_TILES=all) it sweeps the reference's tile list under
    both PvAccum modes (tests.rs:896-915); every tile runs the one CDNA4
    kernel here. Prints one JSON line: prologue and attention times, attention
    TOPS over the merged keys (mod.rs:905-910)."""
    B, H, D, frames = 1, args.heads, args.head_dim, args.frames
    layout = S.FrameLayout(frames, 17, 21, 32, 0)
    N = frames * layout.tokens_per_frame()
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn((B, N, H, D), generator=g, device="cuda").to(torch.bfloat16)
    k = (torch.randn((B, N, H, D), generator=g, device="cuda")
         + 2.0 * torch.randn((H, D), generator=g, device="cuda")).to(torch.bfloat16)
    v = torch.randn((B, N, H, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    stream = torch.cuda.current_stream()
    base = S.Config.for_head_dim(D).tile
    tiles = [base]
    if args.tiles == "all":
        for t in (S.Tile(4, 2, 2), S.Tile(4, 2, 4), S.Tile(4, 1, 3), S.Tile(8, 1, 3), S.Tile(8, 1, 4)):
            if t != base and not (D > 64 and t.m_tiles > 1):
                tiles.append(t)
        configs = [S.Config(t, pv) for pv in (S.PvAccum.F32, S.PvAccum.F16) for t in tiles]
    else:
        configs = [S.Config(base, S.PvAccum.F16 if args.pv16 else S.PvAccum.F32)]
    merge = S.KvMerge.Pool(args.merge, layout) if args.merge > 1 else S.KvMerge.Dense
    qk_norm = None
    if args.qk_norm:
        lnp = torch.cat([1 + 0.5 * torch.randn(D, generator=g, device="cuda"), 0.8 * torch.randn(D, generator=g, device="cuda"),
                         1 + 0.5 * torch.randn(D, generator=g, device="cuda"), 0.8 * torch.randn(D, generator=g, device="cuda")])
        qk_norm = S.QkNorm(lnp.float().contiguous(), 1e-5)
    opts = S.Options(qk_norm=qk_norm)
    qt, kt, vt, ot = S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out)
    reps = max(args.steps, 5)
    rows = []
    for cfg in configs:
        sa = S.SageAttention(stream, D, cfg)
        ws = sa.workspace(S.Shape(B, H, N), merge)
        plan = ws.plan()
        ops = S.flops(plan, D)
        sa.prepare(ws, qt, kt, vt, opts)
        for _ in range(args.warmup):
            sa.attend(ws, ot)
        torch.cuda.synchronize()
        attn_ms = time_events(torch, stream, lambda: sa.attend(ws, ot), reps)
        prep_ms = time_events(torch, stream, lambda: sa.prepare(ws, qt, kt, vt, opts), reps)
        step_ms = time_events(torch, stream, lambda: sa.forward(ws, qt, kt, vt, ot, opts), reps)
        attn_tops = ops / (attn_ms * 1e-3) / 1e12
        t = cfg.tile
        rows.append({"tile": f"{t.warps}w{t.m_tiles}m{t.stages}s", "pv_accum": cfg.pv_accum.name,
                     "prologue_ms": round(prep_ms, 4), "attention_ms": round(attn_ms, 4),
                     "attention_tops": round(attn_tops, 1),
                     "attention_frac_of_peak": round(attn_tops / VENDOR_PEAK_TOPS, 4), "step_ms": round(step_ms, 4),
                     "step_tops": round(ops / (step_ms * 1e-3) / 1e12, 1)})
        del ws
    regs, spill = sa.attn_resources()
    mode = ("dense" if args.merge == 1 else f"merge{args.merge}") + ("_pv16" if args.pv16 else "") + \
        ("_qknorm" if args.qk_norm else "")
    line = {"workload": "VGGT-Omega global attention (reference gpu_bench)", "mode": mode, "frames": frames,
            "heads": H, "head_dim": D, "tokens": N, "keys": plan.tk}
    if args.tiles == "all":
        line["mode"] = mode.replace("_pv16", "")
        line["configs"] = rows
    else:
        line.update({k: v for k, v in rows[0].items() if k not in ("tile", "pv_accum")})
    line.update({"vgprs_dense_kernel": regs, "spill": spill})
    print(json.dumps(line), flush=True)
    return 0


def _time_ms(torch, stream, fn, reps: int):
    """time_ms (tests.rs:733-748): one warm-up call, then (median, best) of
    `reps` individually event-timed calls."""
    fn()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        fn()
        b.record(stream)
    evs[-1][1].synchronize()
    t = sorted(a.elapsed_time(b) for a, b in evs)
    return t[len(t) // 2], t[0]


def gpu_bench(args, torch, S) -> int:
    """The reference's gpu_bench (tests.rs:817-1022) with its file protocol, so
    its torch_ref.py gen / compare run around this library unchanged: with
    SAGE_RUN=DIR it reads DIR/meta.txt (frames, heads, head_dim, special,
    grid_h, grid_w) and bf16 [T][H][D] q.bin, k.bin, v.bin, and writes
    out_<mode>.bin (out_<mode>_pv16.bin for PvAccum::F16) of the base tile
    there; otherwise it times random inputs of SAGE_FRAMES VGGT frames,
    SAGE_HEADS heads of SAGE_D. Every config (the base tile, or the
    reference's list with SAGE_TILES=all, under both PvAccum modes) runs
    dense, merge2 and merge4, one JSON line each with the reference's keys;
    the lines and the MFMA peaks go to $SAGE_OUT/bench_d<D>_f<frames>.json.
    SAGE_VARIANTS (NVRTC defines of the reference's CUDA source) has no
    counterpart: the kernels here are compiled ahead of time."""
    import numpy as np

    run_dir = os.environ.get("SAGE_RUN")
    if run_dir:
        meta = {}
        with open(os.path.join(run_dir, "meta.txt")) as f:
            for ln in f:
                if "=" in ln:
                    k_, v_ = ln.split("=", 1)
                    meta[k_.strip()] = v_.strip()
        layout = S.FrameLayout(int(meta["frames"]), int(meta["special"]), int(meta["grid_h"]), int(meta["grid_w"]), 0)
        heads, d = int(meta["heads"]), int(meta["head_dim"])
    else:
        layout = S.FrameLayout(args.frames, 17, 21, 32, 0)
        heads, d = args.heads, args.head_dim
    frames = layout.frames
    T = frames * layout.tokens_per_frame()
    n = T * heads * d
    shape = S.Shape(1, heads, T)
    t0 = time.perf_counter()
    if run_dir:
        def load(name):
            raw = np.fromfile(os.path.join(run_dir, name), dtype="<u2")
            if raw.size < n:
                raise SystemExit(f"{name}: input files too small ({raw.size} < {n} elements)")
            return torch.from_numpy(raw[:n].view(np.int16).reshape(T, heads, d)).cuda().view(torch.bfloat16)
        q, k, v = load("q.bin"), load("k.bin"), load("v.bin")
    else:
        # Timing does not depend on the values (tests.rs:875-880).
        g = torch.Generator(device="cuda").manual_seed(1)
        q, k, v = ((torch.randn((T, heads, d), generator=g, device="cuda") * 1.5).to(torch.bfloat16) for _ in range(3))
    q, k, v = (x.unsqueeze(0) for x in (q, k, v))
    print(f"inputs ready in {time.perf_counter() - t0:.1f} s", flush=True)
    stream = torch.cuda.current_stream()
    probe = S.SageAttention(stream, d)
    peaks = {}
    for name, which in (("sg_peak_s8", 0), ("sg_peak_e4m3_f32", 1), ("sg_peak_bf16_f32", 2)):
        peaks[name] = probe.peak(which)
        print(f"peak {name}: {peaks[name]:.1f} TOPS", flush=True)
    base = S.Config.for_head_dim(d).tile
    tiles = [base]
    if os.environ.get("SAGE_TILES") == "all" or args.tiles == "all":
        for t in (S.Tile(4, 2, 2), S.Tile(4, 2, 4), S.Tile(4, 1, 3), S.Tile(8, 1, 3), S.Tile(8, 1, 4)):
            if t != base and not (d > 64 and t.m_tiles > 1):
                tiles.append(t)
    if os.environ.get("SAGE_VARIANTS"):
        print("SAGE_VARIANTS: kernel-source defines do not apply to this build; each config runs once", flush=True)
    out = torch.zeros((1, T, heads, d), dtype=torch.bfloat16, device="cuda")
    qt, kt, vt, ot = S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out)
    dense_plan = S.Plan.new(shape, S.KvMerge.Dense)
    lines = []
    for pv in (S.PvAccum.F32, S.PvAccum.F16):
        for tile in tiles:
            sa = S.SageAttention(stream, d, S.Config(tile, pv))
            regs, spill = sa.attn_resources()
            for mode, merge in (("dense", S.KvMerge.Dense), ("merge2", S.KvMerge.Pool(2, layout)),
                                ("merge4", S.KvMerge.Pool(4, layout))):
                ws = sa.workspace(shape, merge)
                opts = S.Options()
                prep = lambda: sa.prepare(ws, qt, kt, vt, opts)
                prep_ms, _ = _time_ms(torch, stream, prep, 5)
                attn_ms, attn_best = _time_ms(torch, stream, lambda: sa.attend(ws, ot), 3 if mode == "dense" else 5)
                plan = ws.plan()
                tops = S.flops(plan, d) / (attn_ms * 1e-3) / 1e12
                dense_tops = S.flops(dense_plan, d) / ((attn_ms + prep_ms) * 1e-3) / 1e12
                line = {"tile": f"{tile.warps}w{tile.m_tiles}m{tile.stages}s", "variant": "",
                        "pv_accum": "f32" if pv == S.PvAccum.F32 else "f16", "regs": regs, "spill": spill,
                        "mode": mode, "frames": frames, "heads": heads, "head_dim": d, "tokens": T, "keys": plan.tk,
                        "prep_ms": round(prep_ms, 3), "attn_ms": round(attn_ms, 3), "attn_best_ms": round(attn_best, 3),
                        "attn_tops": round(tops, 1), "dense_equiv_tops": round(dense_tops, 1),
                        "workspace_mb": round(ws.bytes() / 1e6, 1)}
                print(json.dumps(line), flush=True)
                lines.append(line)
                if run_dir and tile == base:
                    prep()
                    sa.attend(ws, ot)
                    torch.cuda.synchronize()
                    suffix = "_pv16" if pv == S.PvAccum.F16 else ""
                    out.view(torch.int16).cpu().numpy().astype("<i2").tofile(
                        os.path.join(run_dir, f"out_{mode}{suffix}.bin"))
                del ws
    out_dir = os.environ.get("SAGE_OUT", "/out/sage")
    os.makedirs(out_dir, exist_ok=True)
    path = os.path.join(out_dir, f"bench_d{d}_f{frames}.json")
    with open(path, "w") as f:
        f.write(json.dumps({"peaks_tops": {k_: round(v_, 1) for k_, v_ in peaks.items()}, "runs": lines}) + "\n")
    print(f"wrote {path}", flush=True)
    return 0


def qkv_bench(args, torch, S) -> int:
    """The upstream QKV prologue (qkv.rs, qkv.cu) in front of the chosen
    configuration: the fused projection y (bf16 [B][N][(H + 2 HKV) * D]) with
    per-channel scales and bias, LayerNorm QK-norm and 2D RoPE (VGGT layout
    over a 64-column patch grid). Times, per step, the two-step path the
    reference runs -- QkvPrologue::run writing bf16 Q, K and V, then prepare
    and attend -- against the fused prepare_qkv + attend, which never writes
    or re-reads Q, K and V in bf16. Prints one JSON line."""
    from spl_sage import qkv as Q

    merge = S.KvMerge.Dense
    if args.vggt:
        # The reference caller's layer (vggt/trunk): `frames` frames of 17 special
        # tokens and a 21 x 32 patch grid, 16 heads of 64, the frame-relative VGGT
        # RoPE table, dense or KV-merged keys.
        layout = S.FrameLayout(args.frames, 17, 21, 32, 0)
        B, H, HK, N, D, causal = 1, args.heads, args.heads, args.frames * layout.tokens_per_frame(), args.head_dim, False
        if args.merge > 1:
            merge = S.KvMerge.Pool(args.merge, layout)
        name = (f"VGGT {args.frames} frames H{H} D{D} bf16" + ("" if args.merge == 1 else f" merge{args.merge}"))
    else:
        B, H, HK, N, D, dt, causal, *_ = CONFIGS[args.config]
        name = NAMES[args.config]
    g = torch.Generator(device="cuda").manual_seed(0)
    width = (H + 2 * HK) * D
    y = (torch.randn((B, N, width), generator=g, device="cuda")
         + 0.5 * torch.randn((width,), generator=g, device="cuda")).to(torch.bfloat16)
    chan = (0.5 + torch.rand((width,), generator=g, device="cuda")).float()
    bias = (0.2 * torch.randn((width,), generator=g, device="cuda")).to(torch.bfloat16)
    nw = [(1 + 0.2 * torch.randn((D,), generator=g, device="cuda")).float(),
          (0.1 * torch.randn((D,), generator=g, device="cuda")).float(),
          (1 + 0.2 * torch.randn((D,), generator=g, device="cuda")).float(),
          (0.1 * torch.randn((D,), generator=g, device="cuda")).float()]
    if args.vggt:
        table = Q.RopeTable.vggt(21, 32, 17, 100.0, D)
    else:
        gw = 64
        table = Q.RopeTable.vggt((N + gw - 1) // gw, gw, 0, 100.0, D)
    rope = Q.Rope(table.upload(), Q.RopeLayout.Vggt, table.frame_len)
    norm = Q.QkNorm(Q.NormKind.LayerNorm, nw[0], nw[2], nw[1], nw[3], 1e-6)
    inp = Q.QkvIn(y, width, chan=chan, bias=bias)
    stream = torch.cuda.current_stream()
    sa = S.SageAttention(stream, D)
    ws = sa.workspace(S.Shape(B, H, N, HK if HK != H else 0), merge)
    out = torch.empty((B, N, H, D), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((B, N, H, D), dtype=torch.bfloat16, device="cuda")
    k = torch.empty((B, N, HK, D), dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    pro = Q.QkvPrologue(sa)
    qo = Q.QkvOut(S.TensorMut(q), S.TensorMut(k), S.TensorMut(v))
    opts = S.Options(causal=causal)
    ot = S.TensorMut(out)

    def qkv_only():
        pro.run(inp, N, H, norm, rope, qo, batch=B, kv_heads=HK if HK != H else 0)

    def two_step():
        qkv_only()
        sa.forward(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), ot, opts)

    def fused():
        sa.forward_qkv(ws, inp, ot, norm, rope, opts)

    def prepare_fused():
        sa.prepare_qkv(ws, inp, norm, rope, opts)

    def prepare_plain():
        sa.prepare(ws, S.Tensor(q), S.Tensor(k), S.Tensor(v), opts)

    for _ in range(args.warmup):
        two_step()
        fused()
    torch.cuda.synchronize()
    reps = max(args.steps, 20)
    t2 = time_median(torch, stream, two_step, reps)[0]
    t1 = time_median(torch, stream, fused, reps)[0]
    tq = time_median(torch, stream, qkv_only, reps)[0]
    tpf = time_median(torch, stream, prepare_fused, reps)[0]
    tpp = time_median(torch, stream, prepare_plain, reps)[0]
    ops = S.flops(ws.plan(), D, causal)
    y_bytes = B * N * width * 2
    print(json.dumps({
        "workload": f"QKV prologue + sage, {name} (LayerNorm QK-norm, VGGT RoPE, channel scales, bias)",
        "two_step_ms": round(t2, 4), "fused_ms": round(t1, 4), "speedup": round(t2 / t1, 3),
        "qkv_prologue_ms": round(tq, 4), "prepare_from_bf16_ms": round(tpp, 4), "prepare_qkv_ms": round(tpf, 4),
        "qkv_prologue_gbs": round(2 * y_bytes / (tq * 1e-3) / 1e9, 1),
        "bf16_round_trip_bytes": 2 * y_bytes,
        "two_step_tops": round(ops / (t2 * 1e-3) / 1e12, 1), "fused_tops": round(ops / (t1 * 1e-3) / 1e12, 1),
        "timing": "median of individually event-timed calls",
    }), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # ~100 warm-up steps: the GPU clock ramps over the first ~60 attention launches
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-peak", action="store_true", help="skip the MFMA peak probes")
    ap.add_argument("--tile", default=None,
                    help="WARPS,M_TILES,STAGES: the reference's Tile for the context (default Config::for_head_dim); "
                         "warps 8 selects the eight-wave attention layout")
    ap.add_argument("--vggt", action="store_true",
                    help="instead of the headline line: the reference's gpu_bench workload (tests.rs:817-990), "
                         "VGGT-Omega global attention, 689-token frames (17 special + 21x32 patches), by default 16 heads of 64")
    ap.add_argument("--frames", type=int, default=int(os.environ.get("SAGE_FRAMES", 200)),
                    help="--vggt: frames (200 = 137800 tokens; default $SAGE_FRAMES or 200)")
    ap.add_argument("--heads", type=int, default=int(os.environ.get("SAGE_HEADS", 16)),
                    help="--vggt: heads (default $SAGE_HEADS or 16)")
    ap.add_argument("--head-dim", type=int, default=int(os.environ.get("SAGE_D", 64)), choices=[64, 128],
                    help="--vggt: head dim (default $SAGE_D or 64)")
    ap.add_argument("--tiles", choices=["base", "all"], default="all" if os.environ.get("SAGE_TILES") == "all" else "base",
                    help="--vggt: 'all' sweeps the reference's tile list under both PvAccum modes (SAGE_TILES=all)")
    ap.add_argument("--merge", type=int, default=1, choices=[1, 2, 4], help="--vggt: KV merge stride (1 = dense)")
    ap.add_argument("--pv16", action="store_true", help="--vggt: PvAccum::F16")
    ap.add_argument("--qk-norm", action="store_true", help="--vggt: fused QK LayerNorm")
    ap.add_argument("--gpu-bench", action="store_true",
                    help="the reference's gpu_bench with its file protocol (SAGE_RUN, SAGE_OUT, SAGE_FRAMES, "
                         "SAGE_HEADS, SAGE_D, SAGE_TILES): dense, merge2 and merge4 for every config")
    ap.add_argument("--qkv", action="store_true",
                    help="instead of the headline line: the upstream QKV prologue in front of --config (or, with "
                         "--vggt, of the VGGT layer: --frames, --heads, --head-dim, --merge), the reference's two "
                         "steps against the fused prepare_qkv")
    ap.add_argument("--only", choices=["attend", "prepare", "copy"],
                    help="profiling mode: run only this kernel group --steps times and print its timing "
                         "(copy: a plain 512 MiB device copy, the reference for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import spl_sage as S

    torch.cuda.set_device(0)
    if args.qkv:
        return qkv_bench(args, torch, S)
    if args.vggt:
        return vggt_bench(args, torch, S)
    if args.gpu_bench:
        return gpu_bench(args, torch, S)
    if args.only == "copy":
        n = 512 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        stream = torch.cuda.current_stream()
        for _ in range(args.warmup):
            dst.copy_(src)
        ms = time_events(torch, stream, lambda: dst.copy_(src), args.steps)
        print(json.dumps({"only": "copy", "bytes_read": n, "bytes_written": n, "ms": round(ms, 4),
                          "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    B, H, HK, N, D, dt, causal, *_ = CONFIGS[args.config]
    q, k, v = synthetic(torch, args.config)
    out = torch.empty((B, N, H, D), dtype=q.dtype, device="cuda")
    stream = torch.cuda.current_stream()
    config = None
    if args.tile:
        config = S.Config(S.Tile(*(int(x) for x in args.tile.split(","))), S.PvAccum.F32)
    sa = S.SageAttention(stream, D, config)
    shape = S.Shape(B, H, N, HK if HK != H else 0)
    ws = sa.workspace(shape)
    opts = S.Options(causal=causal)
    qt, kt, vt, ot = S.Tensor(q), S.Tensor(k), S.Tensor(v), S.TensorMut(out)
    plan = ws.plan()
    ops = S.flops(plan, D, causal)

    def step():
        sa.prepare(ws, qt, kt, vt, opts)
        sa.attend(ws, ot)

    if args.only:
        fn = (lambda: sa.attend(ws, ot)) if args.only == "attend" else (lambda: sa.prepare(ws, qt, kt, vt, opts))
        sa.prepare(ws, qt, kt, vt, opts)
        for _ in range(args.warmup):
            fn()
        ms = time_events(torch, stream, fn, args.steps)
        print(json.dumps({"only": args.only, "config": NAMES[args.config], "ms": round(ms, 4),
                          "tops": round(ops / (ms * 1e-3) / 1e12, 2) if args.only == "attend" else None}), flush=True)
        return 0

    # The shader clock ramps over the first ~60 attention launches of a
    # process. Untimed steps before the W warm-up steps bring it to its
    # sustained rate, so that the K timed steps measure that rate whatever W
    # is: SETTLE steps before the timed region in all (reported as
    # clock_settle_steps; none when W >= SETTLE).
    pre = max(0, SETTLE - args.warmup)
    for _ in range(pre):
        step()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_ev = time_events(torch, stream, step, args.steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_per_step = max(ms_ev, wall_ms)

    # Per-kernel: the attention kernel alone and the prologue alone, the median
    # of individually event-timed launches (tests.rs:733-748), after the
    # settled steps above.
    settle = pre + args.warmup + args.steps
    attn_reps = max(args.steps, 20)
    attn_ms, attn_min, attn_mean = time_median(torch, stream, lambda: sa.attend(ws, ot), attn_reps)
    prep_ms, prep_min, prep_mean = time_median(torch, stream, lambda: sa.prepare(ws, qt, kt, vt, opts), attn_reps)
    torch.cuda.synchronize()

    attn_tops = ops / (attn_ms * 1e-3) / 1e12
    value = ops / (ms_per_step * 1e-3) / 1e12
    regs, spill = sa.attn_resources()
    peaks = {}
    if not args.no_peak:
        peaks = {"int8_32x32x32": round(sa.peak(0), 1), "fp8_32x32x64": round(sa.peak(1), 1),
                 "bf16_32x32x16": round(sa.peak(2), 1)}
    # Prologue algorithmic bytes: read Q, K, V (2 B/elem), write q8, k8, v8 (1 B/elem) + scales/stats.
    n_q, n_kv = B * H * N * D, B * HK * N * D
    pro_bytes = 2 * (n_q + 2 * n_kv) + (n_q + 2 * n_kv) + 4 * (B * H * plan.tq_pad // 16 + B * HK * plan.tk_pad // 64
                                                               + B * HK * 4 * D)
    traffic = measured_traffic(args.config)
    line = {
        "metric": "attention TOPS @ B2 H32 N4096 D128; % of INT8/FP8 MFMA peak",
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle_steps": pre,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 QK^T (i32 acc) + e4m3 PV (f32 acc)",
        "data": "synthetic (torch.randn on the GPU; K offset per (head, channel) as the config states)",
        "config": {"workload": NAMES[args.config], "batch": B, "heads": H, "kv_heads": HK, "tokens": N,
                   "head_dim": D, "causal": causal, "inputs": dt,
                   "tile": "{}w{}m{}s".format(*(lambda t: (t.warps, t.m_tiles, t.stages))(sa.config().tile))},
        "frac_of_peak": round(value / VENDOR_PEAK_TOPS, 4),
        "attention": {"ms": round(attn_ms, 4), "ms_min": round(attn_min, 4), "ms_mean": round(attn_mean, 4),
                      "reps": attn_reps, "settle_launches": settle,
                      "timing": "median of individually event-timed launches",
                      "tops": round(attn_tops, 2), "frac_of_peak": round(attn_tops / VENDOR_PEAK_TOPS, 4),
                      "vgprs": regs, "spill": spill},
        "prologue": {"ms": round(prep_ms, 4), "ms_min": round(prep_min, 4), "ms_mean": round(prep_mean, 4),
                     "gbs": round(pro_bytes / (prep_ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm": round(pro_bytes / (prep_ms * 1e-3) / 1e9 / VENDOR_HBM_GBS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(attn_tops, 2), "peak": VENDOR_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(attn_tops / VENDOR_PEAK_TOPS, 4),
                     "traffic": traffic[0] if traffic else None},
        "peaks_measured_tops": peaks,
        # roofline.traffic is not measured by this run: it is the HBM bytes per
        # attention launch of the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
        # summary named here (copy-calibrated), null when none covers the config.
        "traffic_source": (f"committed rocprofv3 summary {traffic[1]} (not measured in this run)"
                           if traffic else None),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(q, k, v, args.config)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
