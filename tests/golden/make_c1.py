"""Writes tests/golden/c1.npz, the golden fixture of benchmark configuration C1
(B1 H2 N256 D64 fp16, Q and V ~ N(0,1), K ~ N(0,1) plus a per-channel offset
~ N(0,2); seed 1), the case the reference runs on its CPU path.

The reference holds no golden vectors for this path (its sage tests generate
their data at run time, tests.rs:300-329), and its Rust/NVRTC code cannot run
here, so the expected values come from this repository's CPU oracle: the
splitmix64 + Box-Muller generator (reference.rs:227-254), the prologue's
codes and scales (sage_quant.cu), the quantised attention (sage_attn.cu,
reference logit arithmetic) and the f64 attention (reference.rs:148-184).
The fixture freezes them, so a change to any of those restatements, or to the
HIP path that is checked against it, shows as a difference from committed data.

    python tests/golden/make_c1.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import pyoracle as O  # noqa: E402

OUT = HERE / "c1.npz"


def make() -> dict:
    p, g = O.config(1)
    q, k, v = O.generate(p, g)
    pro = O.prologue(p, q, k, v)
    _, out16 = O.sage_emulate(p, pro, out_dtype=O.F16)
    f64 = O.attention_f64(p, q, k, v)
    return {"q": q, "k": k, "v": v, "q8": pro["q8"], "q_scale": pro["q_scale"], "k8": pro["k8"],
            "k_scale": pro["k_scale"], "v8": pro["v8"], "stats": pro["stats"], "out16": out16,
            "out_f64": f64}


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
