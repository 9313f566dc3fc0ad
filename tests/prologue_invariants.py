"""The reference's prologue checks (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/sage/tests.rs:476-594, check_prologue), as tolerance
invariants over logical-layout buffers: Q scale within 1e-4 of amax/127*q_mul
and every Q code within half a step; K mean within 1e-3 of the f64 mean; K
scale within 1e-4 of amax/127 and every K code within half a step; V
de-quantised within |v - mean|/16 + scale * 2^-8. With KV merging the keys are
the reference's pooled K and V (reference.rs:113-143: f32 sums in member order,
then / n) and every kbias entry is log2(n) within 1e-6, -inf past the keys.
Under QK LayerNorm the Q and K rows are first normalised by the reference's f64
layer_norm (reference.rs:109-118), as tests.rs:448-466 (reference_head) does."""
from __future__ import annotations

import numpy as np


def pool_kv(p, kk: np.ndarray, vv: np.ndarray):
    """reference.rs:113-143 for one (batch, head): [T,D] -> pooled [tk,D] K and V, member counts."""
    tk = p.tk
    km = np.zeros((tk, kk.shape[1]), np.float32)
    vm = np.zeros_like(km)
    n = np.zeros(tk, np.int64)
    for j in range(tk):
        mem = p.members(j)
        for t in mem:
            km[j] += kk[t]
            vm[j] += vv[t]
        km[j] /= np.float32(len(mem))
        vm[j] /= np.float32(len(mem))
        n[j] = len(mem)
    return km, vm, n


def layer_norm_rows(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """reference.rs:109-118 over the last axis: f64 mean and biased variance,
    1 / sqrt(var + eps), the affine map in f64, rounded to f32."""
    x64 = x.astype(np.float64)
    mean = x64.mean(axis=-1, keepdims=True)
    var = ((x64 - mean) ** 2).mean(axis=-1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + np.float64(np.float32(eps)))
    return ((x64 - mean) * rstd * w.astype(np.float64) + b.astype(np.float64)).astype(np.float32)


def check_prologue(p, qf: np.ndarray, kf: np.ndarray, vf: np.ndarray, pro: dict, smooth: bool = True) -> None:
    """qf, kf, vf: decoded inputs [B,T,H,D] / [B,T,HKV,D] float32."""
    B, T, H, HK, D = p.batch, p.tokens, p.heads, p.hk, p.head_dim
    if p.ln is not None:
        ln = p.ln.reshape(-1)[: 4 * D].reshape(4, D)
        qf = layer_norm_rows(qf, ln[0], ln[1], p.ln_eps)
        kf = layer_norm_rows(kf, ln[2], ln[3], p.ln_eps)
    TK = p.tk
    qmul = np.float32(np.float32(1.4426950408889634) / np.sqrt(np.float32(D))) if p.softmax_scale is None \
        else np.float32(np.float32(p.softmax_scale) * np.float32(1.4426950408889634))
    tq, tk = p.tq_pad, p.tk_pad
    for b in range(B):
        for h in range(H):
            q = np.zeros((tq, D), np.float32)
            q[:T] = qf[b, :, h]
            g = q.reshape(tq // 16, 16, D)
            amax = np.abs(g).max(axis=(1, 2))
            got = pro["q_scale"][b, h]
            want = (amax / np.float32(127.0) * qmul).astype(np.float32)
            assert np.all(np.abs(got - want) <= 1e-4 * np.abs(want) + 1e-30), "q scale"
            step = (amax / np.float32(127.0))[:, None, None]
            qv = pro["q8"][b, h].astype(np.float32).reshape(g.shape) * step
            assert np.all(np.abs(qv - g) <= 0.5 * step * 1.01 + 1e-3 * step), "q codes"
        for h in range(HK):
            st = pro["stats"][b, h]
            kk = kf[b, :, h]
            if smooth:
                m = kk.astype(np.float64).mean(axis=0)
                assert np.all(np.abs(st[0].astype(np.float64) - m) < 1e-3 * (1.0 + np.abs(m))), "k mean"
            else:
                assert np.all(st[:2] == 0.0), "means must be 0 without smoothing"
            km, vm, _ = pool_kv(p, kk, vf[b, :, h]) if p.merge > 1 else (kk, vf[b, :, h], None)
            ks = np.zeros((tk, D), np.float32)
            ks[:TK] = km - st[0]
            blocks = ks.reshape(tk // 64, 64, D)
            amax = np.abs(blocks).max(axis=(1, 2))
            got = pro["k_scale"][b, h]
            assert np.all(np.abs(got - amax / 127.0) <= 1e-4 * amax / 127.0 + 1e-30), "k scale"
            kq = pro["k8"][b, h].astype(np.float32).reshape(blocks.shape) * got[:, None, None]
            assert np.all(np.abs(kq - blocks) <= 0.5 * got[:, None, None] * 1.01 + 1e-4 * amax[:, None, None]), \
                "k codes"
            from oracle import pyoracle

            vdq = pyoracle.e4m3_decode(pro["v8"][b, h, :TK]) * st[2] + st[1]
            want = vm
            tol = np.abs(want - st[1]) / 16.0 + st[2] * 2.0 ** -8
            assert np.all(np.abs(vdq - want) <= tol * 1.01), "v codes"
            assert np.all(pro["v8"][b, h, TK:] == 0) and np.all(pro["k8"][b, h, TK:] == 0), "padding keys"
        for h in range(H):
            assert np.all(pro["q8"][b, h, T:] == 0), "padding queries"
    if p.merge > 1:
        kb = pro["kbias"]
        for j in range(tk):
            if j < TK:
                want = np.log2(np.float32(len(p.members(j))))
                assert abs(float(kb[j]) - float(want)) <= 1e-6, ("bias", j, kb[j], want)
            else:
                assert kb[j] == -np.inf, ("padding bias", j)
