"""The QKV prologue on the GPU (sezer-muhammed/sota-papers-lab,
platform/spl-nn/src/qkv.rs, cuda/qkv.cu), through the C ABI:

- QkvPrologue::run (sage_qkv_prologue) against the oracle's restatement of
  the kernel's fp32 arithmetic, bit for bit (bf16 Q and K, bf16 or fp16 V),
  on the reference test's VGGT layout (689-token frames, tests.rs:447-570)
  and its four option sets, plus head dim 128, grouped heads, batch 2 and the
  reference's head-major output;
- the fused sage_prepare_qkv: the workspace's codes and scales equal the
  oracle prologue of the oracle QKV prologue's bf16 Q, K and V bit for bit,
  and the attention output equals the unfused GPU path (sage_qkv_prologue,
  then prepare and attend) bit for bit, and meets the north-star gate;
- RoPE rows t % frame_len at frame lengths 1, 38, 64 and 4096, both paths;
- seeded random fused problems (every option drawn together), bit for bit
  against the oracle and the two GPU steps;
- the reference's refusals, before any launch."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_device16
from sage_gpu_helpers import assert_prologue_equal, gather_rows, read_workspace, run, sample_rows

pytestmark = pytest.mark.gpu

GRID_H, GRID_W, SPECIAL = 21, 32, 17
FRAME = SPECIAL + GRID_H * GRID_W  # 689


def _spec(O, rng, D, heads, kv, batch, tokens, norm, rope, scaled, ld_pad=8, grid=(GRID_H, GRID_W, SPECIAL)):
    s = O.QkvSpec(batch, tokens, heads, D, kv_heads=kv)
    s.ld = s.width + ld_pad
    if scaled:
        s.tok = (0.5 + rng.random(batch * tokens)).astype(np.float32)
        s.chan = (0.5 + rng.random(s.width)).astype(np.float32)
    s.bias = O.encode16((0.2 * rng.standard_normal(s.width)).astype(np.float32), 0)
    if norm:
        s.norm = norm
        s.norm_w = np.stack([1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
                             1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)]).astype(np.float32)
    if rope is not None:
        s.rope = O.rope_table(rope, D, grid[0], grid[1], grid[2], 100.0)
        s.rope_layout = rope
    y = rng.standard_normal((batch, tokens, s.ld), dtype=np.float32)
    y[..., :s.width] += 0.5 * rng.standard_normal(s.width, dtype=np.float32)  # per-channel offsets
    return s, O.encode16(y, 0)


def _device(torch, s, y):
    """(QkvIn, QkNorm or None, Rope or None) on the GPU."""
    from spl_sage import qkv as Q

    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    inp = Q.QkvIn(bf(y), s.ld, tok=None if s.tok is None else f32(s.tok), chan=None if s.chan is None else f32(s.chan),
                  bias=None if s.bias is None else bf(s.bias), batch_stride=s.tokens * s.ld)
    norm = None
    if s.norm:
        w = [f32(s.norm_w[i]) for i in range(4)]
        norm = Q.QkNorm(Q.NormKind(s.norm), w[0], w[2], w[1], w[3], float(s.eps))
    rope = None
    if s.rope is not None:
        rope = Q.Rope(f32(s.rope.reshape(-1)), Q.RopeLayout(s.rope_layout), s.rope.shape[0])
    return inp, norm, rope


STANDALONE = [  # (D, heads, kv, batch, frames, norm, rope, scaled, head_major)
    (64, 16, 0, 1, 2, 1, 0, False, True),   # tests.rs:457-462, as the reference runs them
    (64, 16, 0, 1, 2, 2, 1, True, True),
    (64, 6, 0, 1, 2, 0, 0, True, True),
    (64, 3, 0, 1, 2, 1, None, False, True),
    (128, 8, 2, 2, 1, 1, 0, True, False),   # extensions
    (128, 4, 0, 1, 1, 2, 1, False, False),
]


@pytest.mark.parametrize("case", range(len(STANDALONE)))
def test_standalone_prologue_is_bit_exact(oracle, torch_gpu, case):
    import spl_sage as S
    from spl_sage import qkv as Q

    torch = torch_gpu
    D, H, kv, B, frames, norm, rope, scaled, head_major = STANDALONE[case]
    HK = kv or H
    T = frames * FRAME
    rng = np.random.default_rng(100 + case)
    s, y = _spec(oracle, rng, D, H, kv, B, T, norm, rope, scaled)
    print(f"case {case}: D{D} H{H}/{HK} B{B} T{T} norm {norm} rope {rope} scaled {scaled}", flush=True)
    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, D)
    for v_f16 in (False, True):
        def buf(h, dt):
            if head_major:
                t = torch.empty((B, h, T, D), dtype=dt, device="cuda")
                return t, S.TensorMut(t, S.Strides.bhtd(T, h, D))
            t = torch.empty((B, T, h, D), dtype=dt, device="cuda")
            return t, S.TensorMut(t)
        (q, qm), (k, km), (v, vm) = buf(H, torch.bfloat16), buf(HK, torch.bfloat16), \
            buf(HK, torch.float16 if v_f16 else torch.bfloat16)
        Q.QkvPrologue(sa).run(inp, T, H, qn, rp, Q.QkvOut(qm, km, vm), batch=B, kv_heads=kv)
        torch.cuda.synchronize()
        s.v_f16 = v_f16
        want = oracle.qkv_prologue(s, y)
        for name, got, w in zip("qkv", (q, k, v), want):
            g = from_device16(got)
            if head_major:
                g = np.ascontiguousarray(g.transpose(0, 2, 1, 3))
            assert np.array_equal(g, w), (name, v_f16, int((g != w).sum()))


FUSED = [  # (D, heads, kv, batch, tokens, norm, rope, scaled, causal, merge, sage_ln)
    (64, 16, 0, 1, 2 * FRAME, 1, 0, True, False, 1, False),
    (64, 16, 0, 1, 2 * FRAME, 2, 1, False, False, 4, False),
    (128, 8, 2, 2, 1000, 1, 0, True, True, 1, False),
    (128, 4, 0, 1, 777, 2, 1, False, False, 1, False),
    (128, 4, 4, 1, 300, 0, None, True, False, 1, False),
    # the sage options' QkNorm on top of the QKV prologue's output (the LN and
    # QKV instantiations together), dense and merged at both head dims
    (64, 8, 0, 1, 2 * FRAME, 1, 0, True, False, 1, True),
    (64, 8, 0, 1, 2 * FRAME, 2, 1, False, False, 4, True),
    (128, 8, 2, 2, 1000, 1, 0, True, True, 1, True),
    (128, 4, 0, 1, 2 * FRAME, 0, 0, True, False, 2, True),
]


@pytest.mark.parametrize("case", range(len(FUSED)))
def test_fused_prepare_equals_the_two_steps(oracle, torch_gpu, case):
    import spl_sage as S
    from spl_sage import qkv as Q

    torch = torch_gpu
    D, H, kv, B, T, norm, rope, scaled, causal, merge, sage_ln = FUSED[case]
    HK = kv or H
    rng = np.random.default_rng(200 + case)
    s, y = _spec(oracle, rng, D, H, kv, B, T, norm, rope, scaled)
    print(f"case {case}: D{D} H{H}/{HK} B{B} T{T} norm {norm} rope {rope} scaled {scaled} causal {causal} "
          f"merge {merge} sage QkNorm {sage_ln}", flush=True)
    layout = (T // FRAME, SPECIAL, GRID_H, GRID_W, 0) if merge > 1 else (1, 0, 0, 0, 0)
    ln = None
    if sage_ln:
        ln = np.concatenate([1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
                             1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)]).astype(np.float32)
    p = oracle.Problem(B, H, T, D, kv_heads=kv, dtype=0, causal=causal, merge=merge, layout=layout, ln=ln,
                       ln_eps=1e-6)
    q16, k16, v16 = oracle.qkv_prologue(s, y)
    want = oracle.prologue(p, q16, k16, v16)

    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, D)
    km = S.KvMerge.Pool(merge, S.FrameLayout(*layout)) if merge > 1 else S.KvMerge.Dense
    ws = sa.workspace(S.Shape(B, H, T, kv), km)
    out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device="cuda")
    qk_norm = S.QkNorm(torch.from_numpy(ln.copy()).to("cuda"), 1e-6) if sage_ln else None
    sa.forward_qkv(ws, inp, S.TensorMut(out), qn, rp, S.Options(causal=causal, qk_norm=qk_norm))
    torch.cuda.synchronize()
    assert_prologue_equal(read_workspace(ws, p), want)
    o_fused = from_device16(out)

    # the two steps on the GPU: QkvPrologue::run into bf16 Q, K, V, then forward
    _, o_two = run(torch, p, q16, k16, v16, want_ws=False)
    assert np.array_equal(o_fused, o_two)

    rows = sample_rows(T, 256, seed=case)
    _, emu16 = oracle.sage_emulate(p, want, rows=rows, out_dtype=0)
    e = oracle.errors(oracle.decode16(gather_rows(o_fused, rows), 0), oracle.decode16(emu16, 0))
    print(f"vs reference arithmetic: {e}")
    assert e["cos"] >= 0.999 and e["max_abs"] <= 2e-2, e


ROPE_FRAMES = [(1, 1, 0), (5, 7, 3), (8, 8, 0), (64, 64, 0)]  # (grid_h, grid_w, special): frame_len 1, 38, 64, 4096


@pytest.mark.parametrize("frame", ROPE_FRAMES)
def test_rope_rows_wrap_at_any_frame_length(oracle, torch_gpu, frame):
    """Token t takes RoPE row t % frame_len (qkv.cu:25,110), which the kernels
    form by a multiply with a host-computed reciprocal: frame lengths of 1, 38,
    64 (a power of two) and 4096 (more than the 300 tokens), at both head dims
    and both layouts, standalone bit for bit against the oracle and fused bit
    for bit against the two GPU steps."""
    import spl_sage as S
    from spl_sage import qkv as Q

    torch = torch_gpu
    T, B = 300, 2
    for D, H, rope in ((64, 4, 0), (128, 2, 1)):
        rng = np.random.default_rng(300 + frame[0] + D)
        s, y = _spec(oracle, rng, D, H, 0, B, T, 1, rope, True, grid=frame)
        print(f"frame {frame}: frame_len {s.rope.shape[0]} D{D} H{H} B{B} T{T} rope {rope}", flush=True)
        inp, qn, rp = _device(torch, s, y)
        sa = S.SageAttention(None, D)
        outs = [torch.empty((B, T, H, D), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
        Q.QkvPrologue(sa).run(inp, T, H, qn, rp, Q.QkvOut(*(S.TensorMut(t) for t in outs)), batch=B)
        torch.cuda.synchronize()
        q16, k16, v16 = oracle.qkv_prologue(s, y)
        for name, got, w in zip("qkv", outs, (q16, k16, v16)):
            g = from_device16(got)
            assert np.array_equal(g, w), (name, int((g != w).sum()))

        p = oracle.Problem(B, H, T, D, dtype=0)
        ws = sa.workspace(S.Shape(B, H, T))
        out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device="cuda")
        sa.forward_qkv(ws, inp, S.TensorMut(out), qn, rp)
        torch.cuda.synchronize()
        assert_prologue_equal(read_workspace(ws, p), oracle.prologue(p, q16, k16, v16))
        _, o_two = run(torch, p, q16, k16, v16, want_ws=False)
        assert np.array_equal(from_device16(out), o_two)


def test_refusals_carry_the_references_text(oracle, torch_gpu):
    """qkv.rs:226-278: ld, LayerNorm biases, RoPE frame length, buffer sizes."""
    import spl_sage as S
    from spl_sage import qkv as Q

    torch = torch_gpu
    rng = np.random.default_rng(7)
    s, y = _spec(oracle, rng, 64, 2, 0, 1, 100, 1, 0, False)
    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, 64)
    outs = Q.QkvOut(*(S.TensorMut(torch.empty((1, 100, 2, 64), dtype=torch.bfloat16, device="cuda"))
                      for _ in range(3)))
    pro = Q.QkvPrologue(sa)
    bad = Q.QkvIn(inp.y, s.ld + 4, inp.tok, inp.chan, inp.bias)
    with pytest.raises(S.SageError, match=r"qkv: ld 396 must be a multiple of 8 and at least 384"):
        pro.run(bad, 100, 2, qn, rp, outs)
    with pytest.raises(S.SageError, match="qkv: LayerNorm QK-norm needs q and k biases"):
        pro.run(inp, 100, 2, Q.QkNorm(Q.NormKind.LayerNorm, qn.q_weight, qn.k_weight), rp, outs)
    with pytest.raises(S.SageError, match="qkv: RoPE frame length is 0"):
        pro.run(inp, 100, 2, qn, Q.Rope(rp.table, rp.layout, 0), outs)
    with pytest.raises(S.SageError, match="qkv y: buffer holds"):
        pro.run(inp, 200, 2, qn, rp, outs)
    with pytest.raises(S.SageError, match="RoPE table: buffer holds"):
        pro.run(inp, 100, 2, qn, Q.Rope(rp.table[:100].clone(), rp.layout, FRAME), outs)
    ws = sa.workspace(S.Shape(1, 2, 100))
    with pytest.raises(S.SageError, match=r"qkv: ld 396 must be a multiple of 8"):
        sa.prepare_qkv(ws, bad, qn, rp)
    pro.run(Q.QkvIn(inp.y, s.ld), 0, 2, None, None, outs)  # empty: a no-op, as the reference


def test_check_order_and_alignment_follow_the_reference(oracle, torch_gpu):
    """qkv.rs:249-279: output sizes are checked before the norm and RoPE
    options, and alignment last, over y, chan, bias, q, k and v only: norm
    weights and a RoPE table at a 4-byte (not 16-byte) offset are accepted
    and give the same bits as aligned copies."""
    import spl_sage as S
    from spl_sage import qkv as Q

    torch = torch_gpu
    rng = np.random.default_rng(8)
    T, H, D = 300, 2, 64
    s, y = _spec(oracle, rng, D, H, 0, 1, T, 1, 0, True)
    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, D)
    pro = Q.QkvPrologue(sa)

    def outs(n=T, offset=0):
        ts = [torch.empty(1 * n * H * D + 8, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
        return ts, Q.QkvOut(*(S.TensorMut(t[offset:offset + n * H * D].view(1, n, H, D)) for t in ts))

    # 4-byte offsets of every norm weight and of the RoPE table
    def shifted(t):
        b = torch.empty(t.numel() + 1, dtype=torch.float32, device="cuda")
        b[1:].copy_(t.reshape(-1))
        return b[1:]
    qn4 = Q.QkNorm(qn.kind, shifted(qn.q_weight), shifted(qn.k_weight), shifted(qn.q_bias), shifted(qn.k_bias),
                   qn.eps)
    rp4 = Q.Rope(shifted(rp.table), rp.layout, rp.frame_len)
    assert qn4.q_weight.data_ptr() % 16 == 4 and rp4.table.data_ptr() % 16 == 4
    (a, o_a), (b, o_b) = outs(), outs()
    pro.run(inp, T, H, qn, rp, o_a)
    pro.run(inp, T, H, qn4, rp4, o_b)
    torch.cuda.synchronize()
    n = T * H * D  # the written elements (each buffer has 8 more)
    for x, z in zip(a, b):
        assert torch.equal(x[:n].view(torch.int16), z[:n].view(torch.int16))
    ws_a, ws_b = sa.workspace(S.Shape(1, H, T)), sa.workspace(S.Shape(1, H, T))
    sa.prepare_qkv(ws_a, inp, qn, rp)
    sa.prepare_qkv(ws_b, inp, qn4, rp4)
    torch.cuda.synchronize()
    for name in ("q8", "k8", "v8", "q_scale", "k_scale", "stats"):
        assert torch.equal(ws_a.tensor(name), ws_b.tensor(name)), name

    # a short output is reported before a LayerNorm without biases
    _, short = outs(T - 1)
    with pytest.raises(S.SageError, match="qkv q: buffer holds"):
        pro.run(inp, T, H, Q.QkNorm(Q.NormKind.LayerNorm, qn.q_weight, qn.k_weight), rp, short)
    # a misaligned output is reported after the RoPE checks, before any launch
    _, skew = outs(offset=2)
    with pytest.raises(S.SageError, match="qkv: RoPE frame length is 0"):
        pro.run(inp, T, H, qn, Q.Rope(rp.table, rp.layout, 0), skew)
    with pytest.raises(S.SageError, match="is not 16-byte aligned"):
        pro.run(inp, T, H, qn, rp, skew)


FUZZ_CASES = 16


def _fuzz_case(rng):
    """A random fused-prologue problem: head dim, heads and grouping, batch,
    ragged token count (past one statistics-fold chunk now and then), norm
    kind, RoPE layout or none, token and channel scales or none, causal or
    KV-merged keys, and the sage QkNorm on top."""
    D = int(rng.choice([64, 128]))
    H = int(rng.integers(1, 7))
    kv = int(rng.choice([x for x in range(1, H + 1) if H % x == 0]))
    B = int(rng.integers(1, 3))
    merge = int(rng.choice([1, 1, 1, 2, 4]))
    if merge > 1:
        grid = (int(rng.integers(2, 9)), int(rng.integers(2, 11)), int(rng.integers(0, 6)))
        frames = int(rng.integers(1, 4))
        T = frames * (grid[2] + grid[0] * grid[1])
        layout = (frames, grid[2], grid[0], grid[1], int(rng.integers(0, frames + 1)))
        causal = False
    else:
        grid = (int(rng.integers(1, 12)), int(rng.integers(1, 40)), int(rng.integers(0, 20)))
        T = int(rng.integers(1, 900))
        if rng.random() < 0.2:  # past one fold chunk (512 tiles), kept to a head or two
            T, H, kv, B = int(rng.integers(65000, 67000)), min(H, 2), 1, 1
        layout = (1, 0, 0, 0, 0)
        causal = bool(rng.random() < 0.3)
    norm = int(rng.integers(0, 3))
    rope = None if rng.random() < 0.25 else int(rng.integers(0, 2))
    return dict(D=D, H=H, kv=kv if kv != H else 0, B=B, T=T, norm=norm, rope=rope, scaled=bool(rng.random() < 0.6),
                causal=causal, merge=merge, layout=layout, grid=grid, sage_ln=bool(rng.random() < 0.25))


@pytest.mark.parametrize("case", range(FUZZ_CASES))
def test_fused_prepare_fuzz(oracle, torch_gpu, case):
    """Seeded random fused problems (the K, V and Q workgroups of the
    statistics pass, the K stash of dense plans, the merged path): the
    workspace equals the oracle prologue of the oracle QKV prologue's bf16 Q,
    K and V bit for bit, and the output equals the two GPU steps' bit for bit."""
    import spl_sage as S

    torch = torch_gpu
    rng = np.random.default_rng(5000 + case)
    c = _fuzz_case(rng)
    D, H, kv, B, T = c["D"], c["H"], c["kv"], c["B"], c["T"]
    print(f"case {case}: {c}", flush=True)
    s, y = _spec(oracle, rng, D, H, kv, B, T, c["norm"], c["rope"], c["scaled"], grid=c["grid"])
    ln = None
    if c["sage_ln"]:
        ln = np.concatenate([1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D),
                             1 + 0.2 * rng.standard_normal(D), 0.1 * rng.standard_normal(D)]).astype(np.float32)
    p = oracle.Problem(B, H, T, D, kv_heads=kv, dtype=0, causal=c["causal"], merge=c["merge"], layout=c["layout"],
                       ln=ln, ln_eps=1e-6)
    q16, k16, v16 = oracle.qkv_prologue(s, y)
    want = oracle.prologue(p, q16, k16, v16)

    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, D)
    km = S.KvMerge.Pool(c["merge"], S.FrameLayout(*c["layout"])) if c["merge"] > 1 else S.KvMerge.Dense
    ws = sa.workspace(S.Shape(B, H, T, kv), km)
    out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device="cuda")
    qk_norm = S.QkNorm(torch.from_numpy(ln.copy()).to("cuda"), 1e-6) if c["sage_ln"] else None
    sa.forward_qkv(ws, inp, S.TensorMut(out), qn, rp, S.Options(causal=c["causal"], qk_norm=qk_norm))
    torch.cuda.synchronize()
    assert_prologue_equal(read_workspace(ws, p), want)
    _, o_two = run(torch, p, q16, k16, v16, want_ws=False)
    assert np.array_equal(from_device16(out), o_two)


def test_fused_prepare_at_the_headline_shape(oracle, torch_gpu):
    """C2's shape (B2 H32 N4096 D128) fed from the fused QKV projection with
    every option of the bench's QKV workload (channel scales, bias, LayerNorm
    QK-norm, VGGT RoPE over a 64-column grid): the workspace bit for bit
    against the oracle, the output bit for bit against the two GPU steps."""
    import spl_sage as S

    torch = torch_gpu
    B, H, T, D = 2, 32, 4096, 128
    rng = np.random.default_rng(4242)
    s, y = _spec(oracle, rng, D, H, 0, B, T, 1, 0, True, grid=(T // 64, 64, 0))
    p = oracle.Problem(B, H, T, D, dtype=0)
    q16, k16, v16 = oracle.qkv_prologue(s, y)
    want = oracle.prologue(p, q16, k16, v16)
    inp, qn, rp = _device(torch, s, y)
    sa = S.SageAttention(None, D)
    ws = sa.workspace(S.Shape(B, H, T))
    out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device="cuda")
    sa.forward_qkv(ws, inp, S.TensorMut(out), qn, rp)
    torch.cuda.synchronize()
    assert_prologue_equal(read_workspace(ws, p), want)
    _, o_two = run(torch, p, q16, k16, v16, want_ws=False)
    assert np.array_equal(from_device16(out), o_two)
