// GPU parity through the C++ host API (include/spl_sage.hpp): the reference's
// gpu_prologue_matches_reference and gpu_attention_matches_float_reference
// (sezer-muhammed/sota-papers-lab, platform/spl-nn/src/sage/tests.rs:606-700)
// restated with spl_sage:: calls, its run_gpu (packed QKV input, tests.rs:
// 372-420), Data::synthetic inputs (seed 11) and ln_params(d, 3). The
// checker is the C oracle (oracle/sage_oracle.h, test infrastructure): every
// workspace buffer must
// equal the oracle's prologue bit for bit, the output must reach cos >= 0.999
// against the oracle's emulation of the reference arithmetic with every
// element within 2e-2 + 2^-8 |emulated| of it, and the reference's own gate
// (cos > 0.999, rel_l2 < 0.04) against f64 attention. It also runs the
// reference's caller (sched.rs) through include/spl_sage_sched.hpp, and the
// QKV prologue through the qkv mirror. Prints one line per case; exit status 0
// when all pass.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "sage_oracle.h"
#include "spl_sage.hpp"
#include "spl_sage_sched.hpp"

using namespace spl_sage;

static int failures = 0;

static void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::printf("HIP error in %s: %s\n", what, hipGetErrorString(e));
        std::fflush(stdout);
        std::exit(2);
    }
}

template <typename T>
struct DeviceBuf {
    T* p = nullptr;
    std::size_t n = 0;
    explicit DeviceBuf(std::size_t count) : n(count) { hip_ok(hipMalloc((void**)&p, count * sizeof(T)), "hipMalloc"); }
    ~DeviceBuf() {
        if (p) (void)hipFree(p);
    }
    DeviceBuf(const DeviceBuf&) = delete;
    DeviceBuf& operator=(const DeviceBuf&) = delete;
};

template <typename T>
static std::vector<T> to_host(const T* dev, std::size_t n) {
    std::vector<T> h(n);
    hip_ok(hipMemcpy(h.data(), dev, n * sizeof(T), hipMemcpyDeviceToHost), "copy to host");
    return h;
}

// tests.rs:422-435 (ln_params): weights 1 + 0.5 N(0,1), biases 0.8 N(0,1).
static std::vector<float> ln_params(std::size_t d, uint64_t seed) {
    uint64_t st = seed;
    std::vector<float> p;
    for (int part = 0; part < 4; part++)
        for (std::size_t i = 0; i < d; i++) {
            const float x = oracle_rng_normal(&st);
            p.push_back(part % 2 == 0 ? 1.0f + 0.5f * x : 0.8f * x);
        }
    return p;
}

struct Case {
    std::string name;
    std::size_t d;
    KvMerge merge;
    bool ln, smooth, pv16;
};

// Bitwise equality of two buffers; reports the first difference.
template <typename T>
static bool same(const char* what, const T* a, const T* b, std::size_t n) {
    if (std::memcmp(a, b, n * sizeof(T)) == 0) return true;
    for (std::size_t i = 0; i < n; i++)
        if (std::memcmp(a + i, b + i, sizeof(T)) != 0) {
            std::printf("    %s differs first at %zu\n", what, i);
            break;
        }
    return false;
}

// The workspace after a forward, and its bf16 output [B][T][H][d], against
// the C oracle on the same host inputs (q, k, v with p's strides): every
// buffer bit for bit, the output within the north-star gate of the emulated
// reference arithmetic and within the reference's own gate against f64.
static bool check_forward(const oracle_problem& p, const Workspace& ws, const uint16_t* qh, const uint16_t* kh,
                          const uint16_t* vh, const uint16_t* dev_out, float scale, bool merged) {
    const Plan& plan = ws.plan();
    const std::size_t B = p.batch, H = p.heads, T = p.tokens, d = p.head_dim;
    const std::size_t tq = plan.tq_pad, tk = plan.tk_pad, nkb = plan.kblocks();
    std::vector<int8_t> q8(B * H * tq * d), k8(B * H * tk * d);
    std::vector<float> qs(B * H * tq / QGROUP), ks(B * H * nkb), stats(B * H * 4 * d), kbias(tk);
    std::vector<uint8_t> v8(B * H * tk * d);
    if (oracle_prologue(&p, qh, kh, vh, q8.data(), qs.data(), k8.data(), ks.data(), v8.data(), stats.data(),
                        kbias.data(), 0) != 0) {
        std::printf("    oracle refused the case\n");
        return false;
    }

    // Workspace buffers, bit for bit (v8 back to logical key order).
    const sage_ws_buffers wb = ws.buffers();
    bool ok = same("q8", to_host(wb.q8, q8.size()).data(), q8.data(), q8.size());
    ok &= same("q_scale", to_host(wb.q_scale, qs.size()).data(), qs.data(), qs.size());
    ok &= same("k8", to_host(wb.k8, k8.size()).data(), k8.data(), k8.size());
    ok &= same("k_scale", to_host(wb.k_scale, ks.size()).data(), ks.data(), ks.size());
    ok &= same("stats", to_host(wb.stats, stats.size()).data(), stats.data(), stats.size());
    {
        const std::vector<uint8_t> raw = to_host(wb.v8, v8.size());
        std::vector<uint8_t> logical(v8.size());
        for (std::size_t bh = 0; bh < B * H; bh++)
            for (std::size_t blk = 0; blk < nkb; blk++)
                for (std::size_t ch = 0; ch < d; ch++)
                    for (int key = 0; key < 64; key++)
                        logical[(bh * tk + blk * 64 + key) * d + ch] =
                            raw[((bh * nkb + blk) * d + ch) * 64 + v8_position(key)];
        ok &= same("v8", logical.data(), v8.data(), v8.size());
    }
    if (merged) ok &= same("kbias", to_host(wb.kbias, tk).data(), kbias.data(), tk);

    // Output against the emulation of the reference arithmetic and against f64.
    const std::vector<uint16_t> o16 = to_host(dev_out, B * T * H * d);
    std::vector<float> ours(B * H * T * d);
    for (std::size_t b = 0; b < B; b++)
        for (std::size_t t = 0; t < T; t++)
            for (std::size_t h = 0; h < H; h++)
                oracle_decode16(&o16[((b * T + t) * H + h) * d], &ours[((b * H + h) * T + t) * d], d, ORACLE_BF16);
    std::vector<float> emu(ours.size()), f64(ours.size());
    std::vector<uint16_t> emu16(ours.size());
    oracle_sage_emulate(&p, 0, q8.data(), qs.data(), k8.data(), ks.data(), v8.data(), stats.data(), kbias.data(),
                        nullptr, (int)T, emu.data(), emu16.data(), ORACLE_BF16, 1, 0);
    oracle_attention_f64(&p, 0, scale, qh, kh, vh, nullptr, (int)T, f64.data(), 0);
    // The arithmetic gate compares the bf16 output with the emulation's fp32
    // output before its own rounding. Data::synthetic outputs reach |out| ~ 10,
    // where bf16's half step (up to 2^-8 |out|, 2^-5 at 8..16) alone exceeds
    // 2e-2, so each element is held to 2e-2 + 2^-8 |emu|: the north-star
    // max-abs bound plus the rounding any bf16 output carries. The
    // reference's own gate for this data is the f64 one (tests.rs:699).
    double e[5], e64[5];
    oracle_errors(ours.data(), emu.data(), ours.size(), e);
    oracle_errors(ours.data(), f64.data(), ours.size(), e64);
    std::size_t over = 0;
    for (std::size_t i = 0; i < ours.size(); i++)
        if (!(std::fabs(ours[i] - emu[i]) <= 2e-2 + std::ldexp(std::fabs(emu[i]), -8))) over++;
    const bool gate = e[0] >= 0.999 && over == 0;
    const bool ref_gate = e64[0] > 0.999 && e64[2] < 0.04;
    std::printf("    prologue %s; vs reference arithmetic cos %.6f max_abs %.3g (|out| <= %.3g, %zu over the bound) %s; "
                "vs f64 cos %.6f rel_l2 %.4f %s\n",
                ok ? "bit-exact" : "DIFFERS", e[0], e[3], e[4], over, gate ? "ok" : "FAIL", e64[0], e64[2],
                ref_gate ? "ok" : "FAIL");
    std::fflush(stdout);
    return ok && gate && ref_gate;
}

static void run_case(const Case& c) {
    std::printf("case %s\n", c.name.c_str());
    std::fflush(stdout);
    const std::size_t d = c.d;
    const FrameLayout layout = c.merge.layout;
    const Shape shape{2, 3, c.merge.is_dense() ? 225 : layout.frames * layout.tokens_per_frame()};
    const std::size_t B = shape.batch, T = shape.tokens, H = shape.heads, hd = H * d;

    // Data::synthetic (tests.rs:300-329), then packed [b][t][3][h][d] as run_gpu uploads it.
    std::vector<uint16_t> q(B * T * hd), k(q.size()), v(q.size());
    oracle_reference_synthetic((int)B, (int)T, (int)H, (int)d, 11, q.data(), k.data(), v.data());
    std::vector<uint16_t> packed(3 * q.size());
    for (std::size_t bt = 0; bt < B * T; bt++) {
        std::memcpy(&packed[(bt * 3 + 0) * hd], &q[bt * hd], hd * 2);
        std::memcpy(&packed[(bt * 3 + 1) * hd], &k[bt * hd], hd * 2);
        std::memcpy(&packed[(bt * 3 + 2) * hd], &v[bt * hd], hd * 2);
    }
    const std::vector<float> lnp = ln_params(d, 3);

    DeviceBuf<uint16_t> dqkv(packed.size()), dout(B * T * hd);
    DeviceBuf<float> dln(lnp.size());
    hip_ok(hipMemcpy(dqkv.p, packed.data(), packed.size() * 2, hipMemcpyHostToDevice), "upload qkv");
    hip_ok(hipMemcpy(dln.p, lnp.data(), lnp.size() * 4, hipMemcpyHostToDevice), "upload ln");

    Config cfg = Config::for_head_dim(d);
    if (c.pv16) cfg.pv_accum = PvAccum::F16;
    const SageAttention sage = SageAttention::with_config(nullptr, d, cfg);
    Workspace ws = sage.workspace(shape, c.merge);
    const Strides st = Strides::packed_qkv(T, H, d);
    Options opts;
    opts.smooth_k = opts.smooth_v = c.smooth;
    if (c.ln) opts.qk_norm = QkNorm{dln.p, lnp.size(), 1e-5f};
    const std::size_t len = packed.size();
    sage.forward(ws, Tensor{dqkv.p, len, st}, Tensor{dqkv.p + hd, len - hd, st},
                 Tensor{dqkv.p + 2 * hd, len - 2 * hd, st}, TensorMut{dout.p, dout.n, Strides::bthd(T, H, d)}, opts);
    hip_ok(hipDeviceSynchronize(), "forward");

    // The oracle on the same inputs (same packed strides).
    oracle_problem p{};
    p.batch = (int)B;
    p.heads = p.kv_heads = (int)H;
    p.tokens = (int)T;
    p.head_dim = (int)d;
    p.dtype = ORACLE_BF16;
    p.q_sb = p.k_sb = p.v_sb = (long long)st.batch;
    p.q_st = p.k_st = p.v_st = (long long)st.token;
    p.q_sh = p.k_sh = p.v_sh = (long long)st.head;
    const float scale = 1.0f / std::sqrt((float)d);
    p.q_mul = scale * 1.44269504088896340736f;
    p.smooth_k = p.smooth_v = c.smooth ? 1 : 0;
    p.v_range = c.pv16 ? PV16_V_RANGE : FP8_MAX;
    p.merge = (int)c.merge.stride;
    p.frames = (int)layout.frames;
    p.special = (int)layout.special;
    p.grid_h = (int)layout.grid_h;
    p.grid_w = (int)layout.grid_w;
    p.dense_frames = (int)layout.dense_frames;
    p.ln = c.ln ? lnp.data() : nullptr;
    p.ln_eps = 1e-5f;
    p.pv16 = c.pv16 ? 1 : 0;
    const uint16_t* hp = packed.data();
    if (!check_forward(p, ws, hp, hp + hd, hp + 2 * hd, dout.p, scale, !c.merge.is_dense())) failures++;

    // The no-allocation entry point (no reference counterpart) on the same
    // inputs: the output equals forward's bit for bit.
    DeviceBuf<uint16_t> dout2(dout.n);
    sage.forward_noalloc(shape, Tensor{dqkv.p, len, st}, Tensor{dqkv.p + hd, len - hd, st},
                         Tensor{dqkv.p + 2 * hd, len - 2 * hd, st}, TensorMut{dout2.p, dout2.n, Strides::bthd(T, H, d)},
                         opts, c.merge);
    hip_ok(hipDeviceSynchronize(), "forward_noalloc");
    std::vector<uint16_t> o1(dout.n), o2(dout.n);
    hip_ok(hipMemcpy(o1.data(), dout.p, o1.size() * 2, hipMemcpyDeviceToHost), "download out");
    hip_ok(hipMemcpy(o2.data(), dout2.p, o2.size() * 2, hipMemcpyDeviceToHost), "download out2");
    const bool same = o1 == o2;
    std::printf("    forward_noalloc %s\n", same ? "equals forward" : "DIFFERS from forward");
    std::fflush(stdout);
    if (!same) failures++;
}

// QkvPrologue::run through the C++ qkv mirror (the reference's
// gpu_qkv_prologue_matches_cpu option sets, tests.rs:447-570, on one 689-token
// VGGT frame at head dim 64): Q, K and V equal the C oracle's restatement bit
// for bit, and prepare_qkv's workspace equals prepare's on those Q, K and V.
static void run_qkv_case(int norm_kind, int layout, bool scaled) {
    using namespace spl_sage::qkv;
    const std::size_t d = 64, heads = 4, tokens = 689, width = 3 * heads * d, ld = width + 8;
    uint64_t st = 1234 + norm_kind * 7 + layout;
    std::vector<float> yf(tokens * ld), chan(width), tok(tokens), biasf(width), w(4 * d);
    for (float& x : yf) x = oracle_rng_normal(&st);
    for (float& x : chan) x = 0.5f + (float)oracle_rng_uniform(&st);
    for (float& x : tok) x = 0.5f + (float)oracle_rng_uniform(&st);
    for (float& x : biasf) x = 0.2f * oracle_rng_normal(&st);
    for (std::size_t i = 0; i < 4 * d; i++) w[i] = (i / d) % 2 == 0 ? 1.0f + 0.2f * oracle_rng_normal(&st)
                                                                   : 0.1f * oracle_rng_normal(&st);
    std::vector<uint16_t> y(yf.size()), bias(width);
    oracle_encode16(yf.data(), y.data(), yf.size(), ORACLE_BF16);
    oracle_encode16(biasf.data(), bias.data(), width, ORACLE_BF16);
    const RopeTable table = layout == 0 ? RopeTable::vggt(21, 32, 17, 100.0) : RopeTable::dinov3(21, 32, 17, 100.0);

    DeviceBuf<uint16_t> yd(y.size()), bd(width);
    DeviceBuf<float> cd(width), td(tokens), wd(4 * d), rd(table.cos_sin.size());
    hip_ok(hipMemcpy(yd.p, y.data(), y.size() * 2, hipMemcpyHostToDevice), "copy y");
    hip_ok(hipMemcpy(bd.p, bias.data(), width * 2, hipMemcpyHostToDevice), "copy bias");
    hip_ok(hipMemcpy(cd.p, chan.data(), width * 4, hipMemcpyHostToDevice), "copy chan");
    hip_ok(hipMemcpy(td.p, tok.data(), tokens * 4, hipMemcpyHostToDevice), "copy tok");
    hip_ok(hipMemcpy(wd.p, w.data(), 4 * d * 4, hipMemcpyHostToDevice), "copy norm");
    hip_ok(hipMemcpy(rd.p, table.cos_sin.data(), table.cos_sin.size() * 4, hipMemcpyHostToDevice), "copy rope");

    QkvIn in;
    in.y = yd.p, in.y_len = yd.n, in.ld = ld, in.bias = bd.p, in.bias_len = width;
    if (scaled) in.tok = td.p, in.tok_len = tokens, in.chan = cd.p, in.chan_len = width;
    spl_sage::qkv::QkNorm qn{norm_kind == 1 ? NormKind::LayerNorm : NormKind::Rms, wd.p, wd.p + d, wd.p + 2 * d, wd.p + 3 * d, d, 1e-6f};
    const Rope rope{rd.p, rd.n, layout == 0 ? RopeLayout::Vggt : RopeLayout::Dinov3, table.frame_len};

    const SageAttention sage = SageAttention::create(nullptr, d);
    const std::size_t n = tokens * heads * d;
    DeviceBuf<uint16_t> q(n), k(n), v(n);
    const Strides bthd = Strides::bthd(tokens, heads, d);
    QkvPrologue(sage).run(in, tokens, heads, norm_kind ? &qn : nullptr, &rope,
                          QkvOut{TensorMut{q.p, n, bthd}, TensorMut{k.p, n, bthd}, TensorMut{v.p, n, bthd}});

    oracle_qkv a{};
    a.batch = 1, a.tokens = (int)tokens, a.heads = (int)heads, a.kv_heads = (int)heads, a.head_dim = (int)d;
    a.ld = (long long)ld, a.batch_stride = (long long)(tokens * ld);
    a.bias = bias.data();
    if (scaled) a.tok = tok.data(), a.chan = chan.data();
    a.norm = norm_kind, a.q_w = w.data(), a.q_b = w.data() + d, a.k_w = w.data() + 2 * d, a.k_b = w.data() + 3 * d;
    a.eps = 1e-6f, a.rope = table.cos_sin.data(), a.rope_layout = layout, a.frame_len = (int)table.frame_len;
    std::vector<uint16_t> wq(n), wk(n), wv(n);
    oracle_qkv_prologue(&a, y.data(), wq.data(), wk.data(), wv.data());
    const auto hq = to_host(q.p, n), hk = to_host(k.p, n), hv = to_host(v.p, n);
    bool ok = same("q", hq.data(), wq.data(), n) && same("k", hk.data(), wk.data(), n) && same("v", hv.data(), wv.data(), n);

    Workspace ws_two = sage.workspace(Shape{1, heads, tokens}), ws_fused = sage.workspace(Shape{1, heads, tokens});
    sage.prepare(ws_two, Tensor{q.p, n, bthd}, Tensor{k.p, n, bthd}, Tensor{v.p, n, bthd});
    prepare_qkv(sage, ws_fused, in, norm_kind ? &qn : nullptr, &rope);
    const sage_ws_buffers b2 = ws_two.buffers(), b1 = ws_fused.buffers();
    ok = ok && same("q8", to_host(b1.q8, b1.q8_len).data(), to_host(b2.q8, b2.q8_len).data(), b1.q8_len) &&
         same("k8", to_host(b1.k8, b1.k8_len).data(), to_host(b2.k8, b2.k8_len).data(), b1.k8_len) &&
         same("v8", to_host(b1.v8, b1.v8_len).data(), to_host(b2.v8, b2.v8_len).data(), b1.v8_len) &&
         same("q_scale", to_host(b1.q_scale, b1.q_scale_len).data(), to_host(b2.q_scale, b2.q_scale_len).data(),
              b1.q_scale_len) &&
         same("k_scale", to_host(b1.k_scale, b1.k_scale_len).data(), to_host(b2.k_scale, b2.k_scale_len).data(),
              b1.k_scale_len) &&
         same("stats", to_host(b1.stats, b1.stats_len).data(), to_host(b2.stats, b2.stats_len).data(), b1.stats_len);
    std::printf("qkv norm %d rope %d scaled %d: %s\n", norm_kind, layout, (int)scaled, ok ? "bit-exact" : "DIFFERS");
    if (!ok) failures++;
    std::fflush(stdout);
}

// The reference's caller (apps/image-to-3d/src/vggt/trunk/sched.rs) through its
// C++ restatement (include/spl_sage_sched.hpp): the shipped `ours+sage` schedule
// (vggt/mod.rs:82-107: frame attention at 3-5, merge4 at 0, 1, 7, 19, register
// attention at 2, 6, 9, 14, 20, the other global layers through sage) at a
// 3-frame VGGT geometry of 7 x 10 patches. Sage::prepare makes one workspace per
// distinct merge, each the size the caller counts (sched.rs:56-71); each sage
// layer runs SageLayer::forward on head-major bf16 Q, K and V (Data::synthetic,
// seed 17) and is checked against the oracle; the caller's errors carry its texts.
static void run_sched_case() {
    using namespace spl_vggt;
    std::printf("case sched: ours+sage schedule, VGGT geometry 3 frames x (17 + 7 x 10)\n");
    std::fflush(stdout);
    const TrunkGeom g{3, 7, 10};
    const std::size_t T = g.rows(), H = HEADS, d = HEAD_DIM, n = H * T * d;
    Schedule sched;
    sched.fill(InterKind::Global);
    for (std::size_t i : {2, 6, 9, 14, 20}) sched[i] = InterKind::Register;
    for (InterKind& a : sched)
        if (a == InterKind::Global) a = InterKind::Sage;
    for (std::size_t i : {3, 4, 5}) sched[i] = InterKind::Frame;
    for (std::size_t i : {0, 1, 7, 19}) sched[i] = InterKind::Merge4;

    Sage sage;
    sage.prepare(nullptr, sched, g);
    bool ok = sage.workspaces() == 2;

    std::vector<uint16_t> q(n), k(n), v(n), qh(n), kh(n), vh(n);
    oracle_reference_synthetic(1, (int)T, (int)H, (int)d, 17, q.data(), k.data(), v.data());
    for (std::size_t t = 0; t < T; t++)
        for (std::size_t h = 0; h < H; h++) {
            std::memcpy(&qh[(h * T + t) * d], &q[(t * H + h) * d], d * 2);
            std::memcpy(&kh[(h * T + t) * d], &k[(t * H + h) * d], d * 2);
            std::memcpy(&vh[(h * T + t) * d], &v[(t * H + h) * d], d * 2);
        }
    DeviceBuf<uint16_t> dq(n), dk(n), dv(n), dout(n);
    hip_ok(hipMemcpy(dq.p, qh.data(), n * 2, hipMemcpyHostToDevice), "upload q");
    hip_ok(hipMemcpy(dk.p, kh.data(), n * 2, hipMemcpyHostToDevice), "upload k");
    hip_ok(hipMemcpy(dv.p, vh.data(), n * 2, hipMemcpyHostToDevice), "upload v");

    for (InterKind kind : {InterKind::Sage, InterKind::Merge4}) {
        const KvMerge m = *merge_of(kind, g);
        const SageLayer layer = sage.layer(kind, g);
        ok &= layer.v_format() == Dtype::Bf16;
        const std::size_t bytes = layer.workspace().bytes(), want = workspace_bytes(g, m);
        std::printf("  %s layer: workspace %zu bytes (the caller counts %zu)\n", kind_name(kind), bytes, want);
        ok &= bytes == want;
        layer.forward(dq.p, n, dk.p, n, dv.p, n, dout.p, n, 1, T);
        hip_ok(hipDeviceSynchronize(), "sage layer forward");
        oracle_problem p{};
        p.batch = 1;
        p.heads = p.kv_heads = (int)H;
        p.tokens = (int)T;
        p.head_dim = (int)d;
        p.dtype = ORACLE_BF16;
        p.q_sb = p.k_sb = p.v_sb = (long long)(H * T * d);
        p.q_st = p.k_st = p.v_st = (long long)d;
        p.q_sh = p.k_sh = p.v_sh = (long long)(T * d);
        p.q_mul = ATTN_SCALE * 1.44269504088896340736f;
        p.smooth_k = p.smooth_v = 1;
        p.v_range = FP8_MAX;
        p.merge = (int)m.stride;
        p.frames = (int)m.layout.frames;
        p.special = (int)m.layout.special;
        p.grid_h = (int)m.layout.grid_h;
        p.grid_w = (int)m.layout.grid_w;
        p.dense_frames = (int)m.layout.dense_frames;
        p.ln_eps = 1e-5f;
        ok &= check_forward(p, layer.workspace(), qh.data(), kh.data(), vh.data(), dout.p, ATTN_SCALE, !m.is_dense());
    }
    // The caller's refusals (sched.rs:150-164, 189-195).
    auto refuses = [&](auto f, const std::string& text) {
        try {
            f();
        } catch (const Error& e) {
            const bool hit = std::string(e.what()) == text;
            std::printf("  refused: \"%s\"%s\n", e.what(), hit ? "" : " (unexpected text)");
            return hit;
        }
        std::printf("  no error (expected \"%s\")\n", text.c_str());
        return false;
    };
    ok &= refuses([&] { sage.layer(InterKind::Sage, g).forward(dq.p, n, dk.p, n, dv.p, n, dout.p, n, 2, T / 2); },
                  "sage layer: workspace for Shape { batch: 1, heads: 16, tokens: 261 }, called with 2 \xc3\x97 130");
    ok &= refuses([&] { sage.layer(InterKind::Merge2, g); },
                  "sage workspace for Merge2 at TrunkGeom { frames: 3, grid_h: 7, grid_w: 10 } not prepared");
    ok &= refuses([&] { sage.layer(InterKind::Frame, g); }, "Frame is not a sage layer");
    // A new geometry drops the old workspaces; one frame has nothing to merge.
    const TrunkGeom one{1, 7, 10};
    sage.prepare(nullptr, sched, one);
    ok &= sage.workspaces() == 1 && sage.layer(InterKind::Merge4, one).workspace().plan().merge.is_dense();
    std::printf("  %s\n", ok ? "ok" : "FAIL");
    if (!ok) failures++;
    std::fflush(stdout);
}

int main() {
    check_device(0);
    run_sched_case();
    run_qkv_case(1, 0, false);
    run_qkv_case(2, 1, true);
    run_qkv_case(0, 0, true);
    const FrameLayout small{3, 5, 7, 10, 1};  // tests.rs:596-605
    std::vector<Case> cases;
    for (std::size_t d : {64, 128}) {
        const std::string s = std::to_string(d);
        // tests.rs:622-628, then PvAccum::F16 (tests.rs:633-648, 655-700).
        cases.push_back({"d" + s + " dense", d, KvMerge::Dense(), false, true, false});
        cases.push_back({"d" + s + " dense nosmooth", d, KvMerge::Dense(), false, false, false});
        cases.push_back({"d" + s + " dense ln", d, KvMerge::Dense(), true, true, false});
        cases.push_back({"d" + s + " pool2", d, KvMerge::Pool(2, small), false, true, false});
        cases.push_back({"d" + s + " pool4 ln", d, KvMerge::Pool(4, small), true, true, false});
        cases.push_back({"d" + s + " dense pv16", d, KvMerge::Dense(), false, true, true});
    }
    for (const Case& c : cases) run_case(c);
    // Errors come back as exceptions with the reference's text (mod.rs:841-843).
    {
        const SageAttention sage = SageAttention::create(nullptr, 64);
        const Workspace ws = sage.workspace(Shape{1, 1, 128});
        DeviceBuf<uint16_t> out(128 * 64);
        try {
            sage.attend(ws, TensorMut{out.p, out.n, Strides::bthd(128, 1, 64)});
            std::printf("attend before prepare: no error\n");
            failures++;
        } catch (const Error& err) {
            const bool ok = err.status() == SAGE_ERR_STATE &&
                            std::string(err.what()).find("has not been prepared") != std::string::npos;
            std::printf("attend before prepare: %s (%s)\n", ok ? "ok" : "FAIL", err.what());
            if (!ok) failures++;
        }
        const auto res = sage.attn_resources();
        std::printf("attention kernel d64: %d VGPRs, %d spill bytes\n", res.first, res.second);
        if (res.second != 0) failures++;
    }
    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
