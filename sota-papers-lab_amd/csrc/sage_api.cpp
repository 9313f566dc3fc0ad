// C ABI of the gfx950 SageAttention2 forward path: the host side of the
// reference's `spl_nn::sage` API (sezer-muhammed/sota-papers-lab,
// platform/spl-nn/src/sage/mod.rs:116-910), re-stated in C++ over the HIP
// runtime. Validation order and error text follow the reference so that a
// caller sees the same failures before any launch.
#include "../../include/sage_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace {

thread_local std::string g_last_error;

sage_status fail(sage_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

sage_status hip_fail(hipError_t e, const char* what) {
    return fail(SAGE_ERR_DEVICE, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

sage_status ok() {
    g_last_error.clear();
    return SAGE_OK;
}

using u64 = unsigned long long;

std::string shape_dbg(const sage_shape& s) {
    char b[256];
    if (s.kv_heads && s.kv_heads != s.heads)
        snprintf(b, sizeof b, "Shape { batch: %llu, heads: %llu, tokens: %llu, kv_heads: %llu }", (u64)s.batch,
                 (u64)s.heads, (u64)s.tokens, (u64)s.kv_heads);
    else
        snprintf(b, sizeof b, "Shape { batch: %llu, heads: %llu, tokens: %llu }", (u64)s.batch, (u64)s.heads,
                 (u64)s.tokens);
    return b;
}

std::string layout_dbg(const sage_frame_layout& l) {
    char b[256];
    snprintf(b, sizeof b, "FrameLayout { frames: %llu, special: %llu, grid_h: %llu, grid_w: %llu, dense_frames: %llu }",
             (u64)l.frames, (u64)l.special, (u64)l.grid_h, (u64)l.grid_w, (u64)l.dense_frames);
    return b;
}

std::string strides_dbg(const sage_strides& s) {
    char b[160];
    snprintf(b, sizeof b, "Strides { batch: %llu, token: %llu, head: %llu }", (u64)s.batch, (u64)s.token,
             (u64)s.head);
    return b;
}

std::string tile_dbg(const sage_tile& t) {
    char b[128];
    snprintf(b, sizeof b, "Tile { warps: %u, m_tiles: %u, stages: %u }", t.warps, t.m_tiles, t.stages);
    return b;
}

uint64_t div_ceil(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
uint64_t round_up(uint64_t a, uint64_t m) { return div_ceil(a, m) * m; }

// FrameLayout::tokens_per_frame / merged_per_frame / merged_keys (mod.rs:284-300).
uint64_t tokens_per_frame(const sage_frame_layout& l) { return l.special + l.grid_h * l.grid_w; }
uint64_t merged_per_frame(const sage_frame_layout& l, uint64_t s) {
    return l.special + div_ceil(l.grid_h, s) * div_ceil(l.grid_w, s);
}
uint64_t merged_keys(const sage_frame_layout& l, uint64_t s) {
    const uint64_t d = l.dense_frames < l.frames ? l.dense_frames : l.frames;
    return d * tokens_per_frame(l) + (l.frames - d) * merged_per_frame(l, s);
}

// `int` (mod.rs:387-389).
bool fits_i32(uint64_t v, const char* what, sage_status* st) {
    if (v > 2147483647ull) {
        *st = fail(SAGE_ERR_INVALID, "%s = %llu does not fit in i32", what, (u64)v);
        return false;
    }
    return true;
}

uint64_t kv_heads_of(const sage_shape& s) { return s.kv_heads ? s.kv_heads : s.heads; }

}  // namespace

struct sage_workspace {
    sage_plan plan;
    uint64_t head_dim;
    int device;
    int8_t* q8 = nullptr;
    float* q_scale = nullptr;
    int8_t* k8 = nullptr;
    float* k_scale = nullptr;
    uint8_t* v8 = nullptr;
    float* stats = nullptr;
    float* kbias = nullptr;
    float* part = nullptr;
    uint64_t n_q8 = 0, n_q_scale = 0, n_k8 = 0, n_k_scale = 0, n_v8 = 0, n_stats = 0, n_kbias = 0, n_part = 0;
    bool prepared = false;
    sage::Geom geom{};
};

extern "C" {

const char* sage_last_error(void) { return g_last_error.c_str(); }

sage_status sage_plan_new(const sage_shape* shape, const sage_kv_merge* merge, sage_plan* out) {
    if (!shape || !merge || !out) return fail(SAGE_ERR_INVALID, "null argument");
    const sage_shape& s = *shape;
    if (s.batch == 0 || s.heads == 0 || s.tokens == 0)
        return fail(SAGE_ERR_INVALID, "empty attention shape %s", shape_dbg(s).c_str());
    // Counts so large that padding or a product would wrap 64 bits cannot fit the
    // i32 indexing either; report them with the same text as the checks below.
    if (s.tokens > 0x7fffffffull)
        return fail(SAGE_ERR_INVALID, "padded queries = %llu does not fit in i32", (u64)s.tokens);
    if (s.batch > 0x7fffffffull || s.heads > 0x7fffffffull)
        return fail(SAGE_ERR_INVALID, "batch × heads = %llu × %llu does not fit in i32", (u64)s.batch, (u64)s.heads);
    const uint64_t hk = kv_heads_of(s);
    if (s.heads % hk != 0)
        return fail(SAGE_ERR_INVALID, "%llu query heads are not a multiple of %llu KV heads", (u64)s.heads, (u64)hk);
    uint64_t tk;
    if (merge->stride == 1) {
        tk = s.tokens;
    } else {
        if (merge->stride != 2 && merge->stride != 4)
            return fail(SAGE_ERR_INVALID, "KV merge stride must be 2 or 4, got %u", merge->stride);
        const sage_frame_layout& l = merge->layout;
        if (l.grid_h == 0 || l.grid_w == 0)
            return fail(SAGE_ERR_INVALID, "KV merge needs a patch grid: %s", layout_dbg(l).c_str());
        // A layout whose token count wraps 64 bits covers more tokens than any sequence.
        uint64_t cells, per_frame, covered;
        if (__builtin_mul_overflow(l.grid_h, l.grid_w, &cells) || __builtin_add_overflow(cells, l.special, &per_frame) ||
            __builtin_mul_overflow(l.frames, per_frame, &covered))
            return fail(SAGE_ERR_INVALID, "frame layout %s covers more than 2^64 tokens, the sequence has %llu",
                        layout_dbg(l).c_str(), (u64)s.tokens);
        if (covered != s.tokens)
            return fail(SAGE_ERR_INVALID, "frame layout %s covers %llu tokens, the sequence has %llu",
                        layout_dbg(l).c_str(), (u64)covered, (u64)s.tokens);
        tk = merged_keys(l, merge->stride);
    }
    sage_plan p{};
    p.shape = s;
    p.shape.kv_heads = hk;
    p.merge = *merge;
    p.tq_pad = round_up(s.tokens, SAGE_QTILE);
    p.tk = tk;
    p.tk_pad = round_up(tk, SAGE_KBLOCK);
    sage_status st = SAGE_OK;
    if (!fits_i32(p.tq_pad, "padded queries", &st) || !fits_i32(p.tk_pad, "padded keys", &st) ||
        !fits_i32(s.batch * s.heads, "batch × heads", &st))
        return st;
    *out = p;
    return ok();
}

double sage_flops(const sage_plan* plan, uint64_t head_dim, int32_t causal) {
    if (!plan) return 0.0;
    const double bh = (double)(plan->shape.batch * plan->shape.heads);
    if (causal) return 2.0 * bh * (double)head_dim * (double)plan->shape.tokens * ((double)plan->shape.tokens + 1.0);
    return 4.0 * bh * (double)plan->shape.tokens * (double)plan->tk * (double)head_dim;
}

sage_status sage_strides_check(const sage_strides* s, const char* what) {
    if (!s) return fail(SAGE_ERR_INVALID, "null strides");
    if (s->batch % 8 || s->token % 8 || s->head % 8)
        return fail(SAGE_ERR_INVALID, "%s strides must be multiples of 8 elements: %s", what ? what : "tensor",
                    strides_dbg(*s).c_str());
    return ok();
}

uint64_t sage_strides_extent(const sage_strides* s, uint64_t batch, uint64_t tokens, uint64_t heads,
                             uint64_t head_dim) {
    if (!s || batch == 0 || tokens == 0 || heads == 0) return 0;
    // A view whose extent does not fit 64 bits needs more than any buffer holds.
    uint64_t a, b, c, e;
    if (__builtin_mul_overflow(batch - 1, s->batch, &a) || __builtin_mul_overflow(tokens - 1, s->token, &b) ||
        __builtin_mul_overflow(heads - 1, s->head, &c) || __builtin_add_overflow(a, b, &e) ||
        __builtin_add_overflow(e, c, &e) || __builtin_add_overflow(e, head_dim, &e))
        return UINT64_MAX;
    return e;
}

// Tile::validate (mod.rs:158-167): warps in {2, 4, 8}, m_tiles in {1, 2, 4},
// stages 2..6, and the reference's rows per CTA (16 * m_tiles * warps)
// dividing the 128-query tile. The tile picks the workgroup layout only
// (attend_view): warps = 8 runs the eight-wave layout (score and output
// waves) for dense and causal attention, every other tile the four-wave one;
// outputs do not depend on it.
sage_status sage_tile_validate(const sage_tile* t) {
    if (!t) return fail(SAGE_ERR_INVALID, "null tile");
    const bool warps_ok = t->warps == 2 || t->warps == 4 || t->warps == 8;
    const bool mt_ok = t->m_tiles == 1 || t->m_tiles == 2 || t->m_tiles == 4;
    const bool stages_ok = t->stages >= 2 && t->stages <= 6;
    if (!warps_ok || !mt_ok || !stages_ok || SAGE_QTILE % (16u * t->m_tiles * t->warps) != 0)
        return fail(SAGE_ERR_INVALID, "unsupported sage tile %s", tile_dbg(*t).c_str());
    return ok();
}

// Config::for_head_dim (mod.rs:194-200) with Tile::for_head_dim (:128-147):
// Tile::D128 {4, 1, 3} above head dim 64, Tile::DEFAULT {4, 2, 3} otherwise.
sage_config sage_config_for_head_dim(uint64_t head_dim) {
    sage_config c{};
    c.tile.warps = 4;
    c.tile.m_tiles = head_dim > 64 ? 1 : 2;
    c.tile.stages = 3;
    c.pv_accum = SAGE_PV_F32;
    return c;
}

sage_status sage_check_device(int ordinal) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "device count");
    if (ordinal < 0 || ordinal >= n)
        return fail(SAGE_ERR_DEVICE, "no HIP device %d (%d visible)", ordinal, n);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, ordinal);
    if (e != hipSuccess) return hip_fail(e, "device properties");
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(SAGE_ERR_DEVICE,
                    "sage attention needs INT8 and FP8 MFMA of an MI355X-class GPU (gfx950); this GPU is %s",
                    p.gcnArchName);
    return ok();
}

sage_status sage_new(void* stream, uint64_t head_dim, const sage_config* config, sage_attention** out) {
    if (!out) return fail(SAGE_ERR_INVALID, "null output");
    *out = nullptr;
    if (head_dim != 64 && head_dim != 128)
        return fail(SAGE_ERR_INVALID, "sage attention supports head dim 64 or 128, got %llu", (u64)head_dim);
    const sage_config cfg = config ? *config : sage_config_for_head_dim(head_dim);
    sage_status st = sage_tile_validate(&cfg.tile);
    if (st != SAGE_OK) return st;
    if (cfg.pv_accum != SAGE_PV_F32 && cfg.pv_accum != SAGE_PV_F16)
        return fail(SAGE_ERR_INVALID, "unknown PvAccum %d", cfg.pv_accum);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "current device");
    st = sage_check_device(dev);
    if (st != SAGE_OK) return st;
    // sage_forward_noalloc's scratch address on this device, looked up now so
    // that the entry point itself only launches kernels.
    st = sage::noalloc_init(dev);
    if (st != SAGE_OK) return st;
    // No C++ exception may cross the C ABI: allocation failure is a status.
    sage_attention* s = new (std::nothrow) sage_attention;
    if (!s) return fail(SAGE_ERR_DEVICE, "out of host memory");
    s->stream = static_cast<hipStream_t>(stream);
    s->device = dev;
    s->head_dim = head_dim;
    s->config = cfg;
    *out = s;
    return ok();
}

void sage_destroy(sage_attention* s) { delete s; }
uint64_t sage_head_dim(const sage_attention* s) { return s ? s->head_dim : 0; }
sage_config sage_get_config(const sage_attention* s) { return s ? s->config : sage_config{}; }
void* sage_stream(const sage_attention* s) { return s ? static_cast<void*>(s->stream) : nullptr; }

sage_status sage_attn_resources(const sage_attention* s, int32_t* regs, int32_t* spill, int32_t* lds) {
    return sage_attn_kernel_resources(s, SAGE_KERNEL_DENSE, regs, spill, lds);
}

sage_status sage_attn_kernel_resources(const sage_attention* s, int32_t kernel, int32_t* regs, int32_t* spill,
                                       int32_t* lds) {
    if (!s || !regs || !spill || !lds) return fail(SAGE_ERR_INVALID, "null argument");
    if (kernel != SAGE_KERNEL_DENSE && kernel != SAGE_KERNEL_CAUSAL && kernel != SAGE_KERNEL_MERGED)
        return fail(SAGE_ERR_INVALID, "unknown attention kernel %d", kernel);
    int r = 0, sp = 0, l = 0;
    hipError_t e = sage::attention_resources((int)s->head_dim, kernel == SAGE_KERNEL_CAUSAL,
                                             kernel == SAGE_KERNEL_MERGED, s->config.tile.warps == 8, &r, &sp, &l);
    if (e != hipSuccess) return hip_fail(e, "registers");
    *regs = r;
    *spill = sp;
    *lds = l;
    return ok();
}

static void ws_free(sage_workspace* w) {
    void* bufs[] = {w->q8, w->q_scale, w->k8, w->k_scale, w->v8, w->stats, w->kbias, w->part};
    for (void* p : bufs)
        if (p) (void)hipFree(p);
}

}  // extern "C"

namespace sage {

sage_status set_error(sage_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

sage_status workspace_layout(const sage_attention* s, const sage_shape* shape, const sage_kv_merge* merge,
                             sage_plan* plan_out, WsSizes* n) {
    sage_kv_merge dense{};
    dense.stride = 1;
    sage_plan plan;
    sage_status st = sage_plan_new(shape, merge ? merge : &dense, &plan);
    if (st != SAGE_OK) return st;
    const uint64_t b = plan.shape.batch, h = plan.shape.heads, hk = plan.shape.kv_heads, d = s->head_dim;
    // Every buffer size, and their sum in bytes, must be addressable: the
    // plan's i32 checks bound each factor, not their products. The code
    // buffers and the partials dominate; capping them at 2^62 bytes keeps the
    // scale, statistics and bias buffers' small additions from wrapping too.
    uint64_t n_q8, n_k8, n_part, total;
    const bool wraps = __builtin_mul_overflow(b * h, plan.tq_pad, &n_q8) || __builtin_mul_overflow(n_q8, d, &n_q8) ||
                       __builtin_mul_overflow(b * hk, plan.tk_pad, &n_k8) || __builtin_mul_overflow(n_k8, d, &n_k8) ||
                       __builtin_mul_overflow(b * hk * 4 * d, plan.tq_pad / SAGE_QTILE, &n_part) ||
                       __builtin_mul_overflow(n_part, (uint64_t)4, &total) ||
                       __builtin_add_overflow(total, n_q8, &total) || __builtin_add_overflow(total, n_k8, &total) ||
                       __builtin_add_overflow(total, n_k8, &total) || total > (1ull << 62);
    if (wraps)
        return fail(SAGE_ERR_INVALID, "sage workspace for %s is too large to address", shape_dbg(*shape).c_str());
    n->q8 = n_q8;
    n->q_scale = b * h * plan.tq_pad / SAGE_QGROUP;
    n->k8 = n_k8;
    n->k_scale = b * hk * plan.tk_pad / SAGE_KBLOCK;
    n->v8 = n_k8;
    n->stats = b * hk * 4 * d;
    n->kbias = plan.tk_pad;
    n->part = n_part;
    *plan_out = plan;
    return SAGE_OK;
}

}  // namespace sage

extern "C" {

sage_status sage_workspace_new(const sage_attention* s, const sage_shape* shape, const sage_kv_merge* merge,
                           sage_workspace** out) {
    if (!s || !shape || !out) return fail(SAGE_ERR_INVALID, "null argument");
    *out = nullptr;
    sage_plan plan;
    sage::WsSizes n;
    sage_status st = sage::workspace_layout(s, shape, merge, &plan, &n);
    if (st != SAGE_OK) return st;
    sage_workspace* w = new (std::nothrow) sage_workspace;
    if (!w) return fail(SAGE_ERR_DEVICE, "out of host memory");
    w->plan = plan;
    w->head_dim = s->head_dim;
    w->device = s->device;
    w->n_q8 = n.q8;
    w->n_q_scale = n.q_scale;
    w->n_k8 = n.k8;
    w->n_k_scale = n.k_scale;
    w->n_v8 = n.v8;
    w->n_stats = n.stats;
    w->n_kbias = n.kbias;
    w->n_part = n.part;
    struct {
        void** p;
        uint64_t bytes;
    } allocs[] = {
        {(void**)&w->q8, w->n_q8},       {(void**)&w->q_scale, w->n_q_scale * 4}, {(void**)&w->k8, w->n_k8},
        {(void**)&w->k_scale, w->n_k_scale * 4}, {(void**)&w->v8, w->n_v8},       {(void**)&w->stats, w->n_stats * 4},
        {(void**)&w->kbias, w->n_kbias * 4},     {(void**)&w->part, w->n_part * 4},
    };
    for (auto& a : allocs) {
        hipError_t e = hipMalloc(a.p, a.bytes);
        if (e == hipSuccess) e = hipMemsetAsync(*a.p, 0, a.bytes, s->stream);
        if (e != hipSuccess) {
            ws_free(w);
            delete w;
            return hip_fail(e, "allocate sage workspace");
        }
    }
    *out = w;
    return ok();
}

void sage_workspace_destroy(sage_workspace* ws) {
    if (!ws) return;
    ws_free(ws);
    delete ws;
}

uint64_t sage_workspace_bytes(const sage_workspace* w) {
    if (!w) return 0;
    return w->n_q8 + 4 * w->n_q_scale + w->n_k8 + 4 * w->n_k_scale + w->n_v8 + 4 * w->n_stats + 4 * w->n_kbias +
           4 * w->n_part;
}

sage_status sage_workspace_plan(const sage_workspace* ws, sage_plan* out) {
    if (!ws || !out) return fail(SAGE_ERR_INVALID, "null argument");
    *out = ws->plan;
    return ok();
}

sage_status sage_workspace_buffers(const sage_workspace* w, sage_ws_buffers* out) {
    if (!w || !out) return fail(SAGE_ERR_INVALID, "null argument");
    out->q8 = w->q8;
    out->q_scale = w->q_scale;
    out->k8 = w->k8;
    out->k_scale = w->k_scale;
    out->v8 = w->v8;
    out->stats = w->stats;
    out->kbias = w->kbias;
    out->q8_len = w->n_q8;
    out->q_scale_len = w->n_q_scale;
    out->k8_len = w->n_k8;
    out->k_scale_len = w->n_k_scale;
    out->v8_len = w->n_v8;
    out->stats_len = w->n_stats;
    out->kbias_len = w->n_kbias;
    return ok();
}

static sage_status check_tensor(const sage_strides& st, const void* data, uint64_t len, const sage_plan& plan,
                                uint64_t heads, uint64_t d, const char* what) {
    sage_status r = sage_strides_check(&st, what);
    if (r != SAGE_OK) return r;
    const uint64_t need = sage_strides_extent(&st, plan.shape.batch, plan.shape.tokens, heads, d);
    if (len < need)
        return fail(SAGE_ERR_INVALID, "%s holds %llu elements, its shape and strides need %llu", what, (u64)len,
                    (u64)need);
    if (!data || (reinterpret_cast<uintptr_t>(data) & 15u))
        return fail(SAGE_ERR_INVALID, "%s must start at a 16-byte aligned device address", what);
    return SAGE_OK;
}

}  // extern "C"

namespace sage {

sage_status prepare_view(const sage_attention* s, const WsView& w, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_options* opts, Geom* geom, const QkvDev* qa) {
    const sage_plan& plan = w.plan;
    const uint64_t d = s->head_dim;
    const struct {
        const sage_tensor* t;
        uint64_t heads;
        const char* what;
    } ins[] = {{q, plan.shape.heads, "Q"}, {k, plan.shape.kv_heads, "K"}, {v, plan.shape.kv_heads, "V"}};
    for (auto& in : ins) {
        sage_status r = check_tensor(in.t->strides, in.t->data, in.t->len, plan, in.heads, d, in.what);
        if (r != SAGE_OK) return r;
    }
    if (q->dtype != k->dtype || q->dtype != v->dtype)
        return fail(SAGE_ERR_INVALID, "Q, K and V must share one element type");
    if (q->dtype != SAGE_BF16 && q->dtype != SAGE_F16) return fail(SAGE_ERR_INVALID, "unknown dtype %d", q->dtype);
    if (opts->qk_norm_params && opts->qk_norm_len < 4 * d)
        return fail(SAGE_ERR_INVALID, "QK-norm params hold %llu floats, need %llu", (u64)opts->qk_norm_len,
                    (u64)(4 * d));
    // Causal masking (an extension) is defined over token positions; merged
    // keys have none.
    if (opts->causal && plan.merge.stride != 1)
        return fail(SAGE_ERR_UNSUPPORTED, "causal masking over merged keys (KvMerge::Pool) is not supported");
    int flags = 0;
    if (opts->qk_norm_params) flags |= F_LN_Q | F_LN_K;  // mod.rs:715-717
    if (opts->smooth_k) flags |= F_SMOOTH_K;
    if (opts->smooth_v) flags |= F_SMOOTH_V;
    if (opts->causal) flags |= F_CAUSAL;
    if (q->dtype == SAGE_F16) flags |= F_IN_F16;
    const float scale = opts->has_softmax_scale ? opts->softmax_scale : 1.0f / std::sqrt((float)d);
    const float log2e = 1.44269504088896340736f;

    Geom g{};
    g.q_sb = (long long)q->strides.batch;
    g.q_st = (long long)q->strides.token;
    g.q_sh = (long long)q->strides.head;
    g.k_sb = (long long)k->strides.batch;
    g.k_st = (long long)k->strides.token;
    g.k_sh = (long long)k->strides.head;
    g.v_sb = (long long)v->strides.batch;
    g.v_st = (long long)v->strides.token;
    g.v_sh = (long long)v->strides.head;
    g.batch = (int)plan.shape.batch;
    g.heads = (int)plan.shape.heads;
    g.kv_heads = (int)plan.shape.kv_heads;
    g.group = (int)(plan.shape.heads / plan.shape.kv_heads);
    g.tokens = (int)plan.shape.tokens;
    g.tq_pad = (int)plan.tq_pad;
    g.tk = (int)plan.tk;
    g.tk_pad = (int)plan.tk_pad;
    g.q_tiles = (int)(plan.tq_pad / SAGE_QTILE);
    g.kblocks = (int)(plan.tk_pad / SAGE_KBLOCK);
    g.flags = flags;
    g.q_mul = scale * log2e;
    // PvAccum::F16 quantises V to +-2.25 (mod.rs:763-766). gfx950's FP8 MFMA
    // accumulates in fp32 only, so the block partials stay fp32 either way.
    g.v_range = s->config.pv_accum == SAGE_PV_F16 ? SAGE_PV16_V_RANGE : SAGE_FP8_MAX;
    g.ln_eps = opts->qk_norm_params ? opts->qk_norm_eps : 1e-5f;
    // Merge geometry (mod.rs:727-770): a dense plan is one frame of `tokens`
    // tokens with merge = 1.
    const sage_frame_layout& l = plan.merge.layout;
    const uint64_t ms = plan.merge.stride;
    g.merge = (int)ms;
    if (ms > 1) {
        g.frame_tokens = (int)tokens_per_frame(l);
        g.special = (int)l.special;
        g.grid_h = (int)l.grid_h;
        g.grid_w = (int)l.grid_w;
        g.merged_frame = (int)merged_per_frame(l, ms);
        g.merged_w = (int)((l.grid_w + ms - 1) / ms);
        g.dense_frames = (int)(l.dense_frames < l.frames ? l.dense_frames : l.frames);
    }

    PrologueBufs bufs{w.q8, w.q_scale, w.k8, w.k_scale, w.v8, w.stats, w.part, w.kbias};
    hipError_t e = launch_prologue((int)d, static_cast<const uint16_t*>(q->data), static_cast<const uint16_t*>(k->data),
                                   static_cast<const uint16_t*>(v->data), opts->qk_norm_params, bufs, g, qa,
                                   s->stream);
    if (e != hipSuccess) return hip_fail(e, "launch sage prologue");
    *geom = g;
    return SAGE_OK;
}

sage_status attend_view(const sage_attention* s, const WsView& w, const Geom& geom, const sage_tensor_mut* out) {
    const sage_plan& plan = w.plan;
    sage_status r = check_tensor(out->strides, out->data, out->len, plan, plan.shape.heads, s->head_dim, "output");
    if (r != SAGE_OK) return r;
    if (out->dtype != SAGE_BF16 && out->dtype != SAGE_F16)
        return fail(SAGE_ERR_INVALID, "unknown dtype %d", out->dtype);
    Geom g = geom;
    g.o_sb = (long long)out->strides.batch;
    g.o_st = (long long)out->strides.token;
    g.o_sh = (long long)out->strides.head;
    g.flags = (g.flags & ~(F_OUT_F16 | F_WAVES8)) | (out->dtype == SAGE_F16 ? F_OUT_F16 : 0) |
              (s->config.tile.warps == 8 ? F_WAVES8 : 0);
    AttendBufs bufs{w.q8, w.q_scale, w.k8, w.k_scale, w.v8, w.stats, w.kbias, out->data};
    hipError_t e = launch_attention((int)s->head_dim, bufs, g, s->stream);
    if (e != hipSuccess) return hip_fail(e, "launch sage attention");
    return SAGE_OK;
}

}  // namespace sage

extern "C" {

static sage::WsView view_of(const sage_workspace* w) {
    return sage::WsView{w->plan, w->q8, w->q_scale, w->k8, w->k_scale, w->v8, w->stats, w->kbias, w->part};
}

sage_status sage_prepare(const sage_attention* s, sage_workspace* ws, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_options* opts) {
    if (!s || !ws || !q || !k || !v || !opts) return fail(SAGE_ERR_INVALID, "null argument");
    if (ws->head_dim != s->head_dim)
        return fail(SAGE_ERR_INVALID, "workspace was made for head dim %llu, kernels are %llu", (u64)ws->head_dim,
                    (u64)s->head_dim);
    sage::Geom g;
    sage_status r = sage::prepare_view(s, view_of(ws), q, k, v, opts, &g, nullptr);
    if (r != SAGE_OK) return r;
    ws->geom = g;
    ws->prepared = true;
    return ok();
}

sage_status sage_attend(const sage_attention* s, const sage_workspace* ws, const sage_tensor_mut* out) {
    if (!s || !ws || !out) return fail(SAGE_ERR_INVALID, "null argument");
    if (!ws->prepared) return fail(SAGE_ERR_STATE, "sage workspace has not been prepared");
    if (ws->head_dim != s->head_dim)
        return fail(SAGE_ERR_INVALID, "workspace was made for head dim %llu, kernels are %llu", (u64)ws->head_dim,
                    (u64)s->head_dim);
    sage_status r = sage::attend_view(s, view_of(ws), ws->geom, out);
    return r == SAGE_OK ? ok() : r;
}

sage_status sage_forward(const sage_attention* s, sage_workspace* ws, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_tensor_mut* out, const sage_options* opts) {
    sage_status r = sage_prepare(s, ws, q, k, v, opts);
    if (r != SAGE_OK) return r;
    return sage_attend(s, ws, out);
}

}  // extern "C"

// ---------------------------------------------------------------- QKV prologue
namespace {

// Ptrs::input / Ptrs::output (lib.rs:247-287): "<what>: buffer holds N elements, needs M".
bool holds(uint64_t have, uint64_t need, const char* what, sage_status* st) {
    if (have < need) {
        *st = fail(SAGE_ERR_INVALID, "%s: buffer holds %llu elements, needs %llu", what, (u64)have, (u64)need);
        return false;
    }
    return true;
}

// check_aligned (norm.rs:361-366), for `bytes`-byte alignment.
bool aligned(const void* p, uintptr_t bytes, sage_status* st) {
    if (reinterpret_cast<uintptr_t>(p) % bytes) {
        *st = fail(SAGE_ERR_INVALID, "device pointer %#llx is not %u-byte aligned",
                   (u64) reinterpret_cast<uintptr_t>(p), (unsigned)bytes);
        return false;
    }
    return true;
}

// QkvPrologue::run's checks (qkv.rs:226-279) for batch x tokens tokens of
// heads / kv_heads heads of dimension d, in three parts taken in the
// reference's order: the input buffers' sizes (qkv_inputs), then the
// outputs' (the caller's), then the norm and RoPE options (qkv_options), and
// last the alignment of y, chan, bias and the outputs (qkv_aligned; the
// norm weights and the RoPE table, f32, need no more than their type's).
// *bs receives the batch stride of y.
sage_status qkv_inputs(uint64_t batch, uint64_t tokens, uint64_t heads, uint64_t kv, uint64_t d,
                       const sage_qkv_in* in, sage::QkvDev* qa, uint64_t* bs) {
    sage_status st = SAGE_OK;
    const uint64_t width = (heads + 2 * kv) * d;
    const uint64_t stride = in->batch_stride ? in->batch_stride : tokens * in->ld;
    uint64_t a, b2, need;
    if (stride % 8)
        return fail(SAGE_ERR_INVALID, "qkv: batch stride %llu must be a multiple of 8", (u64)stride);
    if (__builtin_mul_overflow(batch - 1, stride, &a) || __builtin_mul_overflow(tokens - 1, in->ld, &b2) ||
        __builtin_add_overflow(a, b2, &need) || __builtin_add_overflow(need, width, &need))
        return fail(SAGE_ERR_INVALID, "qkv y: buffer holds %llu elements, needs more than 2^64", (u64)in->y_len);
    if (!holds(in->y_len, need, "qkv y", &st)) return st;
    if (in->tok && !holds(in->tok_len, batch * tokens, "qkv tok scales", &st)) return st;
    if (in->chan && !holds(in->chan_len, width, "qkv channel scales", &st)) return st;
    if (in->bias && !holds(in->bias_len, width, "qkv bias", &st)) return st;
    *qa = sage::QkvDev{};
    qa->tok = in->tok;
    qa->chan = in->chan;
    qa->bias = in->bias;
    *bs = stride;
    return SAGE_OK;
}

sage_status qkv_options(uint64_t d, const sage_qkv_norm* norm, const sage_qkv_rope* rope, sage::QkvDev* qa) {
    sage_status st = SAGE_OK;
    if (norm) {
        if (norm->kind != SAGE_QKV_LAYER_NORM && norm->kind != SAGE_QKV_RMS_NORM)
            return fail(SAGE_ERR_INVALID, "qkv: unknown QK-norm kind %d", norm->kind);
        if (!norm->q_weight || !holds(norm->len, d, "q norm weight", &st)) return norm->q_weight ? st :
            fail(SAGE_ERR_INVALID, "q norm weight: buffer holds 0 elements, needs %llu", (u64)d);
        if (!norm->k_weight || !holds(norm->len, d, "k norm weight", &st)) return norm->k_weight ? st :
            fail(SAGE_ERR_INVALID, "k norm weight: buffer holds 0 elements, needs %llu", (u64)d);
        if (norm->kind == SAGE_QKV_LAYER_NORM) {
            if (!norm->q_bias || !norm->k_bias)
                return fail(SAGE_ERR_INVALID, "qkv: LayerNorm QK-norm needs q and k biases");
            if (!holds(norm->len, d, "q norm bias", &st) || !holds(norm->len, d, "k norm bias", &st)) return st;
        }
        qa->norm = norm->kind;
        qa->nw[0] = norm->q_weight;
        qa->nw[1] = norm->q_bias;
        qa->nw[2] = norm->k_weight;
        qa->nw[3] = norm->k_bias;
        qa->eps = norm->eps;
    }
    if (rope) {
        if (rope->frame_len == 0) return fail(SAGE_ERR_INVALID, "qkv: RoPE frame length is 0");
        if (rope->layout != SAGE_ROPE_VGGT && rope->layout != SAGE_ROPE_DINOV3)
            return fail(SAGE_ERR_INVALID, "qkv: unknown RoPE layout %d", rope->layout);
        if (rope->frame_len > 0x7fffffffull)
            return fail(SAGE_ERR_INVALID, "frame_len = %llu does not fit in i32", (u64)rope->frame_len);
        if (!rope->table || !holds(rope->table_len, rope->frame_len * d, "RoPE table", &st))
            return rope->table ? st
                               : fail(SAGE_ERR_INVALID, "RoPE table: buffer holds 0 elements, needs %llu",
                                      (u64)(rope->frame_len * d));
        qa->rope = rope->table;
        qa->rope_half = (int)(rope->layout == SAGE_ROPE_VGGT ? d / 4 : d / 2);
        qa->rope_shift = 0;
        while ((1 << qa->rope_shift) < qa->rope_half) qa->rope_shift++;
        qa->frame_len = (int)rope->frame_len;
        // The kernels' t % frame_len by multiplication (Granlund-Montgomery,
        // the form documented at QkvDev::fl_magic).
        const uint64_t fl = rope->frame_len;
        int l = 0;
        while ((1ull << l) < fl) l++;
        qa->fl_shift = l;
        qa->fl_magic = (uint32_t)(((1ull << 32) * ((1ull << l) - fl)) / fl + 1);
    }
    return SAGE_OK;
}

// check_aligned (qkv.rs:279) over y, chan, bias and the outputs (outs, n of
// them; 16-byte vector loads and stores), plus the per-token scales' f32.
sage_status qkv_aligned(const sage_qkv_in* in, const void* const* outs, int n) {
    sage_status st = SAGE_OK;
    if (!aligned(in->y, 16, &st) || (in->chan && !aligned(in->chan, 16, &st)) ||
        (in->bias && !aligned(in->bias, 16, &st)))
        return st;
    for (int i = 0; i < n; i++)
        if (!aligned(outs[i], 16, &st)) return st;
    if (in->tok && !aligned(in->tok, 4, &st)) return st;
    return SAGE_OK;
}

bool qkv_ld_ok(const sage_qkv_in* in, uint64_t width, sage_status* st) {
    if (in->ld < width || in->ld % 8) {
        *st = fail(SAGE_ERR_INVALID, "qkv: ld %llu must be a multiple of 8 and at least %llu", (u64)in->ld, (u64)width);
        return false;
    }
    return true;
}

}  // namespace

extern "C" {

sage_status sage_rope_table(int32_t layout, uint64_t head_dim, uint64_t grid_h, uint64_t grid_w, uint64_t special,
                            double base, float* out, uint64_t out_len) {
    if (!out) return fail(SAGE_ERR_INVALID, "null argument");
    if (layout != SAGE_ROPE_VGGT && layout != SAGE_ROPE_DINOV3)
        return fail(SAGE_ERR_INVALID, "qkv: unknown RoPE layout %d", layout);
    if (head_dim != 64 && head_dim != 128)
        return fail(SAGE_ERR_INVALID, "sage attention supports head dim 64 or 128, got %llu", (u64)head_dim);
    const uint64_t frame_len = special + grid_h * grid_w, pairs = head_dim / 2, axis = pairs / 2;
    sage_status st = SAGE_OK;
    if (!holds(out_len, frame_len * pairs * 2, "RoPE table", &st)) return st;
    const double pi = 3.14159265358979323846;
    for (uint64_t t = 0; t < frame_len; t++)
        for (uint64_t p = 0; p < pairs; p++) {
            double a = 0.0;
            if (t >= special) {
                const uint64_t y = (t - special) / grid_w, x = (t - special) % grid_w;
                if (layout == SAGE_ROPE_VGGT) {
                    const double pos = (double)(p < axis ? y + 1 : x + 1);
                    a = pos * std::pow(base, -(double)(p % axis) / (double)axis);
                } else {
                    const double coord = p < axis ? ((double)y + 0.5) / (double)grid_h * 2.0 - 1.0
                                                  : ((double)x + 0.5) / (double)grid_w * 2.0 - 1.0;
                    a = 2.0 * pi * coord / std::pow(base, (double)(p % axis) / (double)axis);
                }
            }
            out[(t * pairs + p) * 2] = (float)std::cos(a);
            out[(t * pairs + p) * 2 + 1] = (float)std::sin(a);
        }
    return ok();
}

sage_status sage_qkv_prologue(const sage_attention* s, const sage_shape* shape, const sage_qkv_in* in,
                              const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_tensor_mut* q,
                              const sage_tensor_mut* k, const sage_tensor_mut* v) {
    if (!s || !shape || !in || !q || !k || !v) return fail(SAGE_ERR_INVALID, "null argument");
    const uint64_t d = s->head_dim, heads = shape->heads, kv = shape->kv_heads ? shape->kv_heads : shape->heads;
    sage_status st = SAGE_OK;
    if (!qkv_ld_ok(in, (heads + 2 * kv) * d, &st)) return st;
    if (shape->tokens == 0 || heads == 0 || shape->batch == 0) return ok();
    if (heads % kv)
        return fail(SAGE_ERR_INVALID, "%llu query heads are not a multiple of %llu KV heads", (u64)heads, (u64)kv);
    // The kernel's grid takes the part-head slots in y and the batch in z.
    if (shape->tokens > 0x7fffffffull || shape->batch > 65535 || heads + 2 * kv > 65535)
        return fail(SAGE_ERR_INVALID, "qkv: %llu batch items of %llu part-head slots exceed the launch grid",
                    (u64)shape->batch, (u64)(heads + 2 * kv));
    sage::QkvDev qa;
    uint64_t bs = 0;
    st = qkv_inputs(shape->batch, shape->tokens, heads, kv, d, in, &qa, &bs);
    if (st != SAGE_OK) return st;
    const sage_tensor_mut* outs[3] = {q, k, v};
    const char* names[3] = {"qkv q", "qkv k", "qkv v"};
    sage::QkvOutDev o{};
    for (int i = 0; i < 3; i++) {
        const sage_tensor_mut* t = outs[i];
        st = sage_strides_check(&t->strides, names[i]);
        if (st != SAGE_OK) return st;
        const uint64_t need = sage_strides_extent(&t->strides, shape->batch, shape->tokens, i ? kv : heads, d);
        if (!holds(t->len, need, names[i], &st)) return st;
        const bool f16_ok = i == 2;
        if (t->dtype != SAGE_BF16 && !(f16_ok && t->dtype == SAGE_F16))
            return fail(SAGE_ERR_INVALID, "%s must be bf16%s", names[i], f16_ok ? " or fp16" : "");
        o.p[i] = static_cast<uint16_t*>(t->data);
        o.sb[i] = (long long)t->strides.batch;
        o.st[i] = (long long)t->strides.token;
        o.sh[i] = (long long)t->strides.head;
    }
    o.v_f16 = v->dtype == SAGE_F16;
    st = qkv_options(d, norm, rope, &qa);
    if (st != SAGE_OK) return st;
    const void* out_ptrs[3] = {q->data, k->data, v->data};
    st = qkv_aligned(in, out_ptrs, 3);
    if (st != SAGE_OK) return st;
    sage::Geom g{};
    g.batch = (int)shape->batch;
    g.heads = (int)heads;
    g.kv_heads = (int)kv;
    g.tokens = (int)shape->tokens;
    g.q_sb = (long long)bs;
    g.q_st = (long long)in->ld;
    hipError_t e = sage::launch_qkv((int)d, static_cast<const uint16_t*>(in->y), o, g, qa, s->stream);
    if (e != hipSuccess) return hip_fail(e, "qkv_prologue");
    return ok();
}

sage_status sage_prepare_qkv(const sage_attention* s, sage_workspace* ws, const sage_qkv_in* in,
                             const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_options* opts) {
    if (!s || !ws || !in || !opts) return fail(SAGE_ERR_INVALID, "null argument");
    if (ws->head_dim != s->head_dim)
        return fail(SAGE_ERR_INVALID, "workspace was made for head dim %llu, kernels are %llu", (u64)ws->head_dim,
                    (u64)s->head_dim);
    const sage_shape& sh = ws->plan.shape;
    const uint64_t d = s->head_dim, heads = sh.heads, kv = sh.kv_heads;
    sage_status st = SAGE_OK;
    if (!qkv_ld_ok(in, (heads + 2 * kv) * d, &st)) return st;
    sage::QkvDev qa;
    uint64_t bs = 0;
    st = qkv_inputs(sh.batch, sh.tokens, heads, kv, d, in, &qa, &bs);
    if (st == SAGE_OK) st = qkv_options(d, norm, rope, &qa);
    if (st == SAGE_OK) st = qkv_aligned(in, nullptr, 0);
    if (st != SAGE_OK) return st;
    // Q, K and V as views into the projection: q | k | v along the channels.
    const uint16_t* y = static_cast<const uint16_t*>(in->y);
    const sage_strides str{bs, in->ld, d};
    const sage_tensor q{y, in->y_len, str, SAGE_BF16};
    const sage_tensor k{y + heads * d, in->y_len - heads * d, str, SAGE_BF16};
    const sage_tensor v{y + (heads + kv) * d, in->y_len - (heads + kv) * d, str, SAGE_BF16};
    sage::Geom g;
    st = sage::prepare_view(s, view_of(ws), &q, &k, &v, opts, &g, &qa);
    if (st != SAGE_OK) return st;
    ws->geom = g;
    ws->prepared = true;
    return ok();
}

sage_status sage_forward_qkv(const sage_attention* s, sage_workspace* ws, const sage_qkv_in* in,
                             const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_tensor_mut* out,
                             const sage_options* opts) {
    sage_status r = sage_prepare_qkv(s, ws, in, norm, rope, opts);
    if (r != SAGE_OK) return r;
    return sage_attend(s, ws, out);
}

int32_t sage_v8_position(int32_t k) { return (k < 0 || k >= SAGE_KBLOCK) ? -1 : sage::v8_position(k); }

sage_status sage_peak(const sage_attention* s, int32_t which, int32_t iters, double* tops) {
    if (!s || !tops) return fail(SAGE_ERR_INVALID, "null argument");
    if (which < 0 || which > 2) return fail(SAGE_ERR_INVALID, "unknown peak probe %d", which);
    if (iters <= 0) return fail(SAGE_ERR_INVALID, "peak probe needs iters > 0");
    hipError_t e = sage::run_peak(which, iters, s->stream, tops);
    if (e != hipSuccess) return hip_fail(e, "peak probe");
    return ok();
}

}  // extern "C"
