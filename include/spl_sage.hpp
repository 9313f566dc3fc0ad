// spl_sage.hpp -- C++ host API of the MI355X (gfx950) SageAttention2 path.
//
// The reference's host side is the Rust module `spl_nn::sage`
// (sezer-muhammed/sota-papers-lab, platform/spl-nn/src/sage/mod.rs). This
// header restates that API in C++17 over the C ABI of sage_hip.h: the same
// type and method names, argument meanings and error texts. Rust's
// `anyhow::Result` becomes a thrown spl_sage::Error carrying the reference's
// message and the C status; Rust's `CudaSlice` views become (device pointer,
// element count) pairs; `SageAttention::new` is `SageAttention::create`
// (`new` is a C++ keyword). Header-only: link libsage_hip.so.
//
// Like the reference, every GPU call enqueues on the context's stream and
// returns without synchronising (mod.rs:509-510).
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sage_hip.h"

namespace spl_sage {

// mod.rs:70-77, :183-185.
constexpr std::size_t QGROUP = SAGE_QGROUP;
constexpr std::size_t QTILE = SAGE_QTILE;
constexpr std::size_t KBLOCK = SAGE_KBLOCK;
constexpr float FP8_MAX = SAGE_FP8_MAX;
constexpr float PV16_V_RANGE = SAGE_PV16_V_RANGE;

// A failed call: the reference's error text and the C status (SAGE_ERR_*).
class Error : public std::runtime_error {
public:
    Error(sage_status status, const std::string& what) : std::runtime_error(what), status_(status) {}
    sage_status status() const { return status_; }

private:
    sage_status status_;
};

inline void check(sage_status s) {
    if (s != SAGE_OK) throw Error(s, sage_last_error());
}

// Element type of the 16-bit tensors (bf16 as the reference; fp16 is an extension).
enum class Dtype : int32_t { Bf16 = SAGE_BF16, F16 = SAGE_F16 };

// PvAccum (mod.rs:170-181).
enum class PvAccum : int32_t { F32 = SAGE_PV_F32, F16 = SAGE_PV_F16 };

// Tile (mod.rs:116-168): the reference's CTA shape (warps, 16-row m-tiles,
// K/V ring stages). Validated as the reference validates it. It picks the
// workgroup layout, never the results: warps = 8 (dense and causal
// attention) runs eight waves a workgroup (score waves and output waves),
// every other tile four waves that each do a whole block.
struct Tile {
    uint32_t warps = 4, m_tiles = 2, stages = 3;

    static const Tile DEFAULT;  // mod.rs:128-132
    static const Tile D128;     // mod.rs:136-140
    static Tile for_head_dim(std::size_t head_dim);
    std::size_t rows() const { return 16u * m_tiles * warps; }
    sage_tile raw() const { return sage_tile{warps, m_tiles, stages}; }
    void validate() const {
        const sage_tile t = raw();
        check(sage_tile_validate(&t));
    }
};

// Config (mod.rs:187-201).
struct Config {
    Tile tile;
    PvAccum pv_accum = PvAccum::F32;

    static Config for_head_dim(std::size_t head_dim) {
        const sage_config c = sage_config_for_head_dim(head_dim);
        return Config{Tile{c.tile.warps, c.tile.m_tiles, c.tile.stages}, static_cast<PvAccum>(c.pv_accum)};
    }
    sage_config raw() const { return sage_config{tile.raw(), static_cast<int32_t>(pv_accum)}; }
};

inline const Tile Tile::DEFAULT{4, 2, 3};
inline const Tile Tile::D128{4, 1, 3};
inline Tile Tile::for_head_dim(std::size_t head_dim) { return Config::for_head_dim(head_dim).tile; }

// Shape (mod.rs:262-268); kv_heads (0 = heads) is the grouped-query extension.
struct Shape {
    std::size_t batch = 1, heads = 1, tokens = 0, kv_heads = 0;

    std::size_t kv() const { return kv_heads ? kv_heads : heads; }
    sage_shape raw() const { return sage_shape{batch, heads, tokens, kv_heads}; }
};

// Strides (mod.rs:203-260): element strides of [batch][token][head][dim],
// channels contiguous.
struct Strides {
    std::size_t batch = 0, token = 0, head = 0;

    static Strides bthd(std::size_t tokens, std::size_t heads, std::size_t d) {
        return Strides{tokens * heads * d, heads * d, d};
    }
    static Strides bhtd(std::size_t tokens, std::size_t heads, std::size_t d) {
        return Strides{heads * tokens * d, d, tokens * d};
    }
    // Q, K and V of one fused projection, [batch][token][3][head][dim]; K and
    // V views start head * d and 2 * head * d elements in.
    static Strides packed_qkv(std::size_t tokens, std::size_t heads, std::size_t d) {
        return Strides{tokens * 3 * heads * d, 3 * heads * d, d};
    }
    sage_strides raw() const { return sage_strides{batch, token, head}; }
    // Elements from the first to one past the last addressed (mod.rs:244-249).
    std::size_t extent(const Shape& s, std::size_t d) const { return extent(s, d, s.heads); }
    std::size_t extent(const Shape& s, std::size_t d, std::size_t heads) const {
        const sage_strides r = raw();
        return sage_strides_extent(&r, s.batch, s.tokens, heads, d);
    }
    void check(const char* what) const {
        const sage_strides r = raw();
        spl_sage::check(sage_strides_check(&r, what));
    }
};

// FrameLayout (mod.rs:270-300).
struct FrameLayout {
    std::size_t frames = 1, special = 0, grid_h = 0, grid_w = 0, dense_frames = 0;

    std::size_t tokens_per_frame() const { return special + grid_h * grid_w; }
    std::size_t merged_per_frame(std::size_t stride) const {
        return special + ((grid_h + stride - 1) / stride) * ((grid_w + stride - 1) / stride);
    }
    std::size_t merged_keys(std::size_t stride) const {
        const std::size_t d = dense_frames < frames ? dense_frames : frames;
        return d * tokens_per_frame() + (frames - d) * merged_per_frame(stride);
    }
    sage_frame_layout raw() const { return sage_frame_layout{frames, special, grid_h, grid_w, dense_frames}; }
};

// KvMerge (mod.rs:302-311): Dense, or Pool { stride, layout }.
struct KvMerge {
    uint32_t stride = 1;
    FrameLayout layout;

    static KvMerge Dense() { return KvMerge{}; }
    static KvMerge Pool(uint32_t stride, const FrameLayout& layout) { return KvMerge{stride, layout}; }
    bool is_dense() const { return stride == 1; }
    sage_kv_merge raw() const { return sage_kv_merge{stride, layout.raw()}; }
};

// Plan (mod.rs:391-454).
struct Plan {
    Shape shape;
    KvMerge merge;
    std::size_t tq_pad = 0, tk = 0, tk_pad = 0;

    static Plan create(const Shape& shape, const KvMerge& merge = KvMerge::Dense()) {
        const sage_shape s = shape.raw();
        const sage_kv_merge m = merge.raw();
        sage_plan p{};
        spl_sage::check(sage_plan_new(&s, &m, &p));
        return Plan{shape, merge, p.tq_pad, p.tk, p.tk_pad};
    }
    std::size_t q_tiles() const { return tq_pad / QTILE; }
    std::size_t kblocks() const { return tk_pad / KBLOCK; }
    sage_plan raw() const { return sage_plan{shape.raw(), merge.raw(), tq_pad, tk, tk_pad}; }
};

// flops (mod.rs:905-910); causal counts the visible pairs (extension).
inline double flops(const Plan& plan, std::size_t head_dim, bool causal = false) {
    const sage_plan p = plan.raw();
    return sage_flops(&p, head_dim, causal ? 1 : 0);
}

// check_device (mod.rs:552-566), for gfx950.
inline void check_device(int ordinal = 0) { check(sage_check_device(ordinal)); }

// Byte of key k (0..63) within each channel row of a v8 block.
inline int v8_position(int k) { return sage_v8_position(k); }

// QkNorm (mod.rs:337-344): device pointer to [q weight, q bias, k weight,
// k bias], head_dim floats each.
struct QkNorm {
    const float* params = nullptr;
    std::size_t len = 0;
    float eps = 1e-5f;
};

// Options (mod.rs:313-335); `causal` is an extension.
struct Options {
    std::optional<float> softmax_scale;
    bool smooth_k = true;
    bool smooth_v = true;
    std::optional<QkNorm> qk_norm;
    bool causal = false;

    sage_options raw() const {
        sage_options o{};
        o.softmax_scale = softmax_scale.value_or(0.0f);
        o.has_softmax_scale = softmax_scale.has_value() ? 1 : 0;
        o.smooth_k = smooth_k ? 1 : 0;
        o.smooth_v = smooth_v ? 1 : 0;
        if (qk_norm) {
            o.qk_norm_params = qk_norm->params;
            o.qk_norm_len = qk_norm->len;
            o.qk_norm_eps = qk_norm->eps;
        }
        o.causal = causal ? 1 : 0;
        return o;
    }
};

// Tensor / TensorMut (mod.rs:497-507): a device buffer of `len` 16-bit
// elements viewed with `strides`.
struct Tensor {
    const void* data = nullptr;
    std::size_t len = 0;
    Strides strides;
    Dtype dtype = Dtype::Bf16;

    sage_tensor raw() const { return sage_tensor{data, len, strides.raw(), static_cast<int32_t>(dtype)}; }
};

struct TensorMut {
    void* data = nullptr;
    std::size_t len = 0;
    Strides strides;
    Dtype dtype = Dtype::Bf16;

    sage_tensor_mut raw() const { return sage_tensor_mut{data, len, strides.raw(), static_cast<int32_t>(dtype)}; }
};

// Workspace (mod.rs:456-495): owns the device buffers of one plan. The
// buffers are the reference's pub fields, as device pointers.
class Workspace {
public:
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    Workspace(Workspace&& o) noexcept : h_(std::exchange(o.h_, nullptr)), plan_(o.plan_) {}
    Workspace& operator=(Workspace&& o) noexcept {
        if (this != &o) {
            reset();
            h_ = std::exchange(o.h_, nullptr);
            plan_ = o.plan_;
        }
        return *this;
    }
    ~Workspace() { reset(); }

    const Plan& plan() const { return plan_; }
    std::size_t bytes() const { return sage_workspace_bytes(h_); }
    sage_ws_buffers buffers() const {
        sage_ws_buffers b{};
        check(sage_workspace_buffers(h_, &b));
        return b;
    }
    int8_t* q8() const { return buffers().q8; }
    float* q_scale() const { return buffers().q_scale; }
    int8_t* k8() const { return buffers().k8; }
    float* k_scale() const { return buffers().k_scale; }
    uint8_t* v8() const { return buffers().v8; }
    float* stats() const { return buffers().stats; }
    float* kbias() const { return buffers().kbias; }

    sage_workspace* handle() const { return h_; }

private:
    friend class SageAttention;
    Workspace(sage_workspace* h, const Plan& plan) : h_(h), plan_(plan) {}
    void reset() {
        if (h_) sage_workspace_destroy(h_);
        h_ = nullptr;
    }
    sage_workspace* h_;
    Plan plan_;
};

// SageAttention (mod.rs:509-901): the kernels of one head dim and Config,
// bound to one stream (a hipStream_t; nullptr = the null stream).
class SageAttention {
public:
    // SageAttention::new (mod.rs:571-577).
    static SageAttention create(void* stream, std::size_t head_dim) {
        return SageAttention(stream, head_dim, nullptr);
    }
    // SageAttention::with_config (mod.rs:579-626).
    static SageAttention with_config(void* stream, std::size_t head_dim, const Config& config) {
        const sage_config c = config.raw();
        return SageAttention(stream, head_dim, &c);
    }

    SageAttention(const SageAttention&) = delete;
    SageAttention& operator=(const SageAttention&) = delete;
    SageAttention(SageAttention&& o) noexcept : h_(std::exchange(o.h_, nullptr)) {}
    SageAttention& operator=(SageAttention&& o) noexcept {
        if (this != &o) {
            if (h_) sage_destroy(h_);
            h_ = std::exchange(o.h_, nullptr);
        }
        return *this;
    }
    ~SageAttention() {
        if (h_) sage_destroy(h_);
    }

    std::size_t head_dim() const { return sage_head_dim(h_); }
    Config config() const {
        const sage_config c = sage_get_config(h_);
        return Config{Tile{c.tile.warps, c.tile.m_tiles, c.tile.stages}, static_cast<PvAccum>(c.pv_accum)};
    }
    void* stream() const { return sage_stream(h_); }

    // attn_resources (mod.rs:640-646): (VGPRs per lane, spill bytes).
    std::pair<int, int> attn_resources() const {
        int32_t regs = 0, spill = 0, lds = 0;
        check(sage_attn_resources(h_, &regs, &spill, &lds));
        return {regs, spill};
    }

    // SageAttention::workspace (mod.rs:648-670).
    Workspace workspace(const Shape& shape, const KvMerge& merge = KvMerge::Dense()) const {
        const sage_shape s = shape.raw();
        const sage_kv_merge m = merge.raw();
        sage_workspace* w = nullptr;
        check(sage_workspace_new(h_, &s, &m, &w));
        sage_plan p{};
        const sage_status st = sage_workspace_plan(w, &p);
        if (st != SAGE_OK) {
            const std::string msg = sage_last_error();
            sage_workspace_destroy(w);
            throw Error(st, msg);
        }
        return Workspace(w, Plan{shape, merge, p.tq_pad, p.tk, p.tk_pad});
    }

    // SageAttention::prepare (mod.rs:672-836).
    void prepare(Workspace& ws, const Tensor& q, const Tensor& k, const Tensor& v, const Options& opts = {}) const {
        const sage_tensor tq = q.raw(), tk = k.raw(), tv = v.raw();
        const sage_options o = opts.raw();
        check(sage_prepare(h_, ws.h_, &tq, &tk, &tv, &o));
    }

    // SageAttention::attend (mod.rs:838-886).
    void attend(const Workspace& ws, const TensorMut& out) const {
        const sage_tensor_mut to = out.raw();
        check(sage_attend(h_, ws.h_, &to));
    }

    // SageAttention::forward (mod.rs:888-900): prepare, then attend.
    void forward(Workspace& ws, const Tensor& q, const Tensor& k, const Tensor& v, const TensorMut& out,
                 const Options& opts = {}) const {
        prepare(ws, q, k, v, opts);
        attend(ws, out);
    }

    // forward without a workspace (sage_forward_noalloc; no counterpart in the
    // reference): the buffers come from the library's fixed per-GPU scratch
    // array, nothing is allocated; calls that can overlap on one GPU race.
    void forward_noalloc(const Shape& shape, const Tensor& q, const Tensor& k, const Tensor& v, const TensorMut& out,
                         const Options& opts = {}, const KvMerge& merge = KvMerge{}) const {
        const sage_shape sh = shape.raw();
        const sage_kv_merge m = merge.raw();
        const sage_tensor tq = q.raw(), tk = k.raw(), tv = v.raw();
        const sage_tensor_mut to = out.raw();
        const sage_options o = opts.raw();
        check(sage_forward_noalloc(h_, &sh, &m, &tq, &tk, &tv, &to, &o));
    }

    // MFMA peak probe (the analogue of sage_peak.cu): which = 0 INT8, 1 FP8,
    // 2 BF16; synchronises and returns dense TOPS.
    double peak(int which, int iters = 2048) const {
        double tops = 0.0;
        check(sage_peak(h_, which, iters, &tops));
        return tops;
    }

    sage_attention* handle() const { return h_; }

private:
    SageAttention(void* stream, std::size_t head_dim, const sage_config* config) : h_(nullptr) {
        check(sage_new(stream, head_dim, config, &h_));
    }
    sage_attention* h_;
};

// ---------------------------------------------------------------- qkv
// spl_nn::qkv (platform/spl-nn/src/qkv.rs): the QKV prologue that feeds sage.
namespace qkv {

constexpr std::size_t HEAD_DIM = 64;  // the reference's head dim; 128 is an extension

// RopeLayout (qkv.rs:33-58).
enum class RopeLayout : int32_t { Vggt = SAGE_ROPE_VGGT, Dinov3 = SAGE_ROPE_DINOV3 };

inline std::size_t rope_half(RopeLayout l, std::size_t head_dim = HEAD_DIM) {
    return l == RopeLayout::Vggt ? head_dim / 4 : head_dim / 2;
}
inline std::size_t rope_pair(RopeLayout l, std::size_t d, std::size_t head_dim = HEAD_DIM) {
    const std::size_t h = rope_half(l, head_dim);
    return (d / (2 * h)) * h + d % h;
}

// RopeTable (qkv.rs:60-136): cos/sin per (token in frame, pair), host memory.
struct RopeTable {
    RopeLayout layout = RopeLayout::Vggt;
    std::size_t frame_len = 0;
    std::vector<float> cos_sin;  // frame_len x head_dim/2 x 2

    static RopeTable build(RopeLayout l, std::size_t grid_h, std::size_t grid_w, std::size_t special, double base,
                           std::size_t head_dim) {
        RopeTable t;
        t.layout = l;
        t.frame_len = special + grid_h * grid_w;
        t.cos_sin.resize(t.frame_len * head_dim);
        check(sage_rope_table(static_cast<int32_t>(l), head_dim, grid_h, grid_w, special, base, t.cos_sin.data(),
                              t.cos_sin.size()));
        return t;
    }
    static RopeTable vggt(std::size_t gh, std::size_t gw, std::size_t special, double base,
                          std::size_t head_dim = HEAD_DIM) {
        return build(RopeLayout::Vggt, gh, gw, special, base, head_dim);
    }
    static RopeTable dinov3(std::size_t gh, std::size_t gw, std::size_t special, double base,
                            std::size_t head_dim = HEAD_DIM) {
        return build(RopeLayout::Dinov3, gh, gw, special, base, head_dim);
    }
};

// NormKind / QkNorm (qkv.rs:138-156): device pointers to [head_dim] floats each.
enum class NormKind : int32_t { LayerNorm = SAGE_QKV_LAYER_NORM, Rms = SAGE_QKV_RMS_NORM };
struct QkNorm {
    NormKind kind = NormKind::LayerNorm;
    const float* q_weight = nullptr;
    const float* q_bias = nullptr;
    const float* k_weight = nullptr;
    const float* k_bias = nullptr;
    std::size_t len = 0;  // floats each buffer holds
    float eps = 1e-6f;
    sage_qkv_norm raw() const {
        return sage_qkv_norm{static_cast<int32_t>(kind), q_weight, q_bias, k_weight, k_bias, len, eps};
    }
};

// Rope (qkv.rs:158-163): the uploaded table (device floats) and its layout.
struct Rope {
    const float* table = nullptr;
    std::size_t table_len = 0;
    RopeLayout layout = RopeLayout::Vggt;
    std::size_t frame_len = 0;
    sage_qkv_rope raw() const {
        return sage_qkv_rope{table, table_len, static_cast<int32_t>(layout), frame_len};
    }
};

// QkvIn (qkv.rs:165-177), with a batch stride (0 = tokens * ld).
struct QkvIn {
    const uint16_t* y = nullptr;
    std::size_t y_len = 0, ld = 0, batch_stride = 0;
    const float* tok = nullptr;
    std::size_t tok_len = 0;
    const float* chan = nullptr;
    std::size_t chan_len = 0;
    const uint16_t* bias = nullptr;
    std::size_t bias_len = 0;
    sage_qkv_in raw() const {
        return sage_qkv_in{y, y_len, ld, batch_stride, tok, tok_len, chan, chan_len, bias, bias_len};
    }
};

// QkvOut (qkv.rs:188-196): V's dtype is its VFormat (bf16 or fp16).
struct QkvOut {
    TensorMut q, k, v;
};

// QkvPrologue (qkv.rs:198-306) on a SageAttention context's stream and head dim.
class QkvPrologue {
public:
    explicit QkvPrologue(const SageAttention& sa) : sa_(sa) {}
    void run(const QkvIn& in, std::size_t tokens, std::size_t heads, const QkNorm* norm, const Rope* rope,
             const QkvOut& out, std::size_t batch = 1, std::size_t kv_heads = 0) const {
        const sage_shape sh{batch, heads, tokens, kv_heads};
        const sage_qkv_in i = in.raw();
        sage_qkv_norm n{};
        sage_qkv_rope r{};
        if (norm) n = norm->raw();
        if (rope) r = rope->raw();
        const sage_tensor_mut q = out.q.raw(), k = out.k.raw(), v = out.v.raw();
        check(sage_qkv_prologue(sa_.handle(), &sh, &i, norm ? &n : nullptr, rope ? &r : nullptr, &q, &k, &v));
    }

private:
    const SageAttention& sa_;
};

// The fusion of QkvPrologue::run and SageAttention::prepare (no counterpart in
// the reference): the same codes, bit for bit, without storing Q, K and V.
inline void prepare_qkv(const SageAttention& sa, Workspace& ws, const QkvIn& in, const QkNorm* norm, const Rope* rope,
                        const Options& opts = {}) {
    const sage_qkv_in i = in.raw();
    sage_qkv_norm n{};
    sage_qkv_rope r{};
    if (norm) n = norm->raw();
    if (rope) r = rope->raw();
    const sage_options o = opts.raw();
    check(sage_prepare_qkv(sa.handle(), ws.handle(), &i, norm ? &n : nullptr, rope ? &r : nullptr, &o));
}

}  // namespace qkv

}  // namespace spl_sage
