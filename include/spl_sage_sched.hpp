// The reference's caller of SageAttention, restated in C++ over spl_sage.hpp:
// the sage half of the VGGT trunk's inter-frame attention schedule
// (sezer-muhammed/sota-papers-lab, apps/image-to-3d/src/vggt/trunk/sched.rs).
// It maps a schedule entry to a KvMerge, owns the compiled context and one
// workspace per (geometry, merge), and runs a global layer on the head-major
// bf16 Q, K and V the QKV prologue writes. The reference is Rust; this is the
// code a Rust crate over include/sage_hip.h would hold, written against the
// C++ mirror so the caller can be run and tested here.
#pragma once

#include <array>
#include <cstdio>
#include <map>
#include <optional>
#include <string>
#include <tuple>
#include <vector>

#include "spl_sage.hpp"

namespace spl_vggt {

using spl_sage::KvMerge;

// trunk/mod.rs:40-46, 206-207; qkv.rs:30.
constexpr std::size_t HEADS = 16;
constexpr std::size_t HEAD_DIM = 64;
constexpr std::size_t DEPTH = 24;
constexpr std::size_t SPECIAL = 17;
constexpr float ATTN_SCALE = 0.125f;

// TrunkGeom (trunk/mod.rs:73-93): frames of SPECIAL + grid_h x grid_w tokens.
struct TrunkGeom {
    std::size_t frames = 1, grid_h = 0, grid_w = 0;

    std::size_t patches() const { return grid_h * grid_w; }
    std::size_t tokens() const { return SPECIAL + patches(); }
    std::size_t rows() const { return frames * tokens(); }
    bool operator==(const TrunkGeom& o) const {
        return frames == o.frames && grid_h == o.grid_h && grid_w == o.grid_w;
    }
    // Rust's {:?} of the struct.
    std::string debug() const {
        char b[128];
        std::snprintf(b, sizeof b, "TrunkGeom { frames: %zu, grid_h: %zu, grid_w: %zu }", frames, grid_h, grid_w);
        return b;
    }
};

// InterKind (trunk/mod.rs:95-111): what an inter-frame block attends over.
enum class InterKind { Global, Register, Frame, Sage, Merge2, Merge4 };

inline const char* kind_name(InterKind k) {
    switch (k) {
        case InterKind::Global: return "Global";
        case InterKind::Register: return "Register";
        case InterKind::Frame: return "Frame";
        case InterKind::Sage: return "Sage";
        case InterKind::Merge2: return "Merge2";
        case InterKind::Merge4: return "Merge4";
    }
    return "?";
}

inline bool same_merge(const KvMerge& a, const KvMerge& b) {
    if (a.stride != b.stride) return false;
    if (a.is_dense()) return true;
    const auto& x = a.layout;
    const auto& y = b.layout;
    return x.frames == y.frames && x.special == y.special && x.grid_h == y.grid_h && x.grid_w == y.grid_w &&
           x.dense_frames == y.dense_frames;
}

// merge_of (sched.rs:24-46): the KV merge of a schedule entry; none when the
// entry is not a sage layer. Pooling keeps the specials and frame 0 dense; a
// single frame has nothing to merge.
inline std::optional<KvMerge> merge_of(InterKind kind, const TrunkGeom& g) {
    auto pool = [&](uint32_t stride) {
        spl_sage::FrameLayout l;
        l.frames = g.frames;
        l.special = SPECIAL;
        l.grid_h = g.grid_h;
        l.grid_w = g.grid_w;
        l.dense_frames = 1;
        return KvMerge::Pool(stride, l);
    };
    switch (kind) {
        case InterKind::Sage: return KvMerge::Dense();
        case InterKind::Merge2: return g.frames == 1 ? KvMerge::Dense() : pool(2);
        case InterKind::Merge4: return g.frames == 1 ? KvMerge::Dense() : pool(4);
        default: return std::nullopt;
    }
}

// shape (sched.rs:48-54): one sequence of every row, HEADS heads.
inline spl_sage::Shape shape(const TrunkGeom& g) { return spl_sage::Shape{1, HEADS, g.rows(), 0}; }

// workspace_bytes (sched.rs:56-71): the device bytes of one sage workspace as
// the reference's caller counts them (0 when the plan is refused).
inline std::size_t workspace_bytes(const TrunkGeom& g, const KvMerge& merge) {
    spl_sage::Plan p;
    try {
        p = spl_sage::Plan::create(shape(g), merge);
    } catch (const spl_sage::Error&) {
        return 0;
    }
    const std::size_t h = HEADS, d = HEAD_DIM, q_tiles = p.tq_pad / spl_sage::QTILE;
    return h * p.tq_pad * d + h * p.tq_pad / spl_sage::QGROUP * 4 + 2 * h * p.tk_pad * d +
           h * p.tk_pad / spl_sage::KBLOCK * 4 + h * 4 * d * 4 + p.tk_pad * 4 + h * q_tiles * 4 * d * 4;
}

using Schedule = std::array<InterKind, DEPTH>;

// merges (sched.rs:73-85): every distinct sage workspace a schedule needs, in
// first-use order.
inline std::vector<KvMerge> merges(const Schedule& sched, const TrunkGeom& g) {
    std::vector<KvMerge> out;
    for (InterKind k : sched) {
        const std::optional<KvMerge> m = merge_of(k, g);
        if (!m) continue;
        bool seen = false;
        for (const KvMerge& o : out) seen = seen || same_merge(o, *m);
        if (!seen) out.push_back(*m);
    }
    return out;
}

// One global layer through SageAttention, reading the head-major bf16 Q, K
// and V the QKV prologue writes (QK-norm already applied): sched.rs:166-223.
class SageLayer {
public:
    SageLayer(const spl_sage::SageAttention& kernels, spl_sage::Workspace& ws) : kernels_(kernels), ws_(ws) {}

    // InterAttention::v_format (trunk/mod.rs:154-158): the QKV prologue writes V in bf16 for sage.
    spl_sage::Dtype v_format() const { return spl_sage::Dtype::Bf16; }

    // InterAttention::forward (sched.rs:179-222): q, k, v are [HEADS][rows][HEAD_DIM]
    // bf16 device buffers of q_len, k_len, v_len elements; o is [rows][HEADS][HEAD_DIM].
    void forward(const uint16_t* q, std::size_t q_len, const uint16_t* k, std::size_t k_len, const uint16_t* v,
                 std::size_t v_len, uint16_t* o, std::size_t o_len, std::size_t n_seq, std::size_t seq_len) const {
        const std::size_t tokens = n_seq * seq_len;
        const spl_sage::Shape& s = ws_.plan().shape;
        if (n_seq != 1 || s.tokens != tokens) {
            char b[256];
            std::snprintf(b, sizeof b,
                          "sage layer: workspace for Shape { batch: %zu, heads: %zu, tokens: %zu }, called with %zu "
                          "\xc3\x97 %zu",
                          s.batch, s.heads, s.tokens, n_seq, seq_len);
            throw spl_sage::Error(SAGE_ERR_INVALID, b);
        }
        const spl_sage::Strides hm = spl_sage::Strides::bhtd(tokens, HEADS, HEAD_DIM);
        spl_sage::Options opts;
        opts.softmax_scale = ATTN_SCALE;
        kernels_.forward(ws_, spl_sage::Tensor{q, q_len, hm}, spl_sage::Tensor{k, k_len, hm},
                         spl_sage::Tensor{v, v_len, hm},
                         spl_sage::TensorMut{o, o_len, spl_sage::Strides::bthd(tokens, HEADS, HEAD_DIM)}, opts);
    }

    // The workspace the layer prepares (an accessor for tests; the reference keeps it private).
    const spl_sage::Workspace& workspace() const { return ws_; }

private:
    const spl_sage::SageAttention& kernels_;
    spl_sage::Workspace& ws_;
};

// Sage (sched.rs:87-164): the compiled kernels and the workspaces of the
// current geometry.
class Sage {
public:
    explicit Sage(spl_sage::PvAccum pv = spl_sage::PvAccum::F32) : pv_(pv) {}

    void set_pv_accum(spl_sage::PvAccum pv) {
        if (pv != pv_) {
            pv_ = pv;
            kernels_.reset();
        }
    }

    void release() { ws_.clear(); }

    // Compiles the kernels and allocates the workspaces `sched` needs at `g`
    // (dropping those of other geometries). Call outside graph capture.
    void prepare(void* stream, const Schedule& sched, const TrunkGeom& g) {
        const std::vector<KvMerge> need = merges(sched, g);
        if (need.empty()) return;
        if (!kernels_) {
            spl_sage::Config cfg{spl_sage::Tile::for_head_dim(HEAD_DIM), pv_};
            kernels_.emplace(spl_sage::SageAttention::with_config(stream, HEAD_DIM, cfg));
        }
        std::vector<Key> keys;
        for (const KvMerge& m : need) keys.push_back(key(g, m));
        for (auto it = ws_.begin(); it != ws_.end();) {
            bool keep = false;
            for (const Key& k : keys) keep = keep || k == it->first;
            it = keep ? std::next(it) : ws_.erase(it);
        }
        for (const KvMerge& m : need)
            if (ws_.find(key(g, m)) == ws_.end()) ws_.emplace(key(g, m), kernels_->workspace(shape(g), m));
    }

    // The attention for one sage layer of `kind` at `g`.
    SageLayer layer(InterKind kind, const TrunkGeom& g) {
        const std::optional<KvMerge> merge = merge_of(kind, g);
        if (!merge) throw spl_sage::Error(SAGE_ERR_INVALID, std::string(kind_name(kind)) + " is not a sage layer");
        if (!kernels_) throw spl_sage::Error(SAGE_ERR_STATE, "sage kernels not prepared");
        auto it = ws_.find(key(g, *merge));
        if (it == ws_.end())
            throw spl_sage::Error(SAGE_ERR_STATE, std::string("sage workspace for ") + kind_name(kind) + " at " +
                                                      g.debug() + " not prepared");
        return SageLayer(*kernels_, it->second);
    }

    const spl_sage::SageAttention* kernels() const { return kernels_ ? &*kernels_ : nullptr; }
    std::size_t workspaces() const { return ws_.size(); }

private:
    // ws_key (sched.rs:92-98): (frames, grid_h, grid_w, merge stride).
    using Key = std::tuple<std::size_t, std::size_t, std::size_t, std::size_t>;
    static Key key(const TrunkGeom& g, const KvMerge& m) { return Key{g.frames, g.grid_h, g.grid_w, m.stride}; }

    std::optional<spl_sage::SageAttention> kernels_;
    spl_sage::PvAccum pv_;
    std::map<Key, spl_sage::Workspace> ws_;
};

}  // namespace spl_vggt
