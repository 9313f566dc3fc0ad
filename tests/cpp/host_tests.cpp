// CPU tests of the C++ host API (include/spl_sage.hpp) over libsage_hip.so:
// the reference's host-side tests (sezer-muhammed/sota-papers-lab,
// platform/spl-nn/src/sage/tests.rs:17-22, 95-190, 245-262) restated against
// spl_sage:: names, plus the reference's error texts (mod.rs:251-259,
// 405-440). No GPU call is made. Exit status 0 when every check passes.
#include <cmath>
#include <cstdio>
#include <atomic>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "spl_sage.hpp"
#include "spl_sage_sched.hpp"

using namespace spl_sage;

static int failures = 0;

#define CHECK(cond)                                                           \
    do {                                                                      \
        if (!(cond)) {                                                        \
            std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);   \
            failures++;                                                       \
        }                                                                     \
    } while (0)

// Runs f, which must throw an Error whose status is `status` and whose text
// contains `text`.
template <typename F>
static void expect_error(F f, sage_status status, const char* text, int line) {
    try {
        f();
        std::printf("  FAILED line %d: no error (expected \"%s\")\n", line, text);
        failures++;
    } catch (const Error& e) {
        if (e.status() != status || std::string(e.what()).find(text) == std::string::npos) {
            std::printf("  FAILED line %d: status %d \"%s\" (expected %d \"%s\")\n", line, (int)e.status(), e.what(),
                        (int)status, text);
            failures++;
        }
    }
}
#define EXPECT_ERROR(expr, status, text) expect_error([&] { expr; }, status, text, __LINE__)

static FrameLayout vggt_layout(std::size_t frames) { return FrameLayout{frames, 17, 21, 32, 0}; }

// tests.rs:17-22: the engine and its workspace move between threads; here,
// they are move-only owners.
static void engine_handles_are_move_only() {
    static_assert(!std::is_copy_constructible<SageAttention>::value, "");
    static_assert(std::is_nothrow_move_constructible<SageAttention>::value, "");
    static_assert(!std::is_copy_constructible<Workspace>::value, "");
    static_assert(std::is_nothrow_move_constructible<Workspace>::value, "");
}

// tests.rs:17-22 asks for an engine that is Send + Sync. The C ABI's state
// shared across threads is its error channel: eight threads refuse their own
// shapes concurrently, and each reads back its own text.
static void error_text_is_per_thread() {
    std::atomic<int> wrong{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < 8; t++)
        pool.emplace_back([t, &wrong] {
            sage_kv_merge dense{};
            dense.stride = 1;
            for (int i = 0; i < 2000; i++) {
                sage_shape s{};
                s.batch = 1;
                s.heads = 6 + t;
                s.kv_heads = 4;  // divides 6 + t only at t = 2 and t = 6
                s.tokens = 100;
                sage_plan p;
                const sage_status st = sage_plan_new(&s, &dense, &p);
                const bool refused = (6 + t) % 4 != 0;
                const std::string want = std::to_string(6 + t) + " query heads are not a multiple of 4 KV heads";
                if (refused ? (st != SAGE_ERR_INVALID || sage_last_error() != want)
                            : (st != SAGE_OK || sage_last_error()[0] != 0))
                    wrong++;
            }
        });
    for (auto& th : pool) th.join();
    CHECK(wrong.load() == 0);
}

// tests.rs:95-110: 689 dense keys + 2 x (17 + 6 x 8) pooled.
static void dense_first_frame_keeps_its_keys() {
    FrameLayout layout = vggt_layout(3);
    layout.dense_frames = 1;
    const Plan plan = Plan::create(Shape{1, 1, 3 * 689}, KvMerge::Pool(4, layout));
    CHECK(plan.tk == 689 + 2 * 65);
    CHECK(plan.tk_pad == (plan.tk + 63) / 64 * 64);
    CHECK(plan.tq_pad == (3 * 689 + 127) / 128 * 128);
}

// tests.rs:135-150: plan geometry of VGGT-Omega's 200 frames.
static void vggt_merge_geometry() {
    const FrameLayout layout = vggt_layout(200);
    CHECK(layout.tokens_per_frame() == 689);
    const Shape shape{1, 16, 200 * 689};
    const Plan dense = Plan::create(shape, KvMerge::Dense());
    CHECK(dense.tq_pad == 137856 && dense.tk == 137800 && dense.tk_pad == 137856);
    const Plan m2 = Plan::create(shape, KvMerge::Pool(2, layout));
    CHECK(m2.tk == 200 * (17 + 11 * 16));
    const Plan m4 = Plan::create(shape, KvMerge::Pool(4, layout));
    CHECK(m4.tk == 200 * (17 + 6 * 8));
    CHECK(layout.merged_per_frame(2) == 17 + 11 * 16 && layout.merged_keys(4) == m4.tk);
    CHECK(m4.q_tiles() == 137856 / 128 && m4.kblocks() == m4.tk_pad / 64);
}

// tests.rs:174-190.
static void plan_rejects_bad_layouts() {
    const FrameLayout layout = vggt_layout(2);
    EXPECT_ERROR(Plan::create(Shape{1, 2, 1000}, KvMerge::Pool(2, layout)), SAGE_ERR_INVALID, "");
    const Shape shape{1, 2, 2 * 689};
    EXPECT_ERROR(Plan::create(shape, KvMerge::Pool(3, layout)), SAGE_ERR_INVALID, "");
    Plan::create(shape, KvMerge::Pool(4, layout));
    EXPECT_ERROR(Plan::create(Shape{1, 2, 0}, KvMerge::Dense()), SAGE_ERR_INVALID, "");
    // Grouped-query heads must divide the query heads (extension).
    EXPECT_ERROR(Plan::create(Shape{1, 6, 128, 4}, KvMerge::Dense()), SAGE_ERR_INVALID, "");
    const Plan gqa = Plan::create(Shape{1, 32, 8192, 8}, KvMerge::Dense());
    CHECK(gqa.shape.kv() == 8);
}

// tests.rs:245-262.
static void strides_cover_the_tensor() {
    const Shape shape{2, 3, 5};
    const std::size_t d = 64;
    CHECK(Strides::bthd(5, 3, d).extent(shape, d) == 2 * 5 * 3 * d);
    CHECK(Strides::bhtd(5, 3, d).extent(shape, d) == 2 * 3 * 5 * d);
    // A packed QKV view starting at V's offset ends at the buffer's end.
    CHECK(Strides::packed_qkv(5, 3, d).extent(shape, d) + 2 * 3 * d == 2 * 5 * 3 * 3 * d);
    EXPECT_ERROR(Strides::bthd(5, 3, 60).check("x"), SAGE_ERR_INVALID, "x");
    Strides::bthd(5, 3, 64).check("x");
}

// mod.rs:116-201: the reference's tile menu (Tile::validate) and its default
// configs (Tile::DEFAULT, Tile::D128, Config::for_head_dim).
static void tiles_and_config() {
    const Config c64 = Config::for_head_dim(64), c128 = Config::for_head_dim(128);
    CHECK(c64.pv_accum == PvAccum::F32 && c128.pv_accum == PvAccum::F32);
    CHECK(c64.tile.warps == 4 && c64.tile.m_tiles == 2 && c64.tile.stages == 3);
    CHECK(c128.tile.warps == 4 && c128.tile.m_tiles == 1 && c128.tile.stages == 3);
    CHECK(Tile::DEFAULT.rows() == 128 && Tile::D128.rows() == 64);
    int accepted = 0;
    for (uint32_t w = 0; w < 10; w++)
        for (uint32_t m = 0; m < 6; m++)
            for (uint32_t st = 0; st < 8; st++) {
                const bool ref_ok = (w == 2 || w == 4 || w == 8) && (m == 1 || m == 2 || m == 4) && st >= 2 &&
                                    st <= 6 && 128 % (16 * m * w) == 0;
                if (ref_ok) {
                    (Tile{w, m, st}).validate();
                    accepted++;
                } else {
                    EXPECT_ERROR((Tile{w, m, st}.validate()), SAGE_ERR_INVALID, "unsupported sage tile");
                }
            }
    CHECK(accepted == 30);
    (Tile{8, 1, 2}).validate();
    EXPECT_ERROR((Tile{4, 4, 3}.validate()), SAGE_ERR_INVALID, "unsupported sage tile");
}

// mod.rs:905-910 and the benchmark's operation counts.
static void flops_counts_the_pairs() {
    const Plan c2 = Plan::create(Shape{2, 32, 4096}, KvMerge::Dense());
    CHECK(flops(c2, 128) == 4.0 * 2 * 32 * 4096.0 * 4096.0 * 128);
    const Plan c3 = Plan::create(Shape{1, 32, 16384}, KvMerge::Dense());
    CHECK(flops(c3, 128, true) == 2.0 * 32 * 128 * 16384.0 * 16385.0);
    // Merged keys count as keys.
    FrameLayout layout = vggt_layout(2);
    const Plan m = Plan::create(Shape{1, 1, 2 * 689}, KvMerge::Pool(4, layout));
    CHECK(flops(m, 64) == 4.0 * (2 * 689.0) * (double)m.tk * 64);
}

// The v8 key order is a permutation of the 64 keys of a block.
static void v8_positions_are_a_permutation() {
    int seen[64] = {};
    for (int k = 0; k < 64; k++) {
        const int p = v8_position(k);
        CHECK(p >= 0 && p < 64);
        if (p >= 0 && p < 64) seen[p]++;
    }
    for (int p = 0; p < 64; p++) CHECK(seen[p] == 1);
    CHECK(v8_position(64) == -1 && v8_position(-1) == -1);
}

// Options map onto the C struct as the reference's defaults say (mod.rs:326-335).
// qkv.rs:378-421 (layouts_pair_the_right_channels, vggt_table_matches_its_formula,
// dinov3_table_matches_its_formula) through the C++ qkv mirror.
static void qkv_rope_tables() {
    using namespace spl_sage::qkv;
    CHECK(rope_pair(RopeLayout::Vggt, 0) == 0 && rope_pair(RopeLayout::Vggt, 16) == 0 &&
          rope_pair(RopeLayout::Vggt, 15) == 15);
    CHECK(rope_pair(RopeLayout::Vggt, 32) == 16 && rope_pair(RopeLayout::Vggt, 48) == 16 &&
          rope_pair(RopeLayout::Vggt, 63) == 31);
    CHECK(rope_pair(RopeLayout::Dinov3, 0) == 0 && rope_pair(RopeLayout::Dinov3, 32) == 0 &&
          rope_pair(RopeLayout::Dinov3, 31) == 31 && rope_pair(RopeLayout::Dinov3, 63) == 31);
    for (RopeLayout l : {RopeLayout::Vggt, RopeLayout::Dinov3})
        for (std::size_t c = 0; c < HEAD_DIM; c++) CHECK(rope_pair(l, c) == rope_pair(l, c ^ rope_half(l)));
    const RopeTable t = RopeTable::vggt(3, 4, 2, 100.0);
    CHECK(t.frame_len == 14);
    CHECK(t.cos_sin[(1 * 32 + 5) * 2] == 1.0f && t.cos_sin[(1 * 32 + 5) * 2 + 1] == 0.0f);
    double a = 2.0 * std::pow(100.0, -3.0 / 16.0);
    CHECK(std::fabs(t.cos_sin[(9 * 32 + 3) * 2] - std::cos(a)) < 1e-7);
    CHECK(std::fabs(t.cos_sin[(9 * 32 + 3) * 2 + 1] - std::sin(a)) < 1e-7);
    a = 4.0 * std::pow(100.0, -5.0 / 16.0);
    CHECK(std::fabs(t.cos_sin[(9 * 32 + 21) * 2 + 1] - std::sin(a)) < 1e-7);
    const RopeTable d = RopeTable::dinov3(2, 2, 1, 100.0);
    a = 2.0 * M_PI * -0.5;
    CHECK(std::fabs(d.cos_sin[(2 * 32 + 0) * 2 + 1] - std::sin(a)) < 1e-7);
    a = 2.0 * M_PI * 0.5 / std::pow(100.0, 2.0 / 16.0);
    CHECK(std::fabs(d.cos_sin[(2 * 32 + 18) * 2] - std::cos(a)) < 1e-7);
}

static void options_defaults() {
    const sage_options o = Options{}.raw();
    CHECK(o.smooth_k == 1 && o.smooth_v == 1 && o.has_softmax_scale == 0 && o.qk_norm_params == nullptr &&
          o.causal == 0);
    Options with;
    with.softmax_scale = 0.125f;
    with.qk_norm = QkNorm{reinterpret_cast<const float*>(16), 256, 1e-6f};
    const sage_options w = with.raw();
    CHECK(w.has_softmax_scale == 1 && w.softmax_scale == 0.125f && w.qk_norm_len == 256 && w.qk_norm_eps == 1e-6f);
}

// The reference's caller (apps/image-to-3d/src/vggt/trunk/sched.rs) through
// include/spl_sage_sched.hpp, host side: merge_of for every schedule entry
// (sched.rs:24-46), merges of the shipped `ours+sage` schedule (vggt/mod.rs:
// 82-107) in first-use order (sched.rs:73-85), and the refusals Sage::layer
// makes before any kernel exists (sched.rs:150-158).
static void vggt_caller_schedule() {
    using namespace spl_vggt;
    const TrunkGeom g{200, 21, 32};
    CHECK(g.tokens() == 689 && g.rows() == 137800);
    CHECK(merge_of(InterKind::Sage, g)->is_dense());
    for (InterKind k : {InterKind::Global, InterKind::Register, InterKind::Frame}) CHECK(!merge_of(k, g));
    const std::optional<KvMerge> m4 = merge_of(InterKind::Merge4, g), m2 = merge_of(InterKind::Merge2, g);
    CHECK(m4 && m4->stride == 4 && m4->layout.frames == 200 && m4->layout.special == 17 && m4->layout.grid_h == 21 &&
          m4->layout.grid_w == 32 && m4->layout.dense_frames == 1);
    CHECK(m2 && m2->stride == 2 && !same_merge(*m2, *m4));
    // One frame has nothing to merge: frame 0 stays dense.
    const TrunkGeom one{1, 21, 32};
    CHECK(merge_of(InterKind::Merge4, one)->is_dense() && merge_of(InterKind::Merge2, one)->is_dense());
    // The plan of a merge4 layer at 200 frames: 689 dense keys + 199 x (17 + 6 x 8) pooled.
    CHECK(Plan::create(shape(g), *m4).tk == 689 + 199 * 65);

    Schedule sched;
    sched.fill(InterKind::Global);
    for (std::size_t i : {2, 6, 9, 14, 20}) sched[i] = InterKind::Register;
    for (InterKind& a : sched)
        if (a == InterKind::Global) a = InterKind::Sage;
    for (std::size_t i : {3, 4, 5}) sched[i] = InterKind::Frame;
    for (std::size_t i : {0, 1, 7, 19}) sched[i] = InterKind::Merge4;
    const std::vector<KvMerge> need = merges(sched, g);
    CHECK(need.size() == 2 && need[0].stride == 4 && need[1].is_dense());
    CHECK(merges(sched, one).size() == 1);
    Schedule frames_only;
    frames_only.fill(InterKind::Frame);
    CHECK(merges(frames_only, g).empty());
    // The caller's byte count: positive for its plans, 0 for a refused one.
    CHECK(workspace_bytes(g, need[0]) > 0 && workspace_bytes(g, need[1]) > workspace_bytes(g, need[0]));
    CHECK(workspace_bytes(TrunkGeom{0, 21, 32}, KvMerge::Dense()) == 0);
    // sage_workspaces_are_counted (phase2_tests.rs:98-117): the phase-2 schedule's
    // workspaces (dense sage: Q, K and V at a byte each; merge4: Q and pooled K/V)
    // add between 4 and 5 bytes per (head, channel, token) at 200 frames.
    std::size_t extra = 0;
    for (const KvMerge& m : need) extra += workspace_bytes(g, m);
    const std::size_t per = std::size_t(16) * 64 * 200 * 689;
    CHECK(extra > 4 * per && extra < 5 * per);

    Sage sage;
    sage.prepare(nullptr, frames_only, g);  // nothing to prepare: no kernels, no workspaces
    CHECK(sage.kernels() == nullptr && sage.workspaces() == 0);
    EXPECT_ERROR(sage.layer(InterKind::Global, g), SAGE_ERR_INVALID, "Global is not a sage layer");
    EXPECT_ERROR(sage.layer(InterKind::Merge4, g), SAGE_ERR_STATE, "sage kernels not prepared");
}

int main() {
    struct {
        const char* name;
        void (*fn)();
    } tests[] = {
        {"engine_handles_are_move_only", engine_handles_are_move_only},
        {"error_text_is_per_thread", error_text_is_per_thread},
        {"dense_first_frame_keeps_its_keys", dense_first_frame_keeps_its_keys},
        {"vggt_merge_geometry", vggt_merge_geometry},
        {"plan_rejects_bad_layouts", plan_rejects_bad_layouts},
        {"strides_cover_the_tensor", strides_cover_the_tensor},
        {"tiles_and_config", tiles_and_config},
        {"flops_counts_the_pairs", flops_counts_the_pairs},
        {"v8_positions_are_a_permutation", v8_positions_are_a_permutation},
        {"options_defaults", options_defaults},
        {"qkv_rope_tables", qkv_rope_tables},
        {"vggt_caller_schedule", vggt_caller_schedule},
    };
    for (auto& t : tests) {
        const int before = failures;
        try {
            t.fn();
        } catch (const std::exception& e) {
            std::printf("  FAILED: unexpected exception: %s\n", e.what());
            failures++;
        }
        std::printf("%s %s\n", failures == before ? "ok" : "FAIL", t.name);
    }
    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
