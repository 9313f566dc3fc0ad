/* sage_hip.h -- C ABI of the MI355X (gfx950) SageAttention2 forward path.
 *
 * This is the drop-in boundary for the reference's `spl_nn::sage` Rust API
 * (sezer-muhammed/sota-papers-lab, platform/spl-nn/src/sage/mod.rs) and the
 * cudarc backend under it (platform/spl-gpu/src/lib.rs). Each declaration
 * names the reference item it replaces. Plain pointers, sizes and PODs only;
 * device pointers are HIP device addresses, the stream is a hipStream_t.
 *
 * Semantics kept from the reference:
 *   - every call enqueues on the context's stream and returns without
 *     synchronising (mod.rs:509-510); prepare/attend neither allocate nor
 *     synchronise, so they can be captured in a hipGraph (the workspace is
 *     allocated once per shape by sage_workspace_new, mod.rs:649-670);
 *   - every invalid input is reported before any launch, with the reference's
 *     error text, through the return status and sage_last_error()
 *     (mod.rs:251-259,405-440,587-589,681-709,841-852);
 *   - the caller owns Q/K/V/out device memory (borrowed for the call); the
 *     library owns the workspace and frees it in sage_workspace_destroy.
 *
 * Extensions with no reference counterpart (needed by the benchmark
 * configurations): fp16 inputs and output (dtype fields), causal masking
 * (sage_options.causal) and grouped-query heads (sage_shape.kv_heads).
 */
#ifndef SAGE_HIP_H
#define SAGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Query rows per INT8 Q scale, queries per prologue tile, keys per K/V block
 * (mod.rs:70-75, sage_common.cu:33-35) and the E4M3 range V is scaled to
 * (mod.rs:76-77, :183-185). */
#define SAGE_QGROUP 16
#define SAGE_QTILE 128
#define SAGE_KBLOCK 64
#define SAGE_FP8_MAX 448.0f
#define SAGE_PV16_V_RANGE 2.25f

typedef enum sage_status {
    SAGE_OK = 0,
    SAGE_ERR_INVALID = 1,     /* bad argument: the reference's `bail!` */
    SAGE_ERR_UNSUPPORTED = 2, /* a reference feature this build does not implement */
    SAGE_ERR_DEVICE = 3,      /* HIP runtime failure (mod.rs:106-114 `.cuda(what)`) */
    SAGE_ERR_STATE = 4        /* e.g. attend before prepare (mod.rs:841-843) */
} sage_status;

/* Element type of a 16-bit tensor. The reference reads and writes bf16 only
 * (sage_common.cu:66-80); fp16 is an extension. */
typedef enum sage_dtype { SAGE_BF16 = 0, SAGE_F16 = 1 } sage_dtype;

/* PvAccum (mod.rs:170-185). F16 quantises V to +-SAGE_PV16_V_RANGE, as the
 * reference's F16 mode does, so the prologue's codes and scales are that
 * mode's. gfx950's FP8 MFMA accumulates in fp32 only: the P.V block partials
 * stay fp32 under both settings (at least as accurate as f16 partials). */
typedef enum sage_pv_accum { SAGE_PV_F32 = 0, SAGE_PV_F16 = 1 } sage_pv_accum;

/* Tile (mod.rs:116-168): the reference's CTA shape (warps, 16-row m-tiles per
 * warp, K/V ring stages; 16 * m_tiles * warps rows a CTA). Accepted exactly
 * as Tile::validate accepts it. It picks the CDNA4 workgroup layout, never
 * the results (every layout's outputs are bit-identical): warps = 8 (dense
 * and causal attention, either head dim) runs eight wave64s a workgroup, four
 * score waves (QK^T, softmax) and four output waves (rescale, P.V, one block
 * behind) over the same 128 queries; every other tile, the defaults included,
 * runs four wave64s of 32 queries, each doing the whole block. Both
 * double-buffer K and V. KV-merged attention always runs the four-wave
 * layout. */
typedef struct sage_tile {
    uint32_t warps;
    uint32_t m_tiles;
    uint32_t stages;
} sage_tile;

/* Config (mod.rs:187-201). */
typedef struct sage_config {
    sage_tile tile;
    int32_t pv_accum; /* sage_pv_accum */
} sage_config;

/* Shape (mod.rs:262-268) plus kv_heads (0 = heads; extension: grouped-query
 * attention, heads must be a multiple of kv_heads). */
typedef struct sage_shape {
    uint64_t batch;
    uint64_t heads;
    uint64_t tokens;
    uint64_t kv_heads;
} sage_shape;

/* FrameLayout (mod.rs:270-300). */
typedef struct sage_frame_layout {
    uint64_t frames;
    uint64_t special;
    uint64_t grid_h;
    uint64_t grid_w;
    uint64_t dense_frames;
} sage_frame_layout;

/* KvMerge (mod.rs:302-311): stride 1 = Dense, 2 or 4 = Pool{stride, layout}.
 * A pooled plan averages K and V over stride x stride patch cells of every
 * frame past the first `dense_frames` (special tokens stay single) and gives
 * each key a log2(member count) logit bias; queries are never merged. Causal
 * masking (an extension) is refused over merged keys (SAGE_ERR_UNSUPPORTED). */
typedef struct sage_kv_merge {
    uint32_t stride;
    sage_frame_layout layout;
} sage_kv_merge;

/* Plan (mod.rs:391-454). */
typedef struct sage_plan {
    sage_shape shape;
    sage_kv_merge merge;
    uint64_t tq_pad; /* tokens rounded up to SAGE_QTILE */
    uint64_t tk;     /* keys after merging */
    uint64_t tk_pad; /* tk rounded up to SAGE_KBLOCK */
} sage_plan;

/* Strides (mod.rs:203-260): element strides of [batch][token][head][dim]
 * with contiguous channels; each a multiple of 8 elements. */
typedef struct sage_strides {
    uint64_t batch;
    uint64_t token;
    uint64_t head;
} sage_strides;

/* Tensor / TensorMut (mod.rs:497-507): a device buffer of `len` elements. */
typedef struct sage_tensor {
    const void* data;
    uint64_t len;
    sage_strides strides;
    int32_t dtype; /* sage_dtype */
} sage_tensor;

typedef struct sage_tensor_mut {
    void* data;
    uint64_t len;
    sage_strides strides;
    int32_t dtype; /* sage_dtype */
} sage_tensor_mut;

/* Options (mod.rs:313-335). has_softmax_scale = 0 means the default
 * 1/sqrt(head_dim). qk_norm_params != NULL asks for the fused QK LayerNorm
 * (QkNorm, mod.rs:337-344): a device pointer to qk_norm_len >= 4 * head_dim
 * floats, [q weight, q bias, k weight, k bias], applied to every Q and K head
 * row before the statistics and quantisation read it (eps qk_norm_eps);
 * fewer floats is SAGE_ERR_INVALID. causal is an extension (keys j > i are
 * masked). */
typedef struct sage_options {
    float softmax_scale;
    int32_t has_softmax_scale;
    int32_t smooth_k;
    int32_t smooth_v;
    const float* qk_norm_params;
    uint64_t qk_norm_len;
    float qk_norm_eps;
    int32_t causal;
} sage_options;

/* Device addresses of a workspace's buffers (the pub fields of Workspace,
 * mod.rs:456-477), with their element counts. Layouts (b batch, h Q head,
 * g KV head):
 *   q8      i8  [b][h][tq_pad][D]          q_scale f32 [b][h][tq_pad/16]
 *   k8      i8  [b][g][tk_pad][D]          k_scale f32 [b][g][tk_pad/64]
 *   v8      u8  [b][g][tk_pad/64][D][64]   E4M3, key k of a block at byte
 *                                          sage_v8_position(k) of its row
 *   stats   f32 [b][g][4][D]               K mean, V mean, V scale, 1/V scale
 *   kbias   f32 [tk_pad]                   KV-merge bias: log2(member count),
 *                                          -inf past tk (unused when dense) */
typedef struct sage_ws_buffers {
    int8_t* q8;
    float* q_scale;
    int8_t* k8;
    float* k_scale;
    uint8_t* v8;
    float* stats;
    float* kbias;
    uint64_t q8_len, q_scale_len, k8_len, k_scale_len, v8_len, stats_len, kbias_len;
} sage_ws_buffers;

typedef struct sage_attention sage_attention; /* SageAttention (mod.rs:509-520) */
typedef struct sage_workspace sage_workspace; /* Workspace (mod.rs:456-495) */

/* Text of the last error on this thread ("" when none). The reference's
 * anyhow messages, e.g. "sage workspace has not been prepared". */
const char* sage_last_error(void);

/* Plan::new (mod.rs:405-440). Host only; no GPU needed. */
sage_status sage_plan_new(const sage_shape* shape, const sage_kv_merge* merge, sage_plan* out);

/* flops (mod.rs:905-910): 4 * B * H * tokens * tk * D. With causal = 1, the
 * pairs j <= i only: 2 * B * H * D * tokens * (tokens + 1) (extension). */
double sage_flops(const sage_plan* plan, uint64_t head_dim, int32_t causal);

/* Strides::check (mod.rs:251-259); `what` names the tensor in the message. */
sage_status sage_strides_check(const sage_strides* s, const char* what);

/* Strides::extent (mod.rs:244-249) for `heads` heads; UINT64_MAX when the
 * extent does not fit 64 bits. */
uint64_t sage_strides_extent(const sage_strides* s, uint64_t batch, uint64_t tokens, uint64_t heads,
                             uint64_t head_dim);

/* Tile::validate (mod.rs:158-167): warps in {2,4,8}, m_tiles in {1,2,4},
 * stages 2..6, 128 a multiple of 16 * m_tiles * warps; otherwise
 * "unsupported sage tile Tile { .. }". */
sage_status sage_tile_validate(const sage_tile* t);

/* Config::for_head_dim (mod.rs:194-200): Tile::D128 {4,1,3} above head dim
 * 64, Tile::DEFAULT {4,2,3} otherwise (mod.rs:128-147); PvAccum::F32. */
sage_config sage_config_for_head_dim(uint64_t head_dim);

/* check_device (mod.rs:552-566): fails unless device `ordinal` is gfx950. */
sage_status sage_check_device(int ordinal);

/* SageAttention::new / with_config (mod.rs:571-626) on `stream` (a
 * hipStream_t; NULL = the null stream) of the current device.
 * config == NULL means Config::for_head_dim. */
sage_status sage_new(void* stream, uint64_t head_dim, const sage_config* config, sage_attention** out);
void sage_destroy(sage_attention* s);
uint64_t sage_head_dim(const sage_attention* s);             /* mod.rs:628-630 */
sage_config sage_get_config(const sage_attention* s);        /* mod.rs:632-634 */
void* sage_stream(const sage_attention* s);                  /* mod.rs:636-638 */

/* attn_resources (mod.rs:640-646): VGPRs per lane and scratch (spill) bytes
 * of the attention kernel, plus its static LDS bytes. The kernel is the one
 * the context's tile selects: the eight-wave layout for warps 8, else the
 * four-wave kernel. */
sage_status sage_attn_resources(const sage_attention* s, int32_t* regs, int32_t* spill, int32_t* lds);

/* The same for each attention kernel the context can launch (extension: the
 * reference reports its dense kernel only): SAGE_KERNEL_DENSE, _CAUSAL (the
 * causal extension) or _MERGED (KV merging, sg_attn_merge; always the
 * four-wave kernel). */
typedef enum sage_attn_kernel {
    SAGE_KERNEL_DENSE = 0,
    SAGE_KERNEL_CAUSAL = 1,
    SAGE_KERNEL_MERGED = 2
} sage_attn_kernel;
sage_status sage_attn_kernel_resources(const sage_attention* s, int32_t kernel, int32_t* regs, int32_t* spill,
                                       int32_t* lds);

/* SageAttention::workspace (mod.rs:648-670): allocates (and zero-fills) the
 * buffers for `shape` and `merge`. A shape whose buffers would need more than
 * 2^62 bytes in total is refused (SAGE_ERR_INVALID) before any allocation. */
sage_status sage_workspace_new(const sage_attention* s, const sage_shape* shape, const sage_kv_merge* merge,
                           sage_workspace** out);
void sage_workspace_destroy(sage_workspace* ws);
uint64_t sage_workspace_bytes(const sage_workspace* ws);                 /* mod.rs:484-494 */
sage_status sage_workspace_plan(const sage_workspace* ws, sage_plan* out); /* mod.rs:480-482 */
sage_status sage_workspace_buffers(const sage_workspace* ws, sage_ws_buffers* out);

/* SageAttention::prepare (mod.rs:672-836): K smoothing statistics, INT8 Q
 * (per 16 rows), INT8 K (per 64 keys), FP8 V (per channel) into `ws`. */
sage_status sage_prepare(const sage_attention* s, sage_workspace* ws, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_options* opts);

/* SageAttention::attend (mod.rs:838-886): INT8 QK^T, online exp2 softmax,
 * FP8 P.V; writes [batch][token][head][dim] into `out`. */
sage_status sage_attend(const sage_attention* s, const sage_workspace* ws, const sage_tensor_mut* out);

/* SageAttention::forward (mod.rs:888-900): prepare then attend. */
sage_status sage_forward(const sage_attention* s, sage_workspace* ws, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_tensor_mut* out, const sage_options* opts);

/* ---- The QKV prologue (platform/spl-nn/src/qkv.rs, cuda/qkv.cu) ----
 * The step before sage in the reference's transformer block: it splits the
 * fused QKV projection, applies its optional dequantisation scales and bias,
 * QK-norm (LayerNorm or RMSNorm over the head dim, weights shared across
 * heads) and 2D RoPE on q and k, and writes bf16 Q, K and V. Head dim 64 is
 * the reference's; 128 is an extension (the same arithmetic, RoPE pairs D/4
 * or D/2 apart). */

/* QkvIn (qkv.rs:165-177) with a batch dimension: y is bf16 rows of `ld`
 * elements per token (batch items batch_stride elements apart; 0 = tokens *
 * ld), holding q | k | v of heads*D, kv_heads*D and kv_heads*D channels
 * (kv_heads from the shape; equal to heads in the reference). tok: f32
 * [batch * tokens] per-token scales; chan: f32 [(heads + 2 kv_heads) * D]
 * per-channel scales; bias: bf16 [(heads + 2 kv_heads) * D]; NULL = none.
 * The *_len fields give each buffer's element count. */
typedef struct sage_qkv_in {
    const void* y;
    uint64_t y_len;
    uint64_t ld;
    uint64_t batch_stride;
    const float* tok;
    uint64_t tok_len;
    const float* chan;
    uint64_t chan_len;
    const uint16_t* bias;
    uint64_t bias_len;
} sage_qkv_in;

/* NormKind (qkv.rs:138-143) and QkNorm (qkv.rs:145-156): f32 [D] weights
 * (len elements each), biases used (and required) by LayerNorm only. */
typedef enum sage_qkv_norm_kind { SAGE_QKV_LAYER_NORM = 1, SAGE_QKV_RMS_NORM = 2 } sage_qkv_norm_kind;
typedef struct sage_qkv_norm {
    int32_t kind;
    const float* q_weight;
    const float* q_bias;
    const float* k_weight;
    const float* k_bias;
    uint64_t len;
    float eps;
} sage_qkv_norm;

/* RopeLayout (qkv.rs:33-58) and Rope (qkv.rs:158-163): table is f32
 * [frame_len][D/2][2] (cos, sin per rotation pair; table_len elements), row
 * token % frame_len. VGGT rotates pairs (i, i + D/4) inside each half of the
 * head, DINOv3 pairs (i, i + D/2). */
typedef enum sage_rope_layout { SAGE_ROPE_VGGT = 0, SAGE_ROPE_DINOV3 = 1 } sage_rope_layout;
typedef struct sage_qkv_rope {
    const float* table;
    uint64_t table_len;
    int32_t layout;
    uint64_t frame_len;
} sage_qkv_rope;

/* RopeTable::vggt / RopeTable::dinov3 (qkv.rs:87-136), host only: writes the
 * (special + grid_h * grid_w) x (head_dim / 2) x 2 table (cos, sin of the f64
 * angle, rounded to f32) to `out`, which holds out_len floats. */
sage_status sage_rope_table(int32_t layout, uint64_t head_dim, uint64_t grid_h, uint64_t grid_w, uint64_t special,
                            double base, float* out, uint64_t out_len);

/* QkvPrologue::run (qkv.rs:216-306) on the context's stream: shape gives
 * batch, heads, kv_heads and tokens; norm and rope may be NULL. Q and K are
 * written bf16, V bf16 or fp16 (its dtype; VFormat), into [batch][token]
 * [head][dim] views (any strides that are multiples of 8; the reference's
 * [heads][tokens][64] is the bhtd view). Refusals carry the reference's text
 * ("qkv: ld .. must be a multiple of 8 and at least ..", "qkv: LayerNorm
 * QK-norm needs q and k biases", "qkv: RoPE frame length is 0", "<what>:
 * buffer holds .. elements, needs ..", "device pointer .. is not 16-byte
 * aligned") in the reference's order: ld, then the sizes of y, the scales
 * and the bias, of q, k and v, of the norm weights and the RoPE table, and
 * last the alignment of y, chan, bias, q, k and v (16 bytes). The norm
 * weights and the RoPE table, f32, need only their type's alignment, as
 * there. An empty shape is a no-op, as there. */
sage_status sage_qkv_prologue(const sage_attention* s, const sage_shape* shape, const sage_qkv_in* in,
                              const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_tensor_mut* q,
                              const sage_tensor_mut* k, const sage_tensor_mut* v);

/* SageAttention::prepare fed straight from the fused QKV projection (the
 * fusion of the two steps; no counterpart in the reference, which runs
 * QkvPrologue::run, stores bf16 Q, K and V and prepares from them): the
 * workspace receives the codes and scales that QkvPrologue::run followed by
 * sage_prepare would give, bit for bit, without the bf16 round trip. The
 * shape is the workspace's; opts as sage_prepare (QkNorm of the sage options
 * then applies to the QKV prologue's output). */
sage_status sage_prepare_qkv(const sage_attention* s, sage_workspace* ws, const sage_qkv_in* in,
                             const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_options* opts);

/* sage_prepare_qkv then sage_attend. */
sage_status sage_forward_qkv(const sage_attention* s, sage_workspace* ws, const sage_qkv_in* in,
                             const sage_qkv_norm* norm, const sage_qkv_rope* rope, const sage_tensor_mut* out,
                             const sage_options* opts);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): sage_forward (prepare then attend) for `shape` and
 * `merge` (NULL = dense) with no workspace. Its buffers are carved from one
 * device array of SAGE_NOALLOC_MAX_BYTES that the library holds on every GPU
 * it runs on until the process ends; it allocates and frees nothing. A shape
 * whose buffers (sage_workspace_bytes of its workspace, each buffer rounded up
 * to 256 bytes) exceed that is refused with SAGE_ERR_INVALID before any
 * launch. Every call on one GPU shares that GPU's array: calls whose kernels
 * can overlap on one GPU (different streams with no ordering between them)
 * race, so order them on one stream. Outputs equal sage_forward's. */
#define SAGE_NOALLOC_MAX_BYTES (128ull << 20)
sage_status sage_forward_noalloc(const sage_attention* s, const sage_shape* shape, const sage_kv_merge* merge,
                                 const sage_tensor* q, const sage_tensor* k, const sage_tensor* v,
                                 const sage_tensor_mut* out, const sage_options* opts);

/* Byte position of key k (0..63) of a 64-key block inside each channel row
 * of the v8 layout (the CDNA4 counterpart of sg_vpos, sage_common.cu:151-155):
 * the order in which the QK^T accumulator of the 32x32 MFMA hands keys to the
 * FP8 MFMA's operand. Host only. */
int32_t sage_v8_position(int32_t k);

/* MFMA peak probes (the analogue of sage_peak.cu:10-94 and the tests.rs:757-794
 * driver): which = 0 INT8 32x32x32 (i32 acc), 1 FP8 E4M3 32x32x64 (f32 acc),
 * 2 BF16 32x32x16 (f32 acc). Runs on the context's stream, synchronises, and
 * writes the measured dense TOPS. */
sage_status sage_peak(const sage_attention* s, int32_t which, int32_t iters, double* tops);

#ifdef __cplusplus
}
#endif
#endif
