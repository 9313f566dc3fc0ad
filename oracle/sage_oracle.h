/* CPU oracle for the SageAttention2 forward path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the parity tests, the smoke test and the CPU
 * baseline leg of bench.py compare the HIP path against. The product path
 * (libsage_hip.so) never links, loads or calls it.
 *
 * It restates, in plain C, the arithmetic of the reference
 * (sezer-muhammed/sota-papers-lab, platform/spl-nn):
 *   - codecs            src/sage/reference.rs:8-70, cuda/sage_common.cu:76-99
 *   - splitmix64 RNG    src/sage/reference.rs:228-254
 *   - prologue          cuda/sage_quant.cu:59-206 (sg_prep, sg_finalize) and
 *                       :238-326 (sg_quant_kv), fp32 operation order kept;
 *                       QK LayerNorm :34-52, KV merging :210-235
 *   - f64 attention     src/sage/reference.rs:148-184 (+ causal, GQA)
 *   - sage emulator     cuda/sage_attn.cu:262-344,402-421 semantics
 *   - error metrics     src/sage/reference.rs:202-225
 *
 * The header of each function in sage_oracle.c says what pins it; the
 * checks themselves are tests/test_oracle_*.py.
 *
 * Parity unpinned (no known answer, reference check or closed form reaches it):
 *   - the fused rounding fmaf(sum, 1/n, -mean) of KV-merge cells with 3, 6, 9
 *     or 12 members (1/n inexact); cells of 1, 2, 4, 8 and 16 members are pinned;
 *   - inside the PvAccum::F16 emulation, the rounding of NVIDIA's
 *     f16-accumulate mma within each 32-key step (emulated as one f16 rounding
 *     per step);
 *   - the attention output's last bits on NVIDIA hardware (ex2.approx,
 *     ptxas contraction, Ada's FP8 accumulation): outputs are gated by
 *     tolerance, as the north star states.
 * The QK LayerNorm's reciprocal square root is correctly rounded here where
 * the reference takes rsqrtf; that is a stated choice, pinned against the
 * reference's f64 layer_norm, not an unpinned restatement.
 */
#ifndef SAGE_ORACLE_H
#define SAGE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_BF16 = 0, ORACLE_F16 = 1 };

/* Constants of the reference (cuda/sage_common.cu:33-35, src/sage/mod.rs:70-77). */
#define ORACLE_QGROUP 16
#define ORACLE_QTILE 128
#define ORACLE_KBLOCK 64
#define ORACLE_FP8_MAX 448.0f

/* One attention problem. Q has `heads` heads, K and V `kv_heads` (== heads
 * unless grouped-query). Element strides of the 16-bit inputs, channels
 * contiguous. */
typedef struct {
    int batch, heads, kv_heads, tokens, head_dim;
    int dtype; /* ORACLE_BF16 or ORACLE_F16 */
    long long q_sb, q_st, q_sh;
    long long k_sb, k_st, k_sh;
    long long v_sb, v_st, v_sh;
    float q_mul;   /* softmax scale * log2(e), computed in f32 */
    int smooth_k;  /* subtract the per-channel K mean */
    int smooth_v;  /* subtract the per-channel V mean (added back at the end) */
    float v_range; /* 448 */
    /* KV merging (mod.rs:270-311, KvMerge::Pool): merge = 1 is dense; 2 or 4
     * pools each frame's grid_h x grid_w patch grid in merge x merge cells,
     * keeping the `special` tokens of every frame and every token of the
     * first `dense_frames` frames. */
    int merge;
    int frames, special, grid_h, grid_w, dense_frames;
    /* QK LayerNorm (mod.rs:337-344, QkNorm): NULL is off, else [4][D] floats
     * (q weight, q bias, k weight, k bias) applied to every Q and K head row
     * before anything else reads it; V is never normalised. */
    const float* ln;
    float ln_eps;
    /* PvAccum::F16 (mod.rs:170-185): v_range is then 2.25 and the emulator
     * rounds each 64-key block's P.V to f16 after every 32 keys. */
    int pv16;
} oracle_problem;

/* LayerNorm of one D-channel row in the prologue kernels' fp32 arithmetic
 * (restates sage_quant.cu:34-52 with the reciprocal square root correctly
 * rounded; see sage_oracle.c). x and y may alias. */
void oracle_layernorm(const float* x, float* y, int D, const float* w, const float* b, float eps);
/* The reference's own CPU LayerNorm (reference.rs:109-118): f64 mean, biased
 * variance and 1/sqrt, rounded to f32 at the end. x and y may alias. */
void oracle_layernorm_f64(const float* x, float* y, int D, const float* w, const float* b, float eps);

/* Keys after merging (FrameLayout::merged_keys, mod.rs:293-299); tokens when dense. */
int oracle_merged_keys(const oracle_problem* p);
/* Tokens merged key j pools, in the reference's member order (row-major in
 * the cell; reference.rs:79-109, sage_quant.cu:210-235); returns the count
 * (<= 16) and writes the tokens to `tokens` (may be NULL). */
int oracle_members(const oracle_problem* p, int j, int* tokens);
/* log2(n) for n = 1..16, correctly rounded to f32: the KV-merge bias of a key
 * that pools n tokens (sage_quant.cu:321-325). */
float oracle_log2_count(int n);

/* ---- codecs ---- */
float oracle_bf16_to_f32(uint16_t b);
uint16_t oracle_f32_to_bf16(float x);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float x);
float oracle_e4m3_to_f32(uint8_t b);
uint8_t oracle_f32_to_e4m3(float x);
int oracle_s8(float x);
int oracle_vpos_ref(int k);

/* Bulk codec helpers (n elements). */
/* x rounded to the nearest f16 value (ties to even, subnormals kept, inf past
 * the largest finite), returned as a double; the f16 accumulator of the
 * PvAccum::F16 emulation. */
double oracle_round_f16(double x);
/* The QK-norm's rstd: 1 / sqrt(v) with the square root and the divide each
 * correctly rounded (1.0f / sqrtf(v) in IEEE arithmetic). */
float oracle_rstd(float v);

void oracle_decode16(const uint16_t* in, float* out, size_t n, int dtype);
void oracle_encode16(const float* in, uint16_t* out, size_t n, int dtype);
void oracle_e4m3_encode(const float* in, uint8_t* out, size_t n);
void oracle_e4m3_decode(const uint8_t* in, float* out, size_t n);

/* ---- splitmix64 ---- */
uint64_t oracle_rng_next(uint64_t* state);
double oracle_rng_uniform(uint64_t* state);
float oracle_rng_normal(uint64_t* state);

/* Synthetic Q/K/V: layout [b][t][h][d] (K and V with kv_heads heads), 16-bit
 * codes of `dtype`. Q,V ~ N(0,1); K ~ N(0,1)*s + off[h][c], off ~ N(0, k_off_std)
 * with s = outlier_scale on `outlier_channels` random channels per KV head;
 * a fraction `token_frac` of tokens has Q, K and V scaled by token_scale. */
typedef struct {
    int batch, heads, kv_heads, tokens, head_dim, dtype;
    float k_off_std;
    int outlier_channels;
    float outlier_scale;
    float token_frac;
    float token_scale;
    uint64_t seed;
} oracle_gen_spec;
void oracle_generate(const oracle_gen_spec* s, uint16_t* q, uint16_t* k, uint16_t* v);

/* The reference tests' clustered activations (tests.rs:300-329), bf16 codes,
 * layout [b][t][h][d]. */
void oracle_reference_synthetic(int batch, int tokens, int heads, int d, uint64_t seed, uint16_t* q, uint16_t* k,
                                uint16_t* v);

/* ---- prologue (bit-exact restatement) ----
 * Outputs in logical layouts:
 *   q8      [b][h][tq_pad][D]        q_scale [b][h][tq_pad/16]
 *   k8      [b][hkv][tk_pad][D]      k_scale [b][hkv][tk_pad/64]
 *   v8      [b][hkv][tk_pad][D]  E4M3 codes, keys in natural order
 *   stats   [b][hkv][4][D]           K mean, V mean, V scale, 1/V scale
 *   kbias   [tk_pad]                 merged: log2(member count), -inf past tk;
 *                                    dense: left untouched (may be NULL)
 * k8/k_scale/v8 cover the merged keys (tk_pad = merged keys rounded to 64).
 * Returns 0, or -1 for an unsupported head dim. */
int oracle_prologue(const oracle_problem* p, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    int8_t* q8, float* q_scale, int8_t* k8, float* k_scale, uint8_t* v8, float* stats,
                    float* kbias, int threads);

/* ---- attention ----
 * `rows` (nrows entries, each < tokens) selects the query rows computed for
 * every (b, h); NULL computes all rows. Output layout [b][h][nrows][D]. */

/* Textbook softmax attention in f64 of the 16-bit inputs (reference.rs:148-184),
 * with causal masking and grouped-query heads. With KV merging, K and V are
 * pooled as reference.rs:113-143 does (f32 sums in member order, then / n)
 * and key j's logit gains log2(n_j) * ln 2. */
void oracle_attention_f64(const oracle_problem* p, int causal, float scale, const uint16_t* q,
                          const uint16_t* k, const uint16_t* v, const int* rows, int nrows, float* out,
                          int threads);

/* The quantised algorithm on the prologue's tensors: exact int32 S, fp32
 * online softmax in log2 units with a correctly rounded exp2, P -> E4M3,
 * per-64-key fp32 P.V partial folded as O = O*alpha + PV, then
 * out = O/l * v_scale + v_mean. `out` is fp32 before the final 16-bit
 * rounding; `out16` (may be NULL) receives it rounded to `out_dtype`.
 * fast_exp = 1 is the reference's default logit arithmetic (SG_FAST_EXP=1:
 * scores biased by 1.5 * 2^23, the bias removed inside the exp2 FMA);
 * fast_exp = 0 converts the int32 scores exactly (SG_FAST_EXP=0). */
/* With KV merging (kbias from oracle_prologue), the merged kernel's logit
 * arithmetic (sage_attn.cu:264-305 with MERGE): x = fmaf(S', sc, b') with
 * S' = 1.5*2^23 + S and b' = fmaf(-1.5*2^23, sc, kbias) (fast_exp = 1) or
 * S' = S, b' = kbias (fast_exp = 0); m = max(m, max x); p = 2^(x + (log2(448) - m)). */
void oracle_sage_emulate(const oracle_problem* p, int causal, const int8_t* q8, const float* q_scale,
                         const int8_t* k8, const float* k_scale, const uint8_t* v8, const float* stats,
                         const float* kbias, const int* rows, int nrows, float* out, uint16_t* out16,
                         int out_dtype, int fast_exp, int threads);

/* Alternative softmax numerics for oracle_sage_emulate_numerics (each 0 = the
 * reference's): l from the E4M3-rounded P; the running max rounded up to an
 * integer in log2 units (power-of-two rescales); headroom tau above the
 * running max before it moves; p rounded to f16. */
typedef struct {
    int l_from_p8;
    int pow2_max;
    float tau;
    int exp_f16;
} oracle_numerics;

/* oracle_sage_emulate with per-(b, h) rows (rows_stride > 0: the rows of bh
 * start at rows + bh * rows_stride; 0: shared) and optional alternative
 * numerics (nv == NULL: the reference's). */
void oracle_sage_emulate_numerics(const oracle_problem* p, int causal, const int8_t* q8, const float* q_scale,
                                  const int8_t* k8, const float* k_scale, const uint8_t* v8, const float* stats,
                                  const float* kbias, const int* rows, int nrows, int rows_stride, float* out,
                                  uint16_t* out16, int out_dtype, int fast_exp, const oracle_numerics* nv,
                                  int threads);

/* oracle_attention_f64 with per-(b, h) rows, as above. */
void oracle_attention_f64_rows(const oracle_problem* p, int causal, float scale, const uint16_t* q,
                               const uint16_t* k, const uint16_t* v, const int* rows, int nrows, int rows_stride,
                               float* out, int threads);

/* ---- QKV prologue (qkv.cu, qkv.rs) ---- */
enum { ORACLE_NORM_NONE = 0, ORACLE_NORM_LAYER = 1, ORACLE_NORM_RMS = 2 };
enum { ORACLE_ROPE_VGGT = 0, ORACLE_ROPE_DINOV3 = 1 };

/* The fused QKV projection y (bf16 [batch][tokens] rows of ld elements, batch
 * items batch_stride apart; q | k | v, heads*D, kv_heads*D, kv_heads*D wide)
 * and the QkvArgs options of qkv.cu:9-31 (NULL pointers = off). tok is
 * [batch * tokens]; chan and bias are [(heads + 2 kv_heads) * D]; the norm
 * parameters [D] each (biases read under LayerNorm only); rope is
 * [frame_len][D/2][2] (cos, sin). */
typedef struct {
    int batch, tokens, heads, kv_heads, head_dim;
    long long ld, batch_stride;
    const float* tok;
    const float* chan;
    const uint16_t* bias;
    int norm; /* ORACLE_NORM_* */
    const float *q_w, *q_b, *k_w, *k_b;
    float eps;
    const float* rope;
    int rope_layout; /* ORACLE_ROPE_* */
    int frame_len;
    int v_f16; /* V written as f16 codes of its fp32 value (VFormat::F16) */
} oracle_qkv;

int oracle_rope_half(int layout, int D);
int oracle_rope_pair(int layout, int D, int d);
void oracle_rope_table(int layout, int D, int grid_h, int grid_w, int special, double base, float* out);
/* qkv_prologue's fp32 arithmetic, bf16 outputs Q [b][t][heads][D], K and V
 * [b][t][kv_heads][D]. */
void oracle_qkv_prologue(const oracle_qkv* a, const uint16_t* y, uint16_t* q, uint16_t* k, uint16_t* v);
/* qkv::reference (qkv.rs:310-372) in f64, outputs rounded to f32, same layouts. */
void oracle_qkv_reference_f64(const oracle_qkv* a, const uint16_t* y, float* q, float* k, float* v);

/* Errors of `ours` against `ref` (reference.rs:202-225):
 * out[0] cos, [1] rel_l1, [2] rel_l2, [3] max_abs, [4] ref_max. */
void oracle_errors(const float* ours, const float* ref, size_t n, double* out);

#ifdef __cplusplus
}
#endif
#endif
