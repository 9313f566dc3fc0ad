/* CPU oracle of the QKV prologue -- TEST INFRASTRUCTURE ONLY (tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker; the product library never does).
 *
 * Restates, in plain C, the arithmetic of sezer-muhammed/sota-papers-lab,
 * platform/spl-nn:
 *   - cuda/qkv.cu:37-133 (qkv_prologue): the fp32 kernel, bf16 outputs;
 *   - src/qkv.rs:310-372 (reference): the f64 CPU reference its tests gate the
 *     kernel against;
 *   - src/qkv.rs:60-136 (RopeTable::vggt, RopeTable::dinov3, RopeLayout).
 * Head dim 64 is the reference's; 128 is this build's extension (the same
 * arithmetic over 16 lanes of 8 channels, rope pairs D/4 or D/2 apart).
 * Built with -ffp-contract=off: every fused multiply-add is an explicit fmaf.
 */
#include "sage_oracle.h"

#include <math.h>
#include <string.h>

static const double kPi = 3.14159265358979323846;

static inline float bf16f(uint16_t b) { return oracle_bf16_to_f32(b); }

/* RopeLayout::half (qkv.rs:46-52) for head dim D: Vggt D/4, Dinov3 D/2. */
int oracle_rope_half(int layout, int D) { return layout == ORACLE_ROPE_VGGT ? D / 4 : D / 2; }

/* RopeLayout::pair (qkv.rs:55-58): the row of the angle table channel d uses. */
int oracle_rope_pair(int layout, int D, int d) {
    const int h = oracle_rope_half(layout, D);
    return (d / (2 * h)) * h + d % h;
}

/* RopeTable::vggt / ::dinov3 (qkv.rs:87-136): [special + grid_h*grid_w][D/2]
 * of (cos, sin), each the f64 value rounded to f32. With D/2 = P pairs and
 * A = P/2 pairs an axis (16 at D = 64, as the reference), pair p < A follows
 * the row and p >= A the column.
 *   Vggt:   angle = pos * base^(-(p % A) / A), pos = y + 1 or x + 1;
 *   Dinov3: angle = 2 pi coord / base^((p % A) / A), coord = (i + 0.5)/n*2 - 1;
 * special tokens have angle 0. Pinned: the reference's table tests
 * (qkv.rs:396-421) in tests/test_oracle_qkv.py. */
void oracle_rope_table(int layout, int D, int grid_h, int grid_w, int special, double base, float* out) {
    const int P = D / 2, A = P / 2, frame_len = special + grid_h * grid_w;
    for (int t = 0; t < frame_len; t++)
        for (int p = 0; p < P; p++) {
            double a = 0.0;
            if (t >= special) {
                const int y = (t - special) / grid_w, x = (t - special) % grid_w;
                if (layout == ORACLE_ROPE_VGGT) {
                    const double pos = (double)(p < A ? y + 1 : x + 1);
                    a = pos * pow(base, -((double)(p % A)) / (double)A);
                } else {
                    const double coord = p < A ? ((double)y + 0.5) / (double)grid_h * 2.0 - 1.0
                                               : ((double)x + 0.5) / (double)grid_w * 2.0 - 1.0;
                    a = 2.0 * kPi * coord / pow(base, (double)(p % A) / (double)A);
                }
            }
            out[((size_t)t * P + p) * 2] = (float)cos(a);
            out[((size_t)t * P + p) * 2 + 1] = (float)sin(a);
        }
}

/* Channel offset (in the fused projection row) of head h of part 0 (q),
 * 1 (k) or 2 (v): q | k | v, heads*D, kv_heads*D, kv_heads*D wide. */
static int part_channel(const oracle_qkv* a, int part, int h) {
    const int D = a->head_dim;
    return (part == 0 ? h : part == 1 ? a->heads + h : a->heads + a->kv_heads + h) * D;
}

/* One (b, token, part, head) row as qkv_prologue computes it (qkv.cu:50-120),
 * lane c of the D/8 lanes owning channels 8c..8c+7:
 *   x = bf16(y); x *= tok[t]; x *= chan[c]; x += bf16(bias[c]) (each optional,
 *   each rounded: the three sit in separate branches);
 *   QK-norm (q and k only): s_c = ((0 + x_8c) + ..) + x_8c+7, lane sums meeting in
 *   an xor butterfly over 1, 2, .., D/16; mean = s * (1/D) (LayerNorm; 0 for
 *   RMSNorm); ss likewise of fmaf(x - mean, x - mean, ss); r = 1/sqrt(fmaf(ss,
 *   1/D, eps)) correctly rounded (the reference's rsqrtf does not state its
 *   rounding); x = fmaf((x - mean) * r, w, LayerNorm ? b : 0);
 *   RoPE (q and k only): p = x[d ^ half]; (c, s) = table[t % frame_len][pair(d)];
 *   x = fmaf(x, c, +-(p * s)), minus when d & half == 0;
 *   out = bf16(x), round to nearest even.
 * The fused forms are NVRTC's default contraction of the reference's
 * `ss += d * d`, `sum * (1/64) + eps`, `(x - mean) * r * w + b` and
 * `x * c -+ p * s`; which product the last contracts is the compiler's choice,
 * so the rope outputs' last bits are unpinned against the reference GPU. */
static void qkv_row_f32(const oracle_qkv* a, const uint16_t* y, int b, int t, int part, int h, float* x) {
    const int D = a->head_dim, CH = D / 8, c0 = part_channel(a, part, h);
    const uint16_t* yr = y + (size_t)b * a->batch_stride + (size_t)t * a->ld + c0;
    for (int d = 0; d < D; d++) {
        float v = bf16f(yr[d]);
        if (a->tok) v = v * a->tok[(size_t)b * a->tokens + t];
        if (a->chan) v = v * a->chan[c0 + d];
        if (a->bias) v = v + bf16f(a->bias[c0 + d]);
        x[d] = v;
    }
    if (part < 2 && a->norm) {
        const float* w = part == 0 ? a->q_w : a->k_w;
        const float* bb = part == 0 ? a->q_b : a->k_b;
        float ls[16] = {0}, l2[16] = {0}, mean = 0.f;
        if (a->norm == ORACLE_NORM_LAYER) {
            for (int c = 0; c < CH; c++) {
                float s = 0.f;
                for (int e = 0; e < 8; e++) s += x[8 * c + e];
                ls[c] = s;
            }
            for (int o = 1; o < CH; o <<= 1) {
                float tt[16];
                for (int c = 0; c < CH; c++) tt[c] = ls[c] + ls[c ^ o];
                memcpy(ls, tt, sizeof(float) * (size_t)CH);
            }
            mean = ls[0] * (1.0f / (float)D);
        }
        for (int c = 0; c < CH; c++) {
            float s2 = 0.f;
            for (int e = 0; e < 8; e++) {
                const float dv = x[8 * c + e] - mean;
                s2 = fmaf(dv, dv, s2);
            }
            l2[c] = s2;
        }
        for (int o = 1; o < CH; o <<= 1) {
            float tt[16];
            for (int c = 0; c < CH; c++) tt[c] = l2[c] + l2[c ^ o];
            memcpy(l2, tt, sizeof(float) * (size_t)CH);
        }
        const float r = oracle_rstd(fmaf(l2[0], 1.0f / (float)D, a->eps));
        for (int d = 0; d < D; d++)
            x[d] = fmaf((x[d] - mean) * r, w[d], a->norm == ORACLE_NORM_LAYER ? bb[d] : 0.0f);
    }
    if (part < 2 && a->rope) {
        const int half = oracle_rope_half(a->rope_layout, D), P = D / 2;
        const float* row = a->rope + (size_t)(t % a->frame_len) * P * 2;
        float src[128];
        memcpy(src, x, sizeof(float) * (size_t)D);
        for (int d = 0; d < D; d++) {
            const int pr = oracle_rope_pair(a->rope_layout, D, d);
            const float c = row[2 * pr], s = row[2 * pr + 1];
            const float ps = src[d ^ half] * s;
            x[d] = fmaf(src[d], c, (d & half) ? ps : -ps);
        }
    }
}

/* qkv_prologue (qkv.cu:37-133) for every batch item: bf16 Q [b][t][heads][D],
 * K and V [b][t][kv_heads][D] (the layout oracle_prologue reads); with v_f16,
 * V holds f16 codes of the fp32 values (qkv.cu:122-127, cvt.rn.f16x2). */
void oracle_qkv_prologue(const oracle_qkv* a, const uint16_t* y, uint16_t* q, uint16_t* k, uint16_t* v) {
    const int D = a->head_dim, H = a->heads, HK = a->kv_heads;
    float x[128];
    for (int b = 0; b < a->batch; b++)
        for (int t = 0; t < a->tokens; t++)
            for (int part = 0; part < 3; part++) {
                const int nh = part == 0 ? H : HK;
                uint16_t* o = part == 0 ? q : part == 1 ? k : v;
                for (int h = 0; h < nh; h++) {
                    qkv_row_f32(a, y, b, t, part, h, x);
                    uint16_t* r = o + (((size_t)b * a->tokens + t) * nh + h) * D;
                    for (int d = 0; d < D; d++)
                        r[d] = (part == 2 && a->v_f16) ? oracle_f32_to_f16(x[d]) : oracle_f32_to_bf16(x[d]);
                }
            }
}

/* qkv::reference (qkv.rs:310-372): the f64 CPU reference, f32 Q [b][t][heads][D]
 * and K, V [b][t][kv_heads][D] (the f64 values rounded to f32 at the end). */
void oracle_qkv_reference_f64(const oracle_qkv* a, const uint16_t* y, float* q, float* k, float* v) {
    const int D = a->head_dim, H = a->heads, HK = a->kv_heads;
    double x[128], src[128];
    for (int b = 0; b < a->batch; b++)
        for (int t = 0; t < a->tokens; t++)
            for (int part = 0; part < 3; part++) {
                const int nh = part == 0 ? H : HK;
                float* o = part == 0 ? q : part == 1 ? k : v;
                for (int h = 0; h < nh; h++) {
                    const int c0 = part_channel(a, part, h);
                    const uint16_t* yr = y + (size_t)b * a->batch_stride + (size_t)t * a->ld + c0;
                    for (int d = 0; d < D; d++) {
                        double val = (double)bf16f(yr[d]);
                        val *= a->tok ? (double)a->tok[(size_t)b * a->tokens + t] : 1.0;
                        val *= a->chan ? (double)a->chan[c0 + d] : 1.0;
                        x[d] = val + (a->bias ? (double)bf16f(a->bias[c0 + d]) : 0.0);
                    }
                    if (part < 2) {
                        if (a->norm) {
                            const float* w = part == 0 ? a->q_w : a->k_w;
                            const float* bb = part == 0 ? a->q_b : a->k_b;
                            double mean = 0.0, var = 0.0;
                            if (a->norm == ORACLE_NORM_LAYER) {
                                for (int d = 0; d < D; d++) mean += x[d];
                                mean /= (double)D;
                            }
                            for (int d = 0; d < D; d++) var += (x[d] - mean) * (x[d] - mean);
                            var /= (double)D;
                            const double r = 1.0 / sqrt(var + (double)a->eps);
                            for (int d = 0; d < D; d++)
                                x[d] = (x[d] - mean) * r * (double)w[d] +
                                       (a->norm == ORACLE_NORM_LAYER ? (double)bb[d] : 0.0);
                        }
                        if (a->rope) {
                            const int half = oracle_rope_half(a->rope_layout, D), P = D / 2;
                            const float* row = a->rope + (size_t)(t % a->frame_len) * P * 2;
                            memcpy(src, x, sizeof(double) * (size_t)D);
                            for (int d = 0; d < D; d++) {
                                const int pr = oracle_rope_pair(a->rope_layout, D, d);
                                const double c = row[2 * pr], s = row[2 * pr + 1], p = src[d ^ half];
                                x[d] = (d & half) == 0 ? src[d] * c - p * s : src[d] * c + p * s;
                            }
                        }
                    }
                    float* r = o + (((size_t)b * a->tokens + t) * nh + h) * D;
                    for (int d = 0; d < D; d++) r[d] = (float)x[d];
                }
            }
}
