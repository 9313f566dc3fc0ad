/* CPU oracle for the SageAttention2 forward path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, as the checker; the product library never does.
 *
 * Build with -ffp-contract=off: every fused multiply-add below is written as
 * an explicit fmaf() where the reference's arithmetic is one, and nowhere
 * else. Citations are into sezer-muhammed/sota-papers-lab, platform/spl-nn/.
 */
#include "sage_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* ------------------------------------------------------------------ codecs */

/* bf16 bits -> f32, exact. reference.rs:8-10. Pinned: KAT bf16_rounds_to_nearest_even
 * (tests.rs:57-66) and the closed form bits << 16. */
float oracle_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* f32 -> bf16 bits, round to nearest even, NaN stays NaN. reference.rs:13-20.
 * Pinned: KATs tests.rs:57-66; exhaustive check against a rational rounding in tests. */
uint16_t oracle_f32_to_bf16(float x) {
    uint32_t bits = f2u(x);
    if (isnan(x)) return (uint16_t)((bits >> 16) | 0x40);
    uint32_t round = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + round) >> 16);
}

/* IEEE binary16 -> f32 (extension: fp16 inputs have no reference twin).
 * Pinned: numpy float16 over all 65536 codes in tests. */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        float m = (float)man * (1.0f / 16777216.0f); /* man * 2^-24, exact */
        return sign ? -m : m;
    }
    return u2f(sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13));
}

/* f32 -> binary16, round to nearest even (the output extension).
 * Pinned: numpy float16 casts in tests. */
uint16_t oracle_f32_to_f16(float x) {
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                    /* below 2^-14: subnormal */
        double v = (double)u2f(a) * 16777216.0;               /* units of 2^-24, exact */
        double r = nearbyint(v);                              /* ties to even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    r >>= 13;
    return (uint16_t)(sign | (uint16_t)(r - ((127u - 15u) << 10)));
}

/* E4M3 byte -> f32; 0x7f and 0xff are NaN. reference.rs:23-36.
 * Pinned: KAT e4m3_codes_round_trip (tests.rs:24-37). */
float oracle_e4m3_to_f32(uint8_t b) {
    float sign = (b & 0x80) ? -1.0f : 1.0f;
    int exp = (b >> 3) & 0xf;
    float man = (float)(b & 7);
    if (exp == 15 && (b & 7) == 7) return NAN;
    float mag = exp == 0 ? man * ldexpf(1.0f, -9) : (1.0f + man / 8.0f) * ldexpf(1.0f, exp - 7);
    return sign * mag;
}

/* f32 -> E4M3, round to nearest even, saturating at +-448 (reference.rs:40-70,
 * the semantics of cvt.rn.satfinite.e4m3x2.f32 used by sage_common.cu:83-87).
 * Restated on the bit pattern; the reference rounds k = a / 2^(e-3) in f64,
 * which is the same RNE on the same grid. Pinned: KATs tests.rs:24-55 and an
 * exhaustive comparison with an exact rational rounding in tests. */
uint8_t oracle_f32_to_e4m3(float x) {
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7f;           /* NaN */
    if (a >= 0x43e00000u) return sign | 0x7e;   /* |x| >= 448 (and inf) */
    if (a >= 0x3c800000u) {                     /* |x| >= 2^-6: normal grid */
        uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
        return sign | (uint8_t)(r - (120u << 3));
    }
    /* subnormal grid k * 2^-9, k in [0, 8]; k = 8 is the code of 2^-6 */
    float k = nearbyintf(u2f(a) * 512.0f);
    return sign | (uint8_t)k;
}

/* Round to nearest even and clamp to +-127 (sage_common.cu:95-99). */
int oracle_s8(float x) {
    float r = nearbyintf(x);
    if (isnan(r)) return 0;
    if (r > 127.0f) return 127;
    if (r < -127.0f) return -127;
    return (int)r;
}

/* The reference's NVIDIA-fragment key permutation (reference.rs:74-76),
 * kept for its known-answer test (tests.rs:68-83) only. */
/* IEEE single precision: sqrtf and the divide each round to nearest. Pinned
 * by the closed forms of the LayerNorm tests (tests/test_oracle_qknorm.py). */
float oracle_rstd(float v) { return 1.0f / sqrtf(v); }

/* Pinned: numpy's float64 -> float16 conversion on random, tie, subnormal and
 * overflow values (tests/test_oracle_codecs.py). */
double oracle_round_f16(double x) {
    if (x == 0.0 || !isfinite(x)) return x;
    int e;
    frexp(x, &e);             /* |x| in [2^(e-1), 2^e) */
    int q = e - 11;           /* f16 keeps 11 significant bits ... */
    if (q < -24) q = -24;     /* ... down to the subnormal quantum 2^-24 */
    const double s = ldexp(1.0, q);
    const double r = rint(x / s) * s; /* exact scaling; rint rounds ties to even */
    return fabs(r) > 65504.0 ? copysign(INFINITY, x) : r;
}

int oracle_vpos_ref(int k) { return ((k >> 1) & 3) * 4 + ((k >> 3) << 1) + (k & 1); }

void oracle_decode16(const uint16_t* in, float* out, size_t n, int dtype) {
    for (size_t i = 0; i < n; i++) out[i] = dtype == ORACLE_F16 ? oracle_f16_to_f32(in[i]) : oracle_bf16_to_f32(in[i]);
}
void oracle_encode16(const float* in, uint16_t* out, size_t n, int dtype) {
    for (size_t i = 0; i < n; i++) out[i] = dtype == ORACLE_F16 ? oracle_f32_to_f16(in[i]) : oracle_f32_to_bf16(in[i]);
}
void oracle_e4m3_encode(const float* in, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_f32_to_e4m3(in[i]);
}
void oracle_e4m3_decode(const uint8_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_e4m3_to_f32(in[i]);
}

static inline float dec16(uint16_t h, int dtype) {
    return dtype == ORACLE_F16 ? oracle_f16_to_f32(h) : oracle_bf16_to_f32(h);
}

/* ------------------------------------------------------------- splitmix64 */

/* reference.rs:235-241. Pinned: published splitmix64 test vector in tests. */
uint64_t oracle_rng_next(uint64_t* s) {
    *s += 0x9e3779b97f4a7c15ull;
    uint64_t z = *s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
/* reference.rs:244-246 */
double oracle_rng_uniform(uint64_t* s) { return (double)(oracle_rng_next(s) >> 11) / (double)(1ull << 53); }
/* Box-Muller, reference.rs:249-253 */
float oracle_rng_normal(uint64_t* s) {
    double u1 = oracle_rng_uniform(s);
    if (u1 < 1e-300) u1 = 1e-300;
    double u2 = oracle_rng_uniform(s);
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

void oracle_generate(const oracle_gen_spec* sp, uint16_t* q, uint16_t* k, uint16_t* v) {
    uint64_t st = sp->seed;
    const int B = sp->batch, H = sp->heads, HK = sp->kv_heads, T = sp->tokens, D = sp->head_dim;
    float* off = (float*)malloc(sizeof(float) * (size_t)HK * D);
    unsigned char* outl = (unsigned char*)calloc((size_t)HK * D, 1);
    for (int i = 0; i < HK * D; i++) off[i] = sp->k_off_std * oracle_rng_normal(&st);
    for (int h = 0; h < HK; h++) {
        int n = sp->outlier_channels < D ? sp->outlier_channels : D;
        for (int c = 0; c < n;) {
            int ch = (int)(oracle_rng_next(&st) % (uint64_t)D);
            if (!outl[h * D + ch]) { outl[h * D + ch] = 1; c++; }
        }
    }
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) {
            float ts = 1.0f;
            if (sp->token_frac > 0.0f && oracle_rng_uniform(&st) < (double)sp->token_frac) ts = sp->token_scale;
            size_t rq = ((size_t)b * T + t) * H * D, rk = ((size_t)b * T + t) * HK * D;
            for (int i = 0; i < H * D; i++) {
                float x = oracle_rng_normal(&st) * ts;
                q[rq + i] = sp->dtype == ORACLE_F16 ? oracle_f32_to_f16(x) : oracle_f32_to_bf16(x);
            }
            for (int i = 0; i < HK * D; i++) {
                float s = outl[i] ? sp->outlier_scale : 1.0f;
                float xk = (oracle_rng_normal(&st) * s + off[i]) * ts;
                float xv = oracle_rng_normal(&st) * ts;
                k[rk + i] = sp->dtype == ORACLE_F16 ? oracle_f32_to_f16(xk) : oracle_f32_to_bf16(xk);
                v[rk + i] = sp->dtype == ORACLE_F16 ? oracle_f32_to_f16(xv) : oracle_f32_to_bf16(xv);
            }
        }
    free(off);
    free(outl);
}

/* The reference tests' synthetic activations (tests.rs:300-329): 37 token
 * clusters, per (head, channel) K offset 3*N(0,1) and V offset 2*N(0,1),
 * K outlier channels x % 23 == 5 scaled by 6, every value rounded to bf16.
 * Same draw order as the reference: centers, K offsets, V offsets, then per
 * token its cluster and per (head, channel) one normal each for q, k, v.
 * Layout [b][t][h][d], bf16 codes. Pinned: draw order restated from reading;
 * statistics (cluster structure, offsets) checked in tests. */
void oracle_reference_synthetic(int batch, int tokens, int heads, int d, uint64_t seed, uint16_t* q, uint16_t* k,
                                uint16_t* v) {
    uint64_t st = seed;
    const int clusters = 37;
    float* centers = (float*)malloc(sizeof(float) * (size_t)clusters * heads * d);
    float* k_off = (float*)malloc(sizeof(float) * (size_t)heads * d);
    float* v_off = (float*)malloc(sizeof(float) * (size_t)heads * d);
    for (size_t i = 0; i < (size_t)clusters * heads * d; i++) centers[i] = oracle_rng_normal(&st);
    for (int i = 0; i < heads * d; i++) k_off[i] = 3.0f * oracle_rng_normal(&st);
    for (int i = 0; i < heads * d; i++) v_off[i] = 2.0f * oracle_rng_normal(&st);
    for (int b = 0; b < batch; b++)
        for (int t = 0; t < tokens; t++) {
            const int c = (int)(oracle_rng_next(&st) % (uint64_t)clusters);
            for (int h = 0; h < heads; h++)
                for (int x = 0; x < d; x++) {
                    const size_t i = (((size_t)b * tokens + t) * heads + h) * d + x;
                    const float ctr = centers[((size_t)c * heads + h) * d + x];
                    const float outlier = x % 23 == 5 ? 6.0f : 1.0f;
                    const float fq = 1.6f * ctr + 0.6f * oracle_rng_normal(&st);
                    const float fk = (1.6f * ctr + 0.6f * oracle_rng_normal(&st)) * outlier + k_off[h * d + x];
                    const float fv = oracle_rng_normal(&st) + 0.5f * ctr + v_off[h * d + x];
                    q[i] = oracle_f32_to_bf16(fq);
                    k[i] = oracle_f32_to_bf16(fk);
                    v[i] = oracle_f32_to_bf16(fv);
                }
        }
    free(centers);
    free(k_off);
    free(v_off);
}

/* --------------------------------------------------------------- prologue */

static size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

/* ------------------------------------------------------------- LayerNorm */

/* The xor butterfly of n lane values (s_c <- s_c + s_(c^o), o = 1, 2, ..,
 * n/2); every lane ends with the same sum. */
static void lane_butterfly(float* s, int n) {
    float t[32];
    for (int o = 1; o < n; o <<= 1) {
        for (int c = 0; c < n; c++) t[c] = s[c] + s[c ^ o];
        memcpy(s, t, sizeof(float) * (size_t)n);
    }
}

/* sg_layernorm (sage_quant.cu:34-52) as the prologue kernels compute it. Lane
 * c of the D/8 lanes that hold a row owns channels 8c..8c+7:
 *   s_c = ((0 + x_8c) + x_8c+1) + ... + x_8c+7, the lane sums meeting in an
 *   xor butterfly over distances 1, 2, .., D/16; mean = s * (1/D);
 *   the squared deviations the same way, each step fmaf(x - mean, x - mean, s2);
 *   rstd = 1 / sqrt(fmaf(s2, 1/D, eps)), the square root and the divide each
 *   correctly rounded;
 *   y = fmaf((x - mean) * rstd, w, b).
 * The fused forms are NVRTC's default contraction of the reference's
 * `s2 += d * d`, `s2 * (1.0f / D) + eps` and `(x - mean) * rstd * w + b`.
 * The reference takes rsqrtf, an approximation whose rounding it does not
 * state; this build takes the correctly rounded form instead, so a normalised
 * value can differ from the reference GPU's in its last bits.
 * Pinned: against the reference's f64 layer_norm (reference.rs:109-118) on
 * random, offset, eps-dominated and constant rows, and through check_prologue
 * with QK LayerNorm (tests.rs:448-466, 476-594), in tests. */
void oracle_layernorm(const float* x, float* y, int D, const float* w, const float* b, float eps) {
    const int CH = D / 8;
    float ls[32], l2[32];
    for (int c = 0; c < CH; c++) {
        float s = 0.f;
        for (int e = 0; e < 8; e++) s += x[8 * c + e];
        ls[c] = s;
    }
    lane_butterfly(ls, CH);
    const float mean = ls[0] * (1.0f / (float)D);
    for (int c = 0; c < CH; c++) {
        float s2 = 0.f;
        for (int e = 0; e < 8; e++) {
            const float d = x[8 * c + e] - mean;
            s2 = fmaf(d, d, s2);
        }
        l2[c] = s2;
    }
    lane_butterfly(l2, CH);
    const float rstd = oracle_rstd(fmaf(l2[0], 1.0f / (float)D, eps));
    for (int i = 0; i < D; i++) y[i] = fmaf((x[i] - mean) * rstd, w[i], b[i]);
}

/* reference.rs:109-118 (layer_norm): the f64 LayerNorm of the reference's
 * tests. Pinned: numpy float64 and closed forms in tests. */
void oracle_layernorm_f64(const float* x, float* y, int D, const float* w, const float* b, float eps) {
    double mean = 0.0, var = 0.0;
    for (int i = 0; i < D; i++) mean += (double)x[i];
    mean /= (double)D;
    for (int i = 0; i < D; i++) var += ((double)x[i] - mean) * ((double)x[i] - mean);
    var /= (double)D;
    const double rstd = 1.0 / sqrt(var + (double)eps);
    for (int i = 0; i < D; i++) y[i] = (float)(((double)x[i] - mean) * rstd * (double)w[i] + (double)b[i]);
}

/* Head row `tok` of a 16-bit [b][t][h][d] input, decoded. */
static void read_row(const oracle_problem* p, const uint16_t* x, long long sb, long long st, long long sh, int b,
                     int h, int tok, float* out) {
    const uint16_t* r = x + b * sb + (long long)tok * st + h * sh;
    for (int d = 0; d < p->head_dim; d++) out[d] = dec16(r[d], p->dtype);
}

/* Q (is_k = 0) or K (is_k = 1) head row, decoded and, under QK LayerNorm,
 * normalised as the prologue kernels do (sage_quant.cu:89-90, :271). */
static void qk_row(const oracle_problem* p, const uint16_t* x, int is_k, int b, int h, int tok, float* out) {
    const int D = p->head_dim;
    if (is_k) read_row(p, x, p->k_sb, p->k_st, p->k_sh, b, h, tok, out);
    else read_row(p, x, p->q_sb, p->q_st, p->q_sh, b, h, tok, out);
    if (p->ln) oracle_layernorm(out, out, D, p->ln + (is_k ? 2 : 0) * D, p->ln + (is_k ? 3 : 1) * D, p->ln_eps);
}

/* Per (b, kv head) channel statistics in the reference's fp32 order
 * (sage_quant.cu:73-80,97-107,129-159 then :163-205):
 *   slot s of a 128-token tile sums its tokens t*128 + s + TPI*i in i order
 *   from 0.0f (TPI = 256 / (D/8)); a 32-lane warp combines its slots by a
 *   butterfly (D=128: P[2w]+P[2w+1]; D=64: (P[4w]+P[4w+1])+(P[4w+2]+P[4w+3]));
 *   the tile partial folds warps 0..7 left to right; the finalize folds even
 *   and odd tiles separately from 0.0f and adds the two.
 * Pinned: tolerance invariants of check_prologue (tests.rs:526-536) and closed
 * forms in tests; the fold order itself is restated from reading the
 * reference and agreed with by a second restatement (numpy) in tests. */
static void kv_stats(const oracle_problem* p, int b, int hk, const uint16_t* k, const uint16_t* v,
                     float* st /* [4][D] */) {
    const int D = p->head_dim, N = p->tokens, CH = D / 8, TPI = 256 / CH, NI = ORACLE_QTILE / TPI;
    const int q_tiles = (int)(round_up((size_t)N, ORACLE_QTILE) / ORACLE_QTILE);
    float* part = (float*)malloc(sizeof(float) * (size_t)q_tiles * 4 * D);
    float* P = (float*)malloc(sizeof(float) * (size_t)TPI * 4 * D); /* slot partials [s][stat][d] */
    float fk[256], fv[256];
    for (int t = 0; t < q_tiles; t++) {
        for (int s = 0; s < TPI; s++) {
            float* Ps = P + (size_t)s * 4 * D;
            for (int d = 0; d < D; d++) {
                Ps[d] = 0.f;
                Ps[D + d] = 0.f;
                Ps[2 * D + d] = 3.0e38f;
                Ps[3 * D + d] = -3.0e38f;
            }
            for (int i = 0; i < NI; i++) {
                int tok = t * ORACLE_QTILE + s + TPI * i;
                if (tok >= N) continue;
                qk_row(p, k, 1, b, hk, tok, fk);
                read_row(p, v, p->v_sb, p->v_st, p->v_sh, b, hk, tok, fv);
                for (int d = 0; d < D; d++) {
                    Ps[d] += fk[d];
                    Ps[D + d] += fv[d];
                    Ps[2 * D + d] = fminf(Ps[2 * D + d], fv[d]);
                    Ps[3 * D + d] = fmaxf(Ps[3 * D + d], fv[d]);
                }
            }
        }
        const int spw = 32 / CH; /* slots per 32-lane warp: 2 (D=128) or 4 (D=64) */
        for (int stat = 0; stat < 4; stat++)
            for (int d = 0; d < D; d++) {
                float r = 0.f;
                for (int w = 0; w < 8; w++) {
                    const float* x = P + (size_t)stat * D + d;
                    size_t sl = (size_t)4 * D; /* stride between slots */
                    float W;
                    if (spw == 2) {
                        float a = x[(2 * w) * sl], c = x[(2 * w + 1) * sl];
                        W = stat < 2 ? a + c : (stat == 2 ? fminf(a, c) : fmaxf(a, c));
                    } else {
                        float a0 = x[(4 * w) * sl], a1 = x[(4 * w + 1) * sl];
                        float a2 = x[(4 * w + 2) * sl], a3 = x[(4 * w + 3) * sl];
                        if (stat < 2) W = (a0 + a1) + (a2 + a3);
                        else if (stat == 2) W = fminf(fminf(a0, a1), fminf(a2, a3));
                        else W = fmaxf(fmaxf(a0, a1), fmaxf(a2, a3));
                    }
                    if (w == 0) r = W;
                    else r = stat < 2 ? r + W : (stat == 2 ? fminf(r, W) : fmaxf(r, W));
                }
                part[((size_t)t * 4 + stat) * D + d] = r;
            }
    }
    /* sg_finalize (sage_quant.cu:168-205) */
    float fin[4][256];
    for (int stat = 0; stat < 4; stat++)
        for (int d = 0; d < D; d++) {
            float r0 = stat < 2 ? 0.f : (stat == 2 ? 3.0e38f : -3.0e38f), r1 = r0;
            int t = 0;
            for (; t + 1 < q_tiles; t += 2) {
                float x0 = part[((size_t)t * 4 + stat) * D + d], x1 = part[((size_t)(t + 1) * 4 + stat) * D + d];
                if (stat < 2) { r0 += x0; r1 += x1; }
                else if (stat == 2) { r0 = fminf(r0, x0); r1 = fminf(r1, x1); }
                else { r0 = fmaxf(r0, x0); r1 = fmaxf(r1, x1); }
            }
            if (t < q_tiles) {
                float x0 = part[((size_t)t * 4 + stat) * D + d];
                r0 = stat < 2 ? r0 + x0 : (stat == 2 ? fminf(r0, x0) : fmaxf(r0, x0));
            }
            fin[stat][d] = stat < 2 ? r0 + r1 : (stat == 2 ? fminf(r0, r1) : fmaxf(r0, r1));
        }
    for (int d = 0; d < D; d++) {
        const float n = (float)N;
        const float mk = p->smooth_k ? fin[0][d] / n : 0.f;
        const float mv = p->smooth_v ? fin[1][d] / n : 0.f;
        const float amax = fmaxf(fin[3][d] - mv, mv - fin[2][d]);
        const float scale = amax > 0.f ? amax / p->v_range : 1.0f;
        st[d] = mk;
        st[D + d] = mv;
        st[2 * D + d] = scale;
        st[3 * D + d] = 1.0f / scale;
    }
    free(P);
    free(part);
}

/* INT8 Q per 16-row group (sage_quant.cu:95-127): amax over valid rows,
 * inv = 127/amax, code = RNE clamp(q*inv), scale = (amax * (1/127)) * q_mul.
 * Pinned: tolerance invariants tests.rs:496-521 and closed forms in tests. */
static void quant_q(const oracle_problem* p, int b, int h, const uint16_t* q, int8_t* q8, float* qsc) {
    const int D = p->head_dim, N = p->tokens;
    const size_t tq_pad = round_up((size_t)N, ORACLE_QTILE);
    float x[ORACLE_QGROUP][256];
    for (size_t g = 0; g < tq_pad / ORACLE_QGROUP; g++) {
        float amax = 0.f;
        for (int r = 0; r < ORACLE_QGROUP; r++) {
            int tok = (int)(g * ORACLE_QGROUP) + r;
            if (tok < N) qk_row(p, q, 0, b, h, tok, x[r]);
            else memset(x[r], 0, sizeof(float) * (size_t)D);
            for (int d = 0; d < D; d++) amax = fmaxf(amax, fabsf(x[r][d]));
        }
        const float inv = amax > 0.f ? 127.0f / amax : 0.f;
        for (int r = 0; r < ORACLE_QGROUP; r++) {
            int tok = (int)(g * ORACLE_QGROUP) + r;
            for (int d = 0; d < D; d++) q8[(size_t)tok * D + d] = (int8_t)oracle_s8(x[r][d] * inv);
        }
        qsc[g] = amax * (1.0f / 127.0f) * p->q_mul;
    }
}

/* ------------------------------------------------------------ KV merging */

static int merging(const oracle_problem* p) { return p->merge > 1; }

static int frame_tokens(const oracle_problem* p) { return p->special + p->grid_h * p->grid_w; }

static int merged_per_frame(const oracle_problem* p) {
    const int s = p->merge;
    return p->special + ((p->grid_h + s - 1) / s) * ((p->grid_w + s - 1) / s);
}

/* FrameLayout::merged_keys (mod.rs:293-299). */
int oracle_merged_keys(const oracle_problem* p) {
    if (!merging(p)) return p->tokens;
    const int d = p->dense_frames < p->frames ? p->dense_frames : p->frames;
    return d * frame_tokens(p) + (p->frames - d) * merged_per_frame(p);
}

/* reference.rs:79-109 (members, cell_members). Pinned by the reference's
 * KATs (tests.rs:96-173: the first pooled cell of frame 1, member counts of
 * edge cells, every token pooled exactly once), ported in tests. */
int oracle_members(const oracle_problem* p, int j, int* tokens) {
    if (!merging(p)) {
        if (tokens) tokens[0] = j;
        return 1;
    }
    const int s = p->merge, ft = frame_tokens(p), per = merged_per_frame(p);
    const int df = p->dense_frames < p->frames ? p->dense_frames : p->frames;
    const int dense = df * ft;
    if (j < dense) {
        if (tokens) tokens[0] = j;
        return 1;
    }
    const int f = df + (j - dense) / per, loc = (j - dense) % per, base = f * ft;
    if (loc < p->special) {
        if (tokens) tokens[0] = base + loc;
        return 1;
    }
    const int cell = loc - p->special, mw = (p->grid_w + s - 1) / s;
    const int y0 = (cell / mw) * s, x0 = (cell % mw) * s;
    int n = 0;
    for (int y = y0; y < y0 + s && y < p->grid_h; y++)
        for (int x = x0; x < x0 + s && x < p->grid_w; x++) {
            if (tokens) tokens[n] = base + p->special + y * p->grid_w + x;
            n++;
        }
    return n;
}

/* log2(n), n = 1..16, each the f32 nearest the exact value (checked in tests
 * against a 60-digit evaluation and numpy). */
float oracle_log2_count(int n) {
    static const uint32_t bits[17] = {0xff800000u, 0x00000000u, 0x3f800000u, 0x3fcae00du, 0x40000000u, 0x40149a78u,
                                      0x40257007u, 0x4033abb4u, 0x40400000u, 0x404ae00du, 0x40549a78u, 0x405d6754u,
                                      0x40657007u, 0x406cd401u, 0x4073abb4u, 0x407a0a7fu, 0x40800000u};
    return (n >= 0 && n <= 16) ? u2f(bits[n]) : (float)log2((double)n);
}

/* INT8 K per 64-key block and E4M3 V per channel (sage_quant.cu:238-319).
 * Key j pools its members in order from 0.0f (one member when dense):
 *   ks = ((0 + k_0) + k_1) + ...,  rc = 1.0f / n,
 *   kv = fmaf(ks, rc, -mean_k)   code = RNE clamp(kv * (127/amax_blk)), scale = amax_blk / 127,
 *   vq = fmaf(vs, rc, -mean_v) * (1/v_scale)   code = e4m3 RNE satfinite.
 * The fused form follows NVRTC's default contraction of `ks * rc - mean`; it
 * equals the two-rounding form whenever n is a power of two (rc exact), i.e.
 * for every dense key and every full cell. Padded keys are 0.
 * Pinned: tolerance invariants tests.rs:538-581 and closed forms in tests;
 * the fused rounding of 3-, 6-, 9- and 12-member edge cells is unpinned. */
static void quant_kv(const oracle_problem* p, int b, int hk, const uint16_t* k, const uint16_t* v, const float* st,
                     int8_t* k8, float* ksc, uint8_t* v8) {
    const int D = p->head_dim, TK = oracle_merged_keys(p);
    const size_t tk_pad = round_up((size_t)TK, ORACLE_KBLOCK);
    float* kv = (float*)malloc(sizeof(float) * ORACLE_KBLOCK * D);
    float ks[256], vs[256], fk[256], fv[256];
    int mem[16];
    for (size_t blk = 0; blk < tk_pad / ORACLE_KBLOCK; blk++) {
        float amax = 0.f;
        for (int r = 0; r < ORACLE_KBLOCK; r++) {
            int j = (int)(blk * ORACLE_KBLOCK) + r;
            const int n = j < TK ? oracle_members(p, j, mem) : 0;
            const float rc = n > 0 ? 1.0f / (float)n : 0.f;
            for (int d = 0; d < D; d++) ks[d] = vs[d] = 0.f;
            for (int m = 0; m < n; m++) {
                qk_row(p, k, 1, b, hk, mem[m], fk);
                read_row(p, v, p->v_sb, p->v_st, p->v_sh, b, hk, mem[m], fv);
                for (int d = 0; d < D; d++) {
                    ks[d] += fk[d];
                    vs[d] += fv[d];
                }
            }
            for (int d = 0; d < D; d++) {
                float x = 0.f, vq = 0.f;
                if (n > 0) {
                    x = fmaf(ks[d], rc, -st[d]);
                    vq = fmaf(vs[d], rc, -st[D + d]) * st[3 * D + d];
                }
                kv[r * D + d] = x;
                amax = fmaxf(amax, fabsf(x));
                v8[(size_t)j * D + d] = oracle_f32_to_e4m3(vq);
            }
        }
        const float inv = amax > 0.f ? 127.0f / amax : 0.f;
        for (int r = 0; r < ORACLE_KBLOCK; r++) {
            size_t j = blk * ORACLE_KBLOCK + r;
            for (int d = 0; d < D; d++) k8[j * D + d] = (int8_t)oracle_s8(kv[r * D + d] * inv);
        }
        ksc[blk] = amax * (1.0f / 127.0f);
    }
    free(kv);
}

int oracle_prologue(const oracle_problem* p, const uint16_t* q, const uint16_t* k, const uint16_t* v, int8_t* q8,
                    float* q_scale, int8_t* k8, float* k_scale, uint8_t* v8, float* stats, float* kbias,
                    int threads) {
    const int D = p->head_dim;
    if (D != 64 && D != 128) return -1;
    const size_t tq_pad = round_up((size_t)p->tokens, ORACLE_QTILE);
    const int TK = oracle_merged_keys(p);
    const size_t tk_pad = round_up((size_t)TK, ORACLE_KBLOCK);
    if (merging(p) && kbias)
        for (size_t j = 0; j < tk_pad; j++)
            kbias[j] = (int)j < TK ? oracle_log2_count(oracle_members(p, (int)j, NULL)) : -INFINITY;
    set_threads(threads);
    const int B = p->batch, H = p->heads, HK = p->kv_heads;
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * HK; bh++) {
        int b = bh / HK, hk = bh % HK;
        float* st = stats + (size_t)bh * 4 * D;
        kv_stats(p, b, hk, k, v, st);
        quant_kv(p, b, hk, k, v, st, k8 + (size_t)bh * tk_pad * D, k_scale + (size_t)bh * (tk_pad / ORACLE_KBLOCK),
                 v8 + (size_t)bh * tk_pad * D);
    }
#pragma omp parallel for schedule(dynamic)
    for (int bh = 0; bh < B * H; bh++) {
        int b = bh / H, h = bh % H;
        quant_q(p, b, h, q, q8 + (size_t)bh * tq_pad * D, q_scale + (size_t)bh * (tq_pad / ORACLE_QGROUP));
    }
    return 0;
}

/* -------------------------------------------------------------- attention */

/* Softmax attention in f64 (reference.rs:148-184), over the decoded 16-bit
 * inputs; causal rows see keys j <= i; Q head h reads KV head h / (H/HKV).
 * KV merging pools K and V per (b, kv head) first, as reference.rs:113-143
 * does (f32 sums in member order, then / n in f32), and adds
 * log2(n_j) * ln 2 to key j's logits. Under QK LayerNorm the Q and K rows
 * are normalised first by the reference's f64 layer_norm (tests.rs:448-466).
 * Pinned: closed forms in tests (uniform keys give the mean of V; one-hot
 * logits select one V row; V = const gives const), numpy/torch float64, and
 * the reference's merged == dense identity on uniform cells (tests.rs:193-232). */
void oracle_attention_f64_rows(const oracle_problem* p, int causal, float scale, const uint16_t* q,
                               const uint16_t* k, const uint16_t* v, const int* rows, int nrows, int rows_stride,
                               float* out, int threads) {
    const int B = p->batch, H = p->heads, HK = p->kv_heads, N = p->tokens, D = p->head_dim, G = H / HK;
    const int TK = oracle_merged_keys(p);
    const int R = rows ? nrows : N;
    /* K and V as f32 [b][hk][j][d] over the (possibly merged) keys, and the log-count bias. */
    float* kf = (float*)malloc(sizeof(float) * (size_t)B * HK * TK * D);
    float* vf = (float*)malloc(sizeof(float) * (size_t)B * HK * TK * D);
    double* kb = (double*)malloc(sizeof(double) * (size_t)TK);
    int mem[16];
    float rk[256], rv[256];
    for (int j = 0; j < TK; j++) {
        const int n = oracle_members(p, j, mem);
        kb[j] = merging(p) ? (double)oracle_log2_count(n) * 0.69314718055994530942 : 0.0;
        for (int b = 0; b < B; b++)
            for (int hk = 0; hk < HK; hk++) {
                float* ko = kf + (((size_t)b * HK + hk) * TK + j) * D;
                float* vo = vf + (((size_t)b * HK + hk) * TK + j) * D;
                for (int d = 0; d < D; d++) ko[d] = vo[d] = 0.f;
                for (int m = 0; m < n; m++) {
                    read_row(p, k, p->k_sb, p->k_st, p->k_sh, b, hk, mem[m], rk);
                    read_row(p, v, p->v_sb, p->v_st, p->v_sh, b, hk, mem[m], rv);
                    if (p->ln) oracle_layernorm_f64(rk, rk, D, p->ln + 2 * D, p->ln + 3 * D, p->ln_eps);
                    for (int d = 0; d < D; d++) {
                        ko[d] += rk[d];
                        vo[d] += rv[d];
                    }
                }
                for (int d = 0; d < D; d++) {
                    ko[d] /= (float)n;
                    vo[d] /= (float)n;
                }
            }
    }
    set_threads(threads);
#pragma omp parallel
    {
        double* logit = (double*)malloc(sizeof(double) * TK);
        double* acc = (double*)malloc(sizeof(double) * D);
        double* qi = (double*)malloc(sizeof(double) * D);
        float qf[256];
#pragma omp for schedule(dynamic) collapse(2)
        for (int bh = 0; bh < B * H; bh++)
            for (int ri = 0; ri < R; ri++) {
                int b = bh / H, h = bh % H, hk = h / G;
                int i = rows ? rows[(size_t)bh * rows_stride + ri] : ri;
                read_row(p, q, p->q_sb, p->q_st, p->q_sh, b, h, i, qf);
                if (p->ln) oracle_layernorm_f64(qf, qf, D, p->ln, p->ln + D, p->ln_eps);
                for (int d = 0; d < D; d++) qi[d] = qf[d];
                const float* kr0 = kf + ((size_t)b * HK + hk) * TK * D;
                const float* vr0 = vf + ((size_t)b * HK + hk) * TK * D;
                int nk = causal ? i + 1 : TK;
                double mx = -INFINITY;
                for (int j = 0; j < nk; j++) {
                    const float* kr = kr0 + (size_t)j * D;
                    double dot = 0;
                    for (int d = 0; d < D; d++) dot += qi[d] * (double)kr[d];
                    logit[j] = dot * (double)scale + kb[j];
                    if (logit[j] > mx) mx = logit[j];
                }
                double sum = 0;
                for (int d = 0; d < D; d++) acc[d] = 0;
                for (int j = 0; j < nk; j++) {
                    double pj = exp(logit[j] - mx);
                    sum += pj;
                    const float* vr = vr0 + (size_t)j * D;
                    for (int d = 0; d < D; d++) acc[d] += pj * (double)vr[d];
                }
                float* o = out + ((size_t)bh * R + ri) * D;
                for (int d = 0; d < D; d++) o[d] = (float)(acc[d] / sum);
            }
        free(logit);
        free(acc);
        free(qi);
    }
    free(kf);
    free(vf);
    free(kb);
}

void oracle_attention_f64(const oracle_problem* p, int causal, float scale, const uint16_t* q, const uint16_t* k,
                          const uint16_t* v, const int* rows, int nrows, float* out, int threads) {
    oracle_attention_f64_rows(p, causal, scale, q, k, v, rows, nrows, 0, out, threads);
}

/* Correctly rounded exp2 in f32 (the build's stand-in for a hardware exp2;
 * the reference's ex2.approx is an NVIDIA approximation and is not restated). */
static inline float ex2f_cr(float x) { return (float)exp2((double)x); }

/* The reference's attention arithmetic on quantised tensors
 * (sage_attn.cu:262-344, :402-421), sc = qs*ks:
 *   SG_FAST_EXP=0 (fast_exp = 0): x = S (exact int32 as float),
 *     xoff = 0;
 *   SG_FAST_EXP=1 (fast_exp = 1, the reference's default, sage_attn.cu:59-61):
 *     x = 1.5*2^23 + S (the float whose bits are 0x4B400000 + S, exact for
 *     |S| < 2^22; sage_attn.cu:23-25,265-270), xoff = -(1.5*2^23) * sc in
 *     fp32 (sage_attn.cu:284);
 *   then mnew = max(m, fmaf(max x, sc, xoff)); alpha = 2^(m - mnew);
 *   off = (log2(448) - mnew) + xoff; p = 2^fmaf(x, sc, off);
 *   l = fmaf(l, alpha, sum p); P8 = e4m3(p); PV = sum P8*V8 per 64 keys (fp32,
 *   accumulated exactly here; under PvAccum::F16 the f16 accumulator of
 *   sage_attn.cu:328-333: PV = f16(f16(keys 0..31) + keys 32..63), each
 *   32-key chunk summed exactly -- the rounding inside NVIDIA's f16-accumulate
 *   mma is not documented, so that detail is unpinned); O = fmaf(O, alpha, PV);
 *   out = fmaf(O * (1/l), v_scale, v_mean).
 * Masked keys (padding, and j > i when causal) have p = 0.
 * Pinned: closed forms in tests (uniform Q gives the V-code mean; a block of
 * equal scores gives equal weights) and agreement with oracle_attention_f64
 * within the quantisation error; sequential sums replace the GPU's lane order.
 *
 * `nv` (NULL = the reference's numerics above) selects alternative softmax
 * numerics, for judging them against the reference's on the CPU:
 *   l_from_p8: l sums the E4M3-rounded P, so the weights of the output and of
 *     its normaliser round together;
 *   pow2_max:  the running max m moves to ceil(block max) (log2 units), so
 *     alpha = 2^(m_old - m_new) is a power of two and the row's largest P
 *     lies in (224, 448];
 *   tau:       m moves only when a block's max exceeds it, to that max plus
 *     tau (pow2_max: ceil of the max, plus tau); P = 448 * 2^(x - m) keeps
 *     every P at or below 448; tau = 0 with pow2_max = 0 is the reference;
 *   exp_f16:   every p (and alpha) is rounded to the nearest f16 value.
 * `rows_stride` > 0 gives every (b, h) its own rows: rows + bh * rows_stride.
 * Pinned (tests/test_oracle_numerics.py): per-(b, h) rows select what shared
 * rows select; default numerics equal the reference's bit for bit; a query
 * seeing one key returns that value when l sums the E4M3 P; a query seeing two
 * keys matches the float64 closed form of every mode. */
void oracle_sage_emulate_numerics(const oracle_problem* p, int causal, const int8_t* q8, const float* q_scale,
                                  const int8_t* k8, const float* k_scale, const uint8_t* v8, const float* stats,
                                  const float* kbias, const int* rows, int nrows, int rows_stride, float* out,
                                  uint16_t* out16, int out_dtype, int fast_exp, const oracle_numerics* nv,
                                  int threads) {
    const int B = p->batch, H = p->heads, HK = p->kv_heads, N = p->tokens, D = p->head_dim, G = H / HK;
    const float kMagic = 12582912.0f; /* 1.5 * 2^23 */
    const int TK = oracle_merged_keys(p), merged = merging(p);
    const size_t tq_pad = round_up((size_t)N, ORACLE_QTILE), tk_pad = round_up((size_t)TK, ORACLE_KBLOCK);
    const int nblk = (int)(tk_pad / ORACLE_KBLOCK);
    const int R = rows ? nrows : N;
    const float kLog448 = 8.807354922057604f;
    const oracle_numerics ref_nv = {0, 0, 0.f, 0};
    const oracle_numerics nm = nv ? *nv : ref_nv;
    float v8f[256];
    for (int c = 0; c < 256; c++) v8f[c] = oracle_e4m3_to_f32((uint8_t)c);
    set_threads(threads);
#pragma omp parallel
    {
        float* O = (float*)malloc(sizeof(float) * D);
        double* pv = (double*)malloc(sizeof(double) * D);
        int32_t S[ORACLE_KBLOCK];
        float P[ORACLE_KBLOCK];
#pragma omp for schedule(dynamic) collapse(2)
        for (int bh = 0; bh < B * H; bh++)
            for (int ri = 0; ri < R; ri++) {
                const int b = bh / H, h = bh % H, hk = h / G, bhk = b * HK + hk;
                const int i = rows ? rows[(size_t)bh * rows_stride + ri] : ri;
                const int8_t* qi = q8 + ((size_t)bh * tq_pad + i) * D;
                const float qs = q_scale[(size_t)bh * (tq_pad / ORACLE_QGROUP) + i / ORACLE_QGROUP];
                const int8_t* kb = k8 + (size_t)bhk * tk_pad * D;
                const uint8_t* vb = v8 + (size_t)bhk * tk_pad * D;
                float m = -1.0e30f, l = 0.f;
                for (int d = 0; d < D; d++) O[d] = 0.f;
                for (int blk = 0; blk < nblk; blk++) {
                    if (causal && blk * ORACLE_KBLOCK > i) break;
                    const float sc = qs * k_scale[(size_t)bhk * nblk + blk];
                    int have = 0;
                    int32_t smax = 0;
                    for (int r = 0; r < ORACLE_KBLOCK; r++) {
                        int j = blk * ORACLE_KBLOCK + r;
                        int ok = j < TK && (!causal || j <= i);
                        int32_t s = 0;
                        if (ok) {
                            const int8_t* kj = kb + (size_t)j * D;
                            for (int d = 0; d < D; d++) s += (int32_t)qi[d] * (int32_t)kj[d];
                            if (!have || s > smax) smax = s;
                            have = 1;
                        }
                        S[r] = ok ? s : INT32_MIN;
                    }
                    /* x as the reference holds it: exact, or biased by kMagic (both exact floats) */
                    const float bias = fast_exp ? kMagic : 0.f;
                    const float xoff = fast_exp ? -kMagic * sc : 0.f;
                    float mnew = m, off, bmax = -INFINITY;
                    float X[ORACLE_KBLOCK];
                    if (merged) {
                        /* the log2 logit with the log-count bias; padding keys carry -inf */
                        for (int r = 0; r < ORACLE_KBLOCK; r++) {
                            const int j = blk * ORACLE_KBLOCK + r;
                            const float kb = kbias[j];
                            const float bo = fast_exp ? fmaf(-kMagic, sc, kb) : kb;
                            X[r] = S[r] == INT32_MIN ? -INFINITY : fmaf(bias + (float)S[r], sc, bo);
                            bmax = fmaxf(bmax, X[r]);
                        }
                    } else if (have) {
                        bmax = fmaf(bias + (float)smax, sc, xoff);
                    }
                    if (nm.pow2_max || nm.tau != 0.f) {
                        if (bmax > m) mnew = (nm.pow2_max ? ceilf(bmax) : bmax) + nm.tau;
                    } else {
                        mnew = fmaxf(m, bmax);
                    }
                    off = merged ? kLog448 - mnew : (kLog448 - mnew) + xoff;
                    float alpha = ex2f_cr(m - mnew);
                    if (nm.exp_f16) alpha = (float)oracle_round_f16(alpha);
                    m = mnew;
                    float sum = 0.f;
                    for (int r = 0; r < ORACLE_KBLOCK; r++) {
                        float pr;
                        if (S[r] == INT32_MIN) pr = 0.f;
                        else if (merged) pr = ex2f_cr(X[r] + off);
                        else pr = ex2f_cr(fmaf(bias + (float)S[r], sc, off));
                        if (nm.exp_f16) pr = (float)oracle_round_f16(pr);
                        P[r] = pr;
                        sum += nm.l_from_p8 ? v8f[oracle_f32_to_e4m3(pr)] : pr;
                    }
                    l = fmaf(l, alpha, sum);
                    for (int d = 0; d < D; d++) pv[d] = 0;
                    for (int r = 0; r < ORACLE_KBLOCK; r++) {
                        if (P[r] != 0.f) {
                            const double p8 = v8f[oracle_f32_to_e4m3(P[r])];
                            const uint8_t* vr = vb + (size_t)(blk * ORACLE_KBLOCK + r) * D;
                            for (int d = 0; d < D; d++) pv[d] += p8 * v8f[vr[d]];
                        }
                        if (p->pv16 && (r == 31 || r == 63))
                            for (int d = 0; d < D; d++) pv[d] = oracle_round_f16(pv[d]);
                    }
                    for (int d = 0; d < D; d++) O[d] = fmaf(O[d], alpha, (float)pv[d]);
                }
                const float inv = 1.0f / l;
                const float* vmean = stats + (size_t)bhk * 4 * D + D;
                const float* vscale = vmean + D;
                float* o = out + ((size_t)bh * R + ri) * D;
                for (int d = 0; d < D; d++) o[d] = fmaf(O[d] * inv, vscale[d], vmean[d]);
                if (out16)
                    for (int d = 0; d < D; d++)
                        out16[((size_t)bh * R + ri) * D + d] =
                            out_dtype == ORACLE_F16 ? oracle_f32_to_f16(o[d]) : oracle_f32_to_bf16(o[d]);
            }
        free(O);
        free(pv);
    }
}

void oracle_sage_emulate(const oracle_problem* p, int causal, const int8_t* q8, const float* q_scale,
                         const int8_t* k8, const float* k_scale, const uint8_t* v8, const float* stats,
                         const float* kbias, const int* rows, int nrows, float* out, uint16_t* out16, int out_dtype,
                         int fast_exp, int threads) {
    oracle_sage_emulate_numerics(p, causal, q8, q_scale, k8, k_scale, v8, stats, kbias, rows, nrows, 0, out, out16,
                                 out_dtype, fast_exp, NULL, threads);
}

/* reference.rs:202-225 */
void oracle_errors(const float* ours, const float* ref, size_t n, double* out) {
    double dot = 0, na = 0, nr = 0, l1 = 0, l1r = 0, l2 = 0, mx = 0, rmax = 0;
    for (size_t i = 0; i < n; i++) {
        double a = ours[i], r = ref[i];
        dot += a * r;
        na += a * a;
        nr += r * r;
        l1 += fabs(a - r);
        l1r += fabs(r);
        l2 += (a - r) * (a - r);
        if (fabs(a - r) > mx) mx = fabs(a - r);
        if (fabs(r) > rmax) rmax = fabs(r);
    }
    double den = sqrt(na) * sqrt(nr);
    out[0] = dot / (den > 1e-300 ? den : 1e-300);
    out[1] = l1 / (l1r > 1e-300 ? l1r : 1e-300);
    out[2] = sqrt(l2 / (nr > 1e-300 ? nr : 1e-300));
    out[3] = mx;
    out[4] = rmax;
}
