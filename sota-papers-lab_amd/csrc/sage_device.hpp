// Device-side definitions shared by the SageAttention2 kernels for gfx950:
// the parameter block, the bit-exact codecs of the prologue and MFMA vector
// types. Reference semantics: sezer-muhammed/sota-papers-lab,
// platform/spl-nn/cuda/sage_common.cu (codecs :66-99) and src/sage/reference.rs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sage {

constexpr int QGROUP = 16;  // query rows per INT8 Q scale
constexpr int QTILE = 128;  // queries per prologue tile (one K/V statistics partial)
constexpr int KBLOCK = 64;  // keys per K scale and per V block
constexpr int NUM_XCD = 8;  // MI355X's XCDs, each with its own L2; workgroups are dealt to them round-robin

enum : int {
    F_LN_Q = 1,      // flag values of the reference's SgGeom::flags (sage_common.cu:26-29)
    F_LN_K = 2,
    F_SMOOTH_K = 4,
    F_SMOOTH_V = 8,
    F_CAUSAL = 16,   // extensions
    F_IN_F16 = 32,
    F_OUT_F16 = 64,
    F_WAVES8 = 128,  // Tile { warps: 8 }: the eight-wave attention layout (dense and causal)
};

// Kernel parameter block, passed by value. Element strides of the 16-bit
// [batch][token][head][dim] inputs and output; channels contiguous.
struct Geom {
    long long q_sb, q_st, q_sh;
    long long k_sb, k_st, k_sh;
    long long v_sb, v_st, v_sh;
    long long o_sb, o_st, o_sh;
    int batch, heads, kv_heads, group;  // group = heads / kv_heads
    int tokens;                         // queries and keys per batch item
    int tq_pad, tk, tk_pad;             // tokens rounded to QTILE; keys; keys rounded to KBLOCK
    int q_tiles, kblocks;               // tq_pad / QTILE, tk_pad / KBLOCK
    int flags;
    float q_mul;    // softmax scale * log2(e), folded into the Q scales
    float v_range;  // max |V - mean| maps to this E4M3 value (448)
    // KV merging (the reference's SgGeom merge fields, sage_common.cu:39-64):
    // merge = 1 is dense; 2 or 4 pools each frame's grid_h x grid_w patch
    // grid in merge x merge cells (merged_w cells a row, merged_frame keys a
    // frame), keeping the `special` tokens and the first dense_frames frames.
    int merge, frame_tokens, special, grid_h, grid_w, merged_frame, merged_w, dense_frames;
    float ln_eps;  // QK LayerNorm epsilon (F_LN_Q / F_LN_K)
};

// Members of merged key j (sage_quant.cu:210-235): returns the count; member
// m (0 <= m < count) is token base + (m / nx) * grid_w + m % nx.
__device__ __forceinline__ int merged_members(const Geom& g, int j, int& base, int& nx) {
    nx = 1;
    base = j;
    if (g.merge == 1) return 1;
    const int dense = g.dense_frames * g.frame_tokens;
    if (j < dense) return 1;
    const int f = g.dense_frames + (j - dense) / g.merged_frame, loc = (j - dense) % g.merged_frame;
    if (loc < g.special) {
        base = f * g.frame_tokens + loc;
        return 1;
    }
    const int cell = loc - g.special;
    const int y0 = (cell / g.merged_w) * g.merge, x0 = (cell % g.merged_w) * g.merge;
    const int ny = min(g.merge, g.grid_h - y0);
    nx = min(g.merge, g.grid_w - x0);
    base = f * g.frame_tokens + g.special + y0 * g.grid_w + x0;
    return ny * nx;
}

// log2(n) for n = 1..16, each the f32 nearest the exact value: the KV-merge
// bias of a key that pools n tokens (n <= 16 for strides 2 and 4).
__device__ __forceinline__ float log2_count(int n) {
    constexpr uint32_t bits[17] = {0xff800000u, 0x00000000u, 0x3f800000u, 0x3fcae00du, 0x40000000u, 0x40149a78u,
                                   0x40257007u, 0x4033abb4u, 0x40400000u, 0x404ae00du, 0x40549a78u, 0x405d6754u,
                                   0x40657007u, 0x406cd401u, 0x4073abb4u, 0x407a0a7fu, 0x40800000u};
    return __uint_as_float(bits[n]);
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// Eight 16-bit values of one 16-byte vector -> floats.
__device__ __forceinline__ void unpack8(uint4 v, float* f, bool f16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (f16) {
            f[2 * i] = f16_to_f32(w[i] & 0xffffu);
            f[2 * i + 1] = f16_to_f32(w[i] >> 16);
        } else {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
}

// Round to nearest even, clamp to +-127 (sage_common.cu:95-99; NaN -> 0), in
// three instructions: v_rndne_f32; v_cvt_i32_f32, which saturates values
// beyond the i32 range and turns NaN into 0; an integer clamp (v_med3_i32).
// Equal to the oracle's code on all 2^32 f32 inputs (tests/cpp/
// codec_exhaustive.hip).
__device__ __forceinline__ uint32_t s8_code(float x) {
    int c;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(c) : "v"(__builtin_rintf(x)));
    c = max(-127, min(127, c));
    return (uint32_t)c & 0xffu;
}

__device__ __forceinline__ uint32_t s8x4(float a, float b, float c, float d) {
    return s8_code(a) | (s8_code(b) << 8) | (s8_code(c) << 16) | (s8_code(d) << 24);
}

// f32 -> E4M3 (OCP e4m3fn) codes of a (low byte) and b (high byte): round to
// nearest even, saturating at +-448, NaN -> 0x7f, the semantics of
// reference.rs:40-70 (cvt.rn.satfinite). v_cvt_pk_fp8_f32 rounds to nearest
// even, subnormals included, and agrees with those semantics bit for bit on
// every non-NaN input once it is clamped to +-448 (checked over all 2^32 f32
// inputs on gfx950); the clamp gives the saturation and NaN, which the
// converter encodes differently, is patched to 0x7f.
__device__ __forceinline__ uint32_t e4m3_pair(float a, float b) {
    const float ca = fminf(fmaxf(a, -448.0f), 448.0f), cb = fminf(fmaxf(b, -448.0f), 448.0f);
    uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xffffu;
    if (a != a) r = (r & 0xff00u) | 0x7fu;
    if (b != b) r = (r & 0x00ffu) | 0x7f00u;
    return r;
}

// 1 / sqrt(v) with the square root and the reciprocal each correctly rounded:
// 1.0f / sqrtf(v) bit for bit, the QK-norm's rstd. For v in [2^-100, FLT_MAX]
// it takes 12 instructions instead of about 30: v_sqrt_f32 with the +-1 ulp
// FMA correction of LLVM's correctly rounded square root (whose input scaling
// and special cases that range does not need), then v_rcp_f32 with one FMA
// Newton step. That short form equals 1.0f / sqrtf(v) on every float of the
// range (all mantissas of all exponents, checked on gfx950); other inputs
// (zero, subnormals, infinities, NaN, negatives) take the IEEE expressions.
// Equal to the oracle's 1.0f / sqrtf(v) on all 2^32 f32 inputs
// (tests/cpp/codec_exhaustive.hip).
__device__ __forceinline__ float rsqrt_rn2(float v) {
    if (v >= 0x1p-100f && v <= 3.40282347e38f) {
        float s = __builtin_amdgcn_sqrtf(v);
        const float dn = __uint_as_float(__float_as_uint(s) - 1u), up = __uint_as_float(__float_as_uint(s) + 1u);
        const float rdn = __builtin_fmaf(-dn, s, v), rup = __builtin_fmaf(-up, s, v);
        s = rdn <= 0.0f ? dn : s;
        s = rup > 0.0f ? up : s;
        const float y = __builtin_amdgcn_rcpf(s);
        return __builtin_fmaf(__builtin_fmaf(-s, y, 1.0f), y, y);
    }
    return 1.0f / sqrtf(v);
}

// Two f32 -> one register of two bf16 / fp16 (low half first), rounded to
// nearest even like the reference's f32 -> bf16 conversion
// (reference.rs:13-20); a NaN stays a NaN.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2_t));
}

// The QKV prologue's options (the reference's QkvArgs, qkv.cu:9-31): the
// fused projection y holds, per token, q | k | v of heads * D, kv_heads * D
// and kv_heads * D channels; null pointers switch an option off.
struct QkvDev {
    const float* tok;      // [batch * tokens] per-token scales
    const float* chan;     // [(heads + 2 kv_heads) * D] per-channel scales
    const uint16_t* bias;  // bf16 [(heads + 2 kv_heads) * D]
    const float* nw[4];    // [D] each: q weight, q bias, k weight, k bias (biases: LayerNorm)
    const float* rope;     // [frame_len][D / 2][2]: cos, sin of each rotation pair
    int norm;              // 0 none, 1 LayerNorm, 2 RMSNorm
    int rope_half;         // channels between the two of a rotation pair (a power of two)
    int rope_shift;        // log2(rope_half)
    int frame_len;         // rope row of token t: t % frame_len
    // t / frame_len for 0 <= t < 2^31 as (umulhi(fl_magic, t) + t) >> fl_shift
    // (Granlund and Montgomery, "Division by Invariant Integers using
    // Multiplication", 1994, fig. 4.1: l = ceil(log2 frame_len), magic =
    // floor(2^32 (2^l - frame_len) / frame_len) + 1; the sum stays below 2^32).
    uint32_t fl_magic;
    int fl_shift;
    float eps;
};

// The RoPE table row of token t (t % frame_len) without a runtime divide.
__device__ __forceinline__ int rope_row(const QkvDev& a, int t) {
    const uint32_t n = (uint32_t)t;
    const uint32_t q = (__umulhi(a.fl_magic, n) + n) >> a.fl_shift;
    return (int)(n - q * (uint32_t)a.frame_len);
}

// The QKV prologue (qkv.cu:50-120) on one (token, part, head) row whose D
// channels lie on D/8 consecutive lanes, 8 a lane (ch = the lane's chunk;
// every lane of the wave takes part, rows past the sequence on zeros). part
// is 0 (q), 1 (k) or 2 (v). The arithmetic, in fp32:
//   x *= tok[b, t]; x *= chan[c]; x += bias[c] (each rounded);
//   QK-norm (q, k): lane sums meet in an xor butterfly over 1 .. D/16,
//   mean = s * (1/D) (0 for RMSNorm), fused square deviations, r = 1 / sqrt(
//   fmaf(ss, 1/D, eps)) with the square root and the divide correctly
//   rounded (the reference's rsqrtf does not state its rounding), x =
//   fmaf((x - mean) * r, w, LayerNorm ? b : 0);
//   RoPE (q, k): the partner channel d ^ half sits on lane ^ (half / 8);
//   x = fmaf(x, cos, +-(partner * sin)), minus when d & half == 0.
// Loads are split from the arithmetic: QkvLane holds what depends on the
// lane's channels only (loaded once per part and head), QkvTok what depends
// on the token (its scale and the lane's 8 rotation pairs, 64 contiguous
// bytes of the table row since a lane's 8 channels rotate 8 consecutive
// pairs).
// Sum over the CH lanes of a row group (CH = 2, 4, 8 or 16 consecutive lanes,
// aligned), equal to the xor butterfly v += shfl_xor(v, 1), (v, 2), (v, 4),
// (v, 8) bit for bit, on DPP instead of the LDS crossbar: after each step all
// lanes of the quad (then of the half row) hold the same value, so pairing
// the quads by row_half_mirror and the half rows by row_mirror adds the same
// two values that xor 4 and xor 8 would.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CH>
__device__ __forceinline__ float row_sum(float v) {
    v += dpp<0xB1>(v);                    // quad_perm [1, 0, 3, 2]: lane ^ 1
    if (CH > 2) v += dpp<0x4E>(v);        // quad_perm [2, 3, 0, 1]: lane ^ 2
    if (CH > 4) v += dpp<0x141>(v);       // row_half_mirror: the other quad of the 8
    if (CH > 8) v += dpp<0x140>(v);       // row_mirror: the other 8 of the 16
    return v;
}

struct QkvLane {
    float chan[8], bias[8], w[8], nb[8];
};
struct QkvTok {
    float t;
    float4 cs[4];  // (cos, sin) of the lane's pairs 2i (x, y) and 2i + 1 (z, w)
};

__device__ __forceinline__ int qkv_slot(const Geom& g, int part, int h) {
    return part == 0 ? h : (part == 1 ? g.heads + h : g.heads + g.kv_heads + h);
}

template <int D>
__device__ __forceinline__ void qkv_lane(QkvLane& L, const QkvDev& a, const Geom& g, int part, int h, int ch) {
    const int c0 = qkv_slot(g, part, h) * D + ch * 8;
    // f32 arrays need only 4-byte alignment (the reference checks none for
    // the norm weights, qkv.rs:279): 16-byte loads through memcpy assume no
    // more, and gfx950 serves them as one global_load_dwordx4 either way.
    auto load8 = [](const float* p, float* o) {
        float4 u, v;
        __builtin_memcpy(&u, p, 16);
        __builtin_memcpy(&v, p + 4, 16);
        o[0] = u.x, o[1] = u.y, o[2] = u.z, o[3] = u.w, o[4] = v.x, o[5] = v.y, o[6] = v.z, o[7] = v.w;
    };
    if (a.chan) load8(a.chan + c0, L.chan);
    if (a.bias) unpack8(*reinterpret_cast<const uint4*>(a.bias + c0), L.bias, false);
    if (a.norm && part < 2) {
        load8(a.nw[2 * part] + ch * 8, L.w);
        // The bias pointer is valid either way (the weight's under RMSNorm,
        // where the value is selected away).
        load8((a.norm == 1 ? a.nw[2 * part + 1] : a.nw[2 * part]) + ch * 8, L.nb);
    }
}

template <int D>
__device__ __forceinline__ void qkv_tok(QkvTok& T, const QkvDev& a, const Geom& g, int part, int b, int tok, int ch) {
    if (a.tok) T.t = a.tok[(long long)b * g.tokens + min(tok, g.tokens - 1)];
    if (a.rope && part < 2) {
        // Pair of the lane's first channel: (d0 / (2 half)) half + d0 % half.
        const int d0 = ch * 8, sh = a.rope_shift;
        const int pair0 = ((d0 >> (sh + 1)) << sh) + (d0 & (a.rope_half - 1));
        // 4-byte alignment suffices, as for the norm weights (qkv_lane).
        const float* row = a.rope + (long long)rope_row(a, tok) * D + 2 * pair0;
#pragma unroll
        for (int i = 0; i < 4; i++) __builtin_memcpy(&T.cs[i], row + 4 * i, 16);
    }
}

template <int D>
__device__ __forceinline__ void qkv_apply(float* x, const QkvDev& a, const QkvLane& L, const QkvTok& T, int part,
                                          int ch) {
    constexpr int CH = D / 8;
    if (a.tok) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = x[e] * T.t;
    }
    if (a.chan) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = x[e] * L.chan[e];
    }
    if (a.bias) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = x[e] + L.bias[e];
    }
    // The norm's and the rotation's shuffles run on every lane (part need not
    // be uniform across a wave); only the updates depend on the part.
    if (a.norm) {
        // LayerNorm and RMSNorm differ by selects only, with no branch between
        // them: the row sum is formed either way. (A version with the
        // LayerNorm mean behind its own branch was compiled by ROCm 7.2's
        // hipcc into code that left one channel of each K row undefined under
        // RMSNorm.)
        const bool layer = a.norm == 1;
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) sum += x[e];
        sum = row_sum<CH>(sum);
        const float mean = layer ? sum * (1.0f / D) : 0.0f;
        float s2 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float d = x[e] - mean;
            s2 = __builtin_fmaf(d, d, s2);
        }
        s2 = row_sum<CH>(s2);
        if (part < 2) {
            const float r = rsqrt_rn2(__builtin_fmaf(s2, 1.0f / D, a.eps));
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = __builtin_fmaf((x[e] - mean) * r, L.w[e], layer ? L.nb[e] : 0.0f);
        }
    }
    if (a.rope) {
        const int half = a.rope_half, xo = half >> 3;
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; e++) p[e] = __shfl_xor(x[e], xo, 64);
        if (part < 2) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float4 q = T.cs[e >> 1];
                const float c = (e & 1) ? q.z : q.x, sn = (e & 1) ? q.w : q.y;
                const float ps = p[e] * sn;
                x[e] = __builtin_fmaf(x[e], c, ((ch * 8 + e) & half) ? ps : -ps);
            }
        }
    }
}

// Destinations of the standalone QKV prologue: 16-bit [batch][token][head][D]
// views of Q, K and V (p[0..2], element strides sb, st, sh), V in fp16 when
// v_f16 (the reference's VFormat::F16), else bf16 like Q and K.
struct QkvOutDev {
    uint16_t* p[3];
    long long sb[3], st[3], sh[3];
    int v_f16;
};


// Byte position of key k (0..63) of a 64-key block inside each channel row of
// the V tile. The 32x32 INT8 MFMA leaves key 32t + 8j + 4g + r of a column
// in lane-half g, accumulator 4j + r of sub-tile t; packed four to a register
// that is byte 16t + 4j + r of lane-half g's 32-byte FP8 operand, so V's
// channel rows store that key at byte 32g + 16t + 4j + r.
__host__ __device__ __forceinline__ int v8_position(int k) {
    return 32 * ((k >> 2) & 1) + 16 * (k >> 5) + 4 * ((k >> 3) & 3) + (k & 3);
}

// XOR swizzle of 16-byte chunk u of an LDS tile whose rows are CPR chunks
// long (CPR = 4 or 8). gfx950's LDS serves a ds_read_b128 sixteen lanes at a
// time from 64 four-byte banks, i.e. one 256-byte line of sixteen chunks per
// cycle. Sixteen lanes that read the same chunk column of sixteen consecutive
// rows span 16 / CPR rows per line, so the chunk-in-row bits are XORed with
// the line index: the sixteen reads then land in sixteen different chunk slots
// of the line. The XOR touches only bits below the line index, so swz is an
// involution and keeps every chunk inside its row (cpr = 4 or 8).
__device__ __forceinline__ int swz(int u, int cpr) { return u ^ ((u >> 4) & (cpr - 1)); }

}  // namespace sage
