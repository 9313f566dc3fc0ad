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

enum : int {
    F_LN_Q = 1,      // flag values of the reference's SgGeom::flags (sage_common.cu:26-29)
    F_LN_K = 2,
    F_SMOOTH_K = 4,
    F_SMOOTH_V = 8,
    F_CAUSAL = 16,   // extensions
    F_IN_F16 = 32,
    F_OUT_F16 = 64,
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

// Round to nearest even, clamp to +-127 (sage_common.cu:95-99; NaN -> 0).
__device__ __forceinline__ uint32_t s8_code(float x) {
    float r = __builtin_rintf(x);
    r = r != r ? 0.f : fminf(fmaxf(r, -127.f), 127.f);
    return (uint32_t)((int)r) & 0xffu;
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
