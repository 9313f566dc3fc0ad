// SageAttention2 attention kernel for gfx950 (CDNA4 MFMA, wave64).
//
// Semantics follow sezer-muhammed/sota-papers-lab,
// platform/spl-nn/cuda/sage_attn.cu:135-424 (sg_attn<false>): INT8 Q K^T with
// int32 accumulation and the dequant scale q_scale * k_scale folded into the
// exp2 argument, an online softmax in log2 units, P = 448 * 2^(x - m) rounded
// to E4M3, an FP8 P.V with fp32 accumulation, out = O / l * v_scale + v_mean.
// The layout is this build's own, designed for CDNA4:
//
// - One workgroup = 4 wave64s = 128 queries of one (batch, head); each wave
//   owns 32 queries and walks the keys in 64-key blocks.
// - The wave computes S^T = K Q^T with v_mfma_i32_32x32x32_i8: Q^T is the B
//   operand and stays in registers for the whole sweep; K is the A operand,
//   read from LDS. In the 32x32 accumulator a lane holds ONE query (its
//   column) and 16 keys, so every softmax statistic of a query lives in one
//   lane and its partner lane (lane ^ 32): the row max and row sum need a
//   single cross-half exchange.
// - O^T = V^T P^T with v_mfma_scale_f32_32x32x64_f8f6f4 (E4M3, unit scales):
//   P^T is the B operand, built in registers straight from the S^T
//   accumulators (4 keys per register, v_cvt_pk_fp8_f32); V^T is the A
//   operand, stored by the prologue with its keys in that register order
//   (v8_position). P never goes through LDS, and the O^T accumulator again
//   holds one query per lane, so rescaling by alpha is lane-local.
// - The INT8 accumulators start from the bits of 1.5 * 2^23, so each holds the
//   float 1.5 * 2^23 + S exactly (|S| < 2^22 for D <= 128): the row max runs on
//   the integer bits and the exp2 argument is one FMA, with the offset folded
//   into the per-block constant (the reference's SG_FAST_EXP).
// - O accumulates on the MFMA in fp32 across blocks (O = alpha * O + P.V):
//   the MFMA adds its product to C exactly in fp32, so the reference's
//   separate per-block fp32 partial is not needed.
// - K and V tiles are double-buffered in LDS with an XOR swizzle, filled by
//   direct global -> LDS loads (no staging registers); the next block's copy
//   is issued before the current block's MFMAs.
#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace sage {

constexpr int ATTN_BN = 64;  // keys per iteration (one K scale, one V block)
constexpr unsigned NEG_INF_BITS = 0xff800000u;
// Largest q_scale * k_scale for which the biased-accumulator shortcut is used:
// the offset -1.5 * 2^23 * sc folded into the exp2 argument rounds by up to
// about 0.75 * sc in log2 units, so above this the wave converts S exactly.
constexpr float FAST_SC_MAX = 2.0e-4f;

// Two K/V stages as separate LDS objects: the compiler then knows that the
// direct-to-LDS prefetch into one never aliases the MFMA operand reads of the
// other, and lets them overlap.
template <int D>
struct Stages {
    static constexpr int TILE = ATTN_BN * D;  // bytes of one K tile and of one V tile
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void sage_attn(const int8_t* __restrict__ q8, const float* __restrict__ q_scale,
                                                    const int8_t* __restrict__ k8,
                                                    const float* __restrict__ k_scale,
                                                    const uint8_t* __restrict__ v8, const float* __restrict__ stats,
                                                    uint16_t* __restrict__ out, Geom g) {
    constexpr int BN = ATTN_BN;
    constexpr int KS = D / 32;            // INT8 k-steps of 32 channels
    constexpr int DT = D / 32;            // 32-channel tiles of O^T
    constexpr int TILE = Stages<D>::TILE; // bytes of one K tile and of one V tile
    constexpr int CPT = TILE / 16 / 256;  // 16-byte chunks per thread per tile
    constexpr int KCPR = D / 16;          // chunks per K row
    static_assert(CPT >= 1, "tile too small for 256 threads");

    __shared__ __attribute__((aligned(16))) uint8_t lds0[2 * TILE];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[2 * TILE];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, half = lane >> 5;
    const int qt = CAUSAL ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;  // heavy tiles first
    const int h = blockIdx.y, b = blockIdx.z, hk = h / g.group;
    const long long bh = (long long)b * g.heads + h, bhk = (long long)b * g.kv_heads + hk;
    const int q0 = qt * ATTN_ROWS + wave * 32;  // first query of this wave
    const int qi = q0 + col;                    // this lane's query

    // Q^T operand: lane holds channels 32s + 16*half .. +15 of its query.
    v4i qa[KS];
    {
        const int8_t* qrow = q8 + (bh * g.tq_pad + qi) * D + 16 * half;
#pragma unroll
        for (int s = 0; s < KS; s++) qa[s] = *reinterpret_cast<const v4i*>(qrow + 32 * s);
    }
    const float qs = q_scale[bh * (g.tq_pad / QGROUP) + (qi >> 4)];
    // Consume the Q loads here, before the first barrier: otherwise the
    // compiler sinks them into the key loop and waits for every outstanding
    // load there, prefetches included.
#pragma unroll
    for (int s = 0; s < KS; s++) asm volatile("" ::"v"(qa[s]));
    asm volatile("" ::"v"(qs));

    int nblk = g.kblocks;
    if (CAUSAL) nblk = min(nblk, (qt * ATTN_ROWS + ATTN_ROWS - 1) / BN + 1);

    const uint8_t* kg = reinterpret_cast<const uint8_t*>(k8) + bhk * (long long)g.tk_pad * D;
    const uint8_t* vg = v8 + bhk * (long long)g.tk_pad * D;
    const float* ksc = k_scale + bhk * g.kblocks;

    // Direct global -> LDS copy of one block's K and V tiles into `dst`. Lane
    // `lane` of wave `wave` fills physical chunk c of the tile, so it fetches
    // the logical chunk that the swizzle puts there (swz is an involution).
    auto fetch = [&](int blk, uint8_t* dst) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c0 = i * 256 + wave * 64;
            const long long src = (long long)blk * TILE + 16 * swz(c0 + lane);
            __builtin_amdgcn_global_load_lds(kg + src, (__attribute__((address_space(3))) void*)(dst + 16 * c0), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vg + src, (__attribute__((address_space(3))) void*)(dst + TILE + 16 * c0), 16, 0, 0);
        }
    };

    v16f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
    float m = -1.0e30f, l = 0.f;
    const float kMagic = 12582912.0f;          // 1.5 * 2^23
    const float kLog448 = 8.807354922057604f;  // log2(448): P fills the E4M3 range

    // One 64-key block whose K and V tiles are in `cur`; prefetches block
    // blk + 1 into `nxt` first.
    auto step = [&](int blk, const uint8_t* cur, uint8_t* nxt) {
        if (blk + 1 < nblk) fetch(blk + 1, nxt);
        const uint4* lk = reinterpret_cast<const uint4*>(cur);
        const uint4* lv = reinterpret_cast<const uint4*>(cur + TILE);
        const float sc = qs * ksc[blk];
        const bool fast = __all(sc < FAST_SC_MAX);

        // S^T for keys 32t .. 32t + 31 of the block; with `fast` the
        // accumulators start at the bits of 1.5 * 2^23 and then hold the
        // float 1.5 * 2^23 + S exactly.
        v16i s[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int r = 0; r < 16; r++) s[t][r] = fast ? 0x4b400000 : 0;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const uint4 a = lk[swz((32 * t + col) * KCPR + 2 * ks + half)];
                const v4i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w};
                s[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qa[ks], s[t], 0, 0, 0);
            }
        }

        // Keys past the sequence, and keys after the query when causal.
        const bool mask = (blk + 1) * BN > g.tk || (CAUSAL && blk * BN + BN - 1 > q0);
        const int masked = fast ? (int)NEG_INF_BITS : INT_MIN;
        if (mask) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = blk * BN + 32 * t + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (key >= g.tk || (CAUSAL && key > qi)) s[t][r] = masked;
                }
        }
        int mx = s[0][0];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = max(mx, s[t][r]);
        mx = max(mx, __shfl_xor(mx, 32, 64));

        float p[2][16];
        float sum = 0.f, alpha;
        if (fast) {
            const float negms = -kMagic * sc;
            const float mnew = fmaxf(m, fmaf(__int_as_float(mx), sc, negms));
            alpha = __builtin_amdgcn_exp2f(m - mnew);
            m = mnew;
            const float off = (kLog448 - mnew) + negms;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float e = __builtin_amdgcn_exp2f(fmaf(__int_as_float(s[t][r]), sc, off));
                    if (mask && s[t][r] == masked) e = 0.f;
                    p[t][r] = e;
                    sum += e;
                }
        } else {
            const float mblk = mx == INT_MIN ? -INFINITY : (float)mx * sc;
            const float mnew = fmaxf(m, mblk);
            alpha = __builtin_amdgcn_exp2f(m - mnew);
            m = mnew;
            const float off = kLog448 - mnew;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    float e = __builtin_amdgcn_exp2f(fmaf((float)s[t][r], sc, off));
                    if (mask && s[t][r] == masked) e = 0.f;
                    p[t][r] = e;
                    sum += e;
                }
        }
        l = fmaf(l, alpha, sum);

        // P^T operand: register j holds keys of accumulators 4(j%4)..+3 of sub-tile j/4.
        v8i pb;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = j >> 2, r0 = 4 * (j & 3);
            const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0], p[t][r0 + 1], 0, false);
            pb[j] = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0 + 2], p[t][r0 + 3], lo, true);
        }

        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
        }
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const int u = (32 * dt + col) * 4 + 2 * half;  // V^T row = channel, 4 chunks per row
            const uint4 a0 = lv[swz(u)], a1 = lv[swz(u + 1)];
            const v8i av = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            o[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, pb, o[dt], 0, 0, 0, 127, 0, 127);
        }
        // Drains this wave's prefetch and publishes it; nobody reads `cur` after.
        __syncthreads();
    };

    fetch(0, lds0);
    __syncthreads();
    for (int blk = 0; blk < nblk; blk += 2) {
        step(blk, lds0, lds1);
        if (blk + 1 < nblk) step(blk + 1, lds1, lds0);
    }

    // out = O / l * v_scale + v_mean; lane holds channels 32dt + 8j + 4*half + 0..3.
    const float lt = l + __shfl_xor(l, 32, 64);
    const float inv = 1.0f / lt;
    if (qi < g.tokens) {
        const float* vmean = stats + bhk * 4 * D + D;
        const float* vscale = vmean + D;
        uint16_t* orow = out + b * g.o_sb + (long long)qi * g.o_st + h * g.o_sh;
        const bool f16 = g.flags & F_OUT_F16;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d0 = 32 * dt + 8 * j + 4 * half;
                uint32_t bits[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float y = fmaf(o[dt][4 * j + r] * inv, vscale[d0 + r], vmean[d0 + r]);
                    bits[r] = f16 ? f16_bits(y) : bf16_bits(y);
                }
                uint2 w;
                w.x = bits[0] | (bits[1] << 16);
                w.y = bits[2] | (bits[3] << 16);
                *reinterpret_cast<uint2*>(orow + d0) = w;
            }
    }
}

template <int D, bool CAUSAL>
static hipError_t launch_d(const AttendBufs& w, const Geom& g, hipStream_t s) {
    hipLaunchKernelGGL((sage_attn<D, CAUSAL>), dim3(g.tq_pad / ATTN_ROWS, g.heads, g.batch), dim3(256), 0, s, w.q8,
                       w.q_scale, w.k8, w.k_scale, w.v8, w.stats, static_cast<uint16_t*>(w.out), g);
    return hipGetLastError();
}

hipError_t launch_attention(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s) {
    const bool causal = g.flags & F_CAUSAL;
    if (head_dim == 64) return causal ? launch_d<64, true>(w, g, s) : launch_d<64, false>(w, g, s);
    return causal ? launch_d<128, true>(w, g, s) : launch_d<128, false>(w, g, s);
}

hipError_t attention_resources(int head_dim, bool causal, int* regs, int* spill, int* lds) {
    hipFuncAttributes a;
    const void* f;
    if (head_dim == 64)
        f = causal ? reinterpret_cast<const void*>(&sage_attn<64, true>) : reinterpret_cast<const void*>(&sage_attn<64, false>);
    else
        f = causal ? reinterpret_cast<const void*>(&sage_attn<128, true>)
                   : reinterpret_cast<const void*>(&sage_attn<128, false>);
    hipError_t e = hipFuncGetAttributes(&a, f);
    if (e != hipSuccess) return e;
    *regs = a.numRegs;
    *spill = (int)a.localSizeBytes;
    *lds = (int)a.sharedSizeBytes;
    return hipSuccess;
}

}  // namespace sage
