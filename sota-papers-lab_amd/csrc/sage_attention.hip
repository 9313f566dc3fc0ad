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
// - The INT8 accumulators start from the bits of 1.5 * 2^23, so each score
//   register already holds the float 1.5 * 2^23 + S (exact for |S| < 2^22):
//   no int -> float conversions. The row max runs on those bits (positive
//   floats order like their bit patterns, v_max3_i32), and the bias comes
//   off inside the exp2 FMA through xoff = -(1.5 * 2^23) * sc, the
//   reference's default logit arithmetic (SG_FAST_EXP=1, sage_attn.cu:23-31,
//   262-300), in the same fp32 operation order.
// - O is rescaled only in blocks where some row's running max moved.
// - O accumulates on the MFMA in fp32 across blocks (O = alpha * O + P.V):
//   the MFMA adds its product to C exactly in fp32, so the reference's
//   separate per-block fp32 partial is not needed.
// - K and V tiles are double-buffered in LDS with an XOR swizzle over
//   256-byte lines (conflict-free b128 operand reads), filled by direct
//   global -> LDS loads from a uniform SGPR base (no staging registers).
// - A wave runs one block at a time (QK^T, softmax, P.V); the other waves on
//   its SIMD fill the MFMA and VALU gaps: three a SIMD at head dim 128, four
//   at head dim 64. Q^T stays in registers; at head dim 128 the K operands
//   of one 32-key sub-tile at a time make room for it.
// - Workgroups are dealt to XCDs so that the ones sharing a head's K and V
//   share an L2; causal tiles are dealt longest first across each XCD's
//   heads.
// - KV merging (MERGE, the reference's sg_attn_merge, sage_attn.cu:238-246,
//   264-305): every key carries a log2(member count) bias, staged per block
//   in LDS beside K and V. The log2 logit x = S * sc + bias is formed before
//   the row max (fmaf(1.5 * 2^23 + S, sc, fmaf(-1.5 * 2^23, sc, bias))), and
//   P = 2^(x + log2(448) - m); padding keys carry -inf and need no mask.
#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace sage {

constexpr int ATTN_BN = 64;  // keys per iteration (one K scale, one V block)
constexpr int MAGIC_BITS = 0x4B400000;      // bits of 1.5 * 2^23
constexpr float MAGIC = 12582912.0f;        // 1.5 * 2^23
constexpr int NEG_INF_BITS = (int)0xFF800000;  // -inf: below every biased score as an int
constexpr float LOG2_448 = 8.807354922057604f;  // P = 448 for the row max: E4M3's largest finite

// A row statistic held in lane l and its partner lane l ^ 32 (the other half
// of the wave), combined in every lane with one v_permlane32_swap of two copies
// of x: the swap's first result holds the lower half's values in both halves,
// its second the upper half's, so every lane combines the same pair in the
// same order.
__device__ __forceinline__ int max_halves(int x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return max((int)r[0], (int)r[1]);
}
__device__ __forceinline__ float fmax_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    // v_med3_f32 with FLT_MAX: the maximum of two non-NaN values without the
    // canonicalising v_max_f32 that fmaxf puts on each swapped register.
    return __builtin_amdgcn_fmed3f(__int_as_float((int)r[0]), __int_as_float((int)r[1]), 3.4028234663852886e38f);
}
__device__ __forceinline__ float sum_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
    return __int_as_float((int)r[0]) + __int_as_float((int)r[1]);
}
// Floor of the logit scale q_scale * k_scale in masked blocks: a masked score
// is -inf and must stay -inf through the product (0 * -inf would be a NaN),
// so the product is floored where scores are masked. Below 1e-30
// the floor changes no result: every logit difference of the block is then
// under 2^22 * 1e-30 < 1e-23, far below half an ulp of the exp2 argument
// (about 8.8, ulp 2^-20), so every P and alpha come out bit-identical to the
// unfloored product's. Only an exact zero scale (an all-zero 16-row Q group,
// a K head constant over tokens) is changed: the row attends uniformly to its
// visible keys, where the reference's masked keys turn into NaNs.
constexpr float SCALE_FLOOR = 1.0e-30f;
// max(m, x) for the running max: v_med3_f32(m, x, FLT_MAX) in one instruction
// (fmaxf on the loop-carried m costs a canonicalising v_max_f32 m, m every
// block). Neither operand is a NaN: m starts at -1e30 and x is a finite logit
// or -inf.
__device__ __forceinline__ float running_max(float m, float x) {
    return __builtin_amdgcn_fmed3f(m, x, 3.4028234663852886e38f);
}
// Values the compiler may not re-derive or rematerialise: a uniform pointer
// stays in SGPRs and is not reassociated with per-lane offsets; a VGPR value
// stays where it is. (The constraints name AMDGPU register classes, so the
// statements exist only in the device pass.)
__device__ __forceinline__ const uint8_t* opaque_uniform(const uint8_t* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+s"(p));
#endif
    return p;
}
template <typename T>
__device__ __forceinline__ void opaque_vgpr(T& x) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(x));
#endif
}

// The dispatcher deals workgroups to the 8 XCDs round-robin by linear id,
// and each XCD has its own L2. Tile t (query tile fastest, then head, then
// batch) goes to the workgroup that gives XCD x the contiguous range of
// tiles [x * per, (x + 1) * per): the workgroups that share a head's K and V
// then read them through one L2 instead of eight. The last total % 8 tiles
// keep their place.
__device__ __forceinline__ int xcd_tile(int lin, int total) {
    const int per = total / NUM_XCD;
    if (lin >= per * NUM_XCD) return lin;
    return (lin % NUM_XCD) * per + lin / NUM_XCD;
}

// A causal query tile qt sweeps 2 qt + 2 key blocks. Dealt head by head,
// the heavy tiles of an XCD's last head start late and finish alone; dealt
// longest first across the XCD's heads, the short tiles fill the tail. That
// order needs every XCD to hold whole heads (the plain mapping above does
// then too, so the L2 sharing is unchanged).
__device__ __forceinline__ bool causal_longest_first(int total, int ntq) {
    return total % NUM_XCD == 0 && (total / NUM_XCD) % ntq == 0;
}

// This lane's index in the wave, rebuilt from v_mbcnt: values derived from the
// lane are recomputed where a rare path or the epilogue needs them instead of
// being kept live (or spilled) across the key loop.
__device__ __forceinline__ int lane_now() {
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// Workgroups a CU: four at head dim 64 (<= 128 VGPRs), three at head dim 128
// (<= 168); the merged head-dim-128 kernel needs the registers of two.
template <int D, bool CAUSAL, bool MERGE>
__global__ __launch_bounds__(256, D == 64 ? 4 : (MERGE ? 2 : 3)) void sage_attn(const int8_t* __restrict__ q8, const float* __restrict__ q_scale,
                                                    const int8_t* __restrict__ k8,
                                                    const float* __restrict__ k_scale,
                                                    const uint8_t* __restrict__ v8, const float* __restrict__ stats,
                                                    const float* __restrict__ kbias, uint16_t* __restrict__ out,
                                                    Geom g) {
    constexpr int BN = ATTN_BN;
    constexpr int KS = D / 32;            // INT8 k-steps of 32 channels
    constexpr int DT = D / 32;            // 32-channel tiles of O^T
    constexpr int TILE = BN * D;          // bytes of one K tile and of one V tile
    constexpr int CPT = TILE / 16 / 256;  // 16-byte chunks per thread per tile
    constexpr int KCPR = D / 16;          // chunks per K row
    static_assert(CPT >= 1, "tile too small for 256 threads");

    // K and V are double-buffered separately: step j reads K(j) and V(j)
    // while K(j+1) and V(j+1) arrive in the other buffers. Separate LDS
    // objects let the compiler see that the direct-to-LDS prefetch into one
    // buffer never aliases the MFMA operand reads of another.
    __shared__ __attribute__((aligned(16))) uint8_t ldsK0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsK1[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsV0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsV1[TILE];
    // Merge biases of the current and the next block.
    __shared__ __attribute__((aligned(16))) float ldsB0[MERGE ? BN : 4];
    __shared__ __attribute__((aligned(16))) float ldsB1[MERGE ? BN : 4];
    // Merged: each wave's per-key logit offsets bias - 1.5 * 2^23 * scl of the
    // current block, for each of the two Q-scale groups of its 32 queries.
    __shared__ __attribute__((aligned(16))) float ldsC[MERGE ? 4 * 2 * BN : 4];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, half = lane >> 5;
    const int ntq = gridDim.x;
    const int lin = blockIdx.x + ntq * (blockIdx.y + gridDim.y * blockIdx.z), total = ntq * gridDim.y * gridDim.z;
    int qt, hb;  // query tile; head slot b * heads + h
    if (CAUSAL && causal_longest_first(total, ntq)) {
        // XCD x holds head slots [x * hx, (x + 1) * hx); its i-th workgroup
        // takes query tile ntq - 1 - i / hx of head slot x * hx + i % hx, so
        // the XCD deals its tiles longest first across all of its heads.
        const int per = total / NUM_XCD, hx = per / ntq, x = lin % NUM_XCD, i = lin / NUM_XCD;
        qt = ntq - 1 - i / hx;
        hb = x * hx + i % hx;
    } else {
        const int tile = xcd_tile(lin, total);
        qt = CAUSAL ? ntq - 1 - tile % ntq : tile % ntq;  // causal: heavy tiles of a head first
        hb = tile / ntq;
    }
    const int h = hb % g.heads, b = hb / g.heads, hk = h / g.group;
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
    // The Q scale; the key loop floors its product with the K scale (SCALE_FLOOR).
    const float qs = q_scale[bh * (g.tq_pad / QGROUP) + (qi >> 4)];
    // The Q scales of the wave's two 16-query groups (wave-uniform).
    const float qsg0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qs), 0));
    const float qsg1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qs), QGROUP));
    // Consume the Q loads here, before the first barrier: otherwise the
    // compiler sinks them into the key loop and waits for every outstanding
    // load there, prefetches included.
#pragma unroll
    for (int s = 0; s < KS; s++) asm volatile("" ::"v"(qa[s]));
    asm volatile("" ::"v"(qs));

    int nblk = g.kblocks;
    if (CAUSAL) nblk = min(nblk, (qt * ATTN_ROWS + ATTN_ROWS - 1) / BN + 1);
    // Leading blocks no query of the workgroup needs masked: every key exists
    // and (causal) precedes the workgroup's first query. Merged padding keys
    // carry a -inf bias instead.
    int nfull = MERGE ? nblk : min(nblk, g.tk / BN);
    if (CAUSAL) nfull = min(nfull, (qt * ATTN_ROWS + 1) / BN);

    const uint8_t* kg = reinterpret_cast<const uint8_t*>(k8) + bhk * (long long)g.tk_pad * D;
    const uint8_t* vg = v8 + bhk * (long long)g.tk_pad * D;
    const float* ksc = k_scale + bhk * g.kblocks;

    // Direct global -> LDS copy of one tile. Lane `lane` of wave `wave` fills
    // physical chunk c of the tile, so it fetches the logical chunk that the
    // swizzle puts there (swz is an involution).
    // The tile base is uniform and is kept opaque, so that it stays in SGPRs
    // and each load takes it plus a 32-bit lane offset (instead of a 64-bit
    // per-lane address rebuilt every block); the LDS destination is uniform
    // as well (M0).
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    uint32_t foff[CPT][2];  // [chunk][K, V]
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        foff[i][0] = 16u * (uint32_t)swz(i * 256 + wv * 64 + lane, KCPR);
        foff[i][1] = 16u * (uint32_t)swz(i * 256 + wv * 64 + lane, 4);
    }
    // The 64 merge biases of block blk: one dword a lane of wave 0.
    auto fetch_bias = [&](int blk, float* dst) __attribute__((always_inline)) {
        if (MERGE && wv == 0)
            __builtin_amdgcn_global_load_lds(kbias + blk * BN + lane, (__attribute__((address_space(3))) void*)dst, 4,
                                             0, 0);
    };
    auto fetch = [&](const uint8_t* src_base, int blk, uint8_t* dst, int which) __attribute__((always_inline)) {
        const uint8_t* tb = opaque_uniform(src_base + (long long)blk * TILE);
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c0 = i * 256 + wv * 64;
            opaque_vgpr(foff[i][which]);  // widened next to the load: base + zext(offset) form
            __builtin_amdgcn_global_load_lds(tb + (size_t)foff[i][which],
                                             (__attribute__((address_space(3))) void*)(dst + 16 * c0), 16, 0, 0);
        }
    };

    // Per-lane LDS byte offsets of the MFMA operands. K row 32t + col, chunk
    // 2ks + half sits at swz((32t + col) * KCPR + 2ks + half); 32t rows are a
    // whole number of 256-byte lines whose count is a multiple of KCPR, so
    // the XOR term does not depend on t: the sub-tile term 32t * KCPR is a
    // constant offset and only the KS chunk columns need registers. V^T row
    // 32dt + col (4 chunks a row) likewise shares row col's XOR term.
    int koff[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) koff[ks] = 16 * swz(col * KCPR + 2 * ks + half, KCPR);
    const int voff0 = 16 * swz(col * 4 + 2 * half, 4), voff1 = 16 * swz(col * 4 + 2 * half + 1, 4);

    // S^T of one block (keys 32t .. 32t + 31 in s[t]) from the K tile `kt`,
    // each accumulator starting from the 1.5 * 2^23 bias.
    v16i magic;
#pragma unroll
    for (int r = 0; r < 16; r++) magic[r] = MAGIC_BITS;
    opaque_vgpr(magic);  // kept in VGPRs, not rebuilt before every block
    auto qk = [&](const uint8_t* kt, v16i (&s)[2]) __attribute__((always_inline)) {
        const v4i (&qb)[KS] = qa;
        if constexpr (D == 128) {
            // One 32-key sub-tile's K operands at a time: the registers this
            // saves hold the Q^T operands.
#pragma unroll
            for (int t = 0; t < 2; t++) {
                uint4 ka[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    ka[ks] = *reinterpret_cast<const uint4*>(kt + 16 * 32 * t * KCPR + koff[ks]);
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const v4i av = {(int)ka[ks].x, (int)ka[ks].y, (int)ka[ks].z, (int)ka[ks].w};
                    s[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qb[ks], ks ? s[t] : magic, 0, 0, 0);
                }
                if (t == 0) __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            uint4 ka[2][KS];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    ka[t][ks] = *reinterpret_cast<const uint4*>(kt + 16 * 32 * t * KCPR + koff[ks]);
#pragma unroll
            for (int t = 0; t < 2; t++) {
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const v4i av = {(int)ka[t][ks].x, (int)ka[t][ks].y, (int)ka[t][ks].z, (int)ka[t][ks].w};
                    s[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qb[ks], ks ? s[t] : magic, 0, 0, 0);
                }
            }
        }
    };

    v16f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
    // m: the row's running max (log2 units); P = 2^(x - m + log2 448).
    float m = -1.0e30f, l = 0.f;

    v8i pb = {};  // P^T operand of the block whose P.V is next

    // Softmax of block blk (scores sc, biased by 1.5 * 2^23): updates m and l,
    // writes the P^T operand into pn and returns alpha = 2^(m_old - m_new);
    // grow says whether this row's max moved.
    auto softmax = [&](int blk, v16i (&sc)[2], bool masked, v8i& pn, bool& grow, const float* bias)
                       __attribute__((always_inline)) {
        // The reference's fp32 operation order for the logits: no FMA contraction.
#pragma clang fp contract(off)
        // The logit scale q_scale * k_scale, the reference's. A masked block
        // sets scores to -inf, which the product must keep (0 * -inf is a NaN),
        // so there it is floored at SCALE_FLOOR, which changes no result but an
        // exact zero scale's; merged keys are masked by a -inf bias instead.
        const float kscf = ksc[blk];
        float scl = qs * kscf;
        if constexpr (MERGE) {
            // The logit fmaf(1.5 * 2^23 + S, scl, fmaf(-1.5 * 2^23, scl, bias)):
            // the inner term depends only on the key and the query group, so
            // lane l forms it once for key l and both groups (the same value,
            // bit for bit, that each lane of the group would form) and the
            // wave reads it back from LDS in place of the bias. A wave's LDS
            // operations run in order, so the previous block's reads are done.
            float* cw = ldsC + wv * 2 * BN;
            {
                const float bl = bias[lane];
                cw[lane] = fmaf(-MAGIC, qsg0 * kscf, bl);
                cw[BN + lane] = fmaf(-MAGIC, qsg1 * kscf, bl);
            }
            const float* cg = cw + (col >> 4) * BN;
            // Element (t, r) is key 32t + 8(r >> 2) + 4 half + (r & 3): four
            // consecutive keys a 16-byte read.
            float x[32];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 cc = *reinterpret_cast<const float4*>(cg + 32 * t + 8 * j + 4 * half);
                    const float cv[4] = {cc.x, cc.y, cc.z, cc.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = 4 * j + i;
                        x[16 * t + r] = fmaf(__int_as_float(sc[t][r]), scl, cv[i]);
                    }
                }
            // 15 three-input maxima and one two-input in a tree (the logits are
            // FMA results, so fmaxf needs no canonicalising).
            auto fmax3 = [](float a, float b, float c) __attribute__((always_inline)) {
                return fmaxf(fmaxf(a, b), c);
            };
            float f3[10];
#pragma unroll
            for (int i = 0; i < 10; i++) f3[i] = fmax3(x[3 * i], x[3 * i + 1], x[3 * i + 2]);
            float mx = fmaxf(fmax3(fmax3(f3[0], f3[1], f3[2]), fmax3(f3[3], f3[4], f3[5]), fmax3(f3[6], f3[7], f3[8])),
                             fmax3(f3[9], x[30], x[31]));
            mx = fmax_halves(mx);
            const float mnew = running_max(m, mx);
            grow = mnew > m;
            const float alpha = __builtin_amdgcn_exp2f(m - mnew);
            m = mnew;
            const float off = LOG2_448 - mnew;
            float p[2][16];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) p[t][r] = __builtin_amdgcn_exp2f(x[16 * t + r] + off);
            float q16[16];
#pragma unroll
            for (int r = 0; r < 16; r++) q16[r] = p[0][r] + p[1][r];
#pragma unroll
            for (int w = 8; w > 0; w >>= 1)
#pragma unroll
                for (int r = 0; r < w; r++) q16[r] += q16[r + w];
            l = fmaf(l, alpha, q16[0]);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int t = j >> 2, r0 = 4 * (j & 3);
                const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0], p[t][r0 + 1], pn[j], false);
                pn[j] = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0 + 2], p[t][r0 + 3], lo, true);
            }
            return alpha;
        }
        if (masked) {
            // Keys past the sequence, and keys after the query when causal. Element
            // (t, r) is key blk*BN + 4*half + c with the constant c below, so one
            // per-lane limit decides every element.
            const int ln = D == 128 ? lane_now() : lane, hf = ln >> 5;
            int lim = g.tk - blk * BN - 4 * hf;
            if (CAUSAL) lim = min(lim, q0 + (ln & 31) - blk * BN - 4 * hf + 1);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (32 * t + 8 * (r >> 2) + (r & 3) >= lim) sc[t][r] = NEG_INF_BITS;
            scl = fmaxf(scl, SCALE_FLOOR);
        }
        const float xoff = -MAGIC * scl;
        // Row max over this lane's 32 keys (a v_max3 tree), then the partner half.
        // 32 scores in 15 three-input maxima and one two-input: 10 over 30
        // scores, 4 over those and the last two scores, then 1 + 1.
        auto max3 = [](int a, int b, int c) __attribute__((always_inline)) { return max(max(a, b), c); };
        int m3[10];
#pragma unroll
        for (int i = 0; i < 10; i++)
            m3[i] = max3(sc[(3 * i) >> 4][(3 * i) & 15], sc[(3 * i + 1) >> 4][(3 * i + 1) & 15],
                         sc[(3 * i + 2) >> 4][(3 * i + 2) & 15]);
        const int m9 = max3(m3[0], m3[1], m3[2]), m10 = max3(m3[3], m3[4], m3[5]);
        const int m11 = max3(m3[6], m3[7], m3[8]), m12 = max3(m3[9], sc[1][14], sc[1][15]);
        int mx = max(max3(m9, m10, m11), m12);
        mx = max_halves(mx);

        // The running max in log2 units (a fully masked block gives -inf,
        // which leaves m alone); the row's largest score maps to P = 448.
        const float mnew = running_max(m, fmaf(__int_as_float(mx), scl, xoff));
        grow = mnew > m;
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        m = mnew;

        // P = 2^(x sc + off) of the biased scores; a masked one is -inf, so
        // (scl > 0) its exp2 is 0.
        const float off = (LOG2_448 - mnew) + xoff;
        float p[2][16];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) p[t][r] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(sc[t][r]), scl, off));
        // Row sum as a pairwise tree.
        float q16[16];
#pragma unroll
        for (int r = 0; r < 16; r++) q16[r] = p[0][r] + p[1][r];
#pragma unroll
        for (int w = 8; w > 0; w >>= 1)
#pragma unroll
            for (int r = 0; r < w; r++) q16[r] += q16[r + w];
        l = fmaf(l, alpha, q16[0]);

        // P^T operand: register j holds keys of accumulators 4(j%4)..+3 of
        // sub-tile j/4 (both halves are rewritten, so the register's previous
        // value serves as the unused input half and needs no zeroing).
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = j >> 2, r0 = 4 * (j & 3);
            const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0], p[t][r0 + 1], pn[j], false);
            pn[j] = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0 + 2], p[t][r0 + 3], lo, true);
        }
        return alpha;
    };
    // O *= alpha, only when some row of the wave moved its max.
    auto rescale = [&](float alpha, bool grow) __attribute__((always_inline)) {
        if (__any(grow)) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
        }
    };
    // O^T += V^T P^T; V^T operands (row = channel, 4 chunks per 64-byte row)
    // read two channel tiles at a time.
    auto pv = [&](const uint8_t* vt, const v8i& pbx) __attribute__((always_inline)) {
#pragma unroll
        for (int d2 = 0; d2 < DT; d2 += 2) {
            uint4 va[2][2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                va[e][0] = *reinterpret_cast<const uint4*>(vt + 16 * 128 * (d2 + e) + voff0);
                va[e][1] = *reinterpret_cast<const uint4*>(vt + 16 * 128 * (d2 + e) + voff1);
            }
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const v8i av = {(int)va[e][0].x, (int)va[e][0].y, (int)va[e][0].z, (int)va[e][0].w,
                                (int)va[e][1].x, (int)va[e][1].y, (int)va[e][1].z, (int)va[e][1].w};
                o[d2 + e] =
                    __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, pbx, o[d2 + e], 0, 0, 0, 127, 0, 127);
            }
        }
    };
    // One whole block, unpipelined: softmax, rescale, P.V.
    auto softmax_pv = [&](int blk, v16i (&sc)[2], const uint8_t* v_cur, const float* b_cur)
                          __attribute__((always_inline)) {
        bool grow;
        const float alpha = softmax(blk, sc, blk >= nfull, pb, grow, b_cur);
        __builtin_amdgcn_sched_barrier(0);
        rescale(alpha, grow);
        pv(v_cur, pb);
    };

    v16i S0[2];
    // Step j: prefetch K(j+1) and V(j+1) into the other buffers, then
    // QK^T, softmax and P.V of block j; the other waves on the SIMD fill the
    // MFMA and VALU gaps.
    auto step = [&](int blk, const uint8_t* k_cur, uint8_t* k_fill, const uint8_t* v_cur, uint8_t* v_fill,
                    const float* b_cur, float* b_fill) __attribute__((always_inline)) {
        if (blk + 1 < nblk) {
            fetch(kg, blk + 1, k_fill, 0);
            fetch(vg, blk + 1, v_fill, 1);
            fetch_bias(blk + 1, b_fill);
        }
        qk(k_cur, S0);
        softmax_pv(blk, S0, v_cur, b_cur);
        __syncthreads();
    };
    fetch(kg, 0, ldsK0, 0);
    fetch(vg, 0, ldsV0, 1);
    fetch_bias(0, ldsB0);
    __syncthreads();
    for (int blk = 0; blk < nblk; blk += 2) {
        step(blk, ldsK0, ldsK1, ldsV0, ldsV1, ldsB0, ldsB1);
        if (blk + 1 < nblk) step(blk + 1, ldsK1, ldsK0, ldsV1, ldsV0, ldsB1, ldsB0);
    }

    // out = O / l * v_scale + v_mean; lane holds channels 32dt + 8j + 4*half + 0..3.
    const float lt = sum_halves(l);
    const float inv = 1.0f / lt;
    const int ln_e = (D == 128 || MERGE) ? lane_now() : lane, half_e = ln_e >> 5, qi_e = q0 + (ln_e & 31);
    if (qi_e < g.tokens) {
        const float* vmean = stats + bhk * 4 * D + D;
        const float* vscale = vmean + D;
        uint16_t* orow = out + b * g.o_sb + (long long)qi_e * g.o_st + h * g.o_sh;
        // Pairs of outputs go through gfx950's packed converters
        // (v_cvt_pk_bf16_f32, v_cvt_pk_f16_f32: round to nearest even), one
        // uniform branch on the output type.
        auto emit = [&](auto pack) __attribute__((always_inline)) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int d0 = 32 * dt + 8 * j + 4 * half_e;
                    float y[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) y[r] = fmaf(o[dt][4 * j + r] * inv, vscale[d0 + r], vmean[d0 + r]);
                    uint2 w;
                    w.x = pack(y[0], y[1]);
                    w.y = pack(y[2], y[3]);
                    *reinterpret_cast<uint2*>(orow + d0) = w;
                }
        };
        if (g.flags & F_OUT_F16)
            emit([](float a, float b) { return pack_f16x2(a, b); });
        else
            emit([](float a, float b) { return pack_bf16x2(a, b); });
    }
}

#ifndef SAGE_ATTN_MERGED
// Dense and causal, eight waves a workgroup: score waves and output waves
// (the layout of Tile { warps: 8, .. }).
//
// An 8-wave workgroup owns 128 queries of one (batch, head). Waves 0-3, the
// score waves, run QK^T and the online softmax of 32 queries each; waves 4-7,
// the output waves, hold the O^T accumulators of the same queries (wave
// w + 4 those of wave w) and run the rescale and P.V. The dispatcher places a
// workgroup's waves round-robin over the CU's four SIMDs, so waves w and
// w + 4 share a SIMD, and with two workgroups a CU (<= 128 VGPRs) every SIMD
// runs two score waves and two output waves: a score wave's chain is QK^T
// and softmax only, and the FP8 P.V MFMAs run under the softmax.
//
// Step j runs the softmax of block j on the score waves and the P.V of block
// j - 1 on the output waves. A score wave hands each block's P^T operand (32
// bytes a lane, the register layout of the MFMA's B operand) and its
// per-query alpha to the output wave's same lane through LDS, double-buffered
// like K and V; the V ring runs one block behind the K ring. One barrier a
// step. The arithmetic is sage_attn<D, CAUSAL, false>'s, operation for
// operation (the same logits, running max, P codes, row sums, rescale and
// accumulation order), so the outputs are bit-identical to it. It runs two
// query groups a SIMD where sage_attn runs three (head dim 128) or four (64),
// and is the slower of the two on MI355X; the default tiles select sage_attn.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(512, 2) void sage_attn_split(const int8_t* __restrict__ q8,
                                                          const float* __restrict__ q_scale,
                                                          const int8_t* __restrict__ k8,
                                                          const float* __restrict__ k_scale,
                                                          const uint8_t* __restrict__ v8,
                                                          const float* __restrict__ stats,
                                                          uint16_t* __restrict__ out, Geom g) {
    constexpr int BN = ATTN_BN, KS = D / 32, DT = D / 32, TILE = BN * D, KCPR = D / 16;
    // 16-byte chunks a K or V tile: 512 at head dim 128 (one a thread), 256 at
    // 64 (one a thread of four waves: score waves copy K, output waves V).
    constexpr int CHUNKS = TILE / 16;
    static_assert(CHUNKS == 512 || CHUNKS == 256, "head dim 64 or 128");

    __shared__ __attribute__((aligned(16))) uint8_t ldsK0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsK1[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsV0[TILE];
    __shared__ __attribute__((aligned(16))) uint8_t ldsV1[TILE];
    // P^T operands of one block, [group][register half][lane] 16 bytes (a
    // lane's two b128 accesses are 1 KB apart, conflict-free), and alpha
    // [group][lane], double-buffered; the final row sums [group][lane].
    __shared__ __attribute__((aligned(16))) uint4 ldsP0[4 * 2 * 64];
    __shared__ __attribute__((aligned(16))) uint4 ldsP1[4 * 2 * 64];
    __shared__ __attribute__((aligned(16))) float ldsA0[4 * 64];
    __shared__ __attribute__((aligned(16))) float ldsA1[4 * 64];
    __shared__ __attribute__((aligned(16))) float ldsL[4 * 64];

    const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, half = lane >> 5;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), grp = wv & 3;
    const int ntq = gridDim.x;
    const int lin = blockIdx.x + ntq * (blockIdx.y + gridDim.y * blockIdx.z), total = ntq * gridDim.y * gridDim.z;
    int qt, hb;  // query tile; head slot b * heads + h (the same dealing as sage_attn)
    if (CAUSAL && causal_longest_first(total, ntq)) {
        const int per = total / NUM_XCD, hx = per / ntq, x = lin % NUM_XCD, i = lin / NUM_XCD;
        qt = ntq - 1 - i / hx;
        hb = x * hx + i % hx;
    } else {
        const int tile = xcd_tile(lin, total);
        qt = CAUSAL ? ntq - 1 - tile % ntq : tile % ntq;
        hb = tile / ntq;
    }
    const int h = hb % g.heads, b = hb / g.heads, hk = h / g.group;
    const long long bh = (long long)b * g.heads + h, bhk = (long long)b * g.kv_heads + hk;
    const int q0 = qt * ATTN_ROWS + grp * 32;  // first query of this wave's group

    int nblk = g.kblocks;
    if (CAUSAL) nblk = min(nblk, (qt * ATTN_ROWS + ATTN_ROWS - 1) / BN + 1);
    int nfull = min(nblk, g.tk / BN);
    if (CAUSAL) nfull = min(nfull, (qt * ATTN_ROWS + 1) / BN);

    const uint8_t* kg = reinterpret_cast<const uint8_t*>(k8) + bhk * (long long)g.tk_pad * D;
    const uint8_t* vg = v8 + bhk * (long long)g.tk_pad * D;

    // Direct global -> LDS copies of 16-byte chunks: wave slot `sl` fills
    // chunks 64 sl .. 64 sl + 63 of a tile (they land contiguously at M0;
    // lane `lane` fetches the logical chunk the swizzle puts there).
    const int sl = CHUNKS == 512 ? wv : (wv & 3);
    const uint32_t fk = 16u * (uint32_t)swz(sl * 64 + lane, KCPR), fv = 16u * (uint32_t)swz(sl * 64 + lane, 4);
    auto fetch = [&](const uint8_t* src_base, int blk, uint8_t* dst, uint32_t off) __attribute__((always_inline)) {
        const uint8_t* tb = opaque_uniform(src_base + (long long)blk * TILE);
        opaque_vgpr(off);
        __builtin_amdgcn_global_load_lds(tb + (size_t)off,
                                         (__attribute__((address_space(3))) void*)(dst + 16 * 64 * sl), 16, 0, 0);
    };
    const bool copies_k = CHUNKS == 512 || wv < 4, copies_v = CHUNKS == 512 || wv >= 4;
    // Step j's copies: K(j + 1) for the next step's QK^T, V(j) for the next
    // step's P.V.
    auto prefetch = [&](int j, uint8_t* k_fill, uint8_t* v_fill) __attribute__((always_inline)) {
        if (copies_k && j + 1 < nblk) fetch(kg, j + 1, k_fill, fk);
        if (copies_v && j < nblk) fetch(vg, j, v_fill, fv);
    };

    if (copies_k) fetch(kg, 0, ldsK0, fk);
    __syncthreads();

    if (wv < 4) {
        // ---- score wave: QK^T, online softmax, P^T and alpha to LDS ----
        const int qi = q0 + col;
        v4i qa[KS];
        {
            const int8_t* qrow = q8 + (bh * g.tq_pad + qi) * D + 16 * half;
#pragma unroll
            for (int s = 0; s < KS; s++) qa[s] = *reinterpret_cast<const v4i*>(qrow + 32 * s);
        }
        const float qs = q_scale[bh * (g.tq_pad / QGROUP) + (qi >> 4)];
#pragma unroll
        for (int s = 0; s < KS; s++) asm volatile("" ::"v"(qa[s]));
        asm volatile("" ::"v"(qs));
        const float* ksc = k_scale + bhk * g.kblocks;
        int koff[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) koff[ks] = 16 * swz(col * KCPR + 2 * ks + half, KCPR);
        v16i magic;
#pragma unroll
        for (int r = 0; r < 16; r++) magic[r] = MAGIC_BITS;
        opaque_vgpr(magic);
        float m = -1.0e30f, l = 0.f;

        auto block = [&](int blk, const uint8_t* kt, uint4* pdst, float* adst) __attribute__((always_inline)) {
            // The reference's fp32 operation order for the logits: no FMA contraction.
#pragma clang fp contract(off)
            // S^T of the block, keys 32t .. 32t + 31 in sc[t], from 1.5 * 2^23:
            // a sub-tile's four K operand reads in one LDS round trip, then its
            // four MFMAs.
            v16i sc[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                uint4 ka[KS];
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    ka[ks] = *reinterpret_cast<const uint4*>(kt + 16 * 32 * t * KCPR + koff[ks]);
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    const v4i av = {(int)ka[ks].x, (int)ka[ks].y, (int)ka[ks].z, (int)ka[ks].w};
                    sc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qa[ks], ks ? sc[t] : magic, 0, 0, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, KS, 0);  // the four LDS reads
                __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);  // then the four MFMAs
            }
            // The logit scale, floored in masked blocks only (as sage_attn).
            float scl = qs * ksc[blk];
            if (blk >= nfull) {
                // Padding keys, and keys after the query when causal (as sage_attn).
                const int ln = lane_now(), hf = ln >> 5;
                int lim = g.tk - blk * BN - 4 * hf;
                if (CAUSAL) lim = min(lim, q0 + (ln & 31) - blk * BN - 4 * hf + 1);
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        if (32 * t + 8 * (r >> 2) + (r & 3) >= lim) sc[t][r] = NEG_INF_BITS;
                scl = fmaxf(scl, SCALE_FLOOR);
            }
            const float xoff = -MAGIC * scl;
            auto max3 = [](int a, int b, int c) __attribute__((always_inline)) { return max(max(a, b), c); };
            int m3[10];
#pragma unroll
            for (int i = 0; i < 10; i++)
                m3[i] = max3(sc[(3 * i) >> 4][(3 * i) & 15], sc[(3 * i + 1) >> 4][(3 * i + 1) & 15],
                             sc[(3 * i + 2) >> 4][(3 * i + 2) & 15]);
            const int m9 = max3(m3[0], m3[1], m3[2]), m10 = max3(m3[3], m3[4], m3[5]);
            const int m11 = max3(m3[6], m3[7], m3[8]), m12 = max3(m3[9], sc[1][14], sc[1][15]);
            int mx = max(max3(m9, m10, m11), m12);
            mx = max_halves(mx);
            const float mnew = running_max(m, fmaf(__int_as_float(mx), scl, xoff));
            const float alpha = __builtin_amdgcn_exp2f(m - mnew);
            m = mnew;
            const float off = (LOG2_448 - mnew) + xoff;
            float p[2][16];
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) p[t][r] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(sc[t][r]), scl, off));
            float q16[16];
#pragma unroll
            for (int r = 0; r < 16; r++) q16[r] = p[0][r] + p[1][r];
#pragma unroll
            for (int w = 8; w > 0; w >>= 1)
#pragma unroll
                for (int r = 0; r < w; r++) q16[r] += q16[r + w];
            l = fmaf(l, alpha, q16[0]);
            v8i pn;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int t = j >> 2, r0 = 4 * (j & 3);
                const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0], p[t][r0 + 1], 0, false);
                pn[j] = __builtin_amdgcn_cvt_pk_fp8_f32(p[t][r0 + 2], p[t][r0 + 3], lo, true);
            }
            pdst[lane] = make_uint4((uint32_t)pn[0], (uint32_t)pn[1], (uint32_t)pn[2], (uint32_t)pn[3]);
            pdst[64 + lane] = make_uint4((uint32_t)pn[4], (uint32_t)pn[5], (uint32_t)pn[6], (uint32_t)pn[7]);
            adst[lane] = alpha;
            if (blk == nblk - 1) ldsL[grp * 64 + lane] = l;
        };
        for (int j = 0; j <= nblk; j += 2) {
            prefetch(j, ldsK1, ldsV0);
            if (j < nblk) block(j, ldsK0, ldsP0 + grp * 128, ldsA0 + grp * 64);
            __syncthreads();
            if (j + 1 <= nblk) {
                prefetch(j + 1, ldsK0, ldsV1);
                if (j + 1 < nblk) block(j + 1, ldsK1, ldsP1 + grp * 128, ldsA1 + grp * 64);
                __syncthreads();
            }
        }
    } else {
        // ---- output wave: rescale O by alpha, O^T += V^T P^T, epilogue ----
        v16f o[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[dt][r] = 0.f;
        const int voff0 = 16 * swz(col * 4 + 2 * half, 4), voff1 = 16 * swz(col * 4 + 2 * half + 1, 4);
        auto block = [&](const uint8_t* vt, const uint4* psrc, const float* asrc) __attribute__((always_inline)) {
            const float alpha = asrc[lane];
            const uint4 p0 = psrc[lane], p1 = psrc[64 + lane];
            uint4 va[DT][2];
#pragma unroll
            for (int d = 0; d < DT; d++) {
                va[d][0] = *reinterpret_cast<const uint4*>(vt + 16 * 128 * d + voff0);
                va[d][1] = *reinterpret_cast<const uint4*>(vt + 16 * 128 * d + voff1);
            }
            // alpha is exactly 1 in every row whose max did not move (the exp2
            // of 0) and below 1 otherwise; multiplying by 1 changes nothing, so
            // this is sage_attn's rescale.
            if (__any(alpha < 1.0f)) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
            }
            const v8i pb = {(int)p0.x, (int)p0.y, (int)p0.z, (int)p0.w, (int)p1.x, (int)p1.y, (int)p1.z, (int)p1.w};
#pragma unroll
            for (int d = 0; d < DT; d++) {
                const v8i av = {(int)va[d][0].x, (int)va[d][0].y, (int)va[d][0].z, (int)va[d][0].w,
                                (int)va[d][1].x, (int)va[d][1].y, (int)va[d][1].z, (int)va[d][1].w};
                o[d] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, pb, o[d], 0, 0, 0, 127, 0, 127);
            }
        };
        for (int j = 0; j <= nblk; j += 2) {
            prefetch(j, ldsK1, ldsV0);
            if (j >= 1) block(ldsV1, ldsP1 + grp * 128, ldsA1 + grp * 64);  // block j - 1 (odd)
            __syncthreads();
            if (j + 1 <= nblk) {
                prefetch(j + 1, ldsK0, ldsV1);
                block(ldsV0, ldsP0 + grp * 128, ldsA0 + grp * 64);  // block j (even)
                __syncthreads();
            }
        }

        // out = O / l * v_scale + v_mean; lane holds channels 32dt + 8j + 4*half + 0..3.
        const float lt = sum_halves(ldsL[grp * 64 + lane]);
        const float inv = 1.0f / lt;
        const int qi = q0 + col;
        if (qi < g.tokens) {
            const float* vmean = stats + bhk * 4 * D + D;
            const float* vscale = vmean + D;
            uint16_t* orow = out + b * g.o_sb + (long long)qi * g.o_st + h * g.o_sh;
            auto emit = [&](auto pack) __attribute__((always_inline)) {
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int d0 = 32 * dt + 8 * j + 4 * half;
                        float y[4];
#pragma unroll
                        for (int r = 0; r < 4; r++) y[r] = fmaf(o[dt][4 * j + r] * inv, vscale[d0 + r], vmean[d0 + r]);
                        uint2 w;
                        w.x = pack(y[0], y[1]);
                        w.y = pack(y[2], y[3]);
                        *reinterpret_cast<uint2*>(orow + d0) = w;
                    }
            };
            if (g.flags & F_OUT_F16)
                emit([](float a, float b) { return pack_f16x2(a, b); });
            else
                emit([](float a, float b) { return pack_bf16x2(a, b); });
        }
    }
}

template <int D, bool CAUSAL>
static hipError_t launch_split(const AttendBufs& w, const Geom& g, hipStream_t s) {
    hipLaunchKernelGGL((sage_attn_split<D, CAUSAL>), dim3(g.tq_pad / ATTN_ROWS, g.heads, g.batch), dim3(512), 0, s,
                       w.q8, w.q_scale, w.k8, w.k_scale, w.v8, w.stats, static_cast<uint16_t*>(w.out), g);
    return hipGetLastError();
}
#endif

template <int D, bool CAUSAL, bool MERGE>
static hipError_t launch_d(const AttendBufs& w, const Geom& g, hipStream_t s) {
    hipLaunchKernelGGL((sage_attn<D, CAUSAL, MERGE>), dim3(g.tq_pad / ATTN_ROWS, g.heads, g.batch), dim3(256), 0, s,
                       w.q8, w.q_scale, w.k8, w.k_scale, w.v8, w.stats, w.kbias, static_cast<uint16_t*>(w.out), g);
    return hipGetLastError();
}

template <bool CAUSAL, bool MERGE>
static hipError_t resources_of(int head_dim, int* regs, int* spill, int* lds) {
    hipFuncAttributes a;
    const void* f = head_dim == 64 ? reinterpret_cast<const void*>(&sage_attn<64, CAUSAL, MERGE>)
                                   : reinterpret_cast<const void*>(&sage_attn<128, CAUSAL, MERGE>);
    hipError_t e = hipFuncGetAttributes(&a, f);
    if (e != hipSuccess) return e;
    *regs = a.numRegs;
    *spill = (int)a.localSizeBytes;
    *lds = (int)a.sharedSizeBytes;
    return hipSuccess;
}

// This file is compiled twice. The dense and causal kernels (this pass) take
// LLVM's iterative occupancy-keeping pre-RA scheduler and a bottom-up post-RA
// pass, which reorder their instructions only (outputs bit-identical) and are
// faster for them; the merged kernels (SAGE_ATTN_MERGED) are faster with the
// default order and are built in the second pass.
#ifndef SAGE_ATTN_MERGED

// Dense, causal (an extension) or merged (sg_attn_merge); the API refuses
// causal masking over merged keys.
hipError_t launch_attention(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s) {
    if (g.merge > 1) return launch_attention_merged(head_dim, w, g, s);
    if (g.flags & F_WAVES8) {
        if (head_dim == 64)
            return (g.flags & F_CAUSAL) ? launch_split<64, true>(w, g, s) : launch_split<64, false>(w, g, s);
        return (g.flags & F_CAUSAL) ? launch_split<128, true>(w, g, s) : launch_split<128, false>(w, g, s);
    }
    if (head_dim == 64)
        return (g.flags & F_CAUSAL) ? launch_d<64, true, false>(w, g, s) : launch_d<64, false, false>(w, g, s);
    return (g.flags & F_CAUSAL) ? launch_d<128, true, false>(w, g, s) : launch_d<128, false, false>(w, g, s);
}

hipError_t attention_resources(int head_dim, bool causal, bool merge, bool waves8, int* regs, int* spill, int* lds) {
    if (merge) return attention_resources_merged(head_dim, regs, spill, lds);
    if (waves8) {
        hipFuncAttributes a;
        const void* f = head_dim == 64
                            ? (causal ? reinterpret_cast<const void*>(&sage_attn_split<64, true>)
                                      : reinterpret_cast<const void*>(&sage_attn_split<64, false>))
                            : (causal ? reinterpret_cast<const void*>(&sage_attn_split<128, true>)
                                      : reinterpret_cast<const void*>(&sage_attn_split<128, false>));
        hipError_t e = hipFuncGetAttributes(&a, f);
        if (e != hipSuccess) return e;
        *regs = a.numRegs;
        *spill = (int)a.localSizeBytes;
        *lds = (int)a.sharedSizeBytes;
        return hipSuccess;
    }
    return causal ? resources_of<true, false>(head_dim, regs, spill, lds)
                  : resources_of<false, false>(head_dim, regs, spill, lds);
}

#else

hipError_t launch_attention_merged(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s) {
    return head_dim == 64 ? launch_d<64, false, true>(w, g, s) : launch_d<128, false, true>(w, g, s);
}

hipError_t attention_resources_merged(int head_dim, int* regs, int* spill, int* lds) {
    return resources_of<false, true>(head_dim, regs, spill, lds);
}

#endif

}  // namespace sage
