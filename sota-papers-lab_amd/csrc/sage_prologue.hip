// SageAttention2 prologue for gfx950: K/V channel statistics, INT8 Q (one
// scale per 16 rows), INT8 K (one scale per 64 keys), FP8 E4M3 V (one scale
// per channel). Three HBM-bound launches:
//
//   sage_prep      grid ((1 + group) q_tiles, kv_heads, batch): per 128-token
//                  tile, one workgroup writes the partial K sum, V sum, V min,
//                  V max of every channel, and one per query head of the
//                  group that shares the KV head its INT8 Q (Q and K rows
//                  LayerNormed first under QK LayerNorm); fed from the fused
//                  QKV projection, K and V get a workgroup each
//                  ((2 + group) q_tiles)
//   sage_finalize  grid (D / 4 channel groups of every KV head, dealt one
//                  head an XCD): K mean, V mean, V scale, 1/V scale
//   sage_quant_kv  grid (kblocks, kv_heads, batch): smoothed INT8 K and FP8 V,
//                  V transposed per 64-key block into the MFMA operand order;
//                  with KV merging each key pools its members (and the keys'
//                  log2 member counts go to kbias)
//
// Codes and scales are bit-identical to the reference's
// (sezer-muhammed/sota-papers-lab, platform/spl-nn/cuda/sage_quant.cu:59-206,
// 238-319): each fp32 sum keeps that kernel's operation order, which is fixed
// by its 256-thread tile, its 32-lane warp butterfly and its even/odd tile
// fold. A 256-thread workgroup here is four wave64s; each 32-lane half of a
// wave plays one of the reference's warps, so the same partials meet in the
// same order.
//
// Cache policy: sage_quant_kv re-reads the K and V that sage_prep read, and
// MI355X's memory-side cache can hold much of them in between. Everything
// read or written exactly once goes around it (non-temporal): the Q load and
// the q8, k8 and v8 stores. The attention kernel shares its K/V tiles through
// L2, not through that cache.
#include <algorithm>

#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace sage {

typedef unsigned nt_u2 __attribute__((ext_vector_type(2)));
typedef unsigned nt_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16(const uint16_t* p, bool ok) {
    return ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
}
__device__ __forceinline__ uint4 load16_once(const uint16_t* p, bool ok) {
    if (!ok) return make_uint4(0, 0, 0, 0);
    const nt_u4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store8_once(void* p, uint2 w) {
    __builtin_nontemporal_store(nt_u2{w.x, w.y}, reinterpret_cast<nt_u2*>(p));
}
__device__ __forceinline__ void store16_once(void* p, uint4 w) {
    __builtin_nontemporal_store(nt_u4{w.x, w.y, w.z, w.w}, reinterpret_cast<nt_u4*>(p));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// LayerNorm of one head row (sage_quant.cu:34-52) whose D channels lie on
// D/8 consecutive lanes, 8 a lane (ch = lane's chunk); every lane of the wave
// calls it. The lane sums meet in the reference's xor butterfly over
// distances 1 .. D/16; the square deviations accumulate fused (fmaf), the
// variance takes fmaf(s2, 1/D, eps) and the output fmaf((x - mean) * rstd,
// w, b) -- the reference's expressions under NVRTC's default contraction.
// rstd is 1 / sqrt(.) with the square root and the divide each correctly
// rounded (the reference's rsqrtf is an approximation whose rounding it does
// not state), so the kernel and the CPU oracle agree bit for bit.
template <int D>
__device__ __forceinline__ void layernorm8(float* x, const float* __restrict__ w, const float* __restrict__ bias,
                                           int ch, float eps) {
    constexpr int CH = D / 8;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) s += x[e];
#pragma unroll
    for (int o = 1; o < CH; o <<= 1) s += __shfl_xor(s, o, 64);
    const float mean = s * (1.0f / D);
    float s2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float d = x[e] - mean;
        s2 = __builtin_fmaf(d, d, s2);
    }
#pragma unroll
    for (int o = 1; o < CH; o <<= 1) s2 += __shfl_xor(s2, o, 64);
    const float rstd = rsqrt_rn2(__builtin_fmaf(s2, 1.0f / D, eps));
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = __builtin_fmaf((x[e] - mean) * rstd, w[ch * 8 + e], bias[ch * 8 + e]);
}

// One row chunk of the fused QKV projection as the reference's QKV prologue
// leaves it for the sage prologue (qkv.cu:37-133): transformed in fp32
// (qkv_apply), then rounded to bf16 as qkv_prologue's store rounds it, so
// the codes equal those of running that prologue and then this one.
template <int D>
__device__ __forceinline__ void qkv_row(float* x, const QkvDev& qa, const QkvLane& L, const QkvTok& T, int part,
                                        int ch, uint4* packed = nullptr) {
    qkv_apply<D>(x, qa, L, T, part, ch);
    // Pairs through one packed conversion: the low bf16 back to f32 by a
    // shift, the high one by a mask. `packed` receives the bf16 row itself.
    uint32_t u[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        u[e / 2] = pack_bf16x2(x[e], x[e + 1]);
        x[e] = __uint_as_float(u[e / 2] << 16);
        x[e + 1] = __uint_as_float(u[e / 2] & 0xffff0000u);
    }
    if (packed) *packed = make_uint4(u[0], u[1], u[2], u[3]);
}

// The fused prologue's K stash. While sage_prep runs, the workspace's INT8 K
// and FP8 V buffers hold nothing yet, and one 64-key block of them (64 D
// bytes of k8, 64 D of v8) holds exactly that block's 64 K rows in bf16. So
// sage_prep stores each K row as the QKV prologue leaves it (bf16) there --
// keys 0-31 of block j over k8's block j, keys 32-63 over v8's -- and
// sage_quant_kv reads them back instead of re-running the QKV arithmetic on
// the projection; it reads a block's stash before it writes that block's
// codes (its K-scale barrier lies between). Dense plans only: a merged
// plan's blocks pool more tokens than the stash holds.
__device__ __forceinline__ uint8_t* k_stash(int8_t* k8, uint8_t* v8, const Geom& g, long long bhk, int tok, int ch,
                                            int D) {
    const int blk = tok / KBLOCK, kk = tok % KBLOCK;
    uint8_t* base = kk < KBLOCK / 2
                        ? reinterpret_cast<uint8_t*>(k8) + (bhk * g.tk_pad + (long long)blk * KBLOCK) * D
                        : v8 + (bhk * g.kblocks + blk) * (long long)(KBLOCK * D);
    return base + (kk % (KBLOCK / 2)) * 2 * D + ch * 16;
}

// sage_quant.cu:59-160 (sg_prep), split into roles (statistics, Q codes). Under QK LayerNorm (LN, the
// F_LN_Q and F_LN_K flags together as the reference sets them) every K row is
// normalised before the statistics read it and every Q row before its amax;
// the LN-free instantiation keeps the dense kernel's registers.

// K and V channel statistics of one 128-token tile (sage_quant.cu:73-80,
// 97-107, 129-159): the tile's partial K sum, V sum, V min and V max. PART
// selects the rows a workgroup reads: S_KV both (the reference's one block),
// S_K the K rows and their sum, S_V the V rows and their sum, min and max. The
// fused QKV prologue gives K and V workgroups of their own: K rows carry the
// whole QKV arithmetic (norm, RoPE) and V rows little, so one workgroup doing
// both was the slowest role of the launch.
enum { S_KV = 0, S_K = 1, S_V = 2 };
template <int D, bool LN, bool QKV, int PART>
__device__ __forceinline__ void tile_stats(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                           const float* __restrict__ ln, float* __restrict__ part, int8_t* k8,
                                           uint8_t* v8, const Geom& g, const QkvDev& qa, int tile, int hk, int b,
                                           float (*red)[4][D]) {
    constexpr int CH = D / 8;        // 16-byte chunks per head row
    constexpr int TPI = 256 / CH;    // tokens per iteration
    constexpr int NI = QTILE / TPI;  // iterations
    constexpr bool DO_K = PART != S_V, DO_V = PART != S_K;
    const int tid = threadIdx.x, ch = tid % CH, slot = tid / CH;
    const bool f16 = g.flags & F_IN_F16;
    const long long bhk = (long long)b * g.kv_heads + hk;
    float ks[8], vs[8], vmn[8], vmx[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        ks[e] = 0.f;
        vs[e] = 0.f;
        vmn[e] = 3.0e38f;
        vmx[e] = -3.0e38f;
    }
    QkvLane lk, lv;
    if (QKV) {
        if (DO_K) qkv_lane<D>(lk, qa, g, 1, hk, ch);
        if (DO_V) qkv_lane<D>(lv, qa, g, 2, hk, ch);
    }
    // Row i of the thread (token tok) into the running sums, in i order.
    auto accumulate = [&](int tok, float* fk, float* fv) __attribute__((always_inline)) {
        if (LN && DO_K) layernorm8<D>(fk, ln + 2 * D, ln + 3 * D, ch, g.ln_eps);
        if (tok < g.tokens) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                if (DO_K) ks[e] += fk[e];
                if (DO_V) {
                    vs[e] += fv[e];
                    vmn[e] = fminf(vmn[e], fv[e]);
                    vmx[e] = fmaxf(vmx[e], fv[e]);
                }
            }
        }
    };
    if constexpr (QKV && PART == S_V) {
        // V rows carry only the token and channel scales and the bias: all
        // loads first, as for plain inputs.
        uint4 vraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            vraw[i] = load16(v + b * g.v_sb + (long long)tok * g.v_st + hk * g.v_sh + ch * 8, tok < g.tokens);
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            float fv[8];
            QkvTok tt;
            qkv_tok<D>(tt, qa, g, 2, b, tok, ch);
            unpack8(vraw[i], fv, false);
            qkv_row<D>(fv, qa, lv, tt, 2, ch);
            accumulate(tok, nullptr, fv);
        }
    } else if constexpr (QKV) {
        // K rows of the fused projection: every row's load issued first (one
        // row at a time left each wave waiting on its load), then each row's
        // QKV-prologue arithmetic, its stash and its sum.
        static_assert(PART == S_K, "the fused statistics pass splits K and V");
        uint4 kraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            kraw[i] = load16(k + b * g.k_sb + (long long)tok * g.k_st + hk * g.k_sh + ch * 8, tok < g.tokens);
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            const bool ok = tok < g.tokens;
            float fk[8];
            QkvTok tt;
            qkv_tok<D>(tt, qa, g, 1, b, tok, ch);
            unpack8(kraw[i], fk, false);
            uint4 kbf;
            qkv_row<D>(fk, qa, lk, tt, 1, ch, &kbf);
            if (g.merge == 1 && ok) *reinterpret_cast<uint4*>(k_stash(k8, v8, g, bhk, tok, ch, D)) = kbf;
            accumulate(tok, fk, nullptr);
        }
    } else {
        uint4 kraw[NI], vraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            const bool ok = tok < g.tokens;
            kraw[i] = load16(k + b * g.k_sb + (long long)tok * g.k_st + hk * g.k_sh + ch * 8, ok);
            vraw[i] = load16(v + b * g.v_sb + (long long)tok * g.v_st + hk * g.v_sh + ch * 8, ok);
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            float fk[8], fv[8];
            unpack8(kraw[i], fk, f16);
            unpack8(vraw[i], fv, f16);
            accumulate(tok, fk, fv);
        }
    }
    // Lanes of one 32-lane half that hold the same channels, then the halves
    // in order (sage_quant.cu:129-159).
#pragma unroll
    for (int o = CH; o < 32; o <<= 1) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            if (DO_K) ks[e] += __shfl_xor(ks[e], o, 64);
            if (DO_V) {
                vs[e] += __shfl_xor(vs[e], o, 64);
                vmn[e] = fminf(vmn[e], __shfl_xor(vmn[e], o, 64));
                vmx[e] = fmaxf(vmx[e], __shfl_xor(vmx[e], o, 64));
            }
        }
    }
    if ((tid & 31) < CH) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            red[tid >> 5][0][ch * 8 + e] = ks[e];
            red[tid >> 5][1][ch * 8 + e] = vs[e];
            red[tid >> 5][2][ch * 8 + e] = vmn[e];
            red[tid >> 5][3][ch * 8 + e] = vmx[e];
        }
    }
    __syncthreads();
    constexpr int S0 = DO_K ? 0 : 1, S1 = DO_V ? 4 : 1;  // the statistics [S0, S1) this part owns
    for (int c = S0 * D + tid; c < S1 * D; c += 256) {
        const int stat = c / D, d = c % D;
        float r = red[0][stat][d];
#pragma unroll
        for (int w = 1; w < 8; w++) {
            const float x = red[w][stat][d];
            r = stat < 2 ? r + x : (stat == 2 ? fminf(r, x) : fmaxf(r, x));
        }
        part[((bhk * g.q_tiles + tile) * 4 + stat) * D + d] = r;
    }
}

// INT8 Q of one 128-token tile of query head gi of the `group` heads that
// read KV head hk (sage_quant.cu:85-127).
template <int D, bool LN, bool QKV>
__device__ __forceinline__ void tile_q8(const uint16_t* __restrict__ q, const float* __restrict__ ln,
                                        int8_t* __restrict__ q8, float* __restrict__ q_scale, const Geom& g,
                                        const QkvDev& qa, int tile, int hk, int gi, int b, unsigned* gmax,
                                        float* ginv) {
    constexpr int CH = D / 8;
    constexpr int TPI = 256 / CH;
    constexpr int NI = QTILE / TPI;
    const int tid = threadIdx.x, ch = tid % CH, slot = tid / CH;
    const bool f16 = g.flags & F_IN_F16;
    const bool tail = (tile + 1) * QTILE > g.tokens;  // the tile holds padding rows (workgroup-uniform)
    {
        const int h = hk * g.group + gi;
        const long long bh = (long long)b * g.heads + h;
        if (tid < QTILE / QGROUP) gmax[tid] = 0u;
        __syncthreads();
        QkvLane lq;
        if (QKV) qkv_lane<D>(lq, qa, g, 0, h, ch);
        uint4 qraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tok = tile * QTILE + slot + i * TPI;
            qraw[i] = load16_once(q + b * g.q_sb + (long long)tok * g.q_st + h * g.q_sh + ch * 8, tok < g.tokens);
        }
        float qv[NI][8];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            unpack8(qraw[i], qv[i], f16);
            const int tok = tile * QTILE + slot + i * TPI;
            if (QKV) {
                QkvTok tt;
                qkv_tok<D>(tt, qa, g, 0, b, tok, ch);
                qkv_row<D>(qv[i], qa, lq, tt, 0, ch);
            }
            if (LN) layernorm8<D>(qv[i], ln, ln + D, ch, g.ln_eps);
            if ((LN || QKV) && tail && tok >= g.tokens) {
#pragma unroll
                for (int e = 0; e < 8; e++) qv[i][e] = 0.f;  // padding rows stay zero
            }
            float amax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(qv[i][e]));
            // A wave's tokens of one iteration lie in one 16-row group.
            amax = wave_max(amax);
            if ((tid & 63) == 0) atomicMax(&gmax[(slot + i * TPI) / QGROUP], __float_as_uint(amax));
        }
        __syncthreads();
        // Each 16-row group's 127 / amax (0 for an all-zero group), formed once
        // a group and read back by the lanes of its rows.
        if (tid < QTILE / QGROUP) {
            const float amax = __uint_as_float(gmax[tid]);
            ginv[tid] = amax > 0.f ? 127.0f / amax : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int tl = slot + i * TPI;
            const float inv = ginv[tl / QGROUP];
            const float* f = qv[i];
            uint2 w;
            w.x = s8x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
            w.y = s8x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
            store8_once(q8 + (bh * g.tq_pad + tile * QTILE + tl) * D + ch * 8, w);
        }
        if (tid < QTILE / QGROUP)
            q_scale[bh * (g.tq_pad / QGROUP) + tile * (QTILE / QGROUP) + tid] =
                __uint_as_float(gmax[tid]) * (1.0f / 127.0f) * g.q_mul;
        __syncthreads();
    }
}

// STATS + group workgroups a tile: the first STATS the K/V statistics (one,
// or with the fused QKV prologue one for K and one for V), each other the
// INT8 Q of one query head of the KV head's group. The reference's one
// thread block does all of it in turn; split, the streams of loads overlap
// across workgroups, and grouped-query plans spread their Q heads over
// workgroups instead of walking them in one.
template <bool QKV>
constexpr int stat_roles() { return QKV ? 2 : 1; }
template <int D, bool LN, bool QKV>
__global__ __launch_bounds__(256) void sage_prep(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                 const uint16_t* __restrict__ v, const float* __restrict__ ln,
                                                 int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                 float* __restrict__ part, int8_t* __restrict__ k8,
                                                 uint8_t* __restrict__ v8, Geom g, QkvDev qa) {
    __shared__ unsigned gmax[QTILE / QGROUP];
    __shared__ float ginv[QTILE / QGROUP];
    __shared__ float red[8][4][D];
    constexpr int STATS = stat_roles<QKV>();
    const int roles = STATS + g.group, tile = (int)blockIdx.x / roles, role = (int)blockIdx.x % roles;
    const int hk = blockIdx.y, b = blockIdx.z;
    if (role >= STATS) {
        tile_q8<D, LN, QKV>(q, ln, q8, q_scale, g, qa, tile, hk, role - STATS, b, gmax, ginv);
    } else if constexpr (!QKV) {
        tile_stats<D, LN, QKV, S_KV>(k, v, ln, part, k8, v8, g, qa, tile, hk, b, red);
    } else {
        if (role == 0)
            tile_stats<D, LN, QKV, S_K>(k, v, ln, part, k8, v8, g, qa, tile, hk, b, red);
        else
            tile_stats<D, LN, QKV, S_V>(k, v, ln, part, k8, v8, g, qa, tile, hk, b, red);
    }
}

// sage_quant.cu:163-206 (sg_finalize): even and odd tiles folded separately,
// each in tile order, then combined. A workgroup takes FIN_CH channels of one
// KV head, i.e. their 4 * FIN_CH (statistic, channel) columns. Its 256
// threads stage up to FIN_CHUNK tiles of those columns in LDS with every load
// of the chunk in flight at once; wave w then folds statistic w, one lane per
// (channel, parity), in tile order, so the fold's operation is uniform across
// the wave. A long sequence (VGGT's 1077 tiles a head) costs a few load
// round trips instead of one per sixteen tiles. The workgroups of one head
// share every 128-byte line of its partials, so they are dealt to one XCD
// (the dispatcher deals linear ids round-robin over the 8 XCDs): each line
// then comes from HBM into one L2 once.
constexpr int FIN_CH = 4;
constexpr int FIN_CHUNK = 512;
template <int D>
__global__ __launch_bounds__(256) void sage_finalize(const float* __restrict__ part, float* __restrict__ stats,
                                                     Geom g) {
    constexpr int NCG = D / FIN_CH;
    __shared__ float4 tl[FIN_CHUNK][4];  // [tile][statistic]: the workgroup's FIN_CH channels
    __shared__ float fin[4][2][FIN_CH];
    const int lin = (int)blockIdx.x, j = lin / NUM_XCD, tid = threadIdx.x;
    const int cg = j % NCG;
    const long long bhk = (long long)(j / NCG) * NUM_XCD + lin % NUM_XCD;
    if (bhk >= (long long)g.batch * g.kv_heads) return;  // the grid pads heads to a multiple of 8
    const float* base = part + bhk * g.q_tiles * 4 * D + cg * FIN_CH;
    // Folding lanes: statistic = wave (uniform), channel fc, tile parity par.
    const int fs = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int fc = lane & (FIN_CH - 1), par = (lane >> 2) & 1;
    const bool folds = lane < 2 * FIN_CH;
    float r = fs < 2 ? 0.f : (fs == 2 ? 3.0e38f : -3.0e38f);
    // Loading threads: tile tid / 4 + 64 i of the chunk, statistic tid % 4.
    const int ls = tid & 3, lt = tid >> 2;
    // A chunk's loads are all in flight together, and the next chunk's while
    // this one is folded. Only the 64-tile slices a chunk reaches are loaded
    // (a workgroup-uniform count); rows past the sequence inside them are
    // filled from its last tile and never folded.
    const float* src = base + (long long)lt * 4 * D + ls * D;
    const long long last = (long long)(g.q_tiles - 1 - lt) * 4 * D;  // clamp, relative to src
    auto slices = [&](int t0) { return max(0, min(FIN_CHUNK / 64, (g.q_tiles - t0 + 63) / 64)); };
    // (Held as scalars: an array of float4 copied into LDS whole was kept in
    // scratch memory by the compiler.)
    float x[FIN_CHUNK / 64][4];
    auto fetch = [&](int i, long long off) __attribute__((always_inline)) {
        const float4 u = *reinterpret_cast<const float4*>(src + min(off, last));
        x[i][0] = u.x, x[i][1] = u.y, x[i][2] = u.z, x[i][3] = u.w;
    };
    int nl = slices(0);
#pragma unroll
    for (int i = 0; i < FIN_CHUNK / 64; i++)
        if (i < nl) fetch(i, (long long)(64 * i) * 4 * D);
    for (int t0 = 0; t0 < g.q_tiles; t0 += FIN_CHUNK) {
        const int n = min(FIN_CHUNK, g.q_tiles - t0);
#pragma unroll
        for (int i = 0; i < FIN_CHUNK / 64; i++)
            if (i < nl) tl[lt + 64 * i][ls] = make_float4(x[i][0], x[i][1], x[i][2], x[i][3]);
        __syncthreads();
        nl = slices(t0 + FIN_CHUNK);
#pragma unroll
        for (int i = 0; i < FIN_CHUNK / 64; i++)
            if (i < nl) fetch(i, (long long)(t0 + FIN_CHUNK + 64 * i) * 4 * D);
        // t0 is even, so a tile's parity in the chunk is its parity overall.
        if (folds) {
            const float* col = reinterpret_cast<const float*>(&tl[0][fs]) + fc;
            if (fs < 2) {
#pragma unroll 8
                for (int t = par; t < n; t += 2) r += col[t * 16];
            } else if (fs == 2) {
#pragma unroll 8
                for (int t = par; t < n; t += 2) r = fminf(r, col[t * 16]);
            } else {
#pragma unroll 8
                for (int t = par; t < n; t += 2) r = fmaxf(r, col[t * 16]);
            }
        }
        __syncthreads();
    }
    if (folds) fin[fs][par][fc] = r;
    __syncthreads();
    if (tid < FIN_CH) {
        const int c = tid, d = cg * FIN_CH + c;
        float st[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; s2++) {
            const float r0 = fin[s2][0][c], r1 = fin[s2][1][c];
            st[s2] = s2 < 2 ? r0 + r1 : (s2 == 2 ? fminf(r0, r1) : fmaxf(r0, r1));
        }
        const float n = (float)g.tokens;
        const float mk = (g.flags & F_SMOOTH_K) ? st[0] / n : 0.f;
        const float mv = (g.flags & F_SMOOTH_V) ? st[1] / n : 0.f;
        const float amax = fmaxf(st[3] - mv, mv - st[2]);
        const float scale = amax > 0.f ? amax / g.v_range : 1.0f;
        float* o = stats + bhk * 4 * D;
        o[d] = mk;
        o[D + d] = mv;
        o[2 * D + d] = scale;
        o[3 * D + d] = 1.0f / scale;
    }
}

// E4M3 codes of one key's 8 channels (ch * 8 .. + 7) into the transposed V
// tile: channel row r, byte v8_position(kl). Row r keeps its 16 dwords
// XOR-permuted by r >> 3 (= ch): the channel groups of a wave write rows
// 512 bytes apart, which would all fall in one LDS bank, and the permutation
// spreads them over 16 (D = 128) or 8 (D = 64) banks; the copy to HBM undoes it.
__device__ __forceinline__ void put_v(uint8_t* vt, int ch, int kl, const float* vq) {
    const int pos = v8_position(kl) ^ ((ch & 15) << 2);
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const uint32_t two = e4m3_pair(vq[e], vq[e + 1]);
        vt[(ch * 8 + e) * KBLOCK + pos] = (uint8_t)two;
        vt[(ch * 8 + e + 1) * KBLOCK + pos] = (uint8_t)(two >> 8);
    }
}

// sage_quant.cu:238-319 (sg_quant_kv): K - mean -> INT8 per block,
// (V - mean) / scale -> E4M3, V stored [block][channel][v8_position(key)].
// A merged key sums its members in order from 0.0f and takes
// fmaf(sum, 1/n, -mean): NVRTC's default contraction of the reference's
// `sum * rc - mean`, equal to the dense (k + 0) - mean when n = 1.
// Under QK LayerNorm (LN) each K row (each member, when merging) is
// normalised before it is summed (sage_quant.cu:271).
template <int D, bool LN, bool QKV>
__global__ __launch_bounds__(256) void sage_quant_kv(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     const float* __restrict__ ln,
                                                     const float* __restrict__ stats, int8_t* __restrict__ k8,
                                                     float* __restrict__ k_scale, uint8_t* __restrict__ v8,
                                                     float* __restrict__ kbias, Geom g, QkvDev qa) {
    constexpr int CH = D / 8;
    constexpr int TPI = 256 / CH;
    constexpr int NI = KBLOCK / TPI;
    const int blk = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, ch = tid % CH, slot = tid / CH;
    const bool f16 = g.flags & F_IN_F16;
    const long long bhk = (long long)b * g.kv_heads + hk;

    __shared__ unsigned kmax;
    __shared__ __attribute__((aligned(16))) uint8_t vt[D * KBLOCK];
    if (tid == 0) kmax = 0u;

    const float* st = stats + bhk * 4 * D;
    float mk[8], mv[8], iv[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        mk[e] = st[ch * 8 + e];
        mv[e] = st[D + ch * 8 + e];
        iv[e] = st[3 * D + ch * 8 + e];
    }
    float kv[NI][8];
    float amax = 0.f;
    // The reference sums a dense key's (one) member from 0.0f first, so V's
    // -0 becomes +0 before the mean is taken off: (v + 0) - mv. That equals
    // v - mvz with mvz = -0 where mv is a zero of either sign (x - (-0) is
    // x + 0) and mv elsewhere (where -0 - mv and +0 - mv agree), one operation
    // fewer a value. It matters for V's E4M3 code (0x80 against 0x00) but not
    // for K, whose |kv| and INT8 code drop the sign of a zero.
    float mvz[8];
#pragma unroll
    for (int e = 0; e < 8; e++) mvz[e] = mv[e] == 0.0f ? -0.0f : mv[e];
    // A block with no key past the sequence (all but a ragged last one) can
    // run without the per-key guards (workgroup-uniform).
    const bool full = (blk + 1) * KBLOCK <= g.tk;
    if (QKV && g.merge == 1) {
        // Rows of the fused projection: V first, then K, so that only one
        // part's channel constants (QkvLane) and statistics are live at a time.
        __syncthreads();
        {
            QkvLane lv;
            qkv_lane<D>(lv, qa, g, 2, hk, ch);
            uint4 vraw[NI];
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int j = blk * KBLOCK + slot + i * TPI;
                vraw[i] = load16(v + b * g.v_sb + (long long)j * g.v_st + hk * g.v_sh + ch * 8, j < g.tk);
            }
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int kl = slot + i * TPI;
                const bool ok = blk * KBLOCK + kl < g.tk;
                float fv[8], vq[8];
                unpack8(vraw[i], fv, false);
                QkvTok tt;
                qkv_tok<D>(tt, qa, g, 2, b, blk * KBLOCK + kl, ch);
                qkv_row<D>(fv, qa, lv, tt, 2, ch);
#pragma unroll
                for (int e = 0; e < 8; e++) vq[e] = ok ? (fv[e] - mvz[e]) * iv[e] : 0.f;
                put_v(vt, ch, kl, vq);
            }
        }
        // K rows as sage_prep stashed them (bf16, after the QKV arithmetic),
        // over this block's k8 and v8 bytes: every read here is consumed
        // before the K-scale barrier, every code store comes after it.
        uint4 kraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int j = blk * KBLOCK + slot + i * TPI;
            kraw[i] = j < g.tk ? *reinterpret_cast<const uint4*>(k_stash(k8, v8, g, bhk, j, ch, D))
                               : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int kl = slot + i * TPI;
            const bool ok = blk * KBLOCK + kl < g.tk;
            float fk[8];
            unpack8(kraw[i], fk, false);
            if (LN) layernorm8<D>(fk, ln + 2 * D, ln + 3 * D, ch, g.ln_eps);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kv[i][e] = ok ? fk[e] - mk[e] : 0.f;
                amax = fmaxf(amax, fabsf(kv[i][e]));
            }
        }
    } else if (g.merge == 1) {
        uint4 kraw[NI], vraw[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int j = blk * KBLOCK + slot + i * TPI;
            const bool ok = j < g.tk;
            kraw[i] = load16(k + b * g.k_sb + (long long)j * g.k_st + hk * g.k_sh + ch * 8, ok);
            vraw[i] = load16(v + b * g.v_sb + (long long)j * g.v_st + hk * g.v_sh + ch * 8, ok);
        }
        __syncthreads();
        auto rows = [&](bool all) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int kl = slot + i * TPI;
                const bool ok = all || blk * KBLOCK + kl < g.tk;
                float fk[8], fv[8];
                unpack8(kraw[i], fk, f16);
                unpack8(vraw[i], fv, f16);
                if (LN) layernorm8<D>(fk, ln + 2 * D, ln + 3 * D, ch, g.ln_eps);
                float vq[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    kv[i][e] = ok ? fk[e] - mk[e] : 0.f;
                    amax = fmaxf(amax, fabsf(kv[i][e]));
                    vq[e] = ok ? (fv[e] - mvz[e]) * iv[e] : 0.f;
                }
                put_v(vt, ch, kl, vq);
            }
        };
        // (The normed instantiation keeps one copy: two would cost it a wave.)
        if (!LN && full)
            rows(true);
        else
            rows(false);
    } else {
        __syncthreads();
        const int cells = g.merge * g.merge;  // uniform bound of the member loop
        if constexpr (QKV) {
            // Members of the fused projection: V then K, as in the dense path.
            {
                QkvLane lv;
                qkv_lane<D>(lv, qa, g, 2, hk, ch);
#pragma unroll
                for (int i = 0; i < NI; i++) {
                    const int kl = slot + i * TPI;
                    const int j = blk * KBLOCK + kl;
                    const bool ok = j < g.tk;
                    int base = 0, nx = 1;
                    const int cnt = ok ? merged_members(g, j, base, nx) : 0;
                    float vs[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) vs[e] = 0.f;
                    for (int m = 0; m < cells; m++) {
                        const bool mok = m < cnt;
                        const int tok = base + (mok ? (m / nx) * g.grid_w + m % nx : 0);
                        float fv[8];
                        unpack8(load16(v + b * g.v_sb + (long long)tok * g.v_st + hk * g.v_sh + ch * 8, mok), fv, false);
                        QkvTok tt;
                        qkv_tok<D>(tt, qa, g, 2, b, tok, ch);
                        qkv_row<D>(fv, qa, lv, tt, 2, ch);
                        if (mok) {
#pragma unroll
                            for (int e = 0; e < 8; e++) vs[e] += fv[e];
                        }
                    }
                    const float rc = cnt > 0 ? 1.0f / (float)cnt : 0.f;
                    float vq[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) vq[e] = ok ? __builtin_fmaf(vs[e], rc, -mv[e]) * iv[e] : 0.f;
                    put_v(vt, ch, kl, vq);
                }
            }
            QkvLane lk;
            qkv_lane<D>(lk, qa, g, 1, hk, ch);
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int kl = slot + i * TPI;
                const int j = blk * KBLOCK + kl;
                const bool ok = j < g.tk;
                int base = 0, nx = 1;
                const int cnt = ok ? merged_members(g, j, base, nx) : 0;
                float ks[8];
#pragma unroll
                for (int e = 0; e < 8; e++) ks[e] = 0.f;
                for (int m = 0; m < cells; m++) {
                    const bool mok = m < cnt;
                    const int tok = base + (mok ? (m / nx) * g.grid_w + m % nx : 0);
                    float fk[8];
                    unpack8(load16(k + b * g.k_sb + (long long)tok * g.k_st + hk * g.k_sh + ch * 8, mok), fk, false);
                    QkvTok tt;
                    qkv_tok<D>(tt, qa, g, 1, b, tok, ch);
                    qkv_row<D>(fk, qa, lk, tt, 1, ch);
                    if (LN) layernorm8<D>(fk, ln + 2 * D, ln + 3 * D, ch, g.ln_eps);
                    if (mok) {
#pragma unroll
                        for (int e = 0; e < 8; e++) ks[e] += fk[e];
                    }
                }
                const float rc = cnt > 0 ? 1.0f / (float)cnt : 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    kv[i][e] = ok ? __builtin_fmaf(ks[e], rc, -mk[e]) : 0.f;
                    amax = fmaxf(amax, fabsf(kv[i][e]));
                }
            }
        } else {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int kl = slot + i * TPI;
            const int j = blk * KBLOCK + kl;
            const bool ok = j < g.tk;
            int base = 0, nx = 1;
            const int cnt = ok ? merged_members(g, j, base, nx) : 0;
            float ks[8], vs[8];
#pragma unroll
            for (int e = 0; e < 8; e++) ks[e] = vs[e] = 0.f;
            for (int m = 0; m < cells; m++) {
                const bool mok = m < cnt;
                const int tok = base + (mok ? (m / nx) * g.grid_w + m % nx : 0);
                float fk[8], fv[8];
                unpack8(load16(k + b * g.k_sb + (long long)tok * g.k_st + hk * g.k_sh + ch * 8, mok), fk, f16);
                unpack8(load16(v + b * g.v_sb + (long long)tok * g.v_st + hk * g.v_sh + ch * 8, mok), fv, f16);
                if (LN) layernorm8<D>(fk, ln + 2 * D, ln + 3 * D, ch, g.ln_eps);
                if (mok) {
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        ks[e] += fk[e];
                        vs[e] += fv[e];
                    }
                }
            }
            const float rc = cnt > 0 ? 1.0f / (float)cnt : 0.f;
            float vq[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kv[i][e] = ok ? __builtin_fmaf(ks[e], rc, -mk[e]) : 0.f;
                amax = fmaxf(amax, fabsf(kv[i][e]));
                vq[e] = ok ? __builtin_fmaf(vs[e], rc, -mv[e]) * iv[e] : 0.f;
            }
            put_v(vt, ch, kl, vq);
        }
        }
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) atomicMax(&kmax, __float_as_uint(amax));
    __syncthreads();

    const float km = __uint_as_float(kmax);
    const float inv = km > 0.f ? 127.0f / km : 0.f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int kl = slot + i * TPI;
        const float* f = kv[i];
        uint2 w;
        w.x = s8x4(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
        w.y = s8x4(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
        store8_once(k8 + (bhk * g.tk_pad + blk * KBLOCK + kl) * D + ch * 8, w);
    }
    if (tid == 0) k_scale[bhk * g.kblocks + blk] = km * (1.0f / 127.0f);
    // Channel row r of the tile, un-permuting its dwords (see put_v).
    uint8_t* vo = v8 + (bhk * g.kblocks + blk) * (long long)(D * KBLOCK);
    for (int c = tid; c < D * KBLOCK / 16; c += 256) {
        const int r = c >> 2, sw = (r >> 3) & 15;  // row r, 16-byte chunk c & 3
        const uint32_t* row = reinterpret_cast<const uint32_t*>(vt + r * KBLOCK);
        uint4 w;
        w.x = row[(4 * (c & 3) + 0) ^ sw];
        w.y = row[(4 * (c & 3) + 1) ^ sw];
        w.z = row[(4 * (c & 3) + 2) ^ sw];
        w.w = row[(4 * (c & 3) + 3) ^ sw];
        store16_once(reinterpret_cast<uint4*>(vo) + c, w);
    }
    // The merge bias depends on the key alone (sage_quant.cu:321-325).
    if (g.merge > 1 && b == 0 && hk == 0 && tid < KBLOCK) {
        const int j = blk * KBLOCK + tid;
        int base, nx;
        kbias[j] = j < g.tk ? log2_count(merged_members(g, j, base, nx)) : __uint_as_float(0xff800000u);
    }
}

// qkv.cu:37-133 (qkv_prologue) on its own: every (batch, token, part, head)
// row of the fused projection stored as 16-bit rows of Q, K and V (V in fp16
// when asked, from the fp32 value as the reference's cvt.rn.f16x2 takes it).
// A workgroup owns one part-head slot r (blockIdx.y; slot r starts at channel
// r * D of a projection row) of one batch item (blockIdx.z) and walks its
// tokens 256 / (D/8) at a time, D/8 lanes a token, so the lane's channel
// scales, bias and norm weights are loaded once. The projection's strides
// are g.q_sb (batch) and g.q_st (token). Tokens past the end compute on
// zeros, so every lane takes part in the shuffles, and store nothing.
template <int D>
__global__ __launch_bounds__(256) void sage_qkv(const uint16_t* __restrict__ y, QkvOutDev o, Geom g, QkvDev qa) {
    constexpr int CH = D / 8, RPB = 256 / CH;
    const int ch = threadIdx.x % CH, r = blockIdx.y, b = blockIdx.z;
    const int part = r < g.heads ? 0 : (r < g.heads + g.kv_heads ? 1 : 2);
    const int h = part == 0 ? r : (part == 1 ? r - g.heads : r - g.heads - g.kv_heads);
    QkvLane lane;
    qkv_lane<D>(lane, qa, g, part, h, ch);
    const uint16_t* yb = y + b * g.q_sb + (long long)r * D + ch * 8;
    uint16_t* ob = o.p[part] + b * o.sb[part] + h * o.sh[part] + ch * 8;
    const long long ost = o.st[part];
    const bool f16 = part == 2 && o.v_f16;
    for (int t0 = blockIdx.x * RPB; t0 < g.tokens; t0 += gridDim.x * RPB) {
        const int tok = t0 + (int)threadIdx.x / CH;
        const bool valid = tok < g.tokens;
        QkvTok tt;
        qkv_tok<D>(tt, qa, g, part, b, valid ? tok : 0, ch);
        float x[8];
        unpack8(load16(yb + (long long)tok * g.q_st, valid), x, false);
        qkv_apply<D>(x, qa, lane, tt, part, ch);
        if (valid) {
            uint4 w;
            if (f16) {
                w = make_uint4(pack_f16x2(x[0], x[1]), pack_f16x2(x[2], x[3]), pack_f16x2(x[4], x[5]),
                               pack_f16x2(x[6], x[7]));
            } else {
                w = make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                               pack_bf16x2(x[6], x[7]));
            }
            *reinterpret_cast<uint4*>(ob + (long long)tok * ost) = w;
        }
    }
}

hipError_t launch_qkv(int head_dim, const uint16_t* y, const QkvOutDev& o, const Geom& g, const QkvDev& qa,
                      hipStream_t s) {
    const int rpb = 256 / (head_dim / 8);
    const int slots = g.heads + 2 * g.kv_heads;
    // About 16 workgroups a CU in all; each walks its slot's tokens.
    const long long want = std::max(1LL, (256LL * 16 + (long long)slots * g.batch - 1) / ((long long)slots * g.batch));
    const unsigned bx = (unsigned)std::min<long long>(want, (g.tokens + rpb - 1) / rpb);
    const dim3 grid(bx, slots, g.batch);
    if (head_dim == 64)
        hipLaunchKernelGGL(sage_qkv<64>, grid, dim3(256), 0, s, y, o, g, qa);
    else
        hipLaunchKernelGGL(sage_qkv<128>, grid, dim3(256), 0, s, y, o, g, qa);
    return hipGetLastError();
}

template <int D, bool LN, bool QKV>
static hipError_t launch_prologue_d(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ln,
                                    const PrologueBufs& w, const Geom& g, const QkvDev& qa, hipStream_t s) {
    const long long prep_blocks = (long long)(stat_roles<QKV>() + g.group) * g.q_tiles;
    if (prep_blocks > INT32_MAX) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((sage_prep<D, LN, QKV>), dim3((unsigned)prep_blocks, g.kv_heads, g.batch), dim3(256), 0, s,
                       q, k, v, ln,
                       w.q8, w.q_scale, w.part, w.k8, w.v8, g, qa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long long heads8 = ((long long)g.batch * g.kv_heads + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
    if (heads8 * (D / FIN_CH) > INT32_MAX) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(sage_finalize<D>, dim3((unsigned)(heads8 * (D / FIN_CH))), dim3(256), 0, s, w.part, w.stats, g);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((sage_quant_kv<D, LN, QKV>), dim3(g.kblocks, g.kv_heads, g.batch), dim3(256), 0, s, k, v, ln,
                       w.stats, w.k8, w.k_scale, w.v8, w.kbias, g, qa);
    return hipGetLastError();
}

template <int D, bool LN>
static hipError_t launch_prologue_q(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ln,
                                    const PrologueBufs& w, const Geom& g, const QkvDev* qa, hipStream_t s) {
    if (qa) return launch_prologue_d<D, LN, true>(q, k, v, ln, w, g, *qa, s);
    return launch_prologue_d<D, LN, false>(q, k, v, ln, w, g, QkvDev{}, s);
}

hipError_t launch_prologue(int head_dim, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ln,
                           const PrologueBufs& w, const Geom& g, const QkvDev* qa, hipStream_t s) {
    const bool norm = (g.flags & (F_LN_Q | F_LN_K)) == (F_LN_Q | F_LN_K);
    if (head_dim == 64)
        return norm ? launch_prologue_q<64, true>(q, k, v, ln, w, g, qa, s)
                    : launch_prologue_q<64, false>(q, k, v, ln, w, g, qa, s);
    return norm ? launch_prologue_q<128, true>(q, k, v, ln, w, g, qa, s)
                : launch_prologue_q<128, false>(q, k, v, ln, w, g, qa, s);
}

}  // namespace sage
