// The product's device encoders of the prologue against the C oracle's, on
// every one of the 2^32 f32 bit patterns:
// - sage::e4m3_pair (the FP8 V codes) against oracle_f32_to_e4m3 (the
//   reference's cvt.rn.satfinite semantics), in both bytes of the pair;
// - sage::s8_code (the INT8 Q and K codes) against oracle_s8 (sage_common.cu
//   sg_s8: round to nearest even, clamp to +-127, NaN to 0);
// - sage::rsqrt_rn2 (the QK-norm's rstd) against oracle_rstd (1 / sqrt with
//   both steps correctly rounded), NaN results compared as one pattern.
// The GPU reduces each chunk of 2^24 inputs to weighted sums of its codes; the
// host computes the same sums with the oracle (OpenMP) and compares. A
// differing chunk is recomputed code by code and its first difference printed.
// Exit status 0 when all agree.
#include <hip/hip_runtime.h>
#include <omp.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "sage_device.hpp"
#include "sage_oracle.h"

constexpr int CHUNK_BITS = 24;
constexpr int CHUNKS = 1 << (32 - CHUNK_BITS);
constexpr uint32_t PER_THREAD = 1024;

// The second input of an E4M3 pair: a bijection of the first, so each byte sees every input.
__host__ __device__ inline uint32_t partner(uint32_t u) { return u ^ 0x55555555u; }
// splitmix64's finaliser: the weight of input u in a chunk's sum.
__host__ __device__ inline uint64_t weight(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

enum Codec { E4M3 = 0, S8 = 1 };

// Two codes of input u: E4M3 of u and of partner(u), or the INT8 code of u (and 0).
template <int C>
__device__ inline uint32_t device_codes(uint32_t u) {
    if (C == E4M3) return sage::e4m3_pair(__uint_as_float(u), __uint_as_float(partner(u)));
    return sage::s8_code(__uint_as_float(u));
}
static float as_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static uint32_t host_codes(int c, uint32_t u) {
    if (c == E4M3)
        return oracle_f32_to_e4m3(as_float(u)) | ((uint32_t)oracle_f32_to_e4m3(as_float(partner(u))) << 8);
    return (uint32_t)oracle_s8(as_float(u)) & 0xffu;
}

template <int C>
__global__ __launch_bounds__(256) void code_sums(unsigned long long* sums) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;  // 2^22 threads, PER_THREAD inputs each
    uint64_t lo = 0, hi = 0;
    for (uint32_t j = 0; j < PER_THREAD; j++) {
        const uint32_t u = t * PER_THREAD + j;
        const uint32_t two = device_codes<C>(u);
        lo += (uint64_t)((two & 0xffu) + 1u) * weight(u);
        hi += (uint64_t)((two >> 8) + 1u) * weight(partner(u));
    }
    const uint32_t chunk = (t * PER_THREAD) >> CHUNK_BITS;
    atomicAdd(&sums[2 * chunk], (unsigned long long)lo);
    atomicAdd(&sums[2 * chunk + 1], (unsigned long long)hi);
}

template <int C>
__global__ __launch_bounds__(256) void code_chunk(uint32_t first, uint16_t* out) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;  // 2^24 threads
    out[i] = (uint16_t)device_codes<C>(first + i);
}

// Number of differing chunks of codec C, or -1 on a HIP error.
template <int C>
static int check(const char* name, unsigned long long* d_sums, uint16_t* d_out) {
    if (hipMemset(d_sums, 0, 2 * CHUNKS * sizeof(unsigned long long)) != hipSuccess) return -1;
    hipLaunchKernelGGL(code_sums<C>, dim3((1u << 22) / 256), dim3(256), 0, 0, d_sums);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    std::vector<unsigned long long> gpu(2 * CHUNKS), cpu(2 * CHUNKS, 0);
    if (hipMemcpy(gpu.data(), d_sums, gpu.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < CHUNKS; c++) {
        uint64_t lo = 0, hi = 0;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) {
            const uint32_t u = first + i, two = host_codes(C, u);
            lo += (uint64_t)((two & 0xffu) + 1u) * weight(u);
            hi += (uint64_t)((two >> 8) + 1u) * weight(partner(u));
        }
        cpu[2 * c] = lo;
        cpu[2 * c + 1] = hi;
    }
    int bad = 0;
    std::vector<uint16_t> codes(1u << CHUNK_BITS);
    for (int c = 0; c < CHUNKS; c++) {
        if (gpu[2 * c] == cpu[2 * c] && gpu[2 * c + 1] == cpu[2 * c + 1]) continue;
        bad++;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        hipLaunchKernelGGL(code_chunk<C>, dim3((1u << CHUNK_BITS) / 256), dim3(256), 0, 0, first, d_out);
        if (hipMemcpy(codes.data(), d_out, codes.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) return -1;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) {
            const uint32_t u = first + i, want = host_codes(C, u);
            if (codes[i] != want) {
                std::printf("%s chunk %d: input 0x%08x gives 0x%04x, oracle 0x%04x\n", name, c, u, codes[i], want);
                break;
            }
        }
    }
    std::printf("%s: %d of %d chunks differ (%d threads on the host)\n", name, bad, CHUNKS, omp_get_max_threads());
    return bad;
}

// The rstd's f32 bits, every NaN as 0x7fc00000 (payloads are not part of the contract).
__host__ __device__ inline uint32_t canon(uint32_t r) { return (r & 0x7fffffffu) > 0x7f800000u ? 0x7fc00000u : r; }

__global__ __launch_bounds__(256) void rstd_sums(unsigned long long* sums) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;  // 2^22 threads, PER_THREAD inputs each
    uint64_t acc = 0;
    for (uint32_t j = 0; j < PER_THREAD; j++) {
        const uint32_t u = t * PER_THREAD + j;
        acc += (uint64_t)(canon(__float_as_uint(sage::rsqrt_rn2(__uint_as_float(u)))) + 1u) * weight(u);
    }
    atomicAdd(&sums[(t * PER_THREAD) >> CHUNK_BITS], (unsigned long long)acc);
}

__global__ __launch_bounds__(256) void rstd_chunk(uint32_t first, uint32_t* out) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;  // 2^24 threads
    out[i] = canon(__float_as_uint(sage::rsqrt_rn2(__uint_as_float(first + i))));
}

static uint32_t host_rstd(uint32_t u) {
    const float r = oracle_rstd(as_float(u));
    uint32_t b;
    std::memcpy(&b, &r, 4);
    return canon(b);
}

// Number of differing chunks of the rstd, or -1 on a HIP error.
static int check_rstd(unsigned long long* d_sums, uint32_t* d_out) {
    if (hipMemset(d_sums, 0, CHUNKS * sizeof(unsigned long long)) != hipSuccess) return -1;
    hipLaunchKernelGGL(rstd_sums, dim3((1u << 22) / 256), dim3(256), 0, 0, d_sums);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    std::vector<unsigned long long> gpu(CHUNKS), cpu(CHUNKS, 0);
    if (hipMemcpy(gpu.data(), d_sums, gpu.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < CHUNKS; c++) {
        uint64_t acc = 0;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) acc += (uint64_t)(host_rstd(first + i) + 1u) * weight(first + i);
        cpu[c] = acc;
    }
    int bad = 0;
    std::vector<uint32_t> vals(1u << CHUNK_BITS);
    for (int c = 0; c < CHUNKS; c++) {
        if (gpu[c] == cpu[c]) continue;
        bad++;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        hipLaunchKernelGGL(rstd_chunk, dim3((1u << CHUNK_BITS) / 256), dim3(256), 0, 0, first, d_out);
        if (hipMemcpy(vals.data(), d_out, vals.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) {
            const uint32_t u = first + i, want = host_rstd(u);
            if (vals[i] != want) {
                std::printf("rstd chunk %d: input 0x%08x gives 0x%08x, oracle 0x%08x\n", c, u, vals[i], want);
                break;
            }
        }
    }
    std::printf("rstd: %d of %d chunks differ (%d threads on the host)\n", bad, CHUNKS, omp_get_max_threads());
    return bad;
}

int main() {
    unsigned long long* d_sums;
    uint16_t* d_out;
    if (hipMalloc(&d_sums, 2 * CHUNKS * sizeof(unsigned long long)) != hipSuccess) return 2;
    if (hipMalloc(&d_out, (1u << CHUNK_BITS) * sizeof(uint16_t)) != hipSuccess) return 2;
    uint32_t* d_vals;
    if (hipMalloc(&d_vals, (1u << CHUNK_BITS) * sizeof(uint32_t)) != hipSuccess) return 2;
    const int e = check<E4M3>("e4m3", d_sums, d_out);
    const int s = check<S8>("s8", d_sums, d_out);
    const int r = check_rstd(d_sums, d_vals);
    if (e < 0 || s < 0 || r < 0) return 2;
    return (e || s || r) ? 1 : 0;
}
