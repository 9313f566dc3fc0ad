// The product's device E4M3 encoder (sage::e4m3_pair, the FP8 V quantisation
// of the prologue) against the C oracle's encoder (oracle_f32_to_e4m3, the
// reference's cvt.rn.satfinite semantics) on every one of the 2^32 f32 bit
// patterns, in both bytes of the pair. The GPU reduces each chunk of 2^24
// inputs to two weighted sums of its codes; the host computes the same sums
// with the oracle (OpenMP) and compares. A differing chunk is recomputed code
// by code and its first difference printed. Exit status 0 when all agree.
#include <hip/hip_runtime.h>
#include <omp.h>

#include <cstdio>
#include <cstdint>
#include <cstring>
#include <vector>

#include "sage_device.hpp"
#include "sage_oracle.h"

constexpr int CHUNK_BITS = 24;
constexpr int CHUNKS = 1 << (32 - CHUNK_BITS);
constexpr uint32_t PER_THREAD = 1024;

// The second input of the pair: a bijection of the first, so each byte sees every input.
__host__ __device__ inline uint32_t partner(uint32_t u) { return u ^ 0x55555555u; }
// splitmix64's finaliser: the weight of input u in a chunk's sum.
__host__ __device__ inline uint64_t weight(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void encode_sums(unsigned long long* sums) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;  // 2^22 threads, PER_THREAD inputs each
    uint64_t lo = 0, hi = 0;
    for (uint32_t j = 0; j < PER_THREAD; j++) {
        const uint32_t u = t * PER_THREAD + j;
        const uint32_t w = partner(u);
        const uint32_t two = sage::e4m3_pair(__uint_as_float(u), __uint_as_float(w));
        lo += (uint64_t)((two & 0xffu) + 1u) * weight(u);
        hi += (uint64_t)((two >> 8) + 1u) * weight(w);
    }
    const uint32_t chunk = (t * PER_THREAD) >> CHUNK_BITS;
    atomicAdd(&sums[2 * chunk], (unsigned long long)lo);
    atomicAdd(&sums[2 * chunk + 1], (unsigned long long)hi);
}

__global__ __launch_bounds__(256) void encode_chunk(uint32_t first, uint16_t* out) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;  // 2^24 threads
    const uint32_t u = first + i;
    out[i] = (uint16_t)sage::e4m3_pair(__uint_as_float(u), __uint_as_float(partner(u)));
}

static float as_float(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

int main() {
    unsigned long long* d_sums;
    if (hipMalloc(&d_sums, 2 * CHUNKS * sizeof(unsigned long long)) != hipSuccess) return 2;
    if (hipMemset(d_sums, 0, 2 * CHUNKS * sizeof(unsigned long long)) != hipSuccess) return 2;
    hipLaunchKernelGGL(encode_sums, dim3((1u << 22) / 256), dim3(256), 0, 0, d_sums);
    if (hipDeviceSynchronize() != hipSuccess) return 2;
    std::vector<unsigned long long> gpu(2 * CHUNKS), cpu(2 * CHUNKS, 0);
    if (hipMemcpy(gpu.data(), d_sums, gpu.size() * 8, hipMemcpyDeviceToHost) != hipSuccess) return 2;

    // The same sums from the oracle's encoder.
#pragma omp parallel for schedule(static)
    for (int c = 0; c < CHUNKS; c++) {
        uint64_t lo = 0, hi = 0;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) {
            const uint32_t u = first + i, w = partner(u);
            lo += (uint64_t)(oracle_f32_to_e4m3(as_float(u)) + 1u) * weight(u);
            hi += (uint64_t)(oracle_f32_to_e4m3(as_float(w)) + 1u) * weight(w);
        }
        cpu[2 * c] = lo;
        cpu[2 * c + 1] = hi;
    }
    int bad = 0;
    uint16_t* d_out;
    if (hipMalloc(&d_out, (1u << CHUNK_BITS) * sizeof(uint16_t)) != hipSuccess) return 2;
    std::vector<uint16_t> codes(1u << CHUNK_BITS);
    for (int c = 0; c < CHUNKS; c++) {
        if (gpu[2 * c] == cpu[2 * c] && gpu[2 * c + 1] == cpu[2 * c + 1]) continue;
        bad++;
        const uint32_t first = (uint32_t)c << CHUNK_BITS;
        hipLaunchKernelGGL(encode_chunk, dim3((1u << CHUNK_BITS) / 256), dim3(256), 0, 0, first, d_out);
        if (hipMemcpy(codes.data(), d_out, codes.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) return 2;
        for (uint32_t i = 0; i < (1u << CHUNK_BITS); i++) {
            const uint32_t u = first + i;
            const unsigned want_lo = oracle_f32_to_e4m3(as_float(u)), want_hi = oracle_f32_to_e4m3(as_float(partner(u)));
            if ((codes[i] & 0xffu) != want_lo || (codes[i] >> 8) != want_hi) {
                std::printf("chunk %d: input 0x%08x (pair 0x%08x) gives 0x%04x, oracle 0x%02x%02x\n", c, u, partner(u),
                            codes[i], want_hi, want_lo);
                break;
            }
        }
    }
    std::printf("%d of %d chunks differ (%d threads on the host)\n", bad, CHUNKS, omp_get_max_threads());
    return bad ? 1 : 0;
}
