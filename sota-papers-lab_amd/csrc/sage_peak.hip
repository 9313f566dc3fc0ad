// MFMA peak probes for gfx950: the measured denominators of "% of peak"
// (the counterpart of sezer-muhammed/sota-papers-lab,
// platform/spl-nn/cuda/sage_peak.cu:10-94 and its driver in
// src/sage/tests.rs:757-794). Every wave runs 8 independent accumulator
// chains of one MFMA shape; inputs are fixed finite bit patterns.
#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace sage {

constexpr int PEAK_CHAINS = 8;

__global__ __launch_bounds__(256) void peak_i8(int* out, int iters) {
    const v4i a = {(int)threadIdx.x, 3, 5, 7}, bm = {11, (int)threadIdx.x, 13, 17};
    v16i c[PEAK_CHAINS];
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) c[j] = (v16i){};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < PEAK_CHAINS; j++) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bm, c[j], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) s += c[j][0] + c[j][15];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void peak_f8(int* out, int iters) {
    const int one = 0x38383838;  // E4M3 1.0
    const v8i a = {one, one, one, one, one, one, one, (int)threadIdx.x & 0x38};
    v16f c[PEAK_CHAINS];
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) c[j] = (v16f){};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < PEAK_CHAINS; j++)
            c[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, a, c[j], 0, 0, 0, 127, 0, 127);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) s += c[j][0] + c[j][15];
    out[blockIdx.x * blockDim.x + threadIdx.x] = (int)s;
}

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(256) void peak_bf16(int* out, int iters) {
    v8bf a;
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = (__bf16)(1.0f + (float)((threadIdx.x + i) & 1) * 0.0078125f);
    v16f c[PEAK_CHAINS];
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) c[j] = (v16f){};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < PEAK_CHAINS; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, c[j], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PEAK_CHAINS; j++) s += c[j][0] + c[j][15];
    out[blockIdx.x * blockDim.x + threadIdx.x] = (int)s;
}

hipError_t run_peak(int which, int iters, hipStream_t s, double* tops) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    const int blocks = cus * 8, threads = 256;
    int* sink = nullptr;
    e = hipMalloc(&sink, (size_t)blocks * threads * sizeof(int));
    if (e != hipSuccess) return e;
    double ops_per = which == 0 ? 2.0 * 32 * 32 * 32 : (which == 1 ? 2.0 * 32 * 32 * 64 : 2.0 * 32 * 32 * 16);
    auto launch = [&]() {
        if (which == 0) hipLaunchKernelGGL(peak_i8, dim3(blocks), dim3(threads), 0, s, sink, iters);
        else if (which == 1) hipLaunchKernelGGL(peak_f8, dim3(blocks), dim3(threads), 0, s, sink, iters);
        else hipLaunchKernelGGL(peak_bf16, dim3(blocks), dim3(threads), 0, s, sink, iters);
    };
    hipEvent_t a = nullptr, z = nullptr;
    float best = 1e30f;
    e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&z);
    if (e == hipSuccess) {
        launch();  // warm-up
        for (int r = 0; r < 5 && e == hipSuccess; r++) {
            e = hipEventRecord(a, s);
            launch();
            if (e == hipSuccess) e = hipEventRecord(z, s);
            if (e == hipSuccess) e = hipEventSynchronize(z);
            float ms = 0.f;
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, z);
            if (e == hipSuccess && ms < best) best = ms;
        }
    }
    if (e == hipSuccess) e = hipGetLastError();
    if (a) (void)hipEventDestroy(a);
    if (z) (void)hipEventDestroy(z);
    (void)hipFree(sink);
    if (e != hipSuccess) return e;
    const double mfmas = (double)blocks * threads / 64.0 * iters * PEAK_CHAINS;
    *tops = mfmas * ops_per / (best * 1e-3) / 1e12;
    return hipSuccess;
}

}  // namespace sage
