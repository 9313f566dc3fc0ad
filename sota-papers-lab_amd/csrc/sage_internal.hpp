// Host-side declarations shared by the kernel launchers and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sage {

struct Geom;

// Device buffers the prologue writes (a workspace's view).
struct PrologueBufs {
    int8_t* q8;
    float* q_scale;
    int8_t* k8;
    float* k_scale;
    uint8_t* v8;
    float* stats;
    float* part;
    float* kbias;  // [tk_pad]: log2 member count of each merged key, -inf past tk (merged plans)
};

// The attention kernel's inputs.
struct AttendBufs {
    const int8_t* q8;
    const float* q_scale;
    const int8_t* k8;
    const float* k_scale;
    const uint8_t* v8;
    const float* stats;
    const float* kbias;  // merged plans only
    void* out;
};

// ln: [4][head_dim] QK LayerNorm parameters (q weight, q bias, k weight,
// k bias), read only under F_LN_Q / F_LN_K; may be null otherwise.
hipError_t launch_prologue(int head_dim, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ln,
                           const PrologueBufs& w, const Geom& g, hipStream_t s);

// Rows of queries one attention workgroup owns.
constexpr int ATTN_ROWS = 128;

hipError_t launch_attention(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s);

// Kernel resources (VGPRs, scratch, LDS) of the attention kernel for
// head_dim: dense, causal or KV-merged.
hipError_t attention_resources(int head_dim, bool causal, bool merge, int* regs, int* spill, int* lds);

// MFMA peak probe: which 0 = INT8, 1 = FP8, 2 = BF16; returns dense TOPS.
hipError_t run_peak(int which, int iters, hipStream_t s, double* tops);

}  // namespace sage
