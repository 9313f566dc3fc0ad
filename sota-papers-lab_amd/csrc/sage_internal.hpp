// Host-side declarations shared by the kernel launchers and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sage_hip.h"

// SageAttention (mod.rs:509-520): the context behind the C ABI's handle.
struct sage_attention {
    hipStream_t stream;
    int device;
    uint64_t head_dim;
    sage_config config;
};

namespace sage {

struct Geom;
struct QkvDev;
struct QkvOutDev;

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
// qa: the QKV prologue's options when q, k and v point into a fused QKV
// projection (sage_prepare_qkv), or null for plain 16-bit inputs.
hipError_t launch_prologue(int head_dim, const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* ln,
                           const PrologueBufs& w, const Geom& g, const QkvDev* qa, hipStream_t s);

// The reference's qkv_prologue on its own (QkvPrologue::run): the fused
// projection y (strides g.q_sb, g.q_st) to 16-bit Q, K and V rows.
hipError_t launch_qkv(int head_dim, const uint16_t* y, const QkvOutDev& o, const Geom& g, const QkvDev& qa,
                      hipStream_t s);

// Rows of queries one attention workgroup owns.
constexpr int ATTN_ROWS = 128;

hipError_t launch_attention(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s);
// The merged kernels' launch, from the second compilation of the attention
// source (launch_attention calls it for merged plans).
hipError_t launch_attention_merged(int head_dim, const AttendBufs& w, const Geom& g, hipStream_t s);

// Kernel resources (VGPRs, scratch, LDS) of the attention kernel for
// head_dim: dense, causal or KV-merged; waves8 = the eight-wave layout that
// Tile { warps: 8 } selects for dense and causal attention.
hipError_t attention_resources(int head_dim, bool causal, bool merge, bool waves8, int* regs, int* spill, int* lds);
hipError_t attention_resources_merged(int head_dim, int* regs, int* spill, int* lds);

// MFMA peak probe: which 0 = INT8, 1 = FP8, 2 = BF16; returns dense TOPS.
hipError_t run_peak(int which, int iters, hipStream_t s, double* tops);

// Element counts of a workspace's buffers.
struct WsSizes {
    uint64_t q8, q_scale, k8, k_scale, v8, stats, kbias, part;
};

// A workspace's buffers: owned by a sage_workspace, or carved from the
// no-allocation entry point's scratch array.
struct WsView {
    sage_plan plan;
    int8_t* q8;
    float* q_scale;
    int8_t* k8;
    float* k_scale;
    uint8_t* v8;
    float* stats;
    float* kbias;
    float* part;
};

// Resolves the no-allocation entry point's scratch array on `device`, the
// current device (once per device; sage_new calls it).
sage_status noalloc_init(int device);

// Sets this thread's sage_last_error() text; returns st.
sage_status set_error(sage_status st, const char* fmt, ...);

// Plan::new plus the buffer sizes of SageAttention::workspace for shape and
// merge (NULL = dense), with the same refusals.
sage_status workspace_layout(const sage_attention* s, const sage_shape* shape, const sage_kv_merge* merge,
                             sage_plan* plan, WsSizes* n);

// The bodies of prepare and attend on a buffer view: every check before any
// launch, then the launches on s->stream. prepare_view returns the kernel
// parameters attend_view needs.
// qa: the QKV prologue's options when q, k and v are views into a fused
// QKV projection (sage_prepare_qkv), or null.
sage_status prepare_view(const sage_attention* s, const WsView& w, const sage_tensor* q, const sage_tensor* k,
                         const sage_tensor* v, const sage_options* opts, Geom* geom, const QkvDev* qa);
sage_status attend_view(const sage_attention* s, const WsView& w, const Geom& geom, const sage_tensor_mut* out);

}  // namespace sage
