// The no-allocation forward: sage_forward's prologue and attention kernels
// on buffers carved from one file-scope device array instead of a
// workspace, for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The array `scratch` (SAGE_NOALLOC_MAX_BYTES) exists once on every GPU the
// library is loaded on, from the code object's load until the process ends.
// Its device address is looked up with hipGetSymbolAddress once per device,
// with that device current, when a context is created there (sage_new), and
// only that address is handed to kernels: in host code `scratch` names a
// host-side stand-in, not device memory.
//
// Every call on one GPU shares that GPU's array and leaves its contents
// behind. The prologue writes every element the attention kernel reads
// (padded query rows and key blocks included), so nothing needs clearing
// between calls; but calls whose kernels overlap on one GPU (different
// streams, no ordering between them) race on the array.
#include <mutex>
#include <vector>

#include "../../include/sage_hip.h"
#include "sage_device.hpp"
#include "sage_internal.hpp"

namespace {

static __device__ __align__(256) uint8_t scratch[SAGE_NOALLOC_MAX_BYTES];

std::mutex g_mu;
std::vector<void*> g_scratch;  // device address of `scratch`, per device ordinal

// The device address of `scratch` on `device`, as sage_new resolved it. The
// entry point itself makes no HIP runtime call besides its kernel launches,
// so a caller can capture even its first call on a device in a graph.
sage_status scratch_address(int device, void** out) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (device >= 0 && (size_t)device < g_scratch.size() && g_scratch[device]) {
        *out = g_scratch[device];
        return SAGE_OK;
    }
    return sage::set_error(SAGE_ERR_STATE, "no-allocation scratch of device %d was not resolved (sage_new does it)",
                           device);
}

uint64_t round256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

}  // namespace

namespace sage {

// Looks up `scratch`'s device address on `device`, which must be the current
// device (sage_new calls it with the context's device current), once per
// device; later calls find it cached.
sage_status noalloc_init(int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (device < 0) return set_error(SAGE_ERR_DEVICE, "no HIP device %d", device);
    if ((size_t)device < g_scratch.size() && g_scratch[device]) return SAGE_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_error(SAGE_ERR_DEVICE, "no-allocation scratch address on device %d: %s (%s)", device,
                         hipGetErrorName(e), hipGetErrorString(e));
    if ((size_t)device >= g_scratch.size()) g_scratch.resize((size_t)device + 1, nullptr);
    g_scratch[device] = p;
    return SAGE_OK;
}

}  // namespace sage

extern "C" sage_status sage_forward_noalloc(const sage_attention* s, const sage_shape* shape,
                                            const sage_kv_merge* merge, const sage_tensor* q, const sage_tensor* k,
                                            const sage_tensor* v, const sage_tensor_mut* out,
                                            const sage_options* opts) {
    if (!s || !shape || !q || !k || !v || !out || !opts)
        return sage::set_error(SAGE_ERR_INVALID, "null argument");
    sage_plan plan;
    sage::WsSizes n;
    sage_status st = sage::workspace_layout(s, shape, merge, &plan, &n);
    if (st != SAGE_OK) return st;
    // Byte sizes in carving order, each buffer starting on a 256-byte boundary.
    const uint64_t bytes[8] = {n.q8, 4 * n.q_scale, n.k8, 4 * n.k_scale, n.v8, 4 * n.stats, 4 * n.kbias, 4 * n.part};
    uint64_t need = 0;
    for (uint64_t b : bytes) need += round256(b);
    if (need > SAGE_NOALLOC_MAX_BYTES)
        return sage::set_error(SAGE_ERR_INVALID,
                               "sage_forward_noalloc needs %llu bytes of scratch for this shape, more than its "
                               "maximum of %llu; use a workspace (sage_workspace_new)",
                               (unsigned long long)need, (unsigned long long)SAGE_NOALLOC_MAX_BYTES);
    void* base = nullptr;
    st = scratch_address(s->device, &base);
    if (st != SAGE_OK) return st;
    uint8_t* p = static_cast<uint8_t*>(base);
    void* buf[8];
    for (int i = 0; i < 8; i++) {
        buf[i] = p;
        p += round256(bytes[i]);
    }
    const sage::WsView w{plan,
                         static_cast<int8_t*>(buf[0]),
                         static_cast<float*>(buf[1]),
                         static_cast<int8_t*>(buf[2]),
                         static_cast<float*>(buf[3]),
                         static_cast<uint8_t*>(buf[4]),
                         static_cast<float*>(buf[5]),
                         static_cast<float*>(buf[6]),
                         static_cast<float*>(buf[7])};
    sage::Geom g;
    st = sage::prepare_view(s, w, q, k, v, opts, &g, nullptr);
    if (st != SAGE_OK) return st;
    st = sage::attend_view(s, w, g, out);
    if (st != SAGE_OK) return st;
    sage::set_error(SAGE_OK, "%s", "");
    return SAGE_OK;
}
