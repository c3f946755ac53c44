// The layer entry for callers that cannot allocate device memory (code under
// graph capture, serving loops that forbid hipMalloc): the workspace of
// glmmoe_moe_layer_w4a16 is a file-scope device array of kScratchBytes, one
// copy per GPU, held until the process ends. Contract: include/glmmoe.h.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/glmmoe.h"

namespace {

constexpr size_t kScratchBytes = (size_t)32 << 20;
constexpr int kMaxDevices = 64;

// Device-side storage. In host code `scratch` names a host-side stand-in, not
// the device address: kernels get the per-device address from
// hipGetSymbolAddress below.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices];   // scratch's address on each device (null: not looked up yet)

// scratch's address on the current device, looked up once per device.
int scratch_ptr(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GLMMOE_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return GLMMOE_ERR_LAUNCH;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return GLMMOE_OK;
}

}  // namespace

size_t glmmoe_noalloc_scratch_bytes(void) { return kScratchBytes; }

int glmmoe_moe_layer_w4a16_noalloc(const glmmoe_w4a16_layer* L, const uint16_t* x, int n,
                                   float* out, void* stream) {
    // Shape and size first: no device call for a batch that cannot fit.
    const size_t need = glmmoe_layer_workspace_bytes(L, n);
    if (need == 0) return GLMMOE_ERR_ARG;
    if (need > kScratchBytes) return GLMMOE_ERR_WORKSPACE;
    if (n == 0) return GLMMOE_OK;   // no tokens: nothing to compute or write
    void* ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc) return rc;
    // Every field of the workspace is written by the call before it is read
    // (the expert kernels' tickets are cleared by its router or dispatch
    // kernel), so the previous call's contents do not matter.
    return glmmoe_moe_layer_w4a16(L, x, n, out, ws, kScratchBytes, stream);
}
