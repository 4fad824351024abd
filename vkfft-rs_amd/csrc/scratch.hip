// Static device scratch of vkfx_execute_noalloc: a file-scope device array
// that stands in for a plan's workspace, so that entry point allocates
// nothing. Every GPU the library runs on holds its own copy of the array
// (kStaticScratchBytes) until the process ends.
//
// In host code `scratch` names a host-side shadow, not device memory: host
// code only ever uses the address hipGetSymbolAddress returns for the
// current device, obtained once per device below.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.hpp"

namespace vkfx {

namespace {

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
bool g_scratch_done[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};

}  // namespace

// Device address of `device`'s copy of the scratch array. The first call for
// a device must run with that device current (vkfx_context_create does);
// later calls return the cached address or the cached error.
hipError_t static_scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_done[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_err[device] = e;
        g_scratch_ptr[device] = e == hipSuccess ? p : nullptr;
        g_scratch_done[device] = true;
    }
    *out = g_scratch_ptr[device];
    return g_scratch_err[device];
}

}  // namespace vkfx
