// launch.hip -- dispatches a KernelKind to its instantiation and launches it.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace vkfx {

using KernelFn = void (*)(const KArgs);
KernelFn pick_f32_fwd(KernelKind kind);
KernelFn pick_f32_inv(KernelKind kind);
KernelFn pick_f64_fwd(KernelKind kind);
KernelFn pick_f64_inv(KernelKind kind);

static int lds_limit_bytes() {
    static int cached = -1;
    if (cached < 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
            cached = v;
        else
            cached = 65536;
    }
    return cached;
}

size_t max_lds_bytes() { return (size_t)lds_limit_bytes(); }

int launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned grid, unsigned block, size_t lds_bytes,
           hipStream_t stream) {
    if (kind < 0 || kind >= KK_COUNT || (dir != -1 && dir != 1) || (prec != 0 && prec != 1))
        return (int)hipErrorInvalidValue;
    if (grid == 0) return (int)hipSuccess;
    if (block == 0 || block > 512 || a.G < 1 || a.G > kMaxLinesPerBlock || (unsigned)(a.G * a.TT) != block)
        return (int)hipErrorInvalidConfiguration;
    if (a.nstages < 0 || a.nstages > kMaxStages) return (int)hipErrorInvalidValue;
    if (lds_bytes < (size_t)a.G * (size_t)a.LS * (prec ? 16 : 8) || lds_bytes > (size_t)lds_limit_bytes())
        return (int)hipErrorInvalidConfiguration;
    KernelFn fn = prec == 0 ? (dir < 0 ? pick_f32_fwd(kind) : pick_f32_inv(kind))
                            : (dir < 0 ? pick_f64_fwd(kind) : pick_f64_inv(kind));
    if (!fn) return (int)hipErrorInvalidValue;
    if (lds_bytes > 65536) {
        hipError_t e =
            hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(fn, dim3(grid), dim3(block), lds_bytes, stream, a);
    return (int)hipGetLastError();
}

}  // namespace vkfx
