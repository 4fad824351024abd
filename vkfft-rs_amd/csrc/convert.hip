// convert.hip -- element-type conversion passes for mixed storage/compute
// precisions (Precision::F16StorageF32Compute and F64ComputeF32Storage,
// src/config.rs:108-145): the caller's buffers hold the storage type, the FFT
// passes run on the compute type in the plan's workspace.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace vkfx {

template <typename S, typename D>
__global__ __launch_bounds__(256) void k_convert(const S* __restrict__ in, D* __restrict__ out, long long n) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (; i < n; i += stride) out[i] = (D)in[i];
}

template <typename S, typename D>
static int go(const void* in, void* out, long long n, hipStream_t s) {
    const long long blocks = (n + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
    hipLaunchKernelGGL((k_convert<S, D>), dim3(grid), dim3(256), 0, s, (const S*)in, (D*)out, n);
    return (int)hipGetLastError();
}

// Scalar type codes: 0 = binary16 (round to nearest even), 1 = f32, 2 = f64.
int launch_convert(int src, int dst, const void* in, void* out, long long n, hipStream_t s) {
    if (n <= 0) return (int)hipSuccess;
    if (src == 0 && dst == 1) return go<_Float16, float>(in, out, n, s);
    if (src == 1 && dst == 0) return go<float, _Float16>(in, out, n, s);
    if (src == 1 && dst == 2) return go<float, double>(in, out, n, s);
    if (src == 2 && dst == 1) return go<double, float>(in, out, n, s);
    return (int)hipErrorInvalidValue;
}

}  // namespace vkfx
