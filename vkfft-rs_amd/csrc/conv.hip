// conv.hip -- frequency-domain multiply of VkFFT's performConvolution
// (ConvolutionIr / NdConvolutionIr, src/convolution_ir.rs:4252-4344): data
// [system][coordinate][t], kernel spectrum [kernel][plane][t]. Per output
// (system s, coordinate o, t), with s_in = kernel_count > 1 ? 0 : s and
// kid = kernel_count > 1 ? s : 0:
//   matrix M x M:  y = sum_i prep(X[s_in][i][t]) K[kid][plane(o, i)][t]
//   independent:   y = prep(X[s_in][o][t]) K[kid][o][t]
//   otherwise:     y = prep(X[s_in][o][t]) K[kid][0][t]
// prep = conj for ConvolutionConjugation::Sequence; y / |y| with the
// cross-power-spectrum normalization (no zero guard, as upstream).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace vkfx {

__device__ __forceinline__ long long plane_index(int m, bool sym, int o, int i) {
    if (!sym) return (long long)o * m + i;
    // ConvolutionMatrixLayout::kernel_plane_index (convolution_ir.rs:128-147)
    return i < o ? (long long)i * m - i * i + o : (long long)o * m - o * o + i;
}

template <typename T>
__global__ __launch_bounds__(256) void k_conv(const T* __restrict__ X, const T* __restrict__ K, T* __restrict__ Y,
                                              const ConvArgs a) {
    const long long total = a.T * a.coords * a.systems_out;
    for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * blockDim.x) {
        const long long t = idx % a.T;
        const long long so = idx / a.T;  // s * coords + o
        const int o = (int)(so % a.coords);
        const long long s = so / a.coords;
        const long long s_in = a.kernel_count > 1 ? 0 : s;
        const long long kid = a.kernel_count > 1 ? s : 0;
        double re = 0.0, im = 0.0;
        const int terms = a.matrix ? a.matrix : 1;
        for (int i = 0; i < terms; ++i) {
            const int ci = a.matrix ? i : o;
            const long long plane = a.matrix ? plane_index(a.matrix, a.symmetric, o, i) : (a.independent ? o : 0);
            const long long xo = ((s_in * a.coords + ci) * a.T + t) * 2;
            const long long ko = ((kid * a.planes + plane) * a.T + t) * 2;
            const double xr = (double)X[xo], xi = a.conj_seq ? -(double)X[xo + 1] : (double)X[xo + 1];
            const double kr = (double)K[ko], ki = (double)K[ko + 1];
            re += xr * kr - xi * ki;
            im += xr * ki + xi * kr;
        }
        if (a.cross_norm) {
            const double r = 1.0 / sqrt(re * re + im * im);
            re *= r;
            im *= r;
        }
        Y[idx * 2] = (T)re;
        Y[idx * 2 + 1] = (T)im;
    }
}

const void* conv_kernel_fn(int prec) { return prec ? (const void*)k_conv<double> : (const void*)k_conv<float>; }

int launch_conv(int prec, const ConvArgs& a, const void* x, const void* k, void* y, hipStream_t s) {
    const long long total = a.T * a.coords * a.systems_out;
    if (total <= 0 || a.coords < 1 || a.planes < 1) return (int)hipErrorInvalidValue;
    const long long blocks = (total + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
    if (prec)
        hipLaunchKernelGGL((k_conv<double>), dim3(grid), dim3(256), 0, s, (const double*)x, (const double*)k,
                           (double*)y, a);
    else
        hipLaunchKernelGGL((k_conv<float>), dim3(grid), dim3(256), 0, s, (const float*)x, (const float*)k, (float*)y,
                           a);
    return (int)hipGetLastError();
}

}  // namespace vkfx
