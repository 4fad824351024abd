// r2r.hip -- DCT / DST types I-IV (FFTW REDFT00/10/01/11, RODFT00/10/01/11,
// the definitions of src/r2r_ir.rs:2351-2434) as one complex FFT of length L
// between a pre pass and a post pass:
//   a[m] = w(m) x[m - off] exp(-i pi m ph / (2N)),  m - off in [0, N), else 0
//   X[k] = s * sel( exp(-i pi (k + q) pq / (2N)) A[k + r] ),  A = FFT_L(a)
// with sel = Re or -Im. Lines of a strided axis (N-D transforms) are read
// and written in place with element stride `inner`. The per-type parameters (runtime.cpp, r2r_params)
// follow from writing each cosine / sine sum as the real or imaginary part
// of a zero-padded DFT.
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace vkfx {

__device__ __forceinline__ void phase(double num, double den, double* c, double* s) {
    // exp(-i pi num / den)
    double sn, cs;
    sincospi(num / den, &sn, &cs);
    *c = cs;
    *s = -sn;
}

template <typename T>
__global__ __launch_bounds__(256) void k_r2r_pre(const T* __restrict__ x, T* __restrict__ a, const R2rArgs p) {
    const long long total = p.L * p.batch;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long b = i / p.L, m = i - b * p.L;
        const long long j = m - p.off;
        // line b of the axis: element j at (b / inner) * n * inner + b % inner + j * inner
        const long long bo = b / p.inner, bc = b - bo * p.inner;
        double re = 0.0, im = 0.0;
        if (j >= 0 && j < p.n) {
            double w = 1.0;
            if (p.wmode == 1) w = (j == 0 || j == p.n - 1) ? 1.0 : 2.0;      // DCT-I
            else if (p.wmode == 2) w = j == 0 ? 1.0 : 2.0;                    // DCT-III
            else if (p.wmode == 3) w = m == p.n ? 1.0 : 2.0;                  // DST-III
            const double v = w * (double)x[bo * p.n * p.inner + bc + j * p.inner];
            if (p.ph) {
                double c, s;
                phase((double)m, 2.0 * (double)p.n, &c, &s);
                re = v * c;
                im = v * s;
            } else {
                re = v;
            }
        }
        a[2 * i] = (T)re;
        a[2 * i + 1] = (T)im;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_r2r_post(const T* __restrict__ A, T* __restrict__ X, const R2rArgs p) {
    const long long total = p.n * p.batch;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long b = i / p.n, k = i - b * p.n;
        const long long src = b * p.L + k + p.r;
        double re = (double)A[2 * src], im = (double)A[2 * src + 1];
        if (p.pq) {
            double c, s;
            phase((double)k + 0.5 * (double)p.q2, 2.0 * (double)p.n, &c, &s);
            const double r2 = re * c - im * s, i2 = re * s + im * c;
            re = r2;
            im = i2;
        }
        const long long bo = b / p.inner, bc = b - bo * p.inner;
        X[bo * p.n * p.inner + bc + k * p.inner] = (T)(p.s * (p.im ? -im : re));
    }
}

template <typename T>
static int go(bool pre, const R2rArgs& p, const void* in, void* out, hipStream_t s) {
    const long long total = pre ? p.L * p.batch : p.n * p.batch;
    const long long blocks = (total + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
    if (pre)
        hipLaunchKernelGGL((k_r2r_pre<T>), dim3(grid), dim3(256), 0, s, (const T*)in, (T*)out, p);
    else
        hipLaunchKernelGGL((k_r2r_post<T>), dim3(grid), dim3(256), 0, s, (const T*)in, (T*)out, p);
    return (int)hipGetLastError();
}

const void* r2r_kernel_fn(bool pre, int prec) {
    if (prec) return pre ? (const void*)k_r2r_pre<double> : (const void*)k_r2r_post<double>;
    return pre ? (const void*)k_r2r_pre<float> : (const void*)k_r2r_post<float>;
}

int launch_r2r(bool pre, int prec, const R2rArgs& p, const void* in, void* out, hipStream_t s) {
    if (p.n <= 0 || p.L <= 0 || p.batch <= 0 || p.inner <= 0 || p.batch % p.inner) return (int)hipErrorInvalidValue;
    return prec ? go<double>(pre, p, in, out, s) : go<float>(pre, p, in, out, s);
}

}  // namespace vkfx
