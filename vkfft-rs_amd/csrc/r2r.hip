// r2r.hip -- DCT / DST types I-IV (FFTW REDFT00/10/01/11, RODFT00/10/01/11,
// the definitions of src/r2r_ir.rs:2351-2434) as one complex FFT of length L
// between a pre pass and a post pass, with the FFT lengths of the reference's
// reductions (r2r_ir.rs:76-110):
//
// R2R_EXTEND (types I, odd IV; L = 2(N-1), 2(N+1) or 2N):
//   a[m] = w(m) x[m - off] exp(-i pi m ph / (2N)),  m - off in [0, N), else 0
//   X[k] = s * sel( exp(-i pi (k + q) pq / (2N)) A[k + r] ),  A = FFT_L(a)
//   with sel = Re or -Im.
// R2R_REORDER (DCT-II, L = N; Makhoul): v[m] = x[p(m)] with p(m) = 2m for
//   m < ceil(N/2), else 2(N-1-m)+1; X[k] = 2 s Re(exp(-i pi k/(2N)) V[k]).
//   DST-II (flip): x[j] -> (-1)^j x[j] and X[k] taken at N-1-k.
// R2R_SPECTRUM (DCT-III, L = N, inverse FFT): V[j] = exp(i pi j/(2N))
//   (x[j] - i x[N-j]), x[N] = 0; X[p(m)] = s Re(v[m]). DST-III (flip):
//   x reversed on input, X[k] times (-1)^k.
// R2R_HALF (even DCT-IV, L = N/2): z[j] = (x[2j] + i x[N-1-2j])
//   exp(-i pi (4j+1)/(4N)); u[j] = exp(-i pi j/N) Z[j]; X[2j] = 2 s Re u[j],
//   X[N-1-2j] = -2 s Im u[j]. DST-IV (flip): x reversed, X[k] times (-1)^k.
//
// Lines of a strided axis (N-D transforms) are read and written in place
// with element stride `inner`. The per-type parameters are set by plan_r2r
// (runtime.cpp).
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

// Makhoul's reordering: element p(m) of the line lands at m.
__device__ __forceinline__ long long makhoul_src(long long m, long long n) {
    return m < (n + 1) / 2 ? 2 * m : 2 * (n - 1 - m) + 1;
}
// Its inverse: where element j sits after the reordering.
__device__ __forceinline__ long long makhoul_pos(long long j, long long n) {
    return (j & 1) ? n - 1 - (j >> 1) : (j >> 1);
}

template <typename T>
__device__ __forceinline__ void r2r_pre_short(const T* __restrict__ x, T* __restrict__ a, const R2rArgs& p,
                                              long long i, long long b, long long m) {
    const long long bo = b / p.inner, bc = b - bo * p.inner;
    const T* line = x + bo * p.n * p.inner + bc;
    const long long n = p.n;
    auto at = [&](long long j) -> double {  // element j of the line, reversed for the DST forms
        if (j < 0 || j >= n) return 0.0;
        return (double)line[(p.flip ? n - 1 - j : j) * p.inner];
    };
    double re = 0.0, im = 0.0;
    if (p.op == R2R_REORDER) {
        const long long j = makhoul_src(m, n);
        re = (double)line[j * p.inner];
        if (p.flip && (j & 1)) re = -re;
    } else if (p.op == R2R_SPECTRUM) {
        const double u = at(m), v = m == 0 ? 0.0 : at(n - m);
        double sn, cs;
        sincospi((double)m / (2.0 * (double)n), &sn, &cs);  // exp(+i pi m / (2N))
        re = u * cs + v * sn;
        im = u * sn - v * cs;
    } else {  // R2R_HALF
        const double u = at(2 * m), v = at(n - 1 - 2 * m);
        double sn, cs;
        sincospi((double)(4 * m + 1) / (4.0 * (double)n), &sn, &cs);  // exp(-i pi (4m+1)/(4N))
        re = u * cs + v * sn;
        im = v * cs - u * sn;
    }
    a[2 * i] = (T)re;
    a[2 * i + 1] = (T)im;
}

template <typename T>
__device__ __forceinline__ void r2r_post_short(const T* __restrict__ A, T* __restrict__ X, const R2rArgs& p,
                                               long long b, long long k) {
    const long long n = p.n;
    const T* line = A + 2 * b * p.L;
    double out;
    if (p.op == R2R_REORDER) {
        const long long kk = p.flip ? n - 1 - k : k;
        double sn, cs;
        sincospi((double)kk / (2.0 * (double)n), &sn, &cs);  // exp(-i pi kk / (2N)) = cs - i sn
        out = 2.0 * ((double)line[2 * kk] * cs + (double)line[2 * kk + 1] * sn);
    } else if (p.op == R2R_SPECTRUM) {
        out = (double)line[2 * makhoul_pos(k, n)];
        if (p.flip && (k & 1)) out = -out;
    } else {  // R2R_HALF
        const bool even = (k & 1) == 0;
        const long long j = even ? k >> 1 : (n - 1 - k) >> 1;
        double sn, cs;
        sincospi((double)j / (double)n, &sn, &cs);  // exp(-i pi j / N) = cs - i sn
        const double zr = (double)line[2 * j], zi = (double)line[2 * j + 1];
        out = even ? 2.0 * (zr * cs + zi * sn) : -2.0 * (zi * cs - zr * sn);
        if (p.flip && (k & 1)) out = -out;
    }
    const long long bo = b / p.inner, bc = b - bo * p.inner;
    X[bo * n * p.inner + bc + k * p.inner] = (T)(p.s * out);
}

template <typename T>
__global__ __launch_bounds__(256) void k_r2r_pre(const T* __restrict__ x, T* __restrict__ a, const R2rArgs p) {
    const long long total = p.L * p.batch;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long b = i / p.L, m = i - b * p.L;
        if (p.op != R2R_EXTEND) {
            r2r_pre_short(x, a, p, i, b, m);
            continue;
        }
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
        if (p.op != R2R_EXTEND) {
            r2r_post_short(A, X, p, b, k);
            continue;
        }
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
