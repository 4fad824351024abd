// fft_device.hpp -- complex arithmetic, DFT butterflies and the LDS-resident
// Stockham stage used by every gfx950 kernel in this library.
//
// Stage semantics follow vkfft-rs's Stockham definition
// (src/kernel_ir.rs:4565-4608, docs/KERNEL_IR.md:20-37): for a stage of radix
// R whose previous radices multiply to P, butterfly b (0 <= b < N/R) reads
// in(i) = b + i*N/R, multiplies input i by exp(s*2*pi*i*j*i/(P*R)) with
// j = b mod P, runs a length-R DFT and writes out(q) = j + (b-j)*R + q*P.
// After the last stage the sequence is in natural order.
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "radix_constants.hpp"

namespace vkfx {

// Index-map test build (make VARIANT=index, -DVKFX_INDEX_TEST): every
// butterfly, twiddle, chirp, spectrum and scale multiplication is the
// identity, so a C2C kernel only moves data and its output is a permutation
// (plus the zero fill of Bluestein padding) of its input, compared bit for
// bit with the CPU index maps.
#ifdef VKFX_INDEX_TEST
constexpr bool kIndexTest = true;
#else
constexpr bool kIndexTest = false;
#endif

template <typename T>
struct alignas(2 * sizeof(T)) cpx {
    T re, im;
};

template <typename T>
__device__ __forceinline__ cpx<T> mk(T r, T i) {
    cpx<T> v;
    v.re = r;
    v.im = i;
    return v;
}
template <typename T>
__device__ __forceinline__ cpx<T> operator+(cpx<T> a, cpx<T> b) {
    return mk(a.re + b.re, a.im + b.im);
}
template <typename T>
__device__ __forceinline__ cpx<T> operator-(cpx<T> a, cpx<T> b) {
    return mk(a.re - b.re, a.im - b.im);
}
template <typename T>
__device__ __forceinline__ cpx<T> cmul(cpx<T> a, cpx<T> b) {
    if constexpr (kIndexTest) return a;
    return mk(a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re);
}
// a * conj(b)
template <typename T>
__device__ __forceinline__ cpx<T> cmulc(cpx<T> a, cpx<T> b) {
    if constexpr (kIndexTest) return a;
    return mk(a.re * b.re + a.im * b.im, a.im * b.re - a.re * b.im);
}
template <typename T>
__device__ __forceinline__ cpx<T> conj(cpx<T> a) {
    return mk(a.re, -a.im);
}
template <typename T>
__device__ __forceinline__ cpx<T> scale(cpx<T> a, T s) {
    if constexpr (kIndexTest) return a;
    return mk(a.re * s, a.im * s);
}
// (S * i) * a, S = +-1
template <int S, typename T>
__device__ __forceinline__ cpx<T> muli(cpx<T> a) {
    return S > 0 ? mk(-a.im, a.re) : mk(a.im, -a.re);
}
// Twiddle tables hold forward roots exp(-2*pi*i*k/N); the inverse direction
// (S = +1) uses their conjugates.
template <int S, typename T>
__device__ __forceinline__ cpx<T> twmul(cpx<T> a, cpx<T> w) {
    return S < 0 ? cmul(a, w) : cmulc(a, w);
}

// ------------------------------------------------------------- butterflies
// All butterflies compute X[q] = sum_i x[i] * exp(S*2*pi*i*i*q/R) in place.

template <int S, typename T>
__device__ __forceinline__ void dft2(cpx<T>* x) {
    cpx<T> a = x[0];
    x[0] = a + x[1];
    x[1] = a - x[1];
}

template <int S, typename T>
__device__ __forceinline__ void dft4(cpx<T>& x0, cpx<T>& x1, cpx<T>& x2, cpx<T>& x3) {
    cpx<T> t0 = x0 + x2, t1 = x0 - x2, t2 = x1 + x3, t3 = muli<S>(x1 - x3);
    x0 = t0 + t2;
    x2 = t0 - t2;
    x1 = t1 + t3;
    x3 = t1 - t3;
}

template <int S, typename T>
__device__ __forceinline__ void dft8(cpx<T>* x) {
    cpx<T> e0 = x[0], e1 = x[2], e2 = x[4], e3 = x[6];
    cpx<T> o0 = x[1], o1 = x[3], o2 = x[5], o3 = x[7];
    dft4<S>(e0, e1, e2, e3);
    dft4<S>(o0, o1, o2, o3);
    const T c = (T)0.707106781186547524400844362104849039;
    // o1 *= exp(S*i*pi/4), o2 *= S*i, o3 *= exp(S*3*i*pi/4)
    o1 = S < 0 ? mk(c * (o1.re + o1.im), c * (o1.im - o1.re)) : mk(c * (o1.re - o1.im), c * (o1.im + o1.re));
    o2 = muli<S>(o2);
    o3 = S < 0 ? mk(c * (o3.im - o3.re), -c * (o3.re + o3.im)) : mk(-c * (o3.re + o3.im), c * (o3.re - o3.im));
    x[0] = e0 + o0;
    x[4] = e0 - o0;
    x[1] = e1 + o1;
    x[5] = e1 - o1;
    x[2] = e2 + o2;
    x[6] = e2 - o2;
    x[3] = e3 + o3;
    x[7] = e3 - o3;
}

template <int S, typename T>
__device__ __forceinline__ void dft16(cpx<T>* x) {
    cpx<T> e[8], o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        e[i] = x[2 * i];
        o[i] = x[2 * i + 1];
    }
    dft8<S>(e);
    dft8<S>(o);
    // cos/sin(pi*q/8), q = 0..7
    const T C[8] = {(T)1.0,
                    (T)0.923879532511286756128183189396788933,
                    (T)0.707106781186547524400844362104849039,
                    (T)0.382683432365089771728459984030398866,
                    (T)0.0,
                    (T)-0.382683432365089771728459984030398866,
                    (T)-0.707106781186547524400844362104849039,
                    (T)-0.923879532511286756128183189396788933};
    const T Sn[8] = {(T)0.0,
                     (T)0.382683432365089771728459984030398866,
                     (T)0.707106781186547524400844362104849039,
                     (T)0.923879532511286756128183189396788933,
                     (T)1.0,
                     (T)0.923879532511286756128183189396788933,
                     (T)0.707106781186547524400844362104849039,
                     (T)0.382683432365089771728459984030398866};
#pragma unroll
    for (int q = 1; q < 8; ++q) {
        if (q == 4) {
            o[q] = muli<S>(o[q]);
        } else {
            cpx<T> w = mk(C[q], (T)S * Sn[q]);
            o[q] = cmul(o[q], w);
        }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        x[q] = e[q] + o[q];
        x[q + 8] = e[q] - o[q];
    }
}

template <int R>
struct OddTables;
template <>
struct OddTables<3> {
    static __device__ __forceinline__ double c(int j) { return kCos3[j]; }
    static __device__ __forceinline__ double s(int j) { return kSin3[j]; }
};
template <>
struct OddTables<5> {
    static __device__ __forceinline__ double c(int j) { return kCos5[j]; }
    static __device__ __forceinline__ double s(int j) { return kSin5[j]; }
};
template <>
struct OddTables<7> {
    static __device__ __forceinline__ double c(int j) { return kCos7[j]; }
    static __device__ __forceinline__ double s(int j) { return kSin7[j]; }
};
template <>
struct OddTables<11> {
    static __device__ __forceinline__ double c(int j) { return kCos11[j]; }
    static __device__ __forceinline__ double s(int j) { return kSin11[j]; }
};
template <>
struct OddTables<13> {
    static __device__ __forceinline__ double c(int j) { return kCos13[j]; }
    static __device__ __forceinline__ double s(int j) { return kSin13[j]; }
};

// Odd prime R: pair x[m] with x[R-m]; X[q] and X[R-q] share the cosine sum
// and differ in the sign of the (S*i)-rotated sine sum.
template <int R, int S, typename T>
__device__ __forceinline__ void dft_odd(cpx<T>* x) {
    constexpr int H = (R - 1) / 2;
    cpx<T> a[H], b[H];
#pragma unroll
    for (int m = 1; m <= H; ++m) {
        a[m - 1] = x[m] + x[R - m];
        b[m - 1] = x[m] - x[R - m];
    }
    cpx<T> x0 = x[0];
    cpx<T> y0 = x0;
#pragma unroll
    for (int m = 0; m < H; ++m) y0 = y0 + a[m];
    cpx<T> out[R];
    out[0] = y0;
#pragma unroll
    for (int q = 1; q <= H; ++q) {
        cpx<T> A = x0;
        cpx<T> B = mk((T)0, (T)0);
#pragma unroll
        for (int m = 1; m <= H; ++m) {
            const int j = (m * q) % R;
            const T cj = (T)OddTables<R>::c(j);
            const T sj = (T)OddTables<R>::s(j);
            A = mk(A.re + a[m - 1].re * cj, A.im + a[m - 1].im * cj);
            B = mk(B.re + b[m - 1].re * sj, B.im + b[m - 1].im * sj);
        }
        cpx<T> iB = muli<S>(B);
        out[q] = A + iB;
        out[R - q] = A - iB;
    }
#pragma unroll
    for (int q = 0; q < R; ++q) x[q] = out[q];
}

template <int R, int S, typename T>
__device__ __forceinline__ void dft(cpx<T>* x);

// exp(S 2 pi i m / R) for the internal twiddles of composite butterflies,
// folded to compile-time constants after unrolling (m, R constant).
template <int R, int S, typename T>
__device__ __forceinline__ cpx<T> unit_root(int m) {
    constexpr double kTwoPi = 6.283185307179586476925286766559005768;
    m %= R;
    if (m == 0) return mk((T)1, (T)0);
    // exact values at the quarter points keep the error of the multiply at zero
    if (4 * m == R) return mk((T)0, (T)S);
    if (2 * m == R) return mk((T)-1, (T)0);
    if (4 * m == 3 * R) return mk((T)0, (T)-S);
    return mk((T)__builtin_cos(kTwoPi * m / R), (T)(S * __builtin_sin(kTwoPi * m / R)));
}

// Composite DFT of length R = R1 * R2 (n = R2*n1 + n2, k = k1 + R1*k2): R2
// DFTs of length R1, the internal twiddles W_R^(n2*k1), R1 DFTs of length R2.
template <int R1, int R2, int S, typename T>
__device__ __forceinline__ void dft_composite(cpx<T>* x) {
    constexpr int R = R1 * R2;
    cpx<T> y[R];
#pragma unroll
    for (int n2 = 0; n2 < R2; ++n2) {
        cpx<T> col[R1];
#pragma unroll
        for (int n1 = 0; n1 < R1; ++n1) col[n1] = x[R2 * n1 + n2];
        dft<R1, S>(col);
#pragma unroll
        for (int k1 = 0; k1 < R1; ++k1) y[k1 * R2 + n2] = (n2 * k1 % R) == 0 ? col[k1] : cmul(col[k1], unit_root<R, S, T>(n2 * k1));
    }
#pragma unroll
    for (int k1 = 0; k1 < R1; ++k1) {
        cpx<T> row[R2];
#pragma unroll
        for (int n2 = 0; n2 < R2; ++n2) row[n2] = y[k1 * R2 + n2];
        dft<R2, S>(row);
#pragma unroll
        for (int k2 = 0; k2 < R2; ++k2) x[k1 + R1 * k2] = row[k2];
    }
}

template <int R, int S, typename T>
__device__ __forceinline__ void dft(cpx<T>* x) {
    if constexpr (kIndexTest) {
        return;
    } else if constexpr (R == 2) {
        dft2<S>(x);
    } else if constexpr (R == 4) {
        dft4<S>(x[0], x[1], x[2], x[3]);
    } else if constexpr (R == 8) {
        dft8<S>(x);
    } else if constexpr (R == 16) {
        dft16<S>(x);
    } else if constexpr (R == 6) {
        dft_composite<3, 2, S>(x);
    } else if constexpr (R == 9) {
        dft_composite<3, 3, S>(x);
    } else if constexpr (R == 10) {
        dft_composite<5, 2, S>(x);
    } else if constexpr (R == 12) {
        dft_composite<3, 4, S>(x);
    } else if constexpr (R == 18) {
        dft_composite<9, 2, S>(x);
    } else {
        dft_odd<R, S>(x);
    }
}

// DFT of even length R whose inputs R/2..R-1 are zero: the even outputs are
// the R/2-point DFT of x[0..R/2), the odd ones that of x[m] exp(S 2 pi i m / R).
template <int R, int S, typename T>
__device__ __forceinline__ void dft_upper_zero(cpx<T>* x) {
    if constexpr (kIndexTest) return;
    constexpr int H = R / 2;
    cpx<T> e[H], o[H];
#pragma unroll
    for (int m = 0; m < H; ++m) {
        e[m] = x[m];
        o[m] = m == 0 ? x[0] : 4 * m == R ? muli<S>(x[m]) : cmul(x[m], unit_root<R, S, T>(m));
    }
    dft<H, S>(e);
    dft<H, S>(o);
#pragma unroll
    for (int j = 0; j < H; ++j) {
        x[2 * j] = e[j];
        x[2 * j + 1] = o[j];
    }
}

// LDS element index of element e in a line (one pad slot every 2^ps).
__device__ __forceinline__ int lpad(int e, int ps) { return e + (e >> ps); }

// Stage twiddle exp(-2 pi i m/N). Early stages (small P) touch few distinct
// table entries per wave, so they read the full table; late stages would
// scatter a wave over the whole table, so they combine two sqrt(N)-size
// tables (one extra complex multiply, both tables stay in L1).
struct StageTw {
    const void* full;
    const void* lo;
    const void* hi;
    int shift;
};
// Entry i of a complex table in global memory. The explicit address space
// keeps loads in out-of-line functions (whose pointer arguments are generic)
// on global_load instead of flat_load.
template <typename T>
__device__ __forceinline__ cpx<T> ld_table(const void* p, int i) {
    typedef T v2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) v2* gptr;
    const v2 x = ((gptr)p)[i];
    return mk(x.x, x.y);
}
template <typename T>
__device__ __forceinline__ cpx<T> stage_root(const StageTw& w, int m, bool scattered) {
    if (!scattered) return ld_table<T>(w.full, m);
    return cmul(ld_table<T>(w.hi, m >> w.shift), ld_table<T>(w.lo, m & ((1 << w.shift) - 1)));
}
constexpr int kScatterP = 32;  // stages with P >= this use the two-level tables

// p[i] = w^i for i < R from w = p[1] by a product tree of depth <= log2(R):
// w^i = w^(i - 2^m) * w^(2^m), 2^m the highest power of two in i. One table
// lookup per butterfly instead of R-1; the rounding error stays within a few
// ulp (depth <= 4 for R = 16).
template <int R, typename T>
__device__ __forceinline__ void root_powers(cpx<T> w, cpx<T>* p) {
    p[0] = mk((T)1, (T)0);
    if constexpr (R > 1) p[1] = w;
#pragma unroll
    for (int i = 2; i < R; ++i) {
        int hb = 1;
        while (hb * 2 <= i) hb *= 2;
        p[i] = hb == i ? cmul(p[i / 2], p[i / 2]) : cmul(p[i - hb], p[hb]);
    }
}

// Where a runtime-shape stage reads its inputs and writes its outputs.
enum StageMode : int {
    SM_LDS = 0,    // LDS -> LDS, in place
    SM_FIRST = 1,  // the line's contiguous HBM elements -> LDS
    SM_LAST = 2,   // LDS -> the line's contiguous HBM elements (scaled)
};

// One Stockham stage of the runtime-shape kernels. SM_LDS reads every input
// of the thread's butterflies from LDS, synchronises the block and writes in
// place; SM_FIRST loads from HBM and SM_LAST stores to HBM (lines contiguous
// there, consecutive threads on consecutive elements), with no barrier
// between their reads and writes (the two sides are different memories).
// Not inlined: the runtime-radix loop dispatches to one of these per stage,
// and inlined cases share no registers (a dozen radix cases in one body need
// more than 256 VGPRs and spill to scratch).
template <typename T, int S, int R, bool WIDE, int MODE, class Ld, class St>
__device__ __forceinline__ void stage_rt_body(cpx<T>* __restrict__ line, int N, int P, int TT, const int t, int ps,
                                              const StageTw& tw, Ld&& ld, St&& st) {
    // The stage's geometry is uniform over the block; the out-of-line stage
    // receives it in vector registers, so move it to scalar registers and
    // keep everything derived from it scalar.
    N = __builtin_amdgcn_readfirstlane(N);
    P = __builtin_amdgcn_readfirstlane(P);
    TT = __builtin_amdgcn_readfirstlane(TT);
    ps = __builtin_amdgcn_readfirstlane(ps);
    constexpr int MJ = dyn_butterflies_per_thread(R, WIDE);
    const int NB = N / R;
    // LDS slot of element e: e + (e >> ps). When the butterfly stride NB (on
    // the reads) or P (on the writes) is a multiple of the pad period 2^ps,
    // the R slots of a butterfly are one padded base plus a uniform padded
    // stride, one add per element instead of a shift and two adds.
    const int pmask = ps >= 30 ? 0 : (1 << ps) - 1;
    const bool rd_uni = (NB & pmask) == 0, wr_uni = (P & pmask) == 0;
    const int rd_step = NB + (ps >= 30 ? 0 : NB >> ps), wr_step = P + (ps >= 30 ? 0 : P >> ps);
    cpx<T> v[MJ][R];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (b < NB) {
            if constexpr (MODE == SM_FIRST) {
#pragma unroll
                for (int i = 0; i < R; ++i) v[j][i] = ld(b + i * NB);
            } else if (rd_uni) {
                const int a0 = lpad(b, ps);
#pragma unroll
                for (int i = 0; i < R; ++i) v[j][i] = line[a0 + i * rd_step];
            } else {
#pragma unroll
                for (int i = 0; i < R; ++i) v[j][i] = line[lpad(b + i * NB, ps)];
            }
        }
    }
    if constexpr (MODE == SM_LDS) __syncthreads();
    const int step = N / (P * R);
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (b < NB) {
            const int k = (int)((unsigned)b % (unsigned)P);
            if (P > 1) {
                cpx<T> wp[R];
                root_powers<R>(stage_root<T>(tw, k * step, P >= kScatterP), wp);
#pragma unroll
                for (int i = 1; i < R; ++i) v[j][i] = twmul<S>(v[j][i], wp[i]);
            }
            dft<R, S>(v[j]);
            const int base = (b - k) * R + k;
            if constexpr (MODE == SM_LAST) {
#pragma unroll
                for (int q = 0; q < R; ++q) st(base + q * P, v[j][q]);
            } else if (wr_uni) {
                const int w0 = lpad(base, ps);
#pragma unroll
                for (int q = 0; q < R; ++q) line[w0 + q * wr_step] = v[j][q];
            } else {
#pragma unroll
                for (int q = 0; q < R; ++q) line[lpad(base + q * P, ps)] = v[j][q];
            }
        }
    }
    if constexpr (MODE != SM_LAST) __syncthreads();
}

template <typename T, int S, int R, bool WIDE, int MODE>
__device__ __noinline__ void stage_rt(cpx<T>* __restrict__ line, const int N, const int P, const int TT,
                                      const int t, const int ps, const StageTw tw, const cpx<T>* gsrc,
                                      cpx<T>* gdst, const int valid, const T sc) {
    // `line` always points into LDS; without this a non-inlined function
    // addresses it with flat instructions instead of ds_read / ds_write
    // (the builtin exists in the device pass only)
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)line));
#endif
    typedef T v2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) v2* gsrc_t;
    typedef __attribute__((address_space(1))) v2* gdst_t;
    stage_rt_body<T, S, R, WIDE, MODE>(
        line, N, P, TT, t, ps, tw,
        [&](int e) {
            const v2 x = ((gsrc_t)gsrc)[e];
            return mk(x.x, x.y);
        },
        [&](int o, cpx<T> v) {
            if (valid) {
                const cpx<T> y = scale(v, sc);
                v2 x;
                x.x = y.re;
                x.y = y.im;
                ((gdst_t)gdst)[o] = x;
            }
        });
}

// The HBM end of a runtime-shape direct C2C stage with the plan's boundary
// work (KF_EDGE): the HBM side holds storage type U (converted on load,
// rounded to nearest on store), and elements of [zl, zr) read as zero
// (SM_FIRST) or are written as zero (SM_LAST).
template <typename T, int S, int R, bool WIDE, int MODE, typename U>
__device__ __noinline__ void stage_rt_edge(cpx<T>* __restrict__ line, const int N, const int P, const int TT,
                                           const int t, const int ps, const StageTw tw, const cpx<U>* gsrc,
                                           cpx<U>* gdst, const int valid, const T sc, const int zl, const int zr) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)line));
#endif
    typedef U u2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) u2* gsrc_t;
    typedef __attribute__((address_space(1))) u2* gdst_t;
    stage_rt_body<T, S, R, WIDE, MODE>(
        line, N, P, TT, t, ps, tw,
        [&](int e) {
            if (e >= zl && e < zr) return mk((T)0, (T)0);
            const u2 x = ((gsrc_t)gsrc)[e];
            return mk((T)x.x, (T)x.y);
        },
        [&](int o, cpx<T> v) {
            if (valid) {
                const cpx<T> y = (o >= zl && o < zr) ? mk((T)0, (T)0) : scale(v, sc);
                u2 x;
                x.x = (U)y.re;
                x.y = (U)y.im;
                ((gdst_t)gdst)[o] = x;
            }
        });
}

// Dispatch of one stage on its runtime radix. Radix-2 HBM stages are not
// built (their hoisted loads would raise the register count of every
// runtime-shape kernel); the host gives such lines the staged kernel.
template <typename T, int S, bool WIDE, int MODE>
__device__ __forceinline__ void stage_rt_radix(int R, cpx<T>* __restrict__ line, const int N, const int P,
                                               const int TT, const int t, const int ps, const StageTw& tw,
                                               const cpx<T>* gsrc, cpx<T>* gdst, const int valid, const T sc) {
#define VKFX_STAGE_CASE(RR) \
    case RR: stage_rt<T, S, RR, WIDE, MODE>(line, N, P, TT, t, ps, tw, gsrc, gdst, valid, sc); break;
    switch (R) {
        case 2:
            if constexpr (MODE == SM_LDS) stage_rt<T, S, 2, WIDE, MODE>(line, N, P, TT, t, ps, tw, gsrc, gdst, valid, sc);
            break;
        VKFX_STAGE_CASE(3)
        VKFX_STAGE_CASE(4)
        VKFX_STAGE_CASE(5)
        VKFX_STAGE_CASE(6)
        VKFX_STAGE_CASE(7)
        VKFX_STAGE_CASE(8)
        VKFX_STAGE_CASE(9)
        VKFX_STAGE_CASE(10)
        VKFX_STAGE_CASE(11)
        VKFX_STAGE_CASE(12)
        VKFX_STAGE_CASE(13)
        VKFX_STAGE_CASE(16)
        default: break;
    }
#undef VKFX_STAGE_CASE
}

// A Rader stage: prime radix p > kMaxStockhamRadix in a Stockham sequence
// (the mixed-radix Rader of rader_ir.rs / mixed_ir.rs, with the length p-1
// cyclic convolution by direct multiplication). Butterfly b of the stage
// (input i at b + i N/p, j = b mod P) takes the stage twiddles
// W_{P p}^(j i), then X[0] = sum x and X[g^m] = x0 + sum_s x[g^-s] b[m - s]
// with b[n] = exp(S 2 pi i g^n / p), and writes X[q] to j + (b - j) p + q P.
// The twiddled inputs go through `scr` (N more elements of LDS) in Rader
// order; the threads of the line share the N inputs and then the N outputs.
template <typename T, int S>
__device__ __noinline__ void stage_rader(cpx<T>* __restrict__ line, cpx<T>* __restrict__ scr, const int N,
                                         const int P, const int p, const int TT, const int t, const int ps,
                                         const StageTw tw, const unsigned char* rt) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)line));
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)scr));
#endif
    typedef const __attribute__((address_space(1))) int* gint;
    const int L = p - 1, NB = N / p, step = N / (P * p);
    const gint slot = (gint)rt, logq = (gint)rt + p;
    const void* kern = rt + rader_kernel_offset(p) + (S < 0 ? 0 : (size_t)L * sizeof(cpx<T>));
    for (int e = t; e < N; e += TT) {
        const int i = e / NB, b = e - i * NB, j = b % P;
        cpx<T> v = line[lpad(e, ps)];
        if (i > 0 && j > 0) v = twmul<S>(v, stage_root<T>(tw, j * i * step, P >= kScatterP));
        scr[b * p + slot[i]] = v;
    }
    __syncthreads();
    for (int e = t; e < N; e += TT) {
        const int b = e / p, q = e - b * p, j = b % P;
        const cpx<T>* a = scr + b * p;
        cpx<T> acc = a[L];
        if constexpr (kIndexTest) {
            // identity arithmetic: the unit impulse for the kernel and a[0]
            // for the DC sum (the gather and scatter show bit for bit)
            acc = acc + a[q == 0 ? 0 : logq[q]];
        } else if (q == 0) {
            for (int s = 0; s < L; ++s) acc = acc + a[s];
        } else {
            cpx<T> conv = mk((T)0, (T)0);
            int bi = logq[q];
            for (int s = 0; s < L; ++s) {
                conv = conv + cmul(a[s], ld_table<T>(kern, bi));
                bi = bi == 0 ? L - 1 : bi - 1;
            }
            acc = acc + conv;
        }
        line[lpad((b - j) * p + j + q * P, ps)] = acc;
    }
    __syncthreads();
}

// One radix-R stage of the length-L FFTs inside an FFT-mode Rader stage: NB
// sequences at stride q (element stride 1) in `src`, out of place into
// `dst`, Stockham order (natural-order output after the last stage). Stage
// twiddles W_L^(j i L/(Pp R)) from `roots` (exp(-2 pi i k/L)); SG is the
// sign of the sub-FFT.
template <typename T, int SG, int R>
__device__ __noinline__ void rader_sub_stage(const cpx<T>* __restrict__ src, cpx<T>* __restrict__ dst,
                                             const int NB, const int L, const int q, const int Pp, const int TT,
                                             const int t, const void* roots) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)src));
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)dst));
#endif
    const int nb = L / R, total = NB * nb, tstep = L / (Pp * R);
#pragma unroll 1
    for (int u = t; u < total; u += TT) {
        const int seq = u / nb, bb = u - seq * nb, j = bb % Pp;
        const cpx<T>* s = src + seq * q + bb;
        cpx<T> v[R];
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = s[i * nb];
        if (j > 0) {
#pragma unroll
            for (int i = 1; i < R; ++i) v[i] = twmul<SG>(v[i], ld_table<T>(roots, j * i * tstep));
        }
        dft<R, SG>(v);
        cpx<T>* d = dst + seq * q + j + (bb - j) * R;
#pragma unroll
        for (int k = 0; k < R; ++k) d[k * Pp] = v[k];
    }
}

// The same for a prime sub-radix R in (13, kRaderSubPrimeMax]: the R-point
// DFT by direct multiplication (the direct Rader node of the reference's
// tree computes the same sums), pairing x[m] with x[R - m] as dft_odd does
// and writing each output pair as soon as it is formed, so only the paired
// sums stay in registers; the roots are compile-time constants.
template <typename T, int SG, int R>
__device__ __noinline__ void rader_sub_stage_prime(const cpx<T>* __restrict__ src, cpx<T>* __restrict__ dst,
                                                   const int NB, const int L, const int q, const int Pp,
                                                   const int TT, const int t, const void* roots) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)src));
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)dst));
#endif
    constexpr int H = (R - 1) / 2;
    const int nb = L / R, total = NB * nb, tstep = L / (Pp * R);
#pragma unroll 1
    for (int u = t; u < total; u += TT) {
        const int seq = u / nb, bb = u - seq * nb, j = bb % Pp;
        const cpx<T>* s = src + seq * q + bb;
        cpx<T>* d = dst + seq * q + j + (bb - j) * R;
        const cpx<T> x0 = s[0];
        cpx<T> sa[H], sb[H];
#pragma unroll
        for (int m = 1; m <= H; ++m) {
            cpx<T> lo = s[m * nb], hi = s[(R - m) * nb];
            if (j > 0) {
                lo = twmul<SG>(lo, ld_table<T>(roots, j * m * tstep));
                hi = twmul<SG>(hi, ld_table<T>(roots, j * (R - m) * tstep));
            }
            if constexpr (kIndexTest) {
                d[m * Pp] = lo;
                d[(R - m) * Pp] = hi;
            }
            sa[m - 1] = lo + hi;
            sb[m - 1] = lo - hi;
        }
        if constexpr (kIndexTest) {
            d[0] = x0;
            continue;
        }
        cpx<T> y0 = x0;
#pragma unroll
        for (int m = 0; m < H; ++m) y0 = y0 + sa[m];
        d[0] = y0;
#pragma unroll
        for (int k = 1; k <= H; ++k) {
            cpx<T> A = x0;
            cpx<T> B = mk((T)0, (T)0);
#pragma unroll
            for (int m = 1; m <= H; ++m) {
                const cpx<T> w = unit_root<R, -1, T>(m * k);  // cos and -sin of 2 pi m k / R
                A = mk(A.re + sa[m - 1].re * w.re, A.im + sa[m - 1].im * w.re);
                B = mk(B.re - sb[m - 1].re * w.im, B.im - sb[m - 1].im * w.im);
            }
            const cpx<T> iB = muli<SG>(B);
            d[k * Pp] = A + iB;
            d[(R - k) * Pp] = A - iB;
        }
    }
}

template <typename T, int SG>
__device__ __forceinline__ void rader_sub_stage_radix(int R, const cpx<T>* src, cpx<T>* dst, int NB, int L, int q,
                                                      int Pp, int TT, int t, const void* roots) {
    switch (R) {
        case 2: rader_sub_stage<T, SG, 2>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 3: rader_sub_stage<T, SG, 3>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 4: rader_sub_stage<T, SG, 4>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 5: rader_sub_stage<T, SG, 5>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 7: rader_sub_stage<T, SG, 7>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 8: rader_sub_stage<T, SG, 8>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 9: rader_sub_stage<T, SG, 9>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 11: rader_sub_stage<T, SG, 11>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 13: rader_sub_stage<T, SG, 13>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 16: rader_sub_stage<T, SG, 16>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 17: rader_sub_stage_prime<T, SG, 17>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 19: rader_sub_stage_prime<T, SG, 19>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 23: rader_sub_stage_prime<T, SG, 23>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 29: rader_sub_stage_prime<T, SG, 29>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        case 31: rader_sub_stage_prime<T, SG, 31>(src, dst, NB, L, q, Pp, TT, t, roots); break;
        default: break;  // the host plans no other sub-radix (rader_sub_schedule)
    }
}

// FFT-mode Rader stage (prime radix q >= kRaderFftStageMin, table layout in
// kernels.hpp): the gather of stage_rader into `scr` (butterfly b's inputs
// at b*q + slot[i], x0 at b*q + L), the forward length-L FFTs of all NB
// butterflies, the spectrum multiply, the inverse FFTs, and the outputs
// X[0] = x0 + A[0], X[g^m] = x0 + conv[m] written to the Stockham positions
// j + (b - j) q + {0, g^m} P. Once gathered, the line's own LDS region is
// free until the outputs: the length-L FFTs ping-pong between `scr` and the
// line region (unpadded, sequences at the same b*q offsets; an even number
// of sub-stages in all brings the result back to `scr`), and X[0] waits in
// the line region's slot b*q + L, which no sub-stage writes.
template <typename T, int S>
__device__ __noinline__ void stage_rader_fft(cpx<T>* __restrict__ line, cpx<T>* __restrict__ scr, const int N,
                                             const int P, const int q, const int TT, const int t, const int ps,
                                             const StageTw tw, const unsigned char* rt) {
    const int L = q - 1, NB = N / q, step = N / (P * q);
    const int* hdr = (const int*)rt;
    const int* slot = hdr + 16;
    const int* pw = slot + q;
    const unsigned char* data = rt + rader_fft_data_offset(q);
    const void* roots = data;
    const void* spec = data + (size_t)(S < 0 ? 1 : 2) * L * sizeof(cpx<T>);
    const int nsub = hdr[0];
    for (int e = t; e < N; e += TT) {
        const int i = e / NB, b = e - i * NB, j = b % P;
        cpx<T> v = line[lpad(e, ps)];
        if (i > 0 && j > 0) v = twmul<S>(v, stage_root<T>(tw, j * i * step, P >= kScatterP));
        scr[b * q + slot[i]] = v;
    }
    __syncthreads();
    cpx<T>* src = scr;
    cpx<T>* dst = line;
    int Pp = 1;
    for (int k = 0; k < nsub; ++k) {
        const int R = hdr[1 + k];
        rader_sub_stage_radix<T, -1>(R, src, dst, NB, L, q, Pp, TT, t, roots);
        __syncthreads();
        cpx<T>* tmp = src;
        src = dst;
        dst = tmp;
        Pp *= R;
    }
    // A *= FFT_L(b) / L; X[0] = x0 + A[0] parks in line[b*q + L]
    for (int e = t; e < NB * L; e += TT) {
        const int b = e / L, k = e - b * L;
        cpx<T> a = src[b * q + k];
        if (k == 0) line[b * q + L] = scr[b * q + L] + a;
        if constexpr (!kIndexTest) a = cmul(a, ld_table<T>(spec, k));
        src[b * q + k] = a;
    }
    __syncthreads();
    Pp = 1;
    for (int k = 0; k < nsub; ++k) {
        const int R = hdr[1 + k];
        rader_sub_stage_radix<T, 1>(R, src, dst, NB, L, q, Pp, TT, t, roots);
        __syncthreads();
        cpx<T>* tmp = src;
        src = dst;
        dst = tmp;
        Pp *= R;
    }
    // src == scr: conv[m] + x0, then X[0] into the x0 slot
    for (int e = t; e < NB * L; e += TT) {
        const int b = e / L, m = e - b * L;
        scr[b * q + m] = scr[b * q + L] + scr[b * q + m];
    }
    __syncthreads();
    for (int b = t; b < NB; b += TT) scr[b * q + L] = line[b * q + L];
    __syncthreads();
    for (int e = t; e < N; e += TT) {
        const int b = e / q, r = e - b * q, j = b % P;
        const int out = r == L ? 0 : pw[r];
        line[lpad((b - j) * q + j + out * P, ps)] = scr[b * q + r];
    }
    __syncthreads();
}

// Runs every stage of a runtime radix list over the line at `line` (in LDS);
// with RAD, a Rader stage (radix above kMaxStockhamRadix) uses `scr` and its
// table block in `rtab` (RAD instantiations only, so the Rader stages'
// registers stay out of the other kernels).
template <typename T, int S, bool WIDE, bool RAD = false>
__device__ __forceinline__ void run_stages(cpx<T>* __restrict__ line, const int N, const int TT,
                                           const int t, const int ps, const int nst,
                                           const int* __restrict__ radix, const StageTw& tw,
                                           cpx<T>* scr = nullptr, const void* rtab = nullptr,
                                           const int* roff = nullptr) {
    int P = 1;
    for (int s = 0; s < nst; ++s) {
        if (!RAD)
            stage_rt_radix<T, S, WIDE, SM_LDS>(radix[s], line, N, P, TT, t, ps, tw, nullptr, nullptr, 0, (T)1);
        else if (radix[s] > kMaxStockhamRadix && (roff[s] & kRaderFftStage))
            stage_rader_fft<T, S>(line, scr, N, P, radix[s], TT, t, ps, tw,
                                  (const unsigned char*)rtab + (roff[s] & ~kRaderFftStage));
        else if (radix[s] > kMaxStockhamRadix)
            stage_rader<T, S>(line, scr, N, P, radix[s], TT, t, ps, tw, (const unsigned char*)rtab + roff[s]);
        else
            stage_rt_radix<T, S, WIDE, SM_LDS>(radix[s], line, N, P, TT, t, ps, tw, nullptr, nullptr, 0, (T)1);
        P *= radix[s];
    }
}

// The same with only the first stage reading the line from HBM (`src`); the
// result stays in LDS for a staged epilogue. The first radix must not be 2.
template <typename T, int S, bool WIDE>
__device__ __forceinline__ void run_stages_direct_in(cpx<T>* __restrict__ line, const int N, const int TT,
                                                     const int t, const int ps, const int nst,
                                                     const int* __restrict__ radix, const StageTw& tw,
                                                     const cpx<T>* src) {
    stage_rt_radix<T, S, WIDE, SM_FIRST>(radix[0], line, N, 1, TT, t, ps, tw, src, nullptr, 0, (T)1);
    int P = radix[0];
    for (int s = 1; s < nst; ++s) {
        stage_rt_radix<T, S, WIDE, SM_LDS>(radix[s], line, N, P, TT, t, ps, tw, src, nullptr, 0, (T)1);
        P *= radix[s];
    }
}

// The same with the first stage reading the line from HBM (`src`) and the
// last writing it, times `sc`, to HBM (`dst`, skipped when !valid): at least
// two stages, neither end of radix 2.
template <typename T, int S, bool WIDE>
__device__ __forceinline__ void run_stages_direct(cpx<T>* __restrict__ line, const int N, const int TT,
                                                  const int t, const int ps, const int nst,
                                                  const int* __restrict__ radix, const StageTw& tw,
                                                  const cpx<T>* src, cpx<T>* dst, int valid, T sc) {
    stage_rt_radix<T, S, WIDE, SM_FIRST>(radix[0], line, N, 1, TT, t, ps, tw, src, dst, valid, sc);
    int P = radix[0];
    for (int s = 1; s + 1 < nst; ++s) {
        stage_rt_radix<T, S, WIDE, SM_LDS>(radix[s], line, N, P, TT, t, ps, tw, src, dst, valid, sc);
        P *= radix[s];
    }
    stage_rt_radix<T, S, WIDE, SM_LAST>(radix[nst - 1], line, N, P, TT, t, ps, tw, src, dst, valid, sc);
}

// Dispatch of an HBM end with boundary work on its runtime radix (no radix 2,
// as for the plain direct ends).
template <typename T, int S, bool WIDE, int MODE, typename U>
__device__ __forceinline__ void stage_rt_edge_radix(int R, cpx<T>* __restrict__ line, const int N, const int P,
                                                    const int TT, const int t, const int ps, const StageTw& tw,
                                                    const cpx<U>* gsrc, cpx<U>* gdst, const int valid, const T sc,
                                                    const int zl, const int zr) {
#define VKFX_STAGE_CASE(RR) \
    case RR: stage_rt_edge<T, S, RR, WIDE, MODE, U>(line, N, P, TT, t, ps, tw, gsrc, gdst, valid, sc, zl, zr); break;
    switch (R) {
        VKFX_STAGE_CASE(3)
        VKFX_STAGE_CASE(4)
        VKFX_STAGE_CASE(5)
        VKFX_STAGE_CASE(6)
        VKFX_STAGE_CASE(7)
        VKFX_STAGE_CASE(8)
        VKFX_STAGE_CASE(9)
        VKFX_STAGE_CASE(10)
        VKFX_STAGE_CASE(11)
        VKFX_STAGE_CASE(12)
        VKFX_STAGE_CASE(13)
        VKFX_STAGE_CASE(16)
        default: break;
    }
#undef VKFX_STAGE_CASE
}

// run_stages_direct with boundary work at both HBM ends: the first stage
// reads storage type UI with the input zero interval [zil, zir), the last
// writes storage type UO with the output zero interval [zol, zor).
template <typename T, int S, bool WIDE, typename UI, typename UO>
__device__ __forceinline__ void run_stages_direct_edge(cpx<T>* __restrict__ line, const int N, const int TT,
                                                       const int t, const int ps, const int nst,
                                                       const int* __restrict__ radix, const StageTw& tw,
                                                       const cpx<UI>* src, cpx<UO>* dst, int valid, T sc,
                                                       int zil, int zir, int zol, int zor) {
    stage_rt_edge_radix<T, S, WIDE, SM_FIRST, UI>(radix[0], line, N, 1, TT, t, ps, tw, src, nullptr, valid, sc, zil,
                                                  zir);
    int P = radix[0];
    for (int s = 1; s + 1 < nst; ++s) {
        stage_rt_radix<T, S, WIDE, SM_LDS>(radix[s], line, N, P, TT, t, ps, tw, nullptr, nullptr, 0, (T)1);
        P *= radix[s];
    }
    stage_rt_edge_radix<T, S, WIDE, SM_LAST, UO>(radix[nst - 1], line, N, P, TT, t, ps, tw, nullptr, dst, valid, sc,
                                                 zol, zor);
}

}  // namespace vkfx
