// fft_kernels_impl.hpp -- gfx950 kernels of the batched FFT path.
//
// Every kernel is one HBM pass over a set of "lines" (1-D sequences along one
// axis). A block owns G lines; each line is transformed by the Stockham
// stages of fft_device.hpp with LDS exchanges between stages. IO policies
// decide where a line lives in HBM and which pointwise work is fused into the
// load and the store:
//
//   IoPlain       C2C along any axis (contiguous rows or strided columns)
//   IoR2CFull     odd-length R2C through a full complex FFT (real_ir.rs:935-946)
//   IoC2RFull     odd-length C2R by Hermitian expansion (real_ir.rs:1038-1053)
//   IoR2CHalf     even R2C: half-size packed FFT + postprocess (real_ir.rs:952-1000)
//   IoC2RHalf     even C2R: preprocess + half-size packed FFT (real_ir.rs:1072-1105)
//   IoFsA*        four-step column pass with the W_M^(n2*k1) twiddle fused
//                 into the store (kernel_ir.rs:1042-1238 FourStepRight); the
//                 Bluestein variant fuses chirp * x and the zero padding
//                 (bluestein_ir.rs:436-708), the C2R variant fuses the
//                 even-half preprocess
//   IoFsB         four-step row pass with transposed (natural-order) store
//   IoFsAEdge,    the two passes of a mixed-storage two-upload C2C with the
//   IoFsBEdge     storage conversion and zero intervals in their loads / stores
//   IoFsBR2C      row pass that owns mirror rows k1 and N1-k1 so the R2C
//                 postprocess is fused into the store
//   IoBlueB       Bluestein row pass: FFT, kernel-spectrum multiply, IFFT and
//                 the inverse four-step twiddle in one kernel
//   IoFsCBlue     Bluestein column pass: IFFT, chirp multiply, truncate to N
//   IoBlue1       whole Bluestein transform when the convolution fits LDS
//   IoConv1       one-upload convolution: FFT, kernel-spectrum multiply, IFFT
//   IoConvB       two-upload convolution row pass: FFT, natural-order
//                 kernel-spectrum multiply, IFFT, inverse four-step twiddle
//
// Two kernel templates run these policies:
//   k_dyn  -- runtime length and radix list; lines are staged through LDS on
//             both ends (any length the planner accepts).
//   k_fix  -- compile-time shape (length, radices, threads per line, lines per
//             block, lane mapping). When the lane mapping matches the memory
//             layout the first stage reads HBM straight into registers and the
//             last stage writes registers straight to HBM.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "fft_device.hpp"
#include "kernels.hpp"

namespace vkfx {

struct LineInfo {
    long long ib, ob, o, c;
    long long tr;  // four-step twiddle row (c / twdiv)
    int valid;
};

enum Layout : int { LAY_ANY = 0, LAY_ROW = 1, LAY_COL = 2, LAY_STAGED = 3 };

// Runtime dimensions (k_dyn) and compile-time dimensions (k_fix) seen by the
// IO policies through the same interface.
struct DynDims {
    static constexpr bool NTI = false, NTO = false;
    static __device__ __forceinline__ int N(const KArgs& a) { return a.N; }
    static __device__ __forceinline__ int G(const KArgs& a) { return a.G; }
    static __device__ __forceinline__ int LS(const KArgs& a) { return a.LS; }
    static __device__ __forceinline__ int PS(const KArgs& a) { return a.PS; }
};
template <int N_, int G_, int LS_, int PS_, bool NTI_ = false, bool NTO_ = false>
struct FixDims {
    static constexpr bool NTI = NTI_, NTO = NTO_;
    static __device__ __forceinline__ constexpr int N(const KArgs&) { return N_; }
    static __device__ __forceinline__ constexpr int G(const KArgs&) { return G_; }
    static __device__ __forceinline__ constexpr int LS(const KArgs&) { return LS_; }
    static __device__ __forceinline__ constexpr int PS(const KArgs&) { return PS_; }
};

// Group of lines handled by this block. Workgroups are dispatched round-robin
// over the 8 XCDs; with KF_XCD_GROUPS each XCD gets a contiguous range of
// groups instead, so neighbouring groups whose HBM segments share cache lines
// (unaligned pitches, narrow strided segments) meet in the same L2.
__device__ __forceinline__ long long group_index(const KArgs& a) {
    const long long i = blockIdx.x;
    if (!(a.flags & KF_XCD_GROUPS)) return i;
    constexpr long long X = 8;
    const long long n = gridDim.x, q = n / X, r = n % X;
    const long long x = i % X, k = i / X;
    return x * q + (x < r ? x : r) + k;
}

__device__ __forceinline__ LineInfo line_default(const KArgs& a, long long blk, int g) {
    LineInfo L;
    long long line = blk * a.G + g;
    L.valid = line < a.nlines;
    if (!L.valid) line = 0;
    // line = (o * C1 + o1) * C + c; 32-bit division whenever the operands fit
    long long r;
    if (a.C == 1) {
        r = line;
        L.c = 0;
    } else if (line < (1ll << 31) && a.C < (1ll << 31)) {
        r = (long long)((unsigned)line / (unsigned)a.C);
        L.c = line - r * a.C;
    } else {
        r = line / a.C;
        L.c = line - r * a.C;
    }
    long long o1 = 0;
    L.o = r;
    if (a.C1 > 1) {
        L.o = (r < (1ll << 31) && a.C1 < (1ll << 31)) ? (long long)((unsigned)r / (unsigned)a.C1) : r / a.C1;
        o1 = r - L.o * a.C1;
    }
    L.ib = L.o * a.in_os + o1 * a.in_os1 + L.c * a.in_cs;
    L.ob = L.o * a.out_os + o1 * a.out_os1 + L.c * a.out_cs;
    L.tr = a.twdiv > 1 ? L.c / a.twdiv : L.c;
    return L;
}

// Visits (g, e) for g < G, e < n with consecutive threads on consecutive
// addresses: e fastest when lines are contiguous, g fastest otherwise. The
// (slow, fast) pair of idx = slow * d + fast advances by the block size with
// one division up front instead of one per element.
template <class F>
__device__ __forceinline__ void coop_for(int G, int n, bool rowmajor, F&& f) {
    const int total = G * n;
    const int d = rowmajor ? n : G;
    const int step = (int)blockDim.x;
    const int dq = step / d, dr = step - dq * d;
    int slow = (int)threadIdx.x / d;
    int fast = (int)threadIdx.x - slow * d;
    for (int idx = threadIdx.x; idx < total; idx += step) {
        if (rowmajor) {
            f(slow, fast);
        } else {
            f(fast, slow);
        }
        slow += dq;
        fast += dr;
        if (fast >= d) {
            fast -= d;
            ++slow;
        }
    }
}

template <typename T>
__device__ __forceinline__ cpx<T> tw2(const void* lo, const void* hi, int shift, long long k) {
    const cpx<T>* L = (const cpx<T>*)lo;
    const cpx<T>* H = (const cpx<T>*)hi;
    return cmul(H[k >> shift], L[k & ((1ll << shift) - 1)]);
}

template <typename T>
__device__ __forceinline__ cpx<T> zero() {
    return mk((T)0, (T)0);
}

// HBM element access; NT = nontemporal (streamed data that is not re-read
// by this kernel, so it should not displace cached tables).
template <bool NT, typename T>
__device__ __forceinline__ cpx<T> ldg(const cpx<T>* p) {
    if constexpr (NT) {
        return mk(__builtin_nontemporal_load(&p->re), __builtin_nontemporal_load(&p->im));
    } else {
        return *p;
    }
}
template <bool NT, typename T>
__device__ __forceinline__ void stg(cpx<T>* p, cpx<T> v) {
    if constexpr (NT) {
        __builtin_nontemporal_store(v.re, &p->re);
        __builtin_nontemporal_store(v.im, &p->im);
    } else {
        *p = v;
    }
}
// Input/output accessors honouring the per-launch streaming flags.
// (The hint must be a compile-time choice: a runtime branch between the two
// forms is merged into one plain access by the compiler.)
template <bool NT, typename T>
__device__ __forceinline__ cpx<T> ldg_in(const KArgs&, const cpx<T>* p) {
    return ldg<NT>(p);
}
template <bool NT, typename T>
__device__ __forceinline__ void stg_out(const KArgs&, cpx<T>* p, cpx<T> v) {
    stg<NT>(p, v);
}
template <bool NT, typename T>
__device__ __forceinline__ T ldg_s(const T* p) {
    if constexpr (NT) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}
template <bool NT, typename T>
__device__ __forceinline__ void stg_s(T* p, T v) {
    if constexpr (NT) {
        __builtin_nontemporal_store(v, p);
    } else {
        *p = v;
    }
}

// Generic staged prologue/epilogue built from the element functions.
template <class IO, class D, typename T>
__device__ __forceinline__ void staged_load(const KArgs& a, cpx<T>* lds, const LineInfo* li, bool rowmajor) {
    coop_for(D::G(a), D::N(a), rowmajor, [&](int g, int e) {
        lds[g * D::LS(a) + lpad(e, D::PS(a))] =
            li[g].valid ? IO::template load_elem<T, D::NTI>(a, li[g], e) : zero<T>();
    });
}
template <class IO, class D, typename T, int S>
__device__ __forceinline__ void staged_store(const KArgs& a, const cpx<T>* lds, const LineInfo* li, bool rowmajor) {
    coop_for(D::G(a), IO::template out_count<D>(a), rowmajor, [&](int g, int e) {
        if (li[g].valid) IO::template store_elem<T, S, D::NTO>(a, li[g], e, lds[g * D::LS(a) + lpad(e, D::PS(a))]);
    });
}

// ---------------------------------------------------------------- IO kinds

struct IoPlain {
    static constexpr bool kTwoPass = false;
    static constexpr bool kMidFused = false;  // two-pass: mid_elem applied in the first FFT's last stage
    // direct first stage: load_tw(e, w) with w = ltw_root(b) * ltw_root(NB, step)^i for e = b + i*NB
    static constexpr bool kLoadTw = false;
    static constexpr bool kStoreTw = false;  // store multiplies by a per-element pass twiddle
    // direct first stage of a C2R column pass over mirror-pair blocks that
    // loads each pair (X[k], X[M-k]) once for two butterflies (fstage_c2r_pairs)
    static constexpr bool kPairFirst = false;
    static constexpr int kLoad = LAY_ANY;
    static constexpr int kStore = LAY_ANY;
    // elements at or beyond kZeroFrom(N) of a length-N line are known zeros
    // (Bluestein padding); the direct first stage skips their loads and,
    // when a butterfly's upper half is all zeros, uses the half butterfly
    static constexpr int kZeroFrom(int N) { return N; }
    static __device__ LineInfo line(const KArgs& a, long long blk, int g) { return line_default(a, blk, g); }
    template <class D>
    static __device__ __forceinline__ int out_count(const KArgs& a) { return D::N(a); }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        return ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, scale(v, (T)a.scale));
    }
    // Pointer form of the element functions for the direct stages: element
    // e0 + i*step of a line is at in_ptr(e0) + i*step*in_es, so a thread
    // computes one address and steps it by a uniform stride. A policy whose
    // load_elem / store_elem (or store_twiddled) does more than this plain
    // access sets kPtrLoad / kPtrStore false.
    static constexpr bool kPtrLoad = true;
    static constexpr bool kPtrStore = true;
    // Butterfly forms of the element functions for the direct stages of
    // policies whose element functions weigh and mask elements by their
    // position in the line: load_bfly fills the R inputs b + i*NB of a
    // first-stage butterfly, store_bfly stores the R outputs base + q*P of a
    // last-stage butterfly, each stepping its addresses by a uniform stride.
    static constexpr bool kBflyLoad = false;
    static constexpr bool kBflyStore = false;
    template <typename T>
    static __device__ __forceinline__ const cpx<T>* in_ptr(const KArgs& a, const LineInfo& L, int e) {
        return (const cpx<T>*)a.in + L.ib + (long long)e * a.in_es;
    }
    template <typename T>
    static __device__ __forceinline__ cpx<T>* out_ptr(const KArgs& a, const LineInfo& L, int e) {
        return (cpx<T>*)a.out + L.ob + (long long)e * a.out_es;
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_at(const KArgs& a, cpx<T>* p, cpx<T> v) {
        stg_out<NTIO>(a, p, scale(v, (T)a.scale));
    }
    // staged variants used when an end cannot be direct
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoPlain, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};

// IoPlain with both ends staged through LDS (coalesced cooperative copies):
// for short rows, whose first and last Stockham stages would otherwise touch
// HBM in segments narrower than 128 bytes.
struct IoPlainStaged : IoPlain {
    static constexpr int kLoad = LAY_STAGED;
    static constexpr int kStore = LAY_STAGED;
};

// Storage type of half the compute precision (F16StorageF32Compute,
// F64ComputeF32Storage: src/config.rs:108-145).
template <typename T>
struct Narrow;
template <>
struct Narrow<float> {
    using type = _Float16;
};
template <>
struct Narrow<double> {
    using type = float;
};

// IoPlain with the plan's boundary work in its loads and stores (KF_EDGE):
// NI / NO read / write storage of half the compute precision (converted on
// load, rounded to nearest on store), and the element interval [zl, zr) of
// each line reads as zero (KF_ZERO_IN) or is written as zero (KF_ZERO_OUT),
// the logical zero intervals of src/zero_pad_ir.rs:320-345, 607-647. Line
// strides count elements of the storage type.
template <bool NI, bool NO>
struct IoEdge : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        if ((a.flags & KF_ZERO_IN) && e >= a.zl && e < a.zr) return zero<T>();
        if constexpr (NI) {
            using U = typename Narrow<T>::type;
            const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)a.in + L.ib + e * a.in_es);
            return mk((T)v.re, (T)v.im);
        } else {
            return ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es);
        }
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        v = ((a.flags & KF_ZERO_OUT) && e >= a.zl && e < a.zr) ? zero<T>() : scale(v, (T)a.scale);
        if constexpr (NO) {
            using U = typename Narrow<T>::type;
            stg_out<NTIO>(a, (cpx<U>*)a.out + L.ob + e * a.out_es, mk((U)v.re, (U)v.im));
        } else {
            stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, v);
        }
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoEdge, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoEdge, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};

// IoEdge on the fixed one-upload row shapes (KK_PLAIN_EDGE) of mixed-storage
// plans: the ends of the plain shape read and write the caller's storage type of half the compute
// precision (compile time, so the loads of a butterfly stay one batch), and
// the zero intervals of the line replace loaded or stored values by zero.
template <class Base>
struct IoEdgeFixed : Base {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    static constexpr bool kBflyLoad = true, kBflyStore = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        using U = typename Narrow<T>::type;
        const cpx<U>* x = (const cpx<U>*)a.in + L.ib + (long long)b * a.in_es;
        const long long dx = (long long)NB * a.in_es;
        const bool zi = (a.flags & KF_ZERO_IN) != 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const cpx<U> u = ldg_in<NTIO>(a, x + i * dx);
            const int e = b + i * NB;
            v[i] = (zi && e >= a.zl && e < a.zr) ? zero<T>() : mk((T)u.re, (T)u.im);
        }
    }
    template <typename T, int S, bool NTIO, int R, int P>
    static __device__ __forceinline__ void store_bfly(const KArgs& a, const LineInfo& L, int base, const cpx<T>* v) {
        using U = typename Narrow<T>::type;
        cpx<U>* y = (cpx<U>*)a.out + L.ob + (long long)base * a.out_es;
        const long long dy = (long long)P * a.out_es;
        const T sc = (T)a.scale;
        const bool zo = (a.flags & KF_ZERO_OUT) != 0;
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const int e = base + q * P;
            const bool z = zo && e >= a.zl && e < a.zr;
            stg_out<NTIO>(a, y + q * dy, z ? mk((U)0, (U)0) : mk((U)(v[q].re * sc), (U)(v[q].im * sc)));
        }
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        using U = typename Narrow<T>::type;
        const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)a.in + L.ib + e * a.in_es);
        const bool z = (a.flags & KF_ZERO_IN) && e >= a.zl && e < a.zr;
        return z ? zero<T>() : mk((T)v.re, (T)v.im);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        using U = typename Narrow<T>::type;
        const bool z = (a.flags & KF_ZERO_OUT) && e >= a.zl && e < a.zr;
        v = z ? zero<T>() : scale(v, (T)a.scale);
        stg_out<NTIO>(a, (cpx<U>*)a.out + L.ob + e * a.out_es, mk((U)v.re, (U)v.im));
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoEdgeFixed, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoEdgeFixed, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};
using IoPlainEdge = IoEdgeFixed<IoPlain>;

// The first (NI) or last (NO) pass of a mixed-storage N-D chunk on a fixed
// row or column shape: the caller's side in the storage type of half the
// compute precision (compile time), the other side the compute-type stage.
template <bool NI, bool NO>
struct IoEdgeSide : IoPlain {
    static constexpr bool kPtrLoad = !NI, kPtrStore = !NO;
    // direct stages: one storage-type address per butterfly, stepped by the
    // butterfly's element stride
    static constexpr bool kBflyLoad = NI, kBflyStore = NO;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        using U = typename Narrow<T>::type;
        const cpx<U>* x = (const cpx<U>*)a.in + L.ib + (long long)b * a.in_es;
        const long long dx = (long long)NB * a.in_es;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const cpx<U> u = ldg_in<NTIO>(a, x + i * dx);
            v[i] = mk((T)u.re, (T)u.im);
        }
    }
    template <typename T, int S, bool NTIO, int R, int P>
    static __device__ __forceinline__ void store_bfly(const KArgs& a, const LineInfo& L, int base, const cpx<T>* v) {
        using U = typename Narrow<T>::type;
        cpx<U>* y = (cpx<U>*)a.out + L.ob + (long long)base * a.out_es;
        const long long dy = (long long)P * a.out_es;
        const T sc = (T)a.scale;
#pragma unroll
        for (int q = 0; q < R; ++q) stg_out<NTIO>(a, y + q * dy, mk((U)(v[q].re * sc), (U)(v[q].im * sc)));
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        if constexpr (NI) {
            using U = typename Narrow<T>::type;
            const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)a.in + L.ib + e * a.in_es);
            return mk((T)v.re, (T)v.im);
        } else {
            return ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es);
        }
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        v = scale(v, (T)a.scale);
        if constexpr (NO) {
            using U = typename Narrow<T>::type;
            stg_out<NTIO>(a, (cpx<U>*)a.out + L.ob + e * a.out_es, mk((U)v.re, (U)v.im));
        } else {
            stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, v);
        }
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoEdgeSide, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoEdgeSide, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};
using IoPlainEdgeIn = IoEdgeSide<true, false>;
using IoPlainEdgeOut = IoEdgeSide<false, true>;

struct IoR2CFull : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    template <class D>
    static __device__ __forceinline__ int out_count(const KArgs& a) { return (int)a.nout; }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        return mk(ldg_s<NTIO>((const T*)a.in + L.ib + e * a.in_es), (T)0);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        if (e < a.nout) stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, scale(v, (T)a.scale));
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoR2CFull, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoR2CFull, D, T, S>(a, lds, li, true);
    }
};

struct IoC2RFull : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const int n = a.N, h = n / 2 + 1;
        return e < h ? ldg_in<NTIO>(a, in + L.ib + e * a.in_es) : conj(ldg_in<NTIO>(a, in + L.ib + (n - e) * a.in_es));
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        stg_s<NTIO>((T*)a.out + L.ob + e * a.out_es, v.re * (T)a.scale);
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoC2RFull, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoC2RFull, D, T, S>(a, lds, li, true);
    }
};

// Even-length R2C with the half-size FFT (length M = N) in LDS. Input is the
// real line viewed as M complex pairs z[n] = x[2n] + i x[2n+1]; the store
// needs Z[k] and Z[M-k] together, so it is always staged.
struct IoR2CHalf : IoPlain {
    static constexpr int kLoad = LAY_ROW;
    static constexpr int kStore = LAY_STAGED;
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const int M = D::N(a);
        coop_for(D::G(a), M + 1, true, [&](int g, int k) {
            if (!li[g].valid) return;
            const cpx<T>* Z = lds + g * D::LS(a);
            const int k0 = k == M ? 0 : k;
            const int km = k == 0 ? 0 : M - k;
            cpx<T> A = Z[lpad(k0, D::PS(a))];
            cpx<T> B = conj(Z[lpad(km, D::PS(a))]);
            cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
            cpx<T> X = (A + B) + muli<-1>(cmul(A - B, w));
            stg_out<D::NTO>(a, out + li[g].ob + k * a.out_es, scale(X, (T)0.5));
        });
    }
};

// Even-length C2R: Z[k] = (X[k] + conj X[M-k]) + i W_N^-k (X[k] - conj X[M-k]),
// then the inverse half-size FFT; the complex result is the real output pairs.
struct IoC2RHalf : IoPlain {
    static constexpr bool kPtrLoad = false;
    static constexpr int kLoad = LAY_ROW;
    static constexpr int kStore = LAY_ROW;
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int k) {
        return load_tw<T, NTIO>(a, L, k, tw2<T>(a.rlo, a.rhi, a.rshift, k));
    }
    // w = W_N^k = exp(-2 pi i k / 2M)
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_tw(const KArgs& a, const LineInfo& L, int k, cpx<T> w) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        cpx<T> X = ldg_in<NTIO>(a, in + L.ib + k * a.in_es);
        cpx<T> Xm = conj(ldg_in<NTIO>(a, in + L.ib + (a.N - k) * a.in_es));
        return (X + Xm) + muli<1>(cmulc(X - Xm, w));
    }
    static constexpr bool kLoadTw = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> ltw_root(const KArgs& a, const LineInfo&, int m, bool = false) {
        return tw2<T>(a.rlo, a.rhi, a.rshift, m);
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoC2RHalf, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoPlain, D, T, S>(a, lds, li, true);
    }
};

// The even-length R2C and C2R kernels with the 1-D boundary work inside:
// the caller's buffers in the storage type of half the compute precision
// (KF_NARROW_IN / KF_NARROW_OUT) and the zero interval [zl, zr) of the real
// side (KF_ZERO_IN on the R2C input, KF_ZERO_OUT on the C2R output), over
// real elements: element e of the packed line holds reals 2e and 2e + 1.
template <typename T>
__device__ __forceinline__ cpx<T> real_pair_mask(const KArgs& a, long long e, cpx<T> v) {
    const long long r = 2 * e;
    if (r >= a.zl && r < a.zr) v.re = (T)0;
    if (r + 1 >= a.zl && r + 1 < a.zr) v.im = (T)0;
    return v;
}
template <typename T, bool NTIO>
__device__ __forceinline__ cpx<T> ld_storage(const KArgs& a, const void* base, long long i) {
    if (a.flags & KF_NARROW_IN) {
        using U = typename Narrow<T>::type;
        const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)base + i);
        return mk((T)v.re, (T)v.im);
    }
    return ldg_in<NTIO>(a, (const cpx<T>*)base + i);
}
template <typename T, bool NTIO>
__device__ __forceinline__ void st_storage(const KArgs& a, void* base, long long i, cpx<T> v) {
    if (a.flags & KF_NARROW_OUT) {
        using U = typename Narrow<T>::type;
        stg_out<NTIO>(a, (cpx<U>*)base + i, mk((U)v.re, (U)v.im));
    } else {
        stg_out<NTIO>(a, (cpx<T>*)base + i, v);
    }
}

struct IoR2CHalfEdge : IoR2CHalf {
    static constexpr bool kPtrLoad = false;
    // direct first stage: one address per butterfly, the storage type
    // decided once per butterfly so its loads issue together
    static constexpr bool kBflyLoad = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        const long long i0 = L.ib + (long long)b * a.in_es, di = (long long)NB * a.in_es;
        if (a.flags & KF_NARROW_IN) {
            using U = typename Narrow<T>::type;
            const cpx<U>* x = (const cpx<U>*)a.in + i0;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const cpx<U> u = ldg_in<NTIO>(a, x + i * di);
                v[i] = mk((T)u.re, (T)u.im);
            }
        } else {
            const cpx<T>* x = (const cpx<T>*)a.in + i0;
#pragma unroll
            for (int i = 0; i < R; ++i) v[i] = ldg_in<NTIO>(a, x + i * di);
        }
        if (a.flags & KF_ZERO_IN) {
#pragma unroll
            for (int i = 0; i < R; ++i) v[i] = real_pair_mask(a, b + i * NB, v[i]);
        }
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        const cpx<T> v = ld_storage<T, NTIO>(a, a.in, L.ib + (long long)e * a.in_es);
        return (a.flags & KF_ZERO_IN) ? real_pair_mask(a, e, v) : v;
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoR2CHalfEdge, D>(a, lds, li, true);
    }
    // the postprocess of IoR2CHalf, stored in the storage type
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        const int M = D::N(a);
        coop_for(D::G(a), M + 1, true, [&](int g, int k) {
            if (!li[g].valid) return;
            const cpx<T>* Z = lds + g * D::LS(a);
            const int k0 = k == M ? 0 : k;
            const int km = k == 0 ? 0 : M - k;
            cpx<T> A = Z[lpad(k0, D::PS(a))];
            cpx<T> B = conj(Z[lpad(km, D::PS(a))]);
            cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
            cpx<T> X = (A + B) + muli<-1>(cmul(A - B, w));
            st_storage<T, D::NTO>(a, a.out, li[g].ob + (long long)k * a.out_es, scale(X, (T)0.5));
        });
    }
};

struct IoC2RHalfEdge : IoC2RHalf {
    static constexpr bool kPtrStore = false;
    // direct first stage: the pairs (X[k], X[M-k]) of a butterfly read
    // together, the storage type decided once per butterfly, the twiddles
    // W_N^k from the butterfly's root and the powers of its step
    static constexpr bool kBflyLoad = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        cpx<T> X[R], Xm[R];
        const long long di = (long long)NB * a.in_es;
        const long long i0 = L.ib + (long long)b * a.in_es, m0 = L.ib + (long long)(a.N - b) * a.in_es;
        if (a.flags & KF_NARROW_IN) {
            using U = typename Narrow<T>::type;
            const cpx<U>* x = (const cpx<U>*)a.in;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const cpx<U> p = ldg_in<NTIO>(a, x + i0 + i * di), q = ldg_in<NTIO>(a, x + m0 - i * di);
                X[i] = mk((T)p.re, (T)p.im);
                Xm[i] = mk((T)q.re, (T)q.im);
            }
        } else {
            const cpx<T>* x = (const cpx<T>*)a.in;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                X[i] = ldg_in<NTIO>(a, x + i0 + i * di);
                Xm[i] = ldg_in<NTIO>(a, x + m0 - i * di);
            }
        }
        const cpx<T> wb = tw2<T>(a.rlo, a.rhi, a.rshift, b);
        cpx<T> sp[R];
        root_powers<R>(tw2<T>(a.rlo, a.rhi, a.rshift, NB), sp);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const cpx<T> xm = conj(Xm[i]);
            v[i] = (X[i] + xm) + muli<1>(cmulc(X[i] - xm, cmul(wb, sp[i])));
        }
    }
    // direct last stage: one address per butterfly, the storage type decided
    // once per butterfly
    static constexpr bool kBflyStore = true;
    template <typename T, int S, bool NTIO, int R, int P>
    static __device__ __forceinline__ void store_bfly(const KArgs& a, const LineInfo& L, int base, const cpx<T>* v) {
        const long long o0 = L.ob + (long long)base * a.out_es, dq = (long long)P * a.out_es;
        cpx<T> w[R];
#pragma unroll
        for (int q = 0; q < R; ++q) {
            w[q] = scale(v[q], (T)a.scale);
            if (a.flags & KF_ZERO_OUT) w[q] = real_pair_mask(a, base + q * P, w[q]);
        }
        if (a.flags & KF_NARROW_OUT) {
            using U = typename Narrow<T>::type;
            cpx<U>* y = (cpx<U>*)a.out + o0;
#pragma unroll
            for (int q = 0; q < R; ++q) stg_out<NTIO>(a, y + q * dq, mk((U)w[q].re, (U)w[q].im));
        } else {
            cpx<T>* y = (cpx<T>*)a.out + o0;
#pragma unroll
            for (int q = 0; q < R; ++q) stg_out<NTIO>(a, y + q * dq, w[q]);
        }
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int k) {
        return load_tw<T, NTIO>(a, L, k, tw2<T>(a.rlo, a.rhi, a.rshift, k));
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_tw(const KArgs& a, const LineInfo& L, int k, cpx<T> w) {
        cpx<T> X = ld_storage<T, NTIO>(a, a.in, L.ib + (long long)k * a.in_es);
        cpx<T> Xm = conj(ld_storage<T, NTIO>(a, a.in, L.ib + (long long)(a.N - k) * a.in_es));
        return (X + Xm) + muli<1>(cmulc(X - Xm, w));
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        v = scale(v, (T)a.scale);
        if (a.flags & KF_ZERO_OUT) v = real_pair_mask(a, e, v);
        st_storage<T, NTIO>(a, a.out, L.ob + (long long)e * a.out_es, v);
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoC2RHalfEdge, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoC2RHalfEdge, D, T, S>(a, lds, li, true);
    }
};

// Four-step column pass. Line = column n2 of the [N1][N2] view (C = N2);
// FFT over n1 (length N1); store Y[k1][n2] * W_M^(dir * n2 * k1).
struct IoFsA : IoPlain {
    static constexpr int kLoad = LAY_COL;
    static constexpr int kStore = LAY_COL;
    static constexpr bool kStoreTw = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> tw_root(const KArgs& a, long long m) {
        return tw2<T>(a.tlo, a.thi, a.tshift, m);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_twiddled(const KArgs& a, const LineInfo& L, int e, cpx<T> v,
                                                          cpx<T> w) {
        stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, twmul<S>(v, w));
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_tw_at(const KArgs& a, cpx<T>* p, cpx<T> v, cpx<T> w) {
        stg_out<NTIO>(a, p, twmul<S>(v, w));
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        store_twiddled<T, S, NTIO>(a, L, e, v, tw2<T>(a.tlo, a.thi, a.tshift, L.tr * e));
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, false);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoFsA, D, T, S>(a, lds, li, false);
    }
};

struct IoFsABlue : IoFsA {
    static constexpr bool kPtrLoad = false;
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        const long long n = L.c + (long long)e * a.N2;
        if (n >= a.nvalid) return zero<T>();
        return cmul(ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es), ((const cpx<T>*)a.chirp)[n]);
    }
    // element e = b + i*NB sits at n = c + e*N2 of the padded line
    static constexpr bool kBflyLoad = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        long long n = L.c + (long long)b * a.N2;
        const long long dn = (long long)NB * a.N2;
        const cpx<T>* x = (const cpx<T>*)a.in + L.ib + (long long)b * a.in_es;
        const long long dx = (long long)NB * a.in_es;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            v[i] = n < a.nvalid ? cmul(ldg_in<NTIO>(a, x), chirp[n]) : zero<T>();
            n += dn;
            x += dx;
        }
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoFsABlue, D>(a, lds, li, false);
    }
};

struct IoFsAC2R : IoFsA {
    static constexpr bool kPtrLoad = false;
    static constexpr int kLoad = LAY_STAGED;
    // With KF_MIRROR_PAIRS a block owns H = G/2 columns n2 = j*H + g and
    // their mirrors N2 - n2 (column N2/2 stands in for the mirror of column
    // 0): X is read once into LDS and each pair (X[k], X[M-k]) is turned into
    // (Z[k], Z[M-k]) there. Needs N2 % G == 0, G even.
    static __device__ LineInfo line(const KArgs& a, long long blk, int g) {
        if (!(a.flags & KF_MIRROR_PAIRS)) return line_default(a, blk, g);
        const int H = a.G / 2;
        const long long nbk = a.N2 / (2 * H);
        LineInfo L;
        L.o = blk / nbk;
        const long long j = blk - L.o * nbk;
        long long c;
        if (g < H) {
            c = j * H + g;
        } else {
            c = a.N2 - (j * H + (g - H));
            if (c == a.N2) c = a.N2 / 2;
        }
        L.valid = L.o * a.N2 < a.nlines;
        if (!L.valid) L.o = 0;
        L.c = c;
        L.tr = c;
        L.ib = L.o * a.in_os + c * a.in_cs;
        L.ob = L.o * a.out_os + c * a.out_cs;
        return L;
    }
    // Z[k] = (X[k] + conj X[M-k]) + i (X[k] - conj X[M-k]) conj(w_k), w_k = exp(-2 pi i k / 2M)
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        return load_tw<T, NTIO>(a, L, e, tw2<T>(a.rlo, a.rhi, a.rshift, L.c + (long long)e * a.N2));
    }
    // w = W_N^k for k = c + e*N2
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_tw(const KArgs& a, const LineInfo& L, int e, cpx<T> w) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const long long k = L.c + (long long)e * a.N2;
        cpx<T> X = ldg_in<NTIO>(a, in + L.ib + e * a.in_es);
        cpx<T> Xm = conj(in[L.o * a.in_os + (a.M - k)]);
        return (X + Xm) + muli<1>(cmulc(X - Xm, w));
    }
    // Both members of a pair from A = X[k], B = X[M-k]; w_(M-k) = -conj(w_k)
    // (both in the form of load_tw, data operand first).
    template <typename T>
    static __device__ __forceinline__ void pair(const KArgs& a, long long k, cpx<T>& A, cpx<T>& B) {
        const cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
        const cpx<T> zk = (A + conj(B)) + muli<1>(cmulc(A - conj(B), w));
        const cpx<T> zm = (B + conj(A)) + muli<1>(cmulc(B - conj(A), mk(-w.re, w.im)));
        A = zk;
        B = zm;
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        if (!(a.flags & KF_MIRROR_PAIRS)) {
            staged_load<IoFsAC2R, D>(a, lds, li, false);
            return;
        }
        staged_load<IoPlain, D>(a, lds, li, false);  // X of the 2H columns, each element once
        __syncthreads();
        pair_fixup<T, D>(a, lds, li);
    }
    // (X[k], X[M-k]) -> (Z[k], Z[M-k]) in LDS for the mirror-pair layout
    template <typename T, class D>
    static __device__ void pair_fixup(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        if (!(a.flags & KF_MIRROR_PAIRS)) return;
        const int N1 = D::N(a), H = D::G(a) / 2, LS = D::LS(a), PS = D::PS(a);
        const long long N2 = a.N2;
        const bool first = li[0].c == 0;  // the block holding columns 0 and N2/2
        // regular pairs: column c (line g) row e with column N2 - c (line g + H) row N1-1-e
        for (int idx = threadIdx.x; idx < H * N1; idx += blockDim.x) {
            const int e = idx / H, g = idx - e * H;
            if (first && g == 0) continue;
            cpx<T>& A = lds[g * LS + lpad(e, PS)];
            cpx<T>& B = lds[(g + H) * LS + lpad(N1 - 1 - e, PS)];
            pair<T>(a, li[g].c + (long long)e * N2, A, B);
        }
        if (first) {
            // column 0: rows e and N1 - e; row 0 pairs with the Nyquist bin X[M]
            for (int e = threadIdx.x; e <= N1 / 2; e += blockDim.x) {
                cpx<T>& A = lds[lpad(e, PS)];
                if (e == 0) {
                    cpx<T> B = ((const cpx<T>*)a.in)[li[0].o * a.in_os + a.M];
                    pair<T>(a, 0, A, B);
                } else if (2 * e == N1) {
                    cpx<T> B = A;
                    pair<T>(a, (long long)e * N2, A, B);
                } else {
                    pair<T>(a, (long long)e * N2, A, lds[lpad(N1 - e, PS)]);
                }
            }
            // column N2/2 (line H): rows e and N1-1-e
            for (int e = threadIdx.x; e < N1 / 2; e += blockDim.x)
                pair<T>(a, (long long)e * N2 + N2 / 2, lds[H * LS + lpad(e, PS)], lds[H * LS + lpad(N1 - 1 - e, PS)]);
        }
    }
};

// C2R column pass with direct loads: with KF_MIRROR_PAIRS the block owns
// columns and their mirrors, and every element reads its own X[k] and its
// partner X[M-k] (load_elem): the partner's second read is served by the
// L1/L2 of the same CU, and the staged prologue with its LDS pair pass and
// barrier goes away.
struct IoFsAC2RDirect : IoFsAC2R {
    static constexpr int kLoad = LAY_COL;
    static constexpr bool kLoadTw = true;
    static constexpr bool kPairFirst = true;
    // the block holding column 0 and the stand-in column N2/2, whose pairs
    // differ from the regular (c, e) <-> (N2 - c, N1-1-e); g = this line's
    // slot, H = G/2 (the same answer on every thread of a block)
    static __device__ __forceinline__ bool pair_special(const KArgs& a, const LineInfo& L, int g, int H) {
        return g < H ? L.c == g : g == H ? L.c == a.N2 / 2 : L.c == a.N2 - (g - H);
    }
    // root(c + b*N2) for butterfly b; the step NB advances k by NB*N2
    template <typename T>
    static __device__ __forceinline__ cpx<T> ltw_root(const KArgs& a, const LineInfo& L, int m, bool step = false) {
        return tw2<T>(a.rlo, a.rhi, a.rshift, (step ? 0 : L.c) + (long long)m * a.N2);
    }
};

// The first pass of a mixed-storage two-upload C2C: IoFsA reading the
// caller's input in the storage type of half the compute precision
// (KF_NARROW_IN), with the line's input zero interval [zl, zr) read as zero
// (KF_ZERO_IN); element n1 of column n2 is line element n2 + n1 * N2.
struct IoFsAEdge : IoFsA {
    static constexpr bool kPtrLoad = false;
    // direct first stage: one storage-type address per butterfly
    static constexpr bool kBflyLoad = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        using U = typename Narrow<T>::type;
        const cpx<U>* x = (const cpx<U>*)a.in + L.ib + (long long)b * a.in_es;
        const long long dx = (long long)NB * a.in_es;
        const bool zi = (a.flags & KF_ZERO_IN) != 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const cpx<U> u = ldg_in<NTIO>(a, x + i * dx);
            const long long n = L.c + (long long)(b + i * NB) * a.N2;
            v[i] = (zi && n >= a.zl && n < a.zr) ? zero<T>() : mk((T)u.re, (T)u.im);
        }
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        if (a.flags & KF_ZERO_IN) {
            const long long n = L.c + (long long)e * a.N2;
            if (n >= a.zl && n < a.zr) return zero<T>();
        }
        using U = typename Narrow<T>::type;
        const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)a.in + L.ib + e * a.in_es);
        return mk((T)v.re, (T)v.im);
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoFsAEdge, D>(a, lds, li, false);
    }
};

// Four-step row pass. Line = row k1 (C = N1), contiguous in the scratch;
// FFT over n2 (length N2); store X[k1 + N1*k2] (column-coalesced).
struct IoFsB : IoPlain {
    static constexpr int kLoad = LAY_ROW;
    static constexpr int kStore = LAY_COL;
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoPlain, D, T, S>(a, lds, li, false);
    }
};

// The last pass of a mixed-storage two-upload C2C: IoFsB writing the
// caller's output in the storage type of half the compute precision (scaled,
// rounded to nearest, KF_NARROW_OUT), with the line's output zero interval
// [zl, zr) written as zero (KF_ZERO_OUT); element k2 of row k1 is line
// element k1 + k2 * N1.
struct IoFsBEdge : IoFsB {
    static constexpr bool kPtrStore = false;
    // direct last stage: one storage-type address per butterfly
    static constexpr bool kBflyStore = true;
    template <typename T, int S, bool NTIO, int R, int P>
    static __device__ __forceinline__ void store_bfly(const KArgs& a, const LineInfo& L, int base, const cpx<T>* v) {
        using U = typename Narrow<T>::type;
        cpx<U>* y = (cpx<U>*)a.out + L.ob + (long long)base * a.out_es;
        const long long dy = (long long)P * a.out_es;
        const T sc = (T)a.scale;
        const bool zo = (a.flags & KF_ZERO_OUT) != 0;
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const long long k = L.c + (long long)(base + q * P) * a.N1;
            const bool z = zo && k >= a.zl && k < a.zr;
            stg_out<NTIO>(a, y + q * dy, z ? mk((U)0, (U)0) : mk((U)(v[q].re * sc), (U)(v[q].im * sc)));
        }
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        v = scale(v, (T)a.scale);
        if (a.flags & KF_ZERO_OUT) {
            const long long k = L.c + (long long)e * a.N1;
            if (k >= a.zl && k < a.zr) v = zero<T>();
        }
        using U = typename Narrow<T>::type;
        stg_out<NTIO>(a, (cpx<U>*)a.out + L.ob + e * a.out_es, mk((U)v.re, (U)v.im));
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoFsBEdge, D, T, S>(a, lds, li, false);
    }
};

// Row pass of the packed half-size FFT for a large even R2C. A block owns H
// rows k1 = j*H + h and their mirrors N1 - k1 (row N1/2 replaces the mirror of
// row 0), so Z[k] and Z[M-k] are both in its LDS when the postprocess
// X[k] = 1/2 [(Z[k] + conj Z[M-k]) - i W_N^k (Z[k] - conj Z[M-k])] runs.
struct IoFsBR2C : IoPlain {
    static constexpr int kLoad = LAY_ROW;
    static constexpr int kStore = LAY_STAGED;
    static __device__ LineInfo line(const KArgs& a, long long blk, int g) {
        const int H = a.G / 2;
        const long long nbk = a.N1 / (2 * H);
        LineInfo L;
        L.o = blk / nbk;
        const long long j = blk - L.o * nbk;
        long long k1;
        if (g < H) {
            k1 = j * H + g;
        } else {
            k1 = a.N1 - (j * H + (g - H));
            if (k1 == a.N1) k1 = a.N1 / 2;
        }
        L.valid = L.o * a.N1 < a.nlines;
        if (!L.valid) L.o = 0;
        L.c = k1;
        L.tr = k1;
        L.ib = L.o * a.in_os + k1 * a.in_cs;
        L.ob = L.o * a.out_os;
        return L;
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, true);
    }
    // Column-major over (row g, bin k2) with the block size a multiple of G:
    // each thread keeps its row and steps k2 by blockDim/G, so the twiddle
    // W_N^k (k = k1 + N1*k2) advances by one multiplication with W_N^(N1*dk)
    // (at most 32 steps per thread) instead of two table loads per element.
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const int G = D::G(a), H = G / 2;
        const int N2 = D::N(a);
        const int g = (int)threadIdx.x % G;
        const int dk = (int)blockDim.x / G;
        if (!li[g].valid) return;
        const long long k1 = li[g].c;
        const cpx<T>* row = lds + g * D::LS(a);
        int gp, mirror;  // mirror partner: row gp, bin (mirror - k2) or N2 - k2 for row 0
        if (k1 == 0) {
            gp = g;
            mirror = N2;
        } else if (2 * k1 == a.N1) {
            gp = g;
            mirror = N2 - 1;
        } else {
            gp = g < H ? g + H : g - H;
            mirror = N2 - 1;
        }
        const cpx<T>* prow = lds + gp * D::LS(a);
        int k2 = (int)threadIdx.x / G;
        cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k1 + a.N1 * (long long)k2);
        const cpx<T> wstep = tw2<T>(a.rlo, a.rhi, a.rshift, a.N1 * (long long)dk);
        for (; k2 < N2; k2 += dk) {
            const int k2m = (k1 == 0 && k2 == 0) ? 0 : mirror - k2;
            const long long k = k1 + a.N1 * k2;
            cpx<T> A = row[lpad(k2, D::PS(a))];
            cpx<T> B = conj(prow[lpad(k2m, D::PS(a))]);
            cpx<T> X = (A + B) + muli<-1>(cmul(A - B, w));
            stg_out<D::NTO>(a, out + li[g].ob + k, scale(X, (T)0.5));
            if (k == 0) out[li[g].ob + a.M] = mk(A.re - A.im, (T)0);
            w = cmul(w, wstep);
        }
    }
};

// Bluestein row pass: FFT over n2, multiply by the kernel spectrum (stored
// transposed as spec[k1*N2 + k2] with 1/M folded in), inverse FFT over k2 and
// the inverse four-step twiddle W_M^(-k1*m2); rows stay in place.
struct IoBlueB : IoPlain {
    static constexpr bool kPtrStore = false;
    static constexpr bool kTwoPass = true;
    static constexpr int kLoad = LAY_ROW;
    static constexpr int kStore = LAY_ROW;
    template <typename T, class D>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>& v = lds[g * D::LS(a) + lpad(e, D::PS(a))];
            v = cmul(v, spec[li[g].c * D::N(a) + e]);
        });
    }
    static constexpr bool kMidFused = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> mid_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        return cmul(v, ((const cpx<T>*)a.spec)[L.c * a.N + e]);
    }
    static constexpr bool kStoreTw = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> tw_root(const KArgs& a, long long m) {
        return tw2<T>(a.tlo, a.thi, a.tshift, m);
    }
    // the inverse pass twiddle root(-k1*m2) regardless of the kernel direction
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_twiddled(const KArgs& a, const LineInfo& L, int e, cpx<T> v,
                                                          cpx<T> w) {
        stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, cmulc(v, w));
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        store_twiddled<T, S, NTIO>(a, L, e, v, tw2<T>(a.tlo, a.thi, a.tshift, L.c * e));
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, true);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoBlueB, D, T, S>(a, lds, li, true);
    }
};

// Bluestein column pass: inverse FFT over k1 gives conv[m2 + N2*m1]; keep
// m < N and multiply by the chirp (and the caller's scale).
struct IoFsCBlue : IoPlain {
    static constexpr bool kPtrStore = false;
    static constexpr int kLoad = LAY_COL;
    static constexpr int kStore = LAY_COL;
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        const long long m = L.c + (long long)e * a.N2;
        if (m >= a.nout) return;
        stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, scale(cmul(v, ((const cpx<T>*)a.chirp)[m]), (T)a.scale));
    }
    // outputs e = base + q*P sit at m = c + e*N2 of the convolution
    static constexpr bool kBflyStore = true;
    template <typename T, int S, bool NTIO, int R, int P>
    static __device__ __forceinline__ void store_bfly(const KArgs& a, const LineInfo& L, int base, const cpx<T>* v) {
        long long m = L.c + (long long)base * a.N2;
        const long long dm = (long long)P * a.N2;
        cpx<T>* y = (cpx<T>*)a.out + L.ob + (long long)base * a.out_es;
        const long long dy = (long long)P * a.out_es;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        const T sc = (T)a.scale;
#pragma unroll
        for (int q = 0; q < R; ++q) {
            if (m < a.nout) stg_out<NTIO>(a, y, scale(cmul(v[q], chirp[m]), sc));
            m += dm;
            y += dy;
        }
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoPlain, D>(a, lds, li, false);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoFsCBlue, D, T, S>(a, lds, li, false);
    }
};

// Whole Bluestein transform in LDS: a = chirp * x zero-padded to M = N,
// FFT, multiply by the kernel spectrum, IFFT, chirp multiply, truncate.
struct IoBlue1 : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    static constexpr bool kTwoPass = true;
    // M >= 2 N - 1: inputs from (M + 1) / 2 on are padding
    static constexpr int kZeroFrom(int M) { return (M + 1) / 2; }
    template <class D>
    static __device__ __forceinline__ int out_count(const KArgs& a) { return (int)a.nout; }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        if (e >= a.nvalid) return zero<T>();
        return cmul(ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es), ((const cpx<T>*)a.chirp)[e]);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        if (e >= a.nout) return;
        stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, scale(cmul(v, ((const cpx<T>*)a.chirp)[e]), (T)a.scale));
    }
    template <typename T, class D>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>& v = lds[g * D::LS(a) + lpad(e, D::PS(a))];
            v = cmul(v, spec[e]);
        });
    }
    static constexpr bool kMidFused = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> mid_elem(const KArgs& a, const LineInfo&, int e, cpx<T> v) {
        return cmul(v, ((const cpx<T>*)a.spec)[e]);
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoBlue1, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoBlue1, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};

// The one-upload Bluestein kernel with the 1-D boundary work inside: the
// caller's input read in the storage type of half the compute precision
// (KF_NARROW_IN) with the input zero interval [zl, zr) read as zero
// (KF_ZERO_IN) before the chirp weighting, and the output scaled, written in
// the storage type (KF_NARROW_OUT, rounded to nearest) with the output zero
// interval written as zero (KF_ZERO_OUT).
struct IoBlue1Edge : IoBlue1 {
    // direct first stage: one address per butterfly, the storage type decided
    // once per butterfly; padding elements (e >= N) load the line's last
    // element (the address stays inside the line) and are replaced by zero
    static constexpr bool kBflyLoad = true;
    template <typename T, bool NTIO, int R, int NB>
    static __device__ __forceinline__ void load_bfly(const KArgs& a, const LineInfo& L, int b, cpx<T>* v) {
        constexpr int ZF = kZeroFrom(R * NB);
        const long long last = a.nvalid - 1;
        cpx<T> u[R];
        if (a.flags & KF_NARROW_IN) {
            using U = typename Narrow<T>::type;
            const cpx<U>* x = (const cpx<U>*)a.in + L.ib;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                if (i * NB < ZF) {
                    const long long e = b + i * NB;
                    const cpx<U> w = ldg_in<NTIO>(a, x + (e < last ? e : last) * a.in_es);
                    u[i] = mk((T)w.re, (T)w.im);
                }
            }
        } else {
            const cpx<T>* x = (const cpx<T>*)a.in + L.ib;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                if (i * NB < ZF) {
                    const long long e = b + i * NB;
                    u[i] = ldg_in<NTIO>(a, x + (e < last ? e : last) * a.in_es);
                }
            }
        }
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        const bool zi = (a.flags & KF_ZERO_IN) != 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if (i * NB < ZF) {
                const long long e = b + i * NB;
                const long long ec = e < last ? e : last;
                const bool keep = e <= last && !(zi && e >= a.zl && e < a.zr);
                v[i] = keep ? cmul(u[i], chirp[ec]) : zero<T>();
            } else {
                v[i] = zero<T>();
            }
        }
    }
    template <typename T, bool NTIO = false>
    static __device__ __forceinline__ cpx<T> load_elem(const KArgs& a, const LineInfo& L, int e) {
        if (e >= a.nvalid) return zero<T>();
        if ((a.flags & KF_ZERO_IN) && e >= a.zl && e < a.zr) return zero<T>();
        cpx<T> x;
        if (a.flags & KF_NARROW_IN) {
            using U = typename Narrow<T>::type;
            const cpx<U> v = ldg_in<NTIO>(a, (const cpx<U>*)a.in + L.ib + e * a.in_es);
            x = mk((T)v.re, (T)v.im);
        } else {
            x = ldg_in<NTIO>(a, (const cpx<T>*)a.in + L.ib + e * a.in_es);
        }
        return cmul(x, ((const cpx<T>*)a.chirp)[e]);
    }
    template <typename T, int S, bool NTIO = false>
    static __device__ __forceinline__ void store_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        if (e >= a.nout) return;
        v = scale(cmul(v, ((const cpx<T>*)a.chirp)[e]), (T)a.scale);
        if ((a.flags & KF_ZERO_OUT) && e >= a.zl && e < a.zr) v = zero<T>();
        if (a.flags & KF_NARROW_OUT) {
            using U = typename Narrow<T>::type;
            stg_out<NTIO>(a, (cpx<U>*)a.out + L.ob + e * a.out_es, mk((U)v.re, (U)v.im));
        } else {
            stg_out<NTIO>(a, (cpx<T>*)a.out + L.ob + e * a.out_es, v);
        }
    }
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        staged_load<IoBlue1Edge, D>(a, lds, li, a.flags & KF_IN_ROWMAJOR);
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        staged_store<IoBlue1Edge, D, T, S>(a, lds, li, a.flags & KF_OUT_ROWMAJOR);
    }
};

// Convolution of one tensor line in one kernel (performConvolution,
// convolution_ir.rs:4252-4440, with the multiply that the reference fuses
// into its last forward / first inverse upload): staged load, forward FFT,
// spectrum multiply in LDS, inverse FFT, store scaled by 1/N (the inverse
// child is always normalized). Every line (a scalar convolution: one
// coordinate, one kernel) is multiplied by the one kernel-spectrum plane.
struct IoConv1 : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    static constexpr bool kTwoPass = true;
    static constexpr int kLoad = LAY_STAGED;
    static constexpr int kStore = LAY_STAGED;
    // 1-D lines of a fan-out over kernels and coordinates (C = 1, line =
    // o * C1 + o1, spec_os or spec_os1 set): c holds the offset of the line's
    // spectrum plane, o * spec_os + o1 * spec_os1 (N2 = 1)
    static __device__ LineInfo line(const KArgs& a, long long blk, int g) {
        LineInfo L = line_default(a, blk, g);
        if (a.C == 1 && (a.spec_os || a.spec_os1)) {
            const long long o1 = (L.valid ? blk * a.G + g : 0) - L.o * a.C1;
            L.c = L.o * a.spec_os + o1 * a.spec_os1;
        }
        return L;
    }
    // element e of line (o, c) multiplies the spectrum at c + e * N2: a 1-D
    // line (C = 1, N2 = 1) its spectrum plane, an axis-0 line of an N-D
    // tensor (column c of C = N2 = the product of the other axes) its column
    template <typename T, class D>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        if (a.flags & KF_CONV_MATRIX) {
            mid_matrix<T, D>(a, lds, li);
            return;
        }
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>& v = lds[g * D::LS(a) + lpad(e, D::PS(a))];
            cpx<T> x = v;
            if (a.flags & KF_CONV_CONJ) x = conj(x);
            cpx<T> y = cmul(x, spec[li[g].c + (long long)e * a.N2]);
            if (a.flags & KF_CONV_CROSS) {
                const T r = (T)1 / sqrt(y.re * y.re + y.im * y.im);
                y = mk(y.re * r, y.im * r);
            }
            v = y;
        });
    }
    // Matrix convolution (ConvolutionMatrixLayout, convolution_ir.rs:128-147):
    // for the M = C1 coordinate lines g0 .. g0 + M - 1 of a system and each
    // bin e, y_o = sum_i prep(x_i) K[plane(o, i)][e], plane o*M + i, or the
    // upper-triangle index of (min, max) with KF_CONV_SYM; the system's
    // planes start at li[g0].c (its kernel's when there are several).
    template <typename T, class D>
    static __device__ void mid_matrix(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        const int M = (int)a.C1, n = D::N(a), S = D::G(a) / M;
        const bool sym = (a.flags & KF_CONV_SYM) != 0;
        for (int idx = (int)threadIdx.x; idx < S * n; idx += (int)blockDim.x) {
            const int sb = idx / n, e = idx - sb * n, g0 = sb * M;
            if (!li[g0].valid) continue;
            cpx<T> x[kMaxConvMatrix], y[kMaxConvMatrix];
            for (int i = 0; i < M; ++i) {
                x[i] = lds[(g0 + i) * D::LS(a) + lpad(e, D::PS(a))];
                if (a.flags & KF_CONV_CONJ) x[i] = conj(x[i]);
            }
            for (int o = 0; o < M; ++o) {
                cpx<T> acc = zero<T>();
                for (int i = 0; i < M; ++i) {
                    const int lo = i < o ? i : o, hi = i < o ? o : i;
                    const int plane = sym ? lo * M - lo * lo + hi : o * M + i;
                    acc = acc + cmul(x[i], spec[li[g0].c + (long long)plane * n + e]);
                }
                if (a.flags & KF_CONV_CROSS) {
                    const T r = (T)1 / sqrt(acc.re * acc.re + acc.im * acc.im);
                    acc = mk(acc.re * r, acc.im * r);
                }
                y[o] = acc;
            }
            for (int o = 0; o < M; ++o) lds[(g0 + o) * D::LS(a) + lpad(e, D::PS(a))] = y[o];
        }
    }
};

// IoConv1 on the fixed shapes: the first stage reads HBM and the last stage
// writes HBM in the shape's own lane mapping (rows of a 1-D convolution,
// axis-0 columns of an N-D one), and the spectrum product is applied as the
// forward FFT's last stage writes its outputs, so the block exchanges no
// extra LDS pass between the two FFTs.
struct IoConv1F : IoConv1 {
    static constexpr int kLoad = LAY_ANY;
    static constexpr int kStore = LAY_ANY;
    static constexpr bool kPtrLoad = true, kPtrStore = true;  // plain accesses, scale on store
    static constexpr bool kMidFused = true;
    template <typename T>
    static __device__ __forceinline__ cpx<T> mid_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        if constexpr (kIndexTest) return v;
        if (a.flags & KF_CONV_CONJ) v = conj(v);
        cpx<T> y = cmul(v, ((const cpx<T>*)a.spec)[L.c + (long long)e * a.N2]);
        if (a.flags & KF_CONV_CROSS) {
            const T r = (T)1 / sqrt(y.re * y.re + y.im * y.im);
            y = mk(y.re * r, y.im * r);
        }
        return y;
    }
};

// Row pass of a convolution over a two-upload length N = N1 * N2, between the
// forward column pass (KK_FS_A, W_N^(n2*k1) on store) and the inverse column
// pass (KK_FS_A over k1 with no twiddle): FFT of row k1 over n2, multiply by
// the kernel spectrum in natural order K[k1 + N1*k2] as KK_CONV_1 does
// (conjugated sequence, cross-power normalization) and by the 1/N of the
// normalized inverse, inverse FFT over k2, inverse twiddle W_N^(-k1*m2); rows
// stay in place. Three HBM passes instead of the two forward passes, the
// multiply pass and the two inverse passes.
struct IoConvB : IoBlueB {
    template <typename T>
    static __device__ __forceinline__ cpx<T> conv_mul(const KArgs& a, cpx<T> x, long long k) {
        if constexpr (kIndexTest) return x;
        if (a.flags & KF_CONV_CONJ) x = conj(x);
        cpx<T> y = cmul(x, ((const cpx<T>*)a.spec)[k]);
        if (a.flags & KF_CONV_CROSS) {
            const T r = (T)1 / sqrt(y.re * y.re + y.im * y.im);
            y = mk(y.re * r, y.im * r);
        }
        return scale(y, (T)a.scale);
    }
    template <typename T, class D>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>& v = lds[g * D::LS(a) + lpad(e, D::PS(a))];
            v = conv_mul(a, v, li[g].c + (long long)e * a.N1);
        });
    }
    template <typename T>
    static __device__ __forceinline__ cpx<T> mid_elem(const KArgs& a, const LineInfo& L, int e, cpx<T> v) {
        return conv_mul(a, v, L.c + (long long)e * a.N1);
    }
};

// Rader, FFT convolution (rader_ir.rs:1957-2101): a[s] = x[g^-s] gathered
// into LDS, FFT of length p-1 (= N here), multiply by FFT(b)/(p-1) with
// b[n] = exp(dir 2 pi i g^n / p), inverse FFT, X[g^m] = x0 + conv[m] and
// X[0] = x0 + A[0] (the DC of the gathered sequence is sum x - x0). x0 sits
// in the last LDS slot of the line so in-place execution is safe.
struct IoRader : IoPlain {
    static constexpr bool kPtrLoad = false, kPtrStore = false;
    static constexpr bool kTwoPass = true;
    static constexpr int kLoad = LAY_STAGED;
    static constexpr int kStore = LAY_STAGED;
    template <typename T, class D>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>* line = lds + g * D::LS(a);
            line[lpad(e, D::PS(a))] = li[g].valid ? in[li[g].ib + (long long)a.pin[e] * a.in_es] : zero<T>();
            if (e == 0) line[D::LS(a) - 1] = li[g].valid ? in[li[g].ib] : zero<T>();
        });
    }
    template <typename T, class D>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            cpx<T>* line = lds + g * D::LS(a);
            cpx<T>& v = line[lpad(e, D::PS(a))];
            if (e == 0 && li[g].valid)
                ((cpx<T>*)a.out)[li[g].ob] = scale(line[D::LS(a) - 1] + v, (T)a.scale);
            v = cmul(v, spec[e]);
        });
    }
    template <typename T, int S, class D>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        coop_for(D::G(a), D::N(a), true, [&](int g, int e) {
            if (!li[g].valid) return;
            const cpx<T>* line = lds + g * D::LS(a);
            out[li[g].ob + (long long)a.pout[e] * a.out_es] =
                scale(line[D::LS(a) - 1] + line[lpad(e, D::PS(a))], (T)a.scale);
        });
    }
};

// Rader by direct multiplication for small primes whose p-1 is not
// Stockham-smooth (rader_ir.rs:381): one thread per convolution output m,
// conv[m] = sum_s a[s] b[(m - s) mod (p-1)], b[n] = exp(dir 2 pi i g^n / p).
// N = p-1 <= 87, G lines per block, block = G * N threads.
template <typename T>
__global__ __launch_bounds__(512) void k_rader_direct(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    __shared__ LineInfo li[kMaxLinesPerBlock];
    const int tid = threadIdx.x, N = a.N;
    if (tid < a.G) li[tid] = line_default(a, blockIdx.x, tid);
    __syncthreads();
    const cpx<T>* in = (const cpx<T>*)a.in;
    for (int idx = tid; idx < a.G * (N + 1); idx += blockDim.x) {
        const int g = idx / (N + 1), s = idx - g * (N + 1);
        cpx<T> v = zero<T>();
        if (li[g].valid) v = s < N ? in[li[g].ib + (long long)a.pin[s] * a.in_es] : in[li[g].ib];
        lds[g * (N + 1) + s] = v;
    }
    __syncthreads();
    const int g = tid / N, m = tid - g * N;
    if (g >= a.G || !li[g].valid) return;
    const cpx<T>* av = lds + g * (N + 1);
    const cpx<T>* b = (const cpx<T>*)a.spec;
    const cpx<T> x0 = av[N];
    cpx<T>* out = (cpx<T>*)a.out;
    if constexpr (kIndexTest) {
        // identity arithmetic: the convolution with the unit impulse
        // (conv[m] = a[m]) and a[0] for the DC sum, so the gather and the
        // scatter show bit for bit
        out[li[g].ob + (long long)a.pout[m] * a.out_es] = x0 + av[m];
        if (m == 0) out[li[g].ob] = x0 + av[0];
        return;
    }
    cpx<T> acc = zero<T>(), dc = zero<T>();
    int bi = m;
    for (int s = 0; s < N; ++s) {
        acc = acc + cmul(av[s], b[bi]);
        dc = dc + av[s];
        bi = bi == 0 ? N - 1 : bi - 1;
    }
    const T sc = (T)a.scale;
    out[li[g].ob + (long long)a.pout[m] * a.out_es] = scale(x0 + acc, sc);
    if (m == 0) out[li[g].ob] = scale(x0 + dc, sc);
}

// ------------------------------------------------------- dynamic kernel

template <typename T, int S, class IO, bool WIDE, bool RAD = false>
__global__ __launch_bounds__(512) void k_dyn(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    __shared__ LineInfo li[kMaxLinesPerBlock];
    const int tid = threadIdx.x;
    if (tid < a.G) li[tid] = IO::line(a, group_index(a), tid);
    __syncthreads();
    IO::template prologue<T, DynDims>(a, lds, li);
    __syncthreads();
    const int g = tid / a.TT, t = tid - g * a.TT;
    cpx<T>* line = lds + g * a.LS;
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    // Rader stages (radix > kMaxStockhamRadix) stage their inputs in a second
    // region of G lines after the lines themselves
    cpx<T>* scr = RAD ? lds + a.G * a.LS + g * a.LS : nullptr;
    run_stages<T, S, WIDE, RAD>(line, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw, scr, a.rtab, a.roff);
    if constexpr (IO::kTwoPass) {
        IO::template mid<T, DynDims>(a, lds, li);
        __syncthreads();
        run_stages<T, -S, WIDE, RAD>(line, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw, scr, a.rtab, a.roff);
    }
    IO::template epilogue<T, S, DynDims>(a, lds, li);
}

// Runtime-shape C2C over lines contiguous in HBM (KF_DYN_DIRECT, chosen by
// the host): the first stage loads the line straight from HBM into registers
// and the last stage stores registers straight to HBM (threads of a line are
// adjacent lanes), so the line passes through LDS only between stages. Each
// thread computes its own line placement; lines past the end map onto line 0
// (loads in bounds, stores skipped).
template <typename T, int S, bool WIDE>
__global__ __launch_bounds__(512) void k_dyn_direct(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    const int tid = threadIdx.x;
    const int g = tid / a.TT, t = tid - g * a.TT;
    const LineInfo L = line_default(a, group_index(a), g);
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    run_stages_direct<T, S, WIDE>(lds + g * a.LS, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw,
                                  (const cpx<T>*)a.in + L.ib, (cpx<T>*)a.out + L.ob, L.valid, (T)a.scale);
}

// k_dyn_direct with the plan's boundary work at its HBM ends (KF_EDGE):
// storage of half the compute precision on the input (NI) / output (NO)
// side, the zero interval [zl, zr) on the input (KF_ZERO_IN) or the output
// (KF_ZERO_OUT) side.
template <typename T, int S, bool WIDE, bool NI, bool NO>
__global__ __launch_bounds__(512) void k_dyn_direct_edge(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    using UI = std::conditional_t<NI, typename Narrow<T>::type, T>;
    using UO = std::conditional_t<NO, typename Narrow<T>::type, T>;
    const int tid = threadIdx.x;
    const int g = tid / a.TT, t = tid - g * a.TT;
    const LineInfo L = line_default(a, group_index(a), g);
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    const bool zi = (a.flags & KF_ZERO_IN) != 0, zo = (a.flags & KF_ZERO_OUT) != 0;
    run_stages_direct_edge<T, S, WIDE, UI, UO>(lds + g * a.LS, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw,
                                               (const cpx<UI>*)a.in + L.ib, (cpx<UO>*)a.out + L.ob, L.valid,
                                               (T)a.scale, zi ? (int)a.zl : 0, zi ? (int)a.zr : 0,
                                               zo ? (int)a.zl : 0, zo ? (int)a.zr : 0);
}

// Runtime-shape even R2C of one upload (KF_DYN_DIRECT): the first stage loads
// the real input pairs straight from HBM (contiguous lines), the postprocess
// stays the staged epilogue of IoR2CHalf.
template <typename T, int S, bool WIDE>
__global__ __launch_bounds__(512) void k_dyn_r2c_direct(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    __shared__ LineInfo li[kMaxLinesPerBlock];
    const int tid = threadIdx.x;
    if (tid < a.G) li[tid] = IoR2CHalf::line(a, group_index(a), tid);
    __syncthreads();
    const int g = tid / a.TT, t = tid - g * a.TT;
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    run_stages_direct_in<T, S, WIDE>(lds + g * a.LS, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw,
                                     (const cpx<T>*)a.in + li[g].ib);
    IoR2CHalf::template epilogue<T, S, DynDims>(a, lds, li);
}

// First stage of the runtime-shape even C2R (P = 1), loading its inputs
// straight from HBM: element e of the half-length line is the preprocessed
// Z[e] = (X[e] + conj X[N-e]) + i (X[e] - conj X[N-e]) conj(w_e), from bins e
// and N-e of the N+1-bin input spectrum at `gsrc` (IoC2RHalf::load_tw, w_e
// from the two-level table of exp(-i pi e / N)). Written to LDS, then a
// barrier.
template <typename T, int S, int R, bool WIDE>
__device__ __noinline__ void stage_c2r_first(cpx<T>* __restrict__ line, const int N, const int TT, const int t,
                                             const int ps, const cpx<T>* gsrc, const void* rlo, const void* rhi,
                                             const int rshift) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_assume(__builtin_amdgcn_is_shared((const void*)line));
#endif
    typedef T v2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) v2* gsrc_t;
    constexpr int MJ = dyn_butterflies_per_thread(R, WIDE);
    const int NB = N / R;
    const int mask = (1 << rshift) - 1;
    // w_e for e = b + i NB is w_b (w_NB)^i: one two-level lookup per
    // butterfly and the powers of w_NB once per thread, instead of a lookup
    // per element
    cpx<T> sp[R];
    root_powers<R>(cmul(ld_table<T>(rhi, NB >> rshift), ld_table<T>(rlo, NB & mask)), sp);
    cpx<T> v[MJ][R];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (b < NB) {
            const cpx<T> wb = cmul(ld_table<T>(rhi, b >> rshift), ld_table<T>(rlo, b & mask));
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int e = b + i * NB;
                const v2 x = ((gsrc_t)gsrc)[e];
                const v2 y = ((gsrc_t)gsrc)[N - e];
                const cpx<T> X = mk(x.x, x.y), Xm = mk(y.x, -y.y);
                const cpx<T> w = i == 0 ? wb : cmul(wb, sp[i]);
                v[j][i] = (X + Xm) + muli<1>(cmulc(X - Xm, w));
            }
        }
    }
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (b < NB) {
            dft<R, S>(v[j]);
#pragma unroll
            for (int q = 0; q < R; ++q) line[lpad(b * R + q, ps)] = v[j][q];
        }
    }
    __syncthreads();
}

template <typename T, int S, bool WIDE>
__device__ __forceinline__ void stage_c2r_first_radix(int R, cpx<T>* __restrict__ line, const int N, const int TT,
                                                      const int t, const int ps, const cpx<T>* gsrc,
                                                      const void* rlo, const void* rhi, const int rshift) {
#define VKFX_C2R_CASE(RR) \
    case RR: stage_c2r_first<T, S, RR, WIDE>(line, N, TT, t, ps, gsrc, rlo, rhi, rshift); break;
    switch (R) {
        VKFX_C2R_CASE(3)
        VKFX_C2R_CASE(4)
        VKFX_C2R_CASE(5)
        VKFX_C2R_CASE(6)
        VKFX_C2R_CASE(7)
        VKFX_C2R_CASE(8)
        VKFX_C2R_CASE(9)
        VKFX_C2R_CASE(10)
        VKFX_C2R_CASE(11)
        VKFX_C2R_CASE(12)
        VKFX_C2R_CASE(13)
        VKFX_C2R_CASE(16)
        default: break;
    }
#undef VKFX_C2R_CASE
}

// Runtime-shape even C2R of one upload (KF_DYN_DIRECT): the first stage forms
// the preprocessed line from the input spectrum in HBM, the last stage stores
// the real output pairs straight to HBM (contiguous lines), so the line passes
// through LDS only between stages. At least two stages, neither end of radix
// 2. Lines past the end map onto line 0 (loads in bounds, stores skipped).
template <typename T, int S, bool WIDE>
__global__ __launch_bounds__(512) void k_dyn_c2r_direct(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    const int tid = threadIdx.x;
    const int g = tid / a.TT, t = tid - g * a.TT;
    const LineInfo L = IoC2RHalf::line(a, group_index(a), g);
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    cpx<T>* line = lds + g * a.LS;
    stage_c2r_first_radix<T, S, WIDE>(a.radix[0], line, a.N, a.TT, t, a.PS, (const cpx<T>*)a.in + L.ib, a.rlo,
                                      a.rhi, a.rshift);
    int P = a.radix[0];
    for (int s = 1; s + 1 < a.nstages; ++s) {
        stage_rt_radix<T, S, WIDE, SM_LDS>(a.radix[s], line, a.N, P, a.TT, t, a.PS, tw, nullptr, nullptr, 0, (T)1);
        P *= a.radix[s];
    }
    stage_rt_radix<T, S, WIDE, SM_LAST>(a.radix[a.nstages - 1], line, a.N, P, a.TT, t, a.PS, tw, nullptr,
                                        (cpx<T>*)a.out + L.ob, L.valid, (T)a.scale);
}

// Runtime-shape even C2R with KF_DYN_DIRECT but not KF_DYN_PRE: staged
// preprocess (IoC2RHalf prologue), last stage stored straight to HBM. The
// host takes it for lines whose first stage cannot load directly (one stage,
// a radix-2 first stage, or first-stage loads spanning under 128 bytes).
template <typename T, int S, bool WIDE>
__global__ __launch_bounds__(512) void k_dyn_c2r_direct_out(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    __shared__ LineInfo li[kMaxLinesPerBlock];
    const int tid = threadIdx.x;
    if (tid < a.G) li[tid] = IoC2RHalf::line(a, group_index(a), tid);
    __syncthreads();
    IoC2RHalf::template prologue<T, DynDims>(a, lds, li);
    __syncthreads();
    const int g = tid / a.TT, t = tid - g * a.TT;
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    cpx<T>* line = lds + g * a.LS;
    int P = 1;
    for (int s = 0; s + 1 < a.nstages; ++s) {
        stage_rt_radix<T, S, WIDE, SM_LDS>(a.radix[s], line, a.N, P, a.TT, t, a.PS, tw, nullptr, nullptr, 0, (T)1);
        P *= a.radix[s];
    }
    stage_rt_radix<T, S, WIDE, SM_LAST>(a.radix[a.nstages - 1], line, a.N, P, a.TT, t, a.PS, tw, nullptr,
                                        (cpx<T>*)a.out + li[g].ob, li[g].valid, (T)a.scale);
}

// -------------------------------------------------- fixed-shape kernel

template <int... R>
struct RList {};

// N: length, TT: threads per line, G: lines per block, PS: LDS pad shift,
// COL: lane mapping (false: threads of a line are adjacent lanes, for lines
// contiguous in HBM; true: lines are adjacent lanes, for strided lines).
// LS: LDS stride between lines in elements (chosen per shape to keep the
// stage reads and writes free of bank conflicts).
template <int N_, int TT_, int G_, int PS_, int LS_, bool COL_, int... R>
struct Shape {
    static constexpr int WPE = 0;  // waves-per-EU hint (0 = compiler default)
    static constexpr bool NTI = false, NTO = false;  // nontemporal HBM loads / stores
    static constexpr bool PP = false;  // ping-pong LDS buffers (see PingPong)
    static constexpr bool TWT = false;  // per-stage twiddle tables (see StageTables)
    static constexpr bool SPAD = false;  // per-stage LDS pads (see StagePads)
    static constexpr int N = N_, TT = TT_, G = G_, PS = PS_, LS = LS_;
    static constexpr bool COL = COL_;
    static_assert(LS_ >= N_ + ((N_ - 1) >> PS_), "LDS line stride too small");
    static_assert((R * ... * 1) == N_, "radices must multiply to the length");
    static_assert(G_ >= 1 && G_ <= kMaxLinesPerBlock && TT_ >= 1 && G_ * TT_ <= 1024, "block shape");
    using Radices = RList<R...>;
    using Dims = FixDims<N_, G_, LS_, PS_>;
};

// LDS slot of element e0 + i*STEP. When STEP is a multiple of the pad period
// 2^PS the pad of every element is the pad of e0 plus a constant, so the
// slots are one base plus compile-time offsets.
template <int PS, int STEP>
__device__ __forceinline__ int lds_step(int e0, int i) {
    if constexpr (PS >= 30) {
        return e0 + i * STEP;
    } else if constexpr (STEP % (1 << PS) == 0) {
        return lpad(e0, PS) + i * (STEP + (STEP >> PS));
    } else {
        return lpad(e0 + i * STEP, PS);
    }
}
// LDS slot of Stockham output base + q*P of a radix-R butterfly, base =
// (b - k)*R + k with k = b mod P. If P*R divides 2^PS the R outputs stay in
// one pad period of base, so they share its pad.
template <int PS, int P, int R>
__device__ __forceinline__ int lds_out(int base, int q) {
    if constexpr (PS >= 30) {
        return base + q * P;
    } else if constexpr (P % (1 << PS) == 0) {
        return lpad(base, PS) + q * (P + (P >> PS));
    } else if constexpr ((1 << PS) % (P * R) == 0) {
        return lpad(base, PS) + q * P;
    } else {
        return lpad(base + q * P, PS);
    }
}

// One stage with compile-time geometry. SRC/DST: 0 = the line in LDS,
// 1 = HBM through the IO policy's element functions.
// MID: this stage ends the first FFT of a two-pass kernel and applies the
// policy's pointwise product (IO::mid_elem) to its outputs on the way to LDS.
// PP: ping-pong; the stage reads `line` and writes `out` (a second LDS
// buffer), so no barrier separates its reads from its writes. Otherwise it
// works in place on `line` (`out` is unused).
// TOFF >= 0: the stage's twiddles W_{PR}^(k i), i = 1..R-1, are entries
// TOFF + k (R - 1) + i - 1 of the per-stage table at tw.full (FT_STAGE_PR
// layout); otherwise one root per butterfly from the W_N table and a product
// tree for its powers.
// PS: pad shift of the LDS buffer the stage reads; PSO: of the one it writes.
template <typename T, int S, class IO, int N, int P, int R, int TT, int PS, int SRC, int DST, bool NTI, bool NTO,
          bool MID = false, bool PP = false, int TOFF = -1, int PSO = PS>
__device__ __forceinline__ void fstage(const KArgs& a, cpx<T>* __restrict__ line, cpx<T>* __restrict__ out,
                                       const LineInfo& L, int t, const StageTw& tw) {
    cpx<T>* __restrict__ dst = PP ? out : line;
    constexpr int NB = N / R;
    constexpr int MJ = (NB + TT - 1) / TT;
    constexpr bool EXACT = (NB % TT) == 0;
    cpx<T> v[MJ][R];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (EXACT || b < NB) {
            if constexpr (SRC && IO::kPtrLoad) {
                // line() maps a line past the end onto line 0, so these loads
                // stay inside the buffer; such a line's stores are skipped
                const cpx<T>* p = IO::template in_ptr<T>(a, L, b);
                const long long st = (long long)NB * a.in_es;
#pragma unroll
                for (int i = 0; i < R; ++i) v[j][i] = ldg_in<NTI>(a, p + i * st);
            } else if constexpr (SRC && IO::kBflyLoad) {
                if (L.valid) {
                    IO::template load_bfly<T, NTI, R, NB>(a, L, b, v[j]);
                } else {
#pragma unroll
                    for (int i = 0; i < R; ++i) v[j][i] = zero<T>();
                }
            } else if constexpr (SRC && IO::kLoadTw) {
                // inputs b + i*NB carry the load twiddle root(b) * root(NB)^i
                if (L.valid) {
                    const cpx<T> wb = IO::template ltw_root<T>(a, L, b);
                    cpx<T> sp[R];
                    root_powers<R>(IO::template ltw_root<T>(a, L, NB, true), sp);
#pragma unroll
                    for (int i = 0; i < R; ++i)
                        v[j][i] = IO::template load_tw<T, NTI>(a, L, b + i * NB, cmul(wb, sp[i]));
                } else {
#pragma unroll
                    for (int i = 0; i < R; ++i) v[j][i] = zero<T>();
                }
            } else {
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    if constexpr (SRC) {
                        v[j][i] = (L.valid && i * NB < IO::kZeroFrom(N)) ? IO::template load_elem<T, NTI>(a, L, b + i * NB)
                                                                          : zero<T>();
                    } else {
                        v[j][i] = line[lds_step<PS, NB>(b, i)];
                    }
                }
            }
        }
    }
    if constexpr (!SRC && !PP) __syncthreads();
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
        const int b = t + j * TT;
        if (EXACT || b < NB) {
            const int k = b % P;
            if constexpr (P > 1) {
                constexpr int step = N / (P * R);
                cpx<T> wp[R];
                if constexpr (TOFF >= 0) {
#pragma unroll
                    for (int i = 1; i < R; ++i) wp[i] = ld_table<T>(tw.full, TOFF + k * (R - 1) + i - 1);
                } else {
                    root_powers<R>(stage_root<T>(tw, k * step, P >= kScatterP), wp);
                }
#pragma unroll
                for (int i = 1; i < R; ++i) v[j][i] = twmul<S>(v[j][i], wp[i]);
            }
            // a direct first stage whose inputs b + i NB, i >= R/2, are all padding
            constexpr bool kHalf = SRC && P == 1 && (R == 8 || R == 16) && (R / 2) * NB >= IO::kZeroFrom(N);
            if constexpr (kHalf)
                dft_upper_zero<R, S>(v[j]);
            else
                dft<R, S>(v[j]);
            const int base = (b - k) * R + k;
            if constexpr (DST && IO::kStoreTw) {
                // last stage: outputs o = b + q*N/R carry the pass twiddle
                // root(tr*o) = root(tr*b) * root(tr*N/R)^q
                if (L.valid) {
                    const cpx<T> wb = IO::template tw_root<T>(a, L.tr * b);
                    cpx<T> sp[R];
                    root_powers<R>(IO::template tw_root<T>(a, L.tr * NB), sp);
                    if constexpr (IO::kPtrStore) {
                        cpx<T>* p = IO::template out_ptr<T>(a, L, base);
                        const long long st = (long long)P * a.out_es;
#pragma unroll
                        for (int q = 0; q < R; ++q)
                            IO::template store_tw_at<T, S, NTO>(a, p + q * st, v[j][q], cmul(wb, sp[q]));
                    } else {
#pragma unroll
                        for (int q = 0; q < R; ++q)
                            IO::template store_twiddled<T, S, NTO>(a, L, base + q * P, v[j][q], cmul(wb, sp[q]));
                    }
                }
            } else if constexpr (DST && IO::kBflyStore) {
                if (L.valid) IO::template store_bfly<T, S, NTO, R, P>(a, L, base, v[j]);
            } else if constexpr (DST && IO::kPtrStore) {
                if (L.valid) {
                    cpx<T>* p = IO::template out_ptr<T>(a, L, base);
                    const long long st = (long long)P * a.out_es;
#pragma unroll
                    for (int q = 0; q < R; ++q) IO::template store_at<T, S, NTO>(a, p + q * st, v[j][q]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < R; ++q) {
                    if constexpr (DST) {
                        if (L.valid) IO::template store_elem<T, S, NTO>(a, L, base + q * P, v[j][q]);
                    } else {
                        if constexpr (MID) {
                            dst[lds_out<PSO, P, R>(base, q)] = IO::template mid_elem<T>(a, L, base + q * P, v[j][q]);
                        } else {
                            dst[lds_out<PSO, P, R>(base, q)] = v[j][q];
                        }
                    }
                }
            }
        }
    }
    if constexpr (!DST) __syncthreads();
}

// Runs the stages of Sh over one line. With ping-pong buffers stage k
// (1-based) writes `alt` when k is odd and `line` when k is even.
template <int R, int... Rest>
constexpr int rlist_head(RList<R, Rest...>) {
    return R;
}
// Per-stage pad of a stage's output buffer (StagePads shapes): the first
// stage (P = 1) writes its R outputs R slots apart across lanes, which one
// pad slot every R elements spreads over the banks when R is a power of two
// and the next stage's input stride N/Rn is a multiple of R (its reads then
// keep compile-time offsets); every other Stockham write and read is
// contiguous across lanes up to block steps that stay bank-distinct, so
// those buffers carry no pad (and no per-element pad arithmetic).
template <int N, int P, int R, int Rn>
constexpr int stage_pad() {
    return (P == 1 && Rn > 0 && (R & (R - 1)) == 0 && (N / Rn) % R == 0) ? (R == 2 ? 1 : R == 4 ? 2 : R == 8 ? 3 : 4)
                                                                         : 30;
}

// First stage of a C2R column pass over mirror-pair blocks (KF_MIRROR_PAIRS):
// line g < H holds column c, line g + H its mirror N2 - c, and element e of
// column c pairs with element N1-1-e of the mirror (X[M-k] for k = c + e*N2).
// Thread t of line g runs butterfly t of its own line and butterfly NB-1-t
// of the mirror line: the R pairs (X[k], X[M-k]) it loads for the first are,
// in reverse order, the inputs of the second, so every element is read once
// and each pair gives Z[k] and Z[M-k] from one twiddle (w_(M-k) = -conj w_k).
template <typename T, int S, class IO, class Sh, int R, int PSO>
__device__ __forceinline__ void fstage_c2r_pairs(const KArgs& a, cpx<T>* line, const LineInfo& L, int t) {
    constexpr int NB = Sh::N / R, H = Sh::G / 2;
    static_assert(Sh::COL && Sh::G % 2 == 0 && NB == 2 * Sh::TT, "mirror-pair first stage geometry");
    const int g = threadIdx.x % Sh::G;
    cpx<T>* mline = line + (g < H ? H : -H) * Sh::LS;
    cpx<T> v[R], u[R];
    if (L.valid) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const cpx<T>* xm = in + L.o * a.in_os + (a.M - L.c);  // X[M-k] = xm[-e*N2]
        const cpx<T> wb = IO::template ltw_root<T>(a, L, t);
        cpx<T> sp[R];
        root_powers<R>(IO::template ltw_root<T>(a, L, NB, true), sp);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int e = t + i * NB;
            const cpx<T> A = ldg_in<Sh::NTI>(a, in + L.ib + e * a.in_es);
            const cpx<T> B = ldg_in<Sh::NTI>(a, xm - (long long)e * a.N2);
            const cpx<T> w = cmul(wb, sp[i]);
            v[i] = (A + conj(B)) + muli<1>(cmulc(A - conj(B), w));
            u[R - 1 - i] = (B + conj(A)) + muli<1>(cmulc(B - conj(A), mk(-w.re, w.im)));
        }
    } else {
#pragma unroll
        for (int i = 0; i < R; ++i) v[i] = u[i] = zero<T>();
    }
    dft<R, S>(v);
    dft<R, S>(u);
#pragma unroll
    for (int q = 0; q < R; ++q) {
        line[lds_out<PSO, 1, R>(t * R, q)] = v[q];
        mline[lds_out<PSO, 1, R>((NB - 1 - t) * R, q)] = u[q];
    }
    __syncthreads();
}

// TO: offset of this stage's block in the per-stage twiddle table (stages
// with P > 1 hold P (R - 1) entries each, in radix order). PSI: pad of the
// buffer the stage reads.
template <typename T, int S, class IO, class Sh, int SRC0, int DSTL, bool MIDL, int P, int TO = 0,
          int PSI = (Sh::SPAD ? 30 : Sh::PS), int R, int... Rest>
__device__ __forceinline__ void fstages(const KArgs& a, cpx<T>* line, cpx<T>* alt, const LineInfo& L, int t,
                                        const StageTw& tw, RList<R, Rest...>) {
    constexpr bool last = sizeof...(Rest) == 0;
    constexpr int PSO = !Sh::SPAD ? Sh::PS : last ? 30 : stage_pad<Sh::N, P, R, rlist_head(RList<Rest..., 0>{})>();
    // every padded slot of the buffer this stage writes lies inside the line stride
    static_assert(PSO >= 30 || (Sh::N - 1) + ((Sh::N - 1) >> PSO) < Sh::LS, "LDS line stride below the padded length");
    constexpr bool kPairs = IO::kPairFirst && P == 1 && SRC0 && !last && !Sh::PP && !Sh::SPAD && Sh::COL &&
                            Sh::N / R == 2 * Sh::TT;
    if constexpr (kPairs) {
        if ((a.flags & KF_MIRROR_PAIRS) && (a.flags & KF_PAIR_LOADS) &&
            !IO::pair_special(a, L, (int)(threadIdx.x % Sh::G), Sh::G / 2)) {
            fstage_c2r_pairs<T, S, IO, Sh, R, PSO>(a, line, L, t);
        } else {
            fstage<T, S, IO, Sh::N, P, R, Sh::TT, PSI, SRC0, 0, Sh::NTI, Sh::NTO, false, false, -1, PSO>(a, line, alt,
                                                                                                       L, t, tw);
        }
    } else {
        fstage<T, S, IO, Sh::N, P, R, Sh::TT, PSI, (P == 1 ? SRC0 : 0), (last ? DSTL : 0), Sh::NTI, Sh::NTO,
               last && MIDL && !DSTL, Sh::PP, Sh::TWT ? TO : -1, PSO>(a, line, alt, L, t, tw);
    }
    if constexpr (!last)
        fstages<T, S, IO, Sh, SRC0, DSTL, MIDL, P * R, TO + (P > 1 ? P * (R - 1) : 0), PSO>(
            a, Sh::PP ? alt : line, Sh::PP ? line : alt, L, t, tw, RList<Rest...>{});
}
template <int... R>
constexpr int rlist_size(RList<R...>) {
    return (int)sizeof...(R);
}

template <class IO, bool COL>
struct Direct {
    static constexpr int mine = COL ? LAY_COL : LAY_ROW;
    static constexpr bool load = IO::kLoad == LAY_ANY || IO::kLoad == mine;
    static constexpr bool store = IO::kStore == LAY_ANY || IO::kStore == mine;
};

template <typename T, int S, class IO, class Sh>
__device__ __forceinline__ void fix_body(const KArgs& a, cpx<T>* lds, LineInfo* li, long long blk) {
    using D = typename Sh::Dims;
    constexpr bool LD = Direct<IO, Sh::COL>::load;
    constexpr bool SD = Direct<IO, Sh::COL>::store;
    const int tid = threadIdx.x;
    const int g = Sh::G == 1 ? 0 : Sh::COL ? tid % Sh::G : tid / Sh::TT;
    const int t = Sh::G == 1 ? tid : Sh::COL ? tid / Sh::G : tid % Sh::TT;
    // A pass that reads and writes HBM only from its own registers needs
    // nothing but its own line's placement: every thread computes it, with no
    // shared table and no barrier before the first loads. With one line per
    // block the placement is uniform (scalar registers), which also holds for
    // two-pass kernels whose mid product is fused into the stages.
    constexpr bool kOwnLine = LD && SD && (!IO::kTwoPass || (Sh::G == 1 && IO::kMidFused));
    if constexpr (!kOwnLine) {
        if (tid < Sh::G) li[tid] = IO::line(a, blk, tid);
        __syncthreads();
    }
    cpx<T>* line = lds + g * Sh::LS;
    // ping-pong shapes hold a second buffer of G lines behind the first; the
    // prologue fills the first, the stages alternate and the last stage
    // stores to HBM, so the policy's LDS-wide steps never see the second
    static_assert(!Sh::PP || (SD && (!IO::kTwoPass || IO::kMidFused)),
                  "ping-pong shapes need a direct last stage and a fused mid product");
    static_assert(!Sh::SPAD || (LD && SD && (!IO::kTwoPass || IO::kMidFused)),
                  "per-stage pads need direct first and last stages and a fused mid product");
    cpx<T>* alt = Sh::PP ? lds + (Sh::G + g) * Sh::LS : line;
    const StageTw tw{a.tw, a.swlo, a.swhi, a.swshift};
    const LineInfo L = kOwnLine ? IO::line(a, blk, g) : li[g];
    if constexpr (!LD) {
        IO::template prologue<T, D>(a, lds, li);
        __syncthreads();
    }
    if constexpr (IO::kTwoPass) {
        fstages<T, S, IO, Sh, LD ? 1 : 0, 0, IO::kMidFused, 1>(a, line, alt, L, t, tw, typename Sh::Radices{});
        if constexpr (!IO::kMidFused) {
            IO::template mid<T, D>(a, lds, li);
            __syncthreads();
        }
        // the first FFT's output sits in `alt` after an odd number of stages
        constexpr bool odd = (rlist_size(typename Sh::Radices{}) & 1) != 0;
        fstages<T, -S, IO, Sh, 0, SD ? 1 : 0, false, 1>(a, Sh::PP && odd ? alt : line, Sh::PP && odd ? line : alt,
                                                        L, t, tw, typename Sh::Radices{});
    } else {
        fstages<T, S, IO, Sh, LD ? 1 : 0, SD ? 1 : 0, false, 1>(a, line, alt, L, t, tw, typename Sh::Radices{});
    }
    if constexpr (!SD) IO::template epilogue<T, S, D>(a, lds, li);
}

// One block per group of G lines (grid = number of groups).
template <typename T, int S, class IO, class Sh>
__global__ __launch_bounds__(Sh::G* Sh::TT) void k_fix(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ LineInfo li[Sh::G];
    fix_body<T, S, IO, Sh>(a, reinterpret_cast<cpx<T>*>(smem_raw), li, group_index(a));
}

// Two LDS buffers of G lines each: every stage reads one and writes the
// other, one barrier per stage instead of two (for shapes whose LDS use
// leaves room for the second buffer at the residency they already have).
template <class Base>
struct PingPong : Base {
    static constexpr bool PP = true;
};

// Stage twiddles read from a per-stage table (FT_STAGE_PR) instead of one
// root and a product tree per butterfly: R-1 loads in place of R-2 complex
// multiplications (and the two-level lookup of large P).
template <class Base>
struct StageTables : Base {
    static constexpr bool TWT = true;
};

// Each stage's output buffer carries its own pad (stage_pad); Sh::PS is the
// smallest pad any stage uses, so LS covers every buffer.
template <class Base>
struct StagePads : Base {
    static constexpr bool SPAD = true;
};

// Variant shapes for tuning: a waves-per-EU occupancy hint and nontemporal IO.
template <class Base, int W, bool NTIN, bool NTOUT>
struct Tuned : Base {
    static constexpr int WPE = W;
    static constexpr bool NTI = NTIN, NTO = NTOUT;
    using Dims = FixDims<Base::N, Base::G, Base::LS, Base::PS, NTIN, NTOUT>;
};
template <typename T, int S, class IO, class Sh>
__global__ __launch_bounds__(Sh::G* Sh::TT) __attribute__((amdgpu_waves_per_eu(Sh::WPE > 0 ? Sh::WPE : 1, 8))) void k_fix_occ(
    const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ LineInfo li[Sh::G];
    fix_body<T, S, IO, Sh>(a, reinterpret_cast<cpx<T>*>(smem_raw), li, group_index(a));
}

// ------------------------------------------------------------- selection

template <typename T, int S, bool W>
KernelFn pick_dyn(KernelKind kind) {
    switch (kind) {
        case KK_PLAIN: return k_dyn<T, S, IoPlain, W>;
        case KK_R2C_FULL: return k_dyn<T, S, IoR2CFull, W>;
        case KK_C2R_FULL: return k_dyn<T, S, IoC2RFull, W>;
        case KK_R2C_HALF: return k_dyn<T, S, IoR2CHalf, W>;
        case KK_C2R_HALF: return k_dyn<T, S, IoC2RHalf, W>;
        case KK_FS_A: return k_dyn<T, S, IoFsA, W>;
        case KK_FS_A_BLUE: return k_dyn<T, S, IoFsABlue, W>;
        case KK_FS_A_C2R: return k_dyn<T, S, IoFsAC2R, W>;
        case KK_FS_B: return k_dyn<T, S, IoFsB, W>;
        case KK_FS_B_R2C: return k_dyn<T, S, IoFsBR2C, W>;
        case KK_BLUE_B: return k_dyn<T, S, IoBlueB, W>;
        case KK_FS_C_BLUE: return k_dyn<T, S, IoFsCBlue, W>;
        case KK_BLUE_1: return k_dyn<T, S, IoBlue1, W>;
        case KK_RADER_FFT: return k_dyn<T, S, IoRader, W>;
        case KK_RADER_DIRECT: return k_rader_direct<T>;
        case KK_CONV_1: return k_dyn<T, S, IoConv1, W>;
        default: return nullptr;
    }
}
// KK_PLAIN with boundary work (KF_EDGE): edge = 1 + narrow input + 2 * narrow
// output; staged ends, or HBM-direct ends over contiguous lines
template <typename T, int S, bool W>
KernelFn pick_edge(int edge, bool direct) {
    switch (edge) {
        case 1: return direct ? k_dyn_direct_edge<T, S, W, false, false> : k_dyn<T, S, IoEdge<false, false>, W>;
        case 2: return direct ? k_dyn_direct_edge<T, S, W, true, false> : k_dyn<T, S, IoEdge<true, false>, W>;
        case 3: return direct ? k_dyn_direct_edge<T, S, W, false, true> : k_dyn<T, S, IoEdge<false, true>, W>;
        case 4: return direct ? k_dyn_direct_edge<T, S, W, true, true> : k_dyn<T, S, IoEdge<true, true>, W>;
        default: return nullptr;
    }
}
template <typename T, int S>
KernelFn pick(KernelKind kind, bool wide, int direct, int edge, bool rad) {
    if (rad) {
        // Rader stages: the staged kernels of mixed-radix lines and of the
        // FFT-mode Rader kernel with a nested Rader prime
        if (direct || edge) return nullptr;
        if (kind == KK_PLAIN) return wide ? k_dyn<T, S, IoPlain, true, true> : k_dyn<T, S, IoPlain, false, true>;
        if (kind == KK_RADER_FFT) return wide ? k_dyn<T, S, IoRader, true, true> : k_dyn<T, S, IoRader, false, true>;
        return nullptr;
    }
    if (edge) {
        if (kind != KK_PLAIN || direct > 1) return nullptr;
        return wide ? pick_edge<T, S, true>(edge, direct == 1) : pick_edge<T, S, false>(edge, direct == 1);
    }
    if (direct && kind == KK_PLAIN) return wide ? k_dyn_direct<T, S, true> : k_dyn_direct<T, S, false>;
    if (direct && kind == KK_R2C_HALF)
        return wide ? k_dyn_r2c_direct<T, S, true> : k_dyn_r2c_direct<T, S, false>;
    if (direct == 2 && kind == KK_C2R_HALF)
        return wide ? k_dyn_c2r_direct<T, S, true> : k_dyn_c2r_direct<T, S, false>;
    if (direct && kind == KK_C2R_HALF)
        return wide ? k_dyn_c2r_direct_out<T, S, true> : k_dyn_c2r_direct_out<T, S, false>;
    return wide ? pick_dyn<T, S, true>(kind) : pick_dyn<T, S, false>(kind);
}

}  // namespace vkfx

// Registry entry of one fixed-shape instantiation. Radix lists are
// zero-terminated; nst is filled in by the registry lookup.
#define VKFX_FIXED_OCC(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, W, NTI, NTO, ...)                  \
    FixedKernel {                                                                                      \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                               \
            (KernelFn)(k_fix_occ<T, S, IO, Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, W, NTI, NTO>>) \
    }
// A ping-pong shape (two LDS buffers per line, lds_mult 2).
#define VKFX_FIXED_PP(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...)                              \
    FixedKernel {                                                                                              \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                                       \
            (KernelFn)(k_fix_occ<T, S, IO, PingPong<Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, 0, NTI, NTO>>>), \
            FT_STAGE, 2                                                                                        \
    }
// Ping-pong with per-stage twiddle tables.
#define VKFX_FIXED_PPT(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...)                            \
    FixedKernel {                                                                                              \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                                       \
            (KernelFn)(k_fix_occ<T, S, IO,                                                                     \
                                 StageTables<PingPong<Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, 0, NTI, NTO>>>>), \
            FT_STAGE_PR, 2                                                                                     \
    }
// Ping-pong with per-stage twiddle tables and per-stage pads.
#define VKFX_FIXED_PPTS(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...)                           \
    FixedKernel {                                                                                              \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                                       \
            (KernelFn)(k_fix_occ<T, S, IO,                                                                     \
                                 StagePads<StageTables<PingPong<Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, 0, NTI, NTO>>>>>), \
            FT_STAGE_PR, 2                                                                                     \
    }
// In place with per-stage twiddle tables (the shape's own pad).
#define VKFX_FIXED_T(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...)                               \
    FixedKernel {                                                                                              \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                                       \
            (KernelFn)(k_fix_occ<T, S, IO, StageTables<Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, 0, NTI, NTO>>>), \
            FT_STAGE_PR, 1                                                                                     \
    }
// In place (one LDS buffer) with per-stage twiddle tables and pads, and a
// waves-per-EU hint W.
#define VKFX_FIXED_TS(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, W, NTI, NTO, ...)                           \
    FixedKernel {                                                                                              \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                                       \
            (KernelFn)(k_fix_occ<T, S, IO, StagePads<StageTables<Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, W, NTI, NTO>>>>), \
            FT_STAGE_PR, 1                                                                                     \
    }
// A shape with the default launch bounds hint.
#define VKFX_SHAPE(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...)                                \
    FixedKernel {                                                                                      \
        KIND, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, 0, {__VA_ARGS__},                               \
            (KernelFn)(k_fix_occ<T, S, IO, Tuned<Shape<N, TT, G, PS, LS, COL, __VA_ARGS__>, 0, NTI, NTO>>) \
    }
// The same shape with nontemporal HBM streaming (inputs read once, outputs
// written once).
// NTI / NTO: nontemporal loads of the pass input / stores of its output.
#define VKFX_FIXED_NT(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, NTI, NTO, ...) \
    VKFX_FIXED_OCC(KIND, IO, T, PREC, S, N, TT, G, PS, LS, COL, 0, NTI, NTO, __VA_ARGS__)
