// fft_kernels_impl.hpp -- gfx950 kernels of the batched FFT path.
//
// Every kernel is one HBM pass over a set of "lines" (1-D sequences along one
// axis). A block owns G lines; each line is staged in LDS, transformed there
// by the Stockham stages of fft_device.hpp, and written back. IO policies
// decide where a line lives in HBM and which pointwise work is fused into the
// load (prologue) and the store (epilogue):
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
//   IoFsBR2C      row pass that owns mirror rows k1 and N1-k1 so the R2C
//                 postprocess is fused into the store
//   IoBlueB       Bluestein row pass: FFT, kernel-spectrum multiply, IFFT and
//                 the inverse four-step twiddle in one kernel
//   IoFsCBlue     Bluestein column pass: IFFT, chirp multiply, truncate to N
//   IoBlue1       whole Bluestein transform when the convolution fits LDS
#pragma once
#include <hip/hip_runtime.h>

#include "fft_device.hpp"
#include "kernels.hpp"

namespace vkfx {

struct LineInfo {
    long long ib, ob, o, c;
    int valid;
};

__device__ __forceinline__ LineInfo line_default(const KArgs& a, unsigned blk, int g) {
    LineInfo L;
    long long line = (long long)blk * a.G + g;
    L.valid = line < a.nlines;
    if (!L.valid) line = 0;
    L.o = line / a.C;
    L.c = line - L.o * a.C;
    L.ib = L.o * a.in_os + L.c * a.in_cs;
    L.ob = L.o * a.out_os + L.c * a.out_cs;
    return L;
}

// Visits (g, e) for g < G, e < n with consecutive threads on consecutive
// addresses: e fastest when lines are contiguous, g fastest otherwise.
template <class F>
__device__ __forceinline__ void coop_for(int G, int n, bool rowmajor, F&& f) {
    const int total = G * n;
    if (rowmajor) {
        for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
            const int g = idx / n;
            f(g, idx - g * n);
        }
    } else {
        for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
            const int e = idx / G;
            f(idx - e * G, e);
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

// ---------------------------------------------------------------- IO kinds

struct IoPlain {
    static constexpr bool kTwoPass = false;
    static __device__ LineInfo line(const KArgs& a, unsigned blk, int g) { return line_default(a, blk, g); }
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        coop_for(a.G, a.N, a.flags & KF_IN_ROWMAJOR, [&](int g, int e) {
            lds[g * a.LS + lpad(e, a.PS)] = li[g].valid ? in[li[g].ib + e * a.in_es] : zero<T>();
        });
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const T s = (T)a.scale;
        coop_for(a.G, a.N, a.flags & KF_OUT_ROWMAJOR, [&](int g, int e) {
            if (li[g].valid) out[li[g].ob + e * a.out_es] = scale(lds[g * a.LS + lpad(e, a.PS)], s);
        });
    }
};

struct IoR2CFull : IoPlain {
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const T* in = (const T*)a.in;
        coop_for(a.G, a.N, a.flags & KF_IN_ROWMAJOR, [&](int g, int e) {
            lds[g * a.LS + lpad(e, a.PS)] = li[g].valid ? mk(in[li[g].ib + e * a.in_es], (T)0) : zero<T>();
        });
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const T s = (T)a.scale;
        coop_for(a.G, (int)a.nout, a.flags & KF_OUT_ROWMAJOR, [&](int g, int e) {
            if (li[g].valid) out[li[g].ob + e * a.out_es] = scale(lds[g * a.LS + lpad(e, a.PS)], s);
        });
    }
};

struct IoC2RFull : IoPlain {
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const int n = a.N, h = n / 2 + 1;
        coop_for(a.G, n, a.flags & KF_IN_ROWMAJOR, [&](int g, int e) {
            cpx<T> v = zero<T>();
            if (li[g].valid) v = e < h ? in[li[g].ib + e * a.in_es] : conj(in[li[g].ib + (n - e) * a.in_es]);
            lds[g * a.LS + lpad(e, a.PS)] = v;
        });
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        T* out = (T*)a.out;
        const T s = (T)a.scale;
        coop_for(a.G, a.N, a.flags & KF_OUT_ROWMAJOR, [&](int g, int e) {
            if (li[g].valid) out[li[g].ob + e * a.out_es] = lds[g * a.LS + lpad(e, a.PS)].re * s;
        });
    }
};

// Even-length R2C with the half-size FFT (length M = a.N) in LDS. Input is
// the real line viewed as M complex pairs z[n] = x[2n] + i x[2n+1].
struct IoR2CHalf : IoPlain {
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const int M = a.N;
        coop_for(a.G, M + 1, a.flags & KF_OUT_ROWMAJOR, [&](int g, int k) {
            if (!li[g].valid) return;
            const cpx<T>* Z = lds + g * a.LS;
            const int k0 = k == M ? 0 : k;
            const int km = k == 0 ? 0 : M - k;
            cpx<T> A = Z[lpad(k0, a.PS)];
            cpx<T> B = conj(Z[lpad(km, a.PS)]);
            cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
            cpx<T> X = (A + B) + muli<-1>(cmul(w, A - B));
            out[li[g].ob + k * a.out_es] = scale(X, (T)0.5);
        });
    }
};

// Even-length C2R: Z[k] = (X[k] + conj X[M-k]) + i W_N^-k (X[k] - conj X[M-k]),
// then the inverse half-size FFT; the complex result is the real output pairs.
struct IoC2RHalf : IoPlain {
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const int M = a.N;
        coop_for(a.G, M, a.flags & KF_IN_ROWMAJOR, [&](int g, int k) {
            cpx<T> Z = zero<T>();
            if (li[g].valid) {
                cpx<T> X = in[li[g].ib + k * a.in_es];
                cpx<T> Xm = conj(in[li[g].ib + (M - k) * a.in_es]);
                cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
                Z = (X + Xm) + muli<1>(cmulc(X - Xm, w));
            }
            lds[g * a.LS + lpad(k, a.PS)] = Z;
        });
    }
};

// Four-step column pass. Line = column n2 of the [N1][N2] view (C = N2);
// FFT over n1 (length N1 = a.N); store Y[k1][n2] * W_M^(dir * n2 * k1).
struct IoFsA : IoPlain {
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        coop_for(a.G, a.N, false, [&](int g, int e) {
            if (!li[g].valid) return;
            cpx<T> w = tw2<T>(a.tlo, a.thi, a.tshift, li[g].c * e);
            out[li[g].ob + e * a.out_es] = twmul<S>(lds[g * a.LS + lpad(e, a.PS)], w);
        });
    }
};

struct IoFsABlue : IoFsA {
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        coop_for(a.G, a.N, false, [&](int g, int e) {
            const long long n = li[g].c + (long long)e * a.N2;
            cpx<T> v = zero<T>();
            if (li[g].valid && n < a.nvalid) v = cmul(in[li[g].ib + e * a.in_es], chirp[n]);
            lds[g * a.LS + lpad(e, a.PS)] = v;
        });
    }
};

struct IoFsAC2R : IoFsA {
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        coop_for(a.G, a.N, false, [&](int g, int e) {
            cpx<T> Z = zero<T>();
            if (li[g].valid) {
                const long long k = li[g].c + (long long)e * a.N2;
                cpx<T> X = in[li[g].ib + e * a.in_es];
                cpx<T> Xm = conj(in[li[g].o * a.in_os + (a.M - k)]);
                cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
                Z = (X + Xm) + muli<1>(cmulc(X - Xm, w));
            }
            lds[g * a.LS + lpad(e, a.PS)] = Z;
        });
    }
};

// Four-step row pass. Line = row k1 (C = N1), contiguous in the scratch;
// FFT over n2 (length N2 = a.N); store X[k1 + N1*k2] (column-coalesced).
struct IoFsB : IoPlain {
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const T s = (T)a.scale;
        coop_for(a.G, a.N, false, [&](int g, int e) {
            if (li[g].valid) out[li[g].ob + e * a.out_es] = scale(lds[g * a.LS + lpad(e, a.PS)], s);
        });
    }
};

// Row pass of the packed half-size FFT for a large even R2C. A block owns H
// rows k1 = j*H + h and their mirrors N1 - k1 (row N1/2 replaces the mirror of
// row 0), so Z[k] and Z[M-k] are both in its LDS when the postprocess
// X[k] = 1/2 [(Z[k] + conj Z[M-k]) - i W_N^k (Z[k] - conj Z[M-k])] runs.
struct IoFsBR2C : IoPlain {
    static __device__ LineInfo line(const KArgs& a, unsigned blk, int g) {
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
        L.ib = L.o * a.in_os + k1 * a.in_cs;
        L.ob = L.o * a.out_os;
        return L;
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const int H = a.G / 2;
        const int N2 = a.N;
        coop_for(a.G, N2, false, [&](int g, int k2) {
            if (!li[g].valid) return;
            const long long k1 = li[g].c;
            int gp, k2m;
            if (k1 == 0) {
                gp = g;
                k2m = k2 == 0 ? 0 : N2 - k2;
            } else if (2 * k1 == a.N1) {
                gp = g;
                k2m = N2 - 1 - k2;
            } else {
                gp = g < H ? g + H : g - H;
                k2m = N2 - 1 - k2;
            }
            const long long k = k1 + a.N1 * k2;
            cpx<T> A = lds[g * a.LS + lpad(k2, a.PS)];
            cpx<T> B = conj(lds[gp * a.LS + lpad(k2m, a.PS)]);
            cpx<T> w = tw2<T>(a.rlo, a.rhi, a.rshift, k);
            cpx<T> X = (A + B) + muli<-1>(cmul(w, A - B));
            out[li[g].ob + k] = scale(X, (T)0.5);
            if (k == 0) out[li[g].ob + a.M] = mk(A.re - A.im, (T)0);
        });
    }
};

// Bluestein row pass: FFT over n2, multiply by the kernel spectrum (stored
// transposed as spec[k1*N2 + k2] with 1/M folded in), inverse FFT over k2 and
// the inverse four-step twiddle W_M^(-k1*m2); rows stay in place.
struct IoBlueB : IoPlain {
    static constexpr bool kTwoPass = true;
    template <typename T>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        coop_for(a.G, a.N, true, [&](int g, int e) {
            cpx<T>& v = lds[g * a.LS + lpad(e, a.PS)];
            v = cmul(v, spec[li[g].c * a.N + e]);
        });
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        coop_for(a.G, a.N, true, [&](int g, int e) {
            if (!li[g].valid) return;
            cpx<T> w = tw2<T>(a.tlo, a.thi, a.tshift, li[g].c * e);
            out[li[g].ob + e * a.out_es] = cmulc(lds[g * a.LS + lpad(e, a.PS)], w);
        });
    }
};

// Bluestein column pass: inverse FFT over k1 gives conv[m2 + N2*m1]; keep
// m < N and multiply by the chirp (and the caller's scale).
struct IoFsCBlue : IoPlain {
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        const T s = (T)a.scale;
        coop_for(a.G, a.N, false, [&](int g, int e) {
            const long long m = li[g].c + (long long)e * a.N2;
            if (!li[g].valid || m >= a.nout) return;
            out[li[g].ob + e * a.out_es] = scale(cmul(lds[g * a.LS + lpad(e, a.PS)], chirp[m]), s);
        });
    }
};

// Whole Bluestein transform in LDS: a = chirp * x zero-padded to M = a.N,
// FFT, multiply by the kernel spectrum, IFFT, chirp multiply, truncate.
struct IoBlue1 : IoPlain {
    static constexpr bool kTwoPass = true;
    template <typename T>
    static __device__ void prologue(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* in = (const cpx<T>*)a.in;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        coop_for(a.G, a.N, a.flags & KF_IN_ROWMAJOR, [&](int g, int e) {
            cpx<T> v = zero<T>();
            if (li[g].valid && e < a.nvalid) v = cmul(in[li[g].ib + e * a.in_es], chirp[e]);
            lds[g * a.LS + lpad(e, a.PS)] = v;
        });
    }
    template <typename T>
    static __device__ void mid(const KArgs& a, cpx<T>* lds, const LineInfo* li) {
        const cpx<T>* spec = (const cpx<T>*)a.spec;
        coop_for(a.G, a.N, true, [&](int g, int e) {
            cpx<T>& v = lds[g * a.LS + lpad(e, a.PS)];
            v = cmul(v, spec[e]);
        });
    }
    template <typename T, int S>
    static __device__ void epilogue(const KArgs& a, const cpx<T>* lds, const LineInfo* li) {
        cpx<T>* out = (cpx<T>*)a.out;
        const cpx<T>* chirp = (const cpx<T>*)a.chirp;
        const T s = (T)a.scale;
        coop_for(a.G, (int)a.nout, a.flags & KF_OUT_ROWMAJOR, [&](int g, int e) {
            if (li[g].valid)
                out[li[g].ob + e * a.out_es] = scale(cmul(lds[g * a.LS + lpad(e, a.PS)], chirp[e]), s);
        });
    }
};

// ------------------------------------------------------------------ kernel

template <typename T, int S, class IO>
__global__ __launch_bounds__(512) void k_fft(const KArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    cpx<T>* lds = reinterpret_cast<cpx<T>*>(smem_raw);
    __shared__ LineInfo li[kMaxLinesPerBlock];
    const int tid = threadIdx.x;
    if (tid < a.G) li[tid] = IO::line(a, blockIdx.x, tid);
    __syncthreads();
    IO::template prologue<T>(a, lds, li);
    __syncthreads();
    const int g = tid / a.TT, t = tid - g * a.TT;
    cpx<T>* line = lds + g * a.LS;
    const cpx<T>* tw = (const cpx<T>*)a.tw;
    run_stages<T, S>(line, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw);
    if constexpr (IO::kTwoPass) {
        IO::template mid<T>(a, lds, li);
        __syncthreads();
        run_stages<T, -S>(line, a.N, a.TT, t, a.PS, a.nstages, a.radix, tw);
    }
    IO::template epilogue<T, S>(a, lds, li);
}

// ------------------------------------------------------------- selection

using KernelFn = void (*)(const KArgs);

template <typename T, int S>
KernelFn pick(KernelKind kind) {
    switch (kind) {
        case KK_PLAIN: return k_fft<T, S, IoPlain>;
        case KK_R2C_FULL: return k_fft<T, S, IoR2CFull>;
        case KK_C2R_FULL: return k_fft<T, S, IoC2RFull>;
        case KK_R2C_HALF: return k_fft<T, S, IoR2CHalf>;
        case KK_C2R_HALF: return k_fft<T, S, IoC2RHalf>;
        case KK_FS_A: return k_fft<T, S, IoFsA>;
        case KK_FS_A_BLUE: return k_fft<T, S, IoFsABlue>;
        case KK_FS_A_C2R: return k_fft<T, S, IoFsAC2R>;
        case KK_FS_B: return k_fft<T, S, IoFsB>;
        case KK_FS_B_R2C: return k_fft<T, S, IoFsBR2C>;
        case KK_BLUE_B: return k_fft<T, S, IoBlueB>;
        case KK_FS_C_BLUE: return k_fft<T, S, IoFsCBlue>;
        case KK_BLUE_1: return k_fft<T, S, IoBlue1>;
        default: return nullptr;
    }
}

}  // namespace vkfx
