// kernels.hpp -- host-visible launch interface of the gfx950 kernel library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vkfx {

constexpr int kMaxStages = 24;
constexpr int kMaxLinesPerBlock = 64;
constexpr int kMaxConvMatrix = 3;  // coordinates of a matrix convolution (2 x 2, 3 x 3)
// Bytes of the static device scratch behind vkfx_execute_noalloc (one copy
// per GPU), and the device ordinals it tracks.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
hipError_t static_scratch_address(int device, void** out);

// Kernel families. Each is one HBM pass over its lines; see the comments on
// the IO policies in fft_kernels.hip for what each one loads and stores.
enum KernelKind : int {
    KK_PLAIN = 0,      // C2C lines along any axis, scale on store
    KK_R2C_FULL,       // odd-length R2C: real -> complex FFT, keep n/2+1
    KK_C2R_FULL,       // odd-length C2R: Hermitian expand, FFT, keep real
    KK_R2C_HALF,       // even R2C in one kernel: packed half-size FFT + post
    KK_C2R_HALF,       // even C2R in one kernel: pre + packed half-size FFT
    KK_FS_A,           // four-step column pass + W_M twiddle on store
    KK_FS_A_BLUE,      // same, input = chirp * x with zero padding
    KK_FS_A_C2R,       // same, input = even-half C2R preprocess of X
    KK_FS_B,           // four-step row pass, transposed store
    KK_FS_B_R2C,       // four-step row pass + R2C postprocess (mirror rows)
    KK_BLUE_B,         // Bluestein row pass: FFT, spectrum multiply, IFFT, W_M^-1
    KK_FS_C_BLUE,      // Bluestein column pass: IFFT, chirp, truncate
    KK_BLUE_1,         // Bluestein in one kernel (convolution fits LDS)
    KK_RADER_FFT,      // prime length p: gather, FFT(p-1), kernel multiply, IFFT, scatter
    KK_RADER_DIRECT,   // prime length p: gather, O(p^2) cyclic convolution, scatter
    KK_CONV_1,         // convolution in one kernel: FFT, kernel-spectrum multiply, normalized IFFT
    KK_CONV_B,         // four-step convolution row pass: FFT, natural-order spectrum multiply, IFFT, W_M^-1 (fixed shapes only)
    KK_FS_A_EDGE,      // KK_FS_A reading half-precision storage, input zero interval (fixed shapes only)
    KK_FS_B_EDGE,      // KK_FS_B writing half-precision storage, output zero interval (fixed shapes only)
    KK_BLUE_1_EDGE,    // KK_BLUE_1 reading / writing half-precision storage, zero intervals (fixed shapes only)
    KK_R2C_HALF_EDGE,  // KK_R2C_HALF reading / writing half-precision storage, input zero interval (fixed shapes only)
    KK_C2R_HALF_EDGE,  // KK_C2R_HALF reading / writing half-precision storage, output zero interval (fixed shapes only)
    KK_PLAIN_EDGE,     // one-upload 1-D KK_PLAIN rows with storage conversion and zero intervals (fixed shapes only)
    KK_PLAIN_EDGE_IN,  // KK_PLAIN first pass of an N-D chunk reading half-precision storage (fixed shapes only)
    KK_PLAIN_EDGE_OUT, // KK_PLAIN last pass of an N-D chunk writing half-precision storage (fixed shapes only)
    KK_COUNT
};

enum KFlags : int {
    KF_IN_ROWMAJOR = 1,   // a line's elements are contiguous in the input
    KF_OUT_ROWMAJOR = 2,  // a line's elements are contiguous in the output
    KF_MIRROR_PAIRS = 4,  // C2R column pass: a block owns columns and their mirrors
    KF_XCD_GROUPS = 8,    // deal line groups to XCDs in contiguous ranges
    KF_DYN_WIDE = 16,     // runtime-shape kernel holding up to 32 elements per thread per stage
    KF_DYN_DIRECT = 32,   // runtime-shape C2C with HBM-direct first and last stages (contiguous lines)
    KF_DYN_PRE = 64,      // with KF_DYN_DIRECT, even C2R: the first stage forms the preprocess from HBM
    KF_CONV_CONJ = 128,   // KK_CONV_1/B: conjugate the sequence spectrum (ConvolutionConjugation::Sequence)
    KF_CONV_CROSS = 256,  // KK_CONV_1/B: cross-power-spectrum normalization of the product
    // KK_PLAIN in the staged runtime-shape kernel with the plan's boundary
    // work inside its loads and stores (IoEdge): storage of half the compute
    // precision on the input / output side, and the zero interval [zl, zr) of
    // a line's elements read as zero / written as zero
    KF_EDGE = 512,
    KF_NARROW_IN = 1024,
    KF_NARROW_OUT = 2048,
    KF_ZERO_IN = 4096,
    KF_ZERO_OUT = 8192,
    // with KF_MIRROR_PAIRS: the direct first stage loads each (X[k], X[M-k])
    // once for a butterfly of the column and one of its mirror
    KF_PAIR_LOADS = 16384,
    // the radix list has Rader stages (KArgs::rtab): the staged runtime-shape
    // instantiation that carries them (the others leave their registers out)
    KF_RADER = 32768,
    // KK_CONV_1 on the runtime-shape kernel: a block holds whole systems of
    // C1 coordinate lines (G a multiple of C1) and the product mixes them
    // through the M x M kernel matrix (symmetric planes with KF_CONV_SYM)
    KF_CONV_MATRIX = 65536,
    KF_CONV_SYM = 131072,
};

// Butterflies per thread in one radix-R stage of the runtime-shape kernel
// (the host sizes threads per line with the same rule, so that
// threads * butterflies covers every butterfly of every stage). The narrow
// variant holds at most 16 elements per thread and needs about half the
// registers of the wide one, which doubles the waves resident per CU; the
// wide variant serves lengths whose narrow geometry exceeds 512 threads.
constexpr int dyn_butterflies_per_thread(int R, bool wide) {
    return wide ? (R <= 2 ? 16 : R <= 3 ? 10 : R <= 4 ? 8 : R <= 5 ? 6 : R <= 8 ? 4 : 2)
                : (R <= 16 && 16 / R > 1 ? 16 / R : 1);
}

struct KArgs {
    const void* in;
    void* out;
    long long in_es, in_cs, in_os;     // input element / column / outer strides
    long long out_es, out_cs, out_os;  // output strides
    long long C;                       // columns per outer index (line = (o2*C1 + o1)*C + c)
    long long C1;                      // second outer level (1 = single level)
    long long in_os1, out_os1;         // strides of the second outer level
    long long twdiv;                   // four-step twiddle row = c / twdiv
    long long nlines;                  // total lines
    int N;                             // FFT length run in LDS
    int TT;                            // threads per line
    int G;                             // lines per block
    int LS;                            // LDS stride between lines (elements)
    int PS;                            // LDS pad shift
    int nstages;
    int radix[kMaxStages];
    int flags;
    const void* tw;                    // exp(-2 pi i k/N), k < N
    const void* swlo;                  // same roots as two sqrt(N)-size tables:
    const void* swhi;                  //   root(m) = swhi[m >> swshift] * swlo[m & mask]
    int swshift;
    double scale;
    const void* chirp;                 // Bluestein chirp, logical length
    const void* spec;                  // Bluestein kernel spectrum (1/M folded in)
    const void* tlo;                   // two-level table for exp(-2 pi i k/M)
    const void* thi;
    int tshift;
    const void* rlo;                   // two-level table for exp(-2 pi i k/Nreal)
    const void* rhi;
    int rshift;
    long long M;                       // four-step / half-spectrum / convolution length
    long long nvalid;                  // logical input length (zero pad beyond)
    long long nout;                    // logical output length per line (truncate)
    long long N1, N2;                  // four-step factors (M = N1*N2)
    long long nblk;                    // line groups of the launch
    const int* pin;                    // Rader gather: a[s] = x[pin[s]]
    const int* pout;                   // Rader scatter: X[pout[m]] = x0 + conv[m]
    // Rader stages of a runtime radix list (radix > kMaxStockhamRadix): the
    // table block of stage s starts roff[s] bytes into rtab (rader_stage_table)
    const void* rtab;
    int roff[kMaxStages];
    long long zl, zr;                  // KF_ZERO_IN / KF_ZERO_OUT element interval of a line
    // KK_CONV_1 over 1-D lines (C = 1, line = o * C1 + o1): the line's
    // kernel-spectrum plane starts at o * spec_os + o1 * spec_os1
    long long spec_os, spec_os1;
};

// Radices up to this are Stockham butterflies; a larger (prime) radix in a
// runtime radix list is a Rader stage computed by direct multiplication.
constexpr int kMaxStockhamRadix = 16;

// Byte layout of a Rader stage table for prime p (L = p - 1, generator g):
// int slot[p] (slot[0] = L, slot[i] = s with g^-s = i), int logq[p]
// (logq[q] = m with g^m = q), then from byte rader_kernel_offset(p) the
// complex kernels b[n] = exp(-2 pi i g^n / p) (forward) and its conjugate
// (inverse), L entries each.
constexpr int rader_kernel_offset(int p) { return (2 * p * 4 + 15) / 16 * 16; }

// A Rader stage whose prime p is at least kRaderFftStageMin and whose
// L = p - 1 factors into primes up to kRaderSubPrimeMax runs its length-L
// cyclic convolution by FFT (the FFT-Rader node of rader_ir.rs:706-745):
// forward FFT_L of every butterfly's generator-ordered inputs, multiply by
// the kernel spectrum, inverse FFT_L. Its table block (flagged by
// kRaderFftStage in KArgs::roff) is: int hdr[16] (hdr[0] = number of
// sub-radices, hdr[1..] the sub-radices, product L), int slot[p] (as above),
// int pw[L] (pw[m] = g^m mod p), then from byte rader_fft_data_offset(p) the
// complex roots exp(-2 pi i k/L), k < L, and the spectra FFT_L(b)/L of
// b[n] = exp(-2 pi i g^n / p) and of its conjugate. The length-L FFTs
// ping-pong between the stage's scratch region and the line's own region.
constexpr int kRaderFftStageMin = 89;
constexpr int kRaderSubPrimeMax = 31;
constexpr int kRaderFftStage = 1 << 30;
constexpr int rader_fft_data_offset(int p) { return ((16 + p + (p - 1)) * 4 + 15) / 16 * 16; }

using KernelFn = void (*)(const KArgs);

// A kernel instantiated for one compile-time shape (fft_kernels_impl.hpp
// k_fix): the host must launch it with exactly this geometry.
// Twiddle table a fixed shape reads through KArgs::tw: the stage roots
// exp(-2 pi i k/N), k < N (FT_STAGE), or the lane-ordered table of the
// register-exchange 1024-point kernel (FT_WAVE1024, fft_wave.hpp).
// FT_STAGE_PR: per-stage blocks in radix order, one per stage with P > 1
// (P = product of the earlier radices), P (R - 1) entries each: entry
// k (R - 1) + i - 1 = exp(-2 pi i k i / (P R)).
enum FixedTable : int { FT_STAGE = 0, FT_WAVE1024 = 1, FT_STAGE_PR = 2 };
// Complex entries of the FT_WAVE1024 table: 4 x 64 lane roots of the pass-1
// twiddles, then 4 roots of the pass-2 twiddles.
constexpr int kWave1024TableLen = 260;

struct FixedKernel {
    KernelKind kind;
    int prec, dir;
    int N, TT, G, PS, LS;
    bool col;  // lanes run across lines (strided layouts)
    bool nti, nto;  // nontemporal loads of the pass input / stores of its output
    int nst;
    int radix[8];
    KernelFn fn;          // one block per group of G lines
    int table = FT_STAGE;
    int lds_mult = 1;  // 2: ping-pong shapes hold two LDS buffers of G lines
};

// Finds a fixed-shape kernel for (kind, precision, first-FFT direction,
// length, lane mapping); nullptr when only the runtime-shape kernel applies.
// Setting VKFX_DISABLE_FIXED=1 in the environment forces the runtime-shape kernels.
const FixedKernel* find_fixed(KernelKind kind, int prec, int dir, int N, bool col);

// The registered instantiation with the same shape as f and the given
// nontemporal load/store choice; f itself when none is registered.
const FixedKernel* fixed_variant(const FixedKernel* f, bool nti, bool nto);
// The registered shape of another kind with f's geometry (length, threads,
// lines per block, LDS stride and pad, radices), any nontemporal variant;
// null if there is none.
const FixedKernel* kind_variant(const FixedKernel* f, KernelKind kind);

// Launches one kernel. prec: 0 = f32, 1 = f64. dir: -1 forward, +1 inverse
// (direction of the first FFT the kernel runs). fixed: the fixed-shape
// instantiation to run, or nullptr for the runtime-shape kernel. t_begin /
// t_end: when both are set, HIP events bound to this dispatch
// (hipExtLaunchKernel) that read the kernel's own begin and end. Returns a
// hipError_t value.
int launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned grid, unsigned block,
           size_t lds_bytes, hipStream_t stream, const FixedKernel* fixed = nullptr, hipEvent_t t_begin = nullptr,
           hipEvent_t t_end = nullptr);

// Validates one launch against what the kernel it selects assumes (block
// shape, LDS size, flags, fixed-shape geometry, Rader stage scratch); no HIP
// calls. Returns hipSuccess or the error launch() reports.
hipError_t check_launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned block, size_t lds_bytes,
                        size_t lds_limit, const FixedKernel* fixed);

// Largest dynamic LDS a block may request on this device (bytes).
size_t max_lds_bytes();

// Boundary pass: for every logical element (b, c_0..c_{rank-1}) of a batch
// of tensors, out[dst] = zero ? 0 : (D)in[src] with src / dst the strided
// offsets of the two layouts and zero set when any coordinate lies in its
// axis interval [zero_left, zero_right). Scalar types: 0 = binary16,
// 1 = f32, 2 = f64; src_scalars / dst_scalars = 2 for complex elements, 1
// for real (real -> complex fills the imaginary part with 0, complex -> real
// keeps the real part). mode 1 (rank 1): Hermitian expansion of N/2+1 bins
// to N, out[c] = c <= N/2 ? in[c] : conj(in[N - c]) with N = dims[0].
constexpr int kMaxBoundaryRank = 4;
struct BoundaryArgs {
    int rank = 1;
    int src_scalars = 2, dst_scalars = 2;
    int mode = 0;
    int src_type = 1, dst_type = 1;
    long long batch = 0, tensor_len = 0;
    long long dims[kMaxBoundaryRank] = {1, 1, 1, 1};
    long long src_stride[kMaxBoundaryRank] = {0, 0, 0, 0}, dst_stride[kMaxBoundaryRank] = {0, 0, 0, 0};
    long long src_batch = 0, dst_batch = 0;
    long long zero_left[kMaxBoundaryRank] = {0, 0, 0, 0}, zero_right[kMaxBoundaryRank] = {0, 0, 0, 0};
};
int launch_boundary(const BoundaryArgs& a, const void* in, void* out, hipStream_t s);
// Copy of `bytes` (a multiple of 8) for transforms of length 1 (convert.hip).
int launch_copy(const void* in, void* out, size_t bytes, hipStream_t s);
const void* copy_kernel_fn();

// DCT / DST pre and post passes around a length-L complex FFT (r2r.hip):
//   a[m] = w(m) x[m - off] exp(-i pi m ph / (2n))  (m - off in [0, n), else 0)
//   X[k] = s * (im ? -Im : Re)(exp(-i pi (k + q2/2) pq / (2n)) A[k + r])
// wmode: 0 all 1; 1 DCT-I ends 1, else 2; 2 DCT-III first 1, else 2;
// 3 DST-III m == n 1, else 2.
// DCT / DST pre and post passes around a complex FFT of length L (r2r.hip).
// op selects the reduction: R2R_EXTEND writes each type as the real or
// imaginary part of a zero-padded DFT of length L = 2(N-1), 2(N+1) or 2N
// (types I, and odd IV); R2R_REORDER / R2R_SPECTRUM are the length-N forms of
// types II / III (Makhoul's even-odd reordering); R2R_HALF packs even type IV
// into L = N/2 complex points. flip: the DST form of II / III / IV (input sign
// or reversal, output reversal or sign).
enum R2rOp : int { R2R_EXTEND = 0, R2R_REORDER = 1, R2R_SPECTRUM = 2, R2R_HALF = 3 };
struct R2rArgs {
    long long n = 0, L = 0, batch = 0;
    long long inner = 1;  // element stride of a line (lines of a strided axis)
    int off = 0, ph = 0, wmode = 0;
    int r = 0, pq = 0, q2 = 0, im = 0;
    int op = R2R_EXTEND, flip = 0;
    double s = 1.0;
};
int launch_r2r(bool pre, int prec, const R2rArgs& p, const void* in, void* out, hipStream_t s);

// Convolution multiply (conv.hip): spectra [system][coordinate][T], kernel
// [kernel][plane][T]; matrix = 0 (none), 2 or 3.
struct ConvArgs {
    long long T = 0, systems_out = 0;
    int coords = 1, planes = 1, kernel_count = 1;
    int matrix = 0, symmetric = 0, independent = 0;
    int conj_seq = 0, cross_norm = 0;
};
int launch_conv(int prec, const ConvArgs& a, const void* x, const void* k, void* y, hipStream_t s);

// Device functions a launch runs, for resource queries (hipFuncGetAttributes,
// occupancy): the same selection as the launch functions make.
const void* fft_kernel_fn(KernelKind kind, int prec, int dir, const FixedKernel* fixed, int flags);
const void* boundary_kernel_fn(int src_type, int dst_type);
const void* r2r_kernel_fn(bool pre, int prec);
const void* conv_kernel_fn(int prec);

}  // namespace vkfx
