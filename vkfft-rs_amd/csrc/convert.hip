// convert.hip -- boundary passes around a plan's FFT passes: element-type
// conversion for mixed storage/compute precisions (src/config.rs:108-145),
// gathers from / scatters to formatted (strided) device layouts
// (FftConfig::with_*_buffer_axis_stride, src/config.rs:892-1002; the formatted
// copy passes of src/nd_ir.rs:1105-1150), the logical zero intervals of
// zero padding (src/zero_pad_ir.rs:320-345, 607-647), and the real <-> complex
// promotion, truncation and Hermitian expansion of full-complex real
// transforms (src/real_ir.rs:935-946, 1038-1053).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace vkfx {

template <typename S, typename D>
__global__ __launch_bounds__(256) void k_boundary(const S* __restrict__ in, D* __restrict__ out, const BoundaryArgs a) {
    const long long per = a.tensor_len;
    const long long total = per * a.batch;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long b = i / per;
        long long l = i - b * per;
        long long src = b * a.src_batch, dst = b * a.dst_batch;
        bool zero = false, conj = false;
        if (a.mode == 1) {
            const long long n = a.dims[0], c = l;
            conj = 2 * c > n;
            src += (conj ? n - c : c) * a.src_stride[0];
            dst += c * a.dst_stride[0];
        } else {
            for (int ax = a.rank - 1; ax >= 0; --ax) {
                const long long n = a.dims[ax];
                const long long c = l % n;
                l /= n;
                src += c * a.src_stride[ax];
                dst += c * a.dst_stride[ax];
                zero |= c >= a.zero_left[ax] && c < a.zero_right[ax];
            }
        }
        for (int k = 0; k < a.dst_scalars; ++k) {
            D v = (zero || k >= a.src_scalars) ? (D)0 : (D)in[src * a.src_scalars + k];
            if (conj && k == 1) v = -v;
            out[dst * a.dst_scalars + k] = v;
        }
    }
}

// The same boundary work one row of the fastest axis per block and step:
// the row's placement (and its zero test on the slower axes) is decomposed
// once, and the threads walk the row's contiguous elements. For rows of at
// least 1024 elements (launch_boundary's choice: 4096-element rows 20%
// faster than k_boundary, 256-element rows 17% slower).
template <typename S, typename D>
__global__ __launch_bounds__(256) void k_boundary_rows(const S* __restrict__ in, D* __restrict__ out,
                                                       const BoundaryArgs a) {
    const int last = a.rank - 1;
    const long long n = a.dims[last];
    const long long per = a.tensor_len / n;
    const long long rows = per * a.batch;
    const long long zl = a.zero_left[last], zr = a.zero_right[last];
    const long long ss = a.src_stride[last], ds = a.dst_stride[last];
    for (long long row = blockIdx.x; row < rows; row += gridDim.x) {
        const long long b = row / per;
        long long l = row - b * per;
        long long src = b * a.src_batch, dst = b * a.dst_batch;
        bool zero = false;
        for (int ax = last - 1; ax >= 0; --ax) {
            const long long m = a.dims[ax];
            const long long c = l % m;
            l /= m;
            src += c * a.src_stride[ax];
            dst += c * a.dst_stride[ax];
            zero |= c >= a.zero_left[ax] && c < a.zero_right[ax];
        }
        for (long long e = threadIdx.x; e < n; e += blockDim.x) {
            const bool z = zero || (e >= zl && e < zr);
            const long long si = (src + e * ss) * a.src_scalars, di = (dst + e * ds) * a.dst_scalars;
            for (int k = 0; k < a.dst_scalars; ++k) out[di + k] = (z || k >= a.src_scalars) ? (D)0 : (D)in[si + k];
        }
    }
}

template <typename S, typename D>
static int go(const void* in, void* out, const BoundaryArgs& a, hipStream_t s) {
    if (a.mode == 0 && a.dims[a.rank - 1] >= 1024) {
        const long long rows = a.tensor_len / a.dims[a.rank - 1] * a.batch;
        const unsigned grid = (unsigned)(rows < 65536 ? rows : 65536);
        hipLaunchKernelGGL((k_boundary_rows<S, D>), dim3(grid), dim3(256), 0, s, (const S*)in, (D*)out, a);
        return (int)hipGetLastError();
    }
    const long long total = a.tensor_len * a.batch;
    const long long blocks = (total + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
    hipLaunchKernelGGL((k_boundary<S, D>), dim3(grid), dim3(256), 0, s, (const S*)in, (D*)out, a);
    return (int)hipGetLastError();
}

// Dense layouts on both sides, no zero interval, no Hermitian expansion and
// the same scalars per element: the boundary pass is a flat type conversion
// of n scalars, one 16-byte source vector per thread per step (V scalars),
// with the n % V tail converted one scalar at a time by the first threads.
template <typename S, typename D>
__global__ __launch_bounds__(256) void k_convert_flat(const S* __restrict__ in, D* __restrict__ out, long long n) {
    constexpr int V = 16 / (int)sizeof(S);
    typedef S sv __attribute__((ext_vector_type(V)));
    typedef D dv __attribute__((ext_vector_type(V)));
    const long long nv = n / V;
    const long long stride = (long long)gridDim.x * blockDim.x;
    const long long t0 = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (long long i = t0; i < nv; i += stride)
        ((dv*)out)[i] = __builtin_convertvector(((const sv*)in)[i], dv);
    if (t0 < n - nv * V) out[nv * V + t0] = (D)in[nv * V + t0];
}

template <typename S, typename D>
static int go_flat(const void* in, void* out, long long n, hipStream_t s) {
    constexpr int V = 16 / (int)sizeof(S);
    long long blocks = (n / V + 255) / 256;
    blocks = blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks;
    hipLaunchKernelGGL((k_convert_flat<S, D>), dim3((unsigned)blocks), dim3(256), 0, s, (const S*)in, (D*)out, n);
    return (int)hipGetLastError();
}

// Whether the boundary pass is a flat conversion (see k_convert_flat): both
// sides dense, both pointers aligned to the vectors of k_convert_flat.
static bool flat_boundary(const BoundaryArgs& a, const void* in, void* out) {
    if (a.mode != 0 || a.src_scalars != a.dst_scalars || a.src_type == a.dst_type) return false;
    long long dense = 1;
    for (int ax = a.rank - 1; ax >= 0; --ax) {
        if (a.src_stride[ax] != dense || a.dst_stride[ax] != dense || a.zero_left[ax] < a.zero_right[ax]) return false;
        dense *= a.dims[ax];
    }
    if (dense != a.tensor_len || a.src_batch != dense || a.dst_batch != dense) return false;
    return (uintptr_t)in % 16 == 0 && (uintptr_t)out % 16 == 0;
}

// A transform whose only axis has length 1 is a copy (X[0] = x[0], scale 1):
// a grid-stride copy of 16-byte vectors, four per thread per step, with
// nontemporal loads and stores (the data is not re-read), and an 8-byte tail.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(256) void k_copy16(const u32x4* __restrict__ in, u32x4* __restrict__ out, long long n16) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(in + i + k * stride);
#pragma unroll
        for (int k = 0; k < 4; ++k) __builtin_nontemporal_store(v[k], out + i + k * stride);
    }
    for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

__global__ void k_copy8(const u32x2* __restrict__ in, u32x2* __restrict__ out, long long n8) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (long long)gridDim.x * blockDim.x)
        out[i] = in[i];
}

const void* copy_kernel_fn() { return (const void*)k_copy16; }

int launch_copy(const void* in, void* out, size_t bytes, hipStream_t s) {
    if (bytes == 0 || in == out) return (int)hipSuccess;
    if (bytes % 8) return (int)hipErrorInvalidValue;
    const bool aligned = ((uintptr_t)in % 16 == 0) && ((uintptr_t)out % 16 == 0);
    const long long n16 = aligned ? (long long)(bytes / 16) : 0;
    if (n16) {
        long long blocks = (n16 + 1023) / 1024;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(k_copy16, dim3((unsigned)blocks), dim3(256), 0, s, (const u32x4*)in, (u32x4*)out, n16);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    const size_t done = (size_t)n16 * 16;
    const long long n8 = (long long)((bytes - done) / 8);
    if (n8) {
        long long blocks = (n8 + 255) / 256;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(k_copy8, dim3((unsigned)blocks), dim3(256), 0, s, (const u32x2*)((const char*)in + done),
                           (u32x2*)((char*)out + done), n8);
        return (int)hipGetLastError();
    }
    return (int)hipSuccess;
}

const void* boundary_kernel_fn(int src_type, int dst_type) {
    switch (src_type * 3 + dst_type) {
        case 0 * 3 + 1: return (const void*)k_boundary<_Float16, float>;
        case 1 * 3 + 0: return (const void*)k_boundary<float, _Float16>;
        case 1 * 3 + 1: return (const void*)k_boundary<float, float>;
        case 1 * 3 + 2: return (const void*)k_boundary<float, double>;
        case 2 * 3 + 1: return (const void*)k_boundary<double, float>;
        case 2 * 3 + 2: return (const void*)k_boundary<double, double>;
        default: return nullptr;
    }
}

int launch_boundary(const BoundaryArgs& a, const void* in, void* out, hipStream_t s) {
    if (a.tensor_len <= 0 || a.batch <= 0) return (int)hipSuccess;
    if (a.rank < 1 || a.rank > kMaxBoundaryRank || a.src_scalars < 1 || a.src_scalars > 2 || a.dst_scalars < 1 ||
        a.dst_scalars > 2 || (a.mode == 1 && a.rank != 1))
        return (int)hipErrorInvalidValue;
    const int code = a.src_type * 3 + a.dst_type;
    if (flat_boundary(a, in, out)) {
        const long long n = a.batch * a.tensor_len * a.src_scalars;
        switch (code) {
            case 0 * 3 + 1: return go_flat<_Float16, float>(in, out, n, s);
            case 1 * 3 + 0: return go_flat<float, _Float16>(in, out, n, s);
            case 1 * 3 + 2: return go_flat<float, double>(in, out, n, s);
            case 2 * 3 + 1: return go_flat<double, float>(in, out, n, s);
            default: break;
        }
    }
    switch (code) {
        case 0 * 3 + 1: return go<_Float16, float>(in, out, a, s);
        case 1 * 3 + 0: return go<float, _Float16>(in, out, a, s);
        case 1 * 3 + 1: return go<float, float>(in, out, a, s);
        case 1 * 3 + 2: return go<float, double>(in, out, a, s);
        case 2 * 3 + 1: return go<double, float>(in, out, a, s);
        case 2 * 3 + 2: return go<double, double>(in, out, a, s);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // namespace vkfx
