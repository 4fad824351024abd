// launch.hip -- dispatches a KernelKind to its instantiation and launches it.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdlib>
#include <map>
#include <mutex>
#include <string>

#include "kernels.hpp"

namespace vkfx {

KernelFn pick_f32_fwd(KernelKind kind, bool wide, int direct, int edge, bool rad);
KernelFn pick_f32_inv(KernelKind kind, bool wide, int direct, int edge, bool rad);
KernelFn pick_f64_fwd(KernelKind kind, bool wide, int direct, int edge, bool rad);
KernelFn pick_f64_inv(KernelKind kind, bool wide, int direct, int edge, bool rad);
const FixedKernel* fixed_table_wave(int* count);
const FixedKernel* fixed_table_plain(int* count);
const FixedKernel* fixed_table_real(int* count);
const FixedKernel* fixed_table_blue(int* count);
const FixedKernel* fixed_table_nd(int* count);
const FixedKernel* fixed_table_pow2_f32(int* count);
const FixedKernel* fixed_table_pow2_f64(int* count);
const FixedKernel* fixed_table_fam_f32(int* count);
const FixedKernel* fixed_table_fam_f64(int* count);
const FixedKernel* fixed_table_real_rows_f32(int* count);
const FixedKernel* fixed_table_real_rows_f64(int* count);
const FixedKernel* fixed_table_round_f32(int* count);
const FixedKernel* fixed_table_round_f64(int* count);
const FixedKernel* fixed_table_round_nd_f32(int* count);
const FixedKernel* fixed_table_round_nd_f64(int* count);
const FixedKernel* fixed_table_round_real_f32(int* count);
const FixedKernel* fixed_table_round_real_f64(int* count);
const FixedKernel* fixed_table_round_fs_f32(int* count);
const FixedKernel* fixed_table_round_fs_f64(int* count);
const FixedKernel* fixed_table_blue_rows_f32(int* count);
const FixedKernel* fixed_table_blue_rows_f64(int* count);
const FixedKernel* fixed_table_conv(int* count);
const FixedKernel* fixed_table_fs_edge(int* count);
const FixedKernel* fixed_table_conv1(int* count);
const FixedKernel* fixed_table_blue_edge_f32(int* count);
const FixedKernel* fixed_table_blue_edge_f64(int* count);
const FixedKernel* fixed_table_real_edge_f32(int* count);
const FixedKernel* fixed_table_real_edge_f64(int* count);
const FixedKernel* fixed_table_plain_edge_f32(int* count);
const FixedKernel* fixed_table_plain_edge_f64(int* count);
const FixedKernel* fixed_table_nd_edge_f32(int* count);
const FixedKernel* fixed_table_nd_edge_f64(int* count);

// All registered fixed-shape instantiations, merged once (thread-safe
// static initialisation).
static const FixedKernel* registry(int* count) {
    struct Merged {
        const FixedKernel* all;
        int total;
    };
    static const Merged m = [] {
        const FixedKernel* (*tables[])(int*) = {fixed_table_plain, fixed_table_wave, fixed_table_real, fixed_table_blue,
                                                fixed_table_nd, fixed_table_pow2_f32, fixed_table_pow2_f64,
                                                fixed_table_fam_f32, fixed_table_fam_f64, fixed_table_real_rows_f32,
                                                fixed_table_real_rows_f64, fixed_table_round_f32, fixed_table_round_f64,
                                                fixed_table_round_nd_f32, fixed_table_round_nd_f64,
                                                fixed_table_round_real_f32, fixed_table_round_real_f64,
                                                fixed_table_round_fs_f32, fixed_table_round_fs_f64,
                                                fixed_table_blue_rows_f32, fixed_table_blue_rows_f64,
                                                fixed_table_conv, fixed_table_fs_edge,
                                                fixed_table_conv1, fixed_table_blue_edge_f32,
                                                fixed_table_blue_edge_f64, fixed_table_real_edge_f32,
                                                fixed_table_real_edge_f64, fixed_table_plain_edge_f32,
                                                fixed_table_plain_edge_f64, fixed_table_nd_edge_f32,
                                                fixed_table_nd_edge_f64};
        constexpr int kTables = (int)(sizeof(tables) / sizeof(tables[0]));
        int counts[kTables], sum = 0;
        const FixedKernel* ptrs[kTables];
        for (int i = 0; i < kTables; ++i) {
            ptrs[i] = tables[i](&counts[i]);
            sum += counts[i];
        }
        FixedKernel* merged = new FixedKernel[sum];
        int k = 0;
        for (int i = 0; i < kTables; ++i)
            for (int j = 0; j < counts[i]; ++j) {
                merged[k] = ptrs[i][j];
                int n = 0;
                while (n < 8 && merged[k].radix[n]) ++n;
                merged[k].nst = n;
                ++k;
            }
        return Merged{merged, sum};
    }();
    *count = m.total;
    return m.all;
}

const FixedKernel* find_fixed(KernelKind kind, int prec, int dir, int N, bool col) {
    // the knobs are read at each call: plans are built rarely, and a process
    // may build plans under different settings (tests do)
    const char* dis = getenv("VKFX_DISABLE_FIXED");
    if (dis && dis[0] == '1') return nullptr;
    int total = 0;
    const FixedKernel* all = registry(&total);
    // VKFX_REGISTER_EXCHANGE=1 prefers the register-exchange shape of a key
    // (one wave per line, no LDS) where one is registered.
    const char* rx = getenv("VKFX_REGISTER_EXCHANGE");
    if (rx && rx[0] == '1')
        for (int i = 0; i < total; ++i) {
            const FixedKernel& f = all[i];
            if (f.kind == kind && f.prec == prec && f.dir == dir && f.N == N && f.col == col &&
                f.table == FT_WAVE1024)
                return &f;
        }
    // VKFX_FIXED_PICK=k selects the k-th registered variant of a shape key,
    // or its last one if it has fewer (tuning runs); the default is the first.
    // VKFX_FIXED_PICK_K<kind>=k does the same for one KernelKind only.
    const char* pa = getenv("VKFX_FIXED_PICK");
    const int pick_all = pa ? atoi(pa) : 0;
    int pick = pick_all;
    if (kind >= 0 && kind < KK_COUNT) {
        const std::string name = "VKFX_FIXED_PICK_K" + std::to_string((int)kind);
        if (const char* e = getenv(name.c_str())) pick = atoi(e);
    }
    const FixedKernel* last = nullptr;
    int seen = 0;
    for (int i = 0; i < total; ++i) {
        const FixedKernel& f = all[i];
        if (f.kind == kind && f.prec == prec && f.dir == dir && f.N == N && f.col == col) {
            last = &f;
            if (seen++ == pick) return &f;
        }
    }
    return last;
}

const FixedKernel* fixed_variant(const FixedKernel* f, bool nti, bool nto) {
    if (!f || (f->nti == nti && f->nto == nto)) return f;
    int total = 0;
    const FixedKernel* all = registry(&total);
    for (int i = 0; i < total; ++i) {
        const FixedKernel& v = all[i];
        if (v.kind != f->kind || v.prec != f->prec || v.dir != f->dir || v.N != f->N || v.col != f->col ||
            v.TT != f->TT || v.G != f->G || v.PS != f->PS || v.LS != f->LS || v.nst != f->nst || v.nti != nti ||
            v.nto != nto || v.table != f->table || v.lds_mult != f->lds_mult)
            continue;
        bool same = true;
        for (int s = 0; s < v.nst; ++s) same = same && v.radix[s] == f->radix[s];
        if (same) return &v;
    }
    return f;
}

const FixedKernel* kind_variant(const FixedKernel* f, KernelKind kind) {
    if (!f) return nullptr;
    int total = 0;
    const FixedKernel* all = registry(&total);
    for (int i = 0; i < total; ++i) {
        const FixedKernel& v = all[i];
        if (v.kind != kind || v.prec != f->prec || v.dir != f->dir || v.N != f->N || v.col != f->col ||
            v.TT != f->TT || v.G != f->G || v.PS != f->PS || v.LS != f->LS || v.nst != f->nst ||
            v.table != f->table || v.lds_mult != f->lds_mult)
            continue;
        bool same = true;
        for (int s = 0; s < v.nst; ++s) same = same && v.radix[s] == f->radix[s];
        if (same) return &v;
    }
    return nullptr;
}

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

static KernelFn pick_kernel(KernelKind kind, int prec, int dir, int flags) {
    const bool wide = (flags & KF_DYN_WIDE) != 0;
    const int direct = (flags & KF_DYN_DIRECT) ? ((flags & KF_DYN_PRE) ? 2 : 1) : 0;
    const int edge =
        (flags & KF_EDGE) ? 1 + ((flags & KF_NARROW_IN) ? 1 : 0) + ((flags & KF_NARROW_OUT) ? 2 : 0) : 0;
    const bool rad = (flags & KF_RADER) != 0;
    return prec == 0 ? (dir < 0 ? pick_f32_fwd(kind, wide, direct, edge, rad) : pick_f32_inv(kind, wide, direct, edge, rad))
                     : (dir < 0 ? pick_f64_fwd(kind, wide, direct, edge, rad) : pick_f64_inv(kind, wide, direct, edge, rad));
}

// Raises a kernel's dynamic-LDS limit once per (device, kernel) to the
// largest size launched so far: the attribute persists, and setting it on
// every launch costs host time on the launch path.
static int raise_lds_limit(const void* fn, size_t bytes) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, size_t> done;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> lock(mu);
    size_t& have = done[{dev, fn}];
    if (have >= bytes) return (int)hipSuccess;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess) have = bytes;
    return (int)e;
}

const void* fft_kernel_fn(KernelKind kind, int prec, int dir, const FixedKernel* fixed, int flags) {
    if (kind < 0 || kind >= KK_COUNT || (dir != -1 && dir != 1) || (prec != 0 && prec != 1)) return nullptr;
    if (fixed) return (const void*)fixed->fn;
    return (const void*)pick_kernel(kind, prec, dir, flags);
}

int launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned grid, unsigned block, size_t lds_bytes,
           hipStream_t stream, const FixedKernel* fixed, hipEvent_t t_begin, hipEvent_t t_end) {
    if (grid == 0) return (int)hipSuccess;
    const hipError_t bad = check_launch(kind, prec, dir, a, block, lds_bytes, (size_t)lds_limit_bytes(), fixed);
    if (bad != hipSuccess) return (int)bad;
    KernelFn fn = fixed ? fixed->fn : pick_kernel(kind, prec, dir, a.flags);
    if (!fn) return (int)hipErrorInvalidValue;
    KArgs args = a;
    args.nblk = grid;
    if (lds_bytes > 65536) {
        int e = raise_lds_limit((const void*)fn, lds_bytes);
        if (e != (int)hipSuccess) return e;
    }
    if (t_begin && t_end) {
        void* kargs[1] = {&args};
        hipError_t e = hipExtLaunchKernel((const void*)fn, dim3(grid), dim3(block), kargs, lds_bytes, stream, t_begin,
                                          t_end, 0);
        return e != hipSuccess ? (int)e : (int)hipGetLastError();
    }
    hipLaunchKernelGGL(fn, dim3(grid), dim3(block), lds_bytes, stream, args);
    return (int)hipGetLastError();
}

}  // namespace vkfx
