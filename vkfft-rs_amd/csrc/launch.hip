// launch.hip -- dispatches a KernelKind to its instantiation and launches it.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <string>

#include "kernels.hpp"

namespace vkfx {

KernelFn pick_f32_fwd(KernelKind kind, bool wide, int direct, int edge);
KernelFn pick_f32_inv(KernelKind kind, bool wide, int direct, int edge);
KernelFn pick_f64_fwd(KernelKind kind, bool wide, int direct, int edge);
KernelFn pick_f64_inv(KernelKind kind, bool wide, int direct, int edge);
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
                                                fixed_table_blue_rows_f32, fixed_table_blue_rows_f64};
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

// Blocks per CU of a persistent launch (0 = one block per group). Tuning knob:
// VKFX_PERSIST_BLOCKS_PER_CU.
static int persist_blocks_per_cu() {
    static const int v = [] {
        const char* e = getenv("VKFX_PERSIST_BLOCKS_PER_CU");
        return e ? atoi(e) : 0;
    }();
    return v;
}

// Launches whose blocks share HBM cache lines with their neighbours get their
// groups dealt to XCDs in contiguous ranges: the four-step passes that read
// or write the N/2+1-pitch real-transform spectra (unaligned 128-byte
// segments) and the Bluestein passes over pitch-N lines. Measured on C2: the
// C2R column pass reads 1.0x its bytes instead of 2.0x and the R2C row pass
// writes 1.0x instead of 1.19x. VKFX_XCD_GROUPS=0/1 forces it off/on for
// every launch (tuning runs).
static bool xcd_groups(KernelKind kind) {
    static const int forced = [] {
        const char* e = getenv("VKFX_XCD_GROUPS");
        return e ? (e[0] == '1' ? 1 : 0) : -1;
    }();
    if (forced >= 0) return forced == 1;
    return kind == KK_FS_B_R2C || kind == KK_FS_A_C2R || kind == KK_FS_A_BLUE || kind == KK_BLUE_B ||
           kind == KK_FS_C_BLUE;
}

static KernelFn pick_kernel(KernelKind kind, int prec, int dir, int flags) {
    const bool wide = (flags & KF_DYN_WIDE) != 0;
    const int direct = (flags & KF_DYN_DIRECT) ? ((flags & KF_DYN_PRE) ? 2 : 1) : 0;
    const int edge =
        (flags & KF_EDGE) ? 1 + ((flags & KF_NARROW_IN) ? 1 : 0) + ((flags & KF_NARROW_OUT) ? 2 : 0) : 0;
    return prec == 0 ? (dir < 0 ? pick_f32_fwd(kind, wide, direct, edge) : pick_f32_inv(kind, wide, direct, edge))
                     : (dir < 0 ? pick_f64_fwd(kind, wide, direct, edge) : pick_f64_inv(kind, wide, direct, edge));
}

const void* fft_kernel_fn(KernelKind kind, int prec, int dir, const FixedKernel* fixed, int flags) {
    if (kind < 0 || kind >= KK_COUNT || (dir != -1 && dir != 1) || (prec != 0 && prec != 1)) return nullptr;
    if (fixed) return (const void*)fixed->fn;
    return (const void*)pick_kernel(kind, prec, dir, flags);
}

int launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned grid, unsigned block, size_t lds_bytes,
           hipStream_t stream, const FixedKernel* fixed) {
    if (kind < 0 || kind >= KK_COUNT || (dir != -1 && dir != 1) || (prec != 0 && prec != 1))
        return (int)hipErrorInvalidValue;
    if (grid == 0) return (int)hipSuccess;
    // runtime-shape kernels are built for at most 512 threads, fixed shapes
    // for exactly their own G * TT (at most 1024)
    if (block == 0 || block > (fixed ? 1024u : 512u) || a.G < 1 || a.G > kMaxLinesPerBlock ||
        (unsigned)(a.G * a.TT) != block)
        return (int)hipErrorInvalidConfiguration;
    if (a.nstages < 0 || a.nstages > kMaxStages) return (int)hipErrorInvalidValue;
    if (lds_bytes < (size_t)a.G * (size_t)a.LS * (prec ? 16 : 8) * (fixed ? fixed->lds_mult : 1) ||
        lds_bytes > (size_t)lds_limit_bytes())
        return (int)hipErrorInvalidConfiguration;
    if (kind == KK_CONV_1 && !a.spec) return (int)hipErrorInvalidConfiguration;
    if (kind == KK_RADER_DIRECT && (a.TT != a.N || a.LS < a.N + 1 || a.N < 1 || !a.pin || !a.pout))
        return (int)hipErrorInvalidConfiguration;
    if (kind == KK_RADER_FFT && (!a.pin || !a.pout || a.LS < a.N + ((a.N - 1) >> a.PS) + 1))
        return (int)hipErrorInvalidConfiguration;
    KernelFn fn = pick_kernel(kind, prec, dir, a.flags);
    // the direct runtime-shape kernels read (C2C, even R2C, even C2R with
    // KF_DYN_PRE) and write (C2C, even C2R) contiguous lines, with no radix-2
    // stage at a direct end
    if (!fixed && (a.flags & KF_DYN_DIRECT) &&
        !(kind == KK_PLAIN && a.in_es == 1 && a.out_es == 1 && a.nstages >= 2 && a.radix[0] != 2 &&
          a.radix[a.nstages - 1] != 2) &&
        !(kind == KK_R2C_HALF && a.in_es == 1 && a.nstages >= 1 && a.radix[0] != 2) &&
        !(kind == KK_C2R_HALF && a.out_es == 1 && a.nstages >= 1 && a.radix[a.nstages - 1] != 2 &&
          (!(a.flags & KF_DYN_PRE) || (a.in_es == 1 && a.nstages >= 2 && a.radix[0] != 2))))
        return (int)hipErrorInvalidConfiguration;
    // boundary work runs in the runtime-shape C2C kernels only (staged, or
    // HBM-direct under the direct kernel's own conditions below)
    if ((a.flags & (KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_IN | KF_ZERO_OUT)) && !(a.flags & KF_EDGE))
        return (int)hipErrorInvalidValue;
    if ((a.flags & KF_EDGE) && (fixed || kind != KK_PLAIN || (a.flags & KF_DYN_PRE) || a.zl > a.zr || a.zl < 0 ||
                                a.zr > a.N))
        return (int)hipErrorInvalidConfiguration;
    // the register-exchange kernels address contiguous lines (element stride 1)
    if (fixed && fixed->table == FT_WAVE1024 && (a.in_es != 1 || a.out_es != 1 || !a.tw))
        return (int)hipErrorInvalidConfiguration;
    if (fixed && fixed->table == FT_STAGE_PR && !a.tw) return (int)hipErrorInvalidConfiguration;
    if (fixed) {
        // the fixed shape must be launched with exactly its own geometry
        if (fixed->kind != kind || fixed->prec != prec || fixed->dir != dir || fixed->N != a.N ||
            fixed->TT != a.TT || fixed->G != a.G || fixed->PS != a.PS || fixed->LS != a.LS ||
            fixed->nst != a.nstages)
            return (int)hipErrorInvalidConfiguration;
        for (int i = 0; i < fixed->nst; ++i)
            if (fixed->radix[i] != a.radix[i]) return (int)hipErrorInvalidConfiguration;
        fn = fixed->fn;
    }
    if (!fn) return (int)hipErrorInvalidValue;
    KArgs args = a;
    args.nblk = grid;
    if (xcd_groups(kind)) args.flags |= KF_XCD_GROUPS;
    if (fixed && fixed->fn_persist && persist_blocks_per_cu() > 0) {
        // persistent launch: at most the resident capacity, groups by grid stride
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
                cus = 256;
        }
        fn = fixed->fn_persist;
        const unsigned cap = (unsigned)(cus * persist_blocks_per_cu());
        if (grid > cap) grid = cap;
    }
    if (lds_bytes > 65536) {
        hipError_t e =
            hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(fn, dim3(grid), dim3(block), lds_bytes, stream, args);
    return (int)hipGetLastError();
}

}  // namespace vkfx
