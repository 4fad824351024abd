// launch_check.cpp -- host-side validation of one kernel launch (no HIP
// calls: it builds with g++ as well, for the CPU tests of the rejections).
#include "kernels.hpp"

namespace vkfx {

hipError_t check_launch(KernelKind kind, int prec, int dir, const KArgs& a, unsigned block, size_t lds_bytes,
                        size_t lds_limit, const FixedKernel* fixed) {
    if (kind < 0 || kind >= KK_COUNT || (dir != -1 && dir != 1) || (prec != 0 && prec != 1))
        return hipErrorInvalidValue;
    // runtime-shape kernels are built for at most 512 threads, fixed shapes
    // for exactly their own G * TT (at most 1024)
    if (block == 0 || block > (fixed ? 1024u : 512u) || a.G < 1 || a.G > kMaxLinesPerBlock ||
        (unsigned)(a.G * a.TT) != block)
        return hipErrorInvalidConfiguration;
    if (a.nstages < 0 || a.nstages > kMaxStages) return hipErrorInvalidValue;
    if (lds_bytes < (size_t)a.G * (size_t)a.LS * (prec ? 16 : 8) * (fixed ? fixed->lds_mult : 1) ||
        lds_bytes > lds_limit)
        return hipErrorInvalidConfiguration;
    if (kind == KK_CONV_1 && !a.spec) return hipErrorInvalidConfiguration;
    // the matrix product mixes whole systems of C1 coordinate lines in a
    // block of the runtime-shape kernel
    if ((a.flags & (KF_CONV_MATRIX | KF_CONV_SYM)) &&
        (kind != KK_CONV_1 || fixed || !(a.flags & KF_CONV_MATRIX) || a.C != 1 || a.C1 < 2 ||
         a.C1 > kMaxConvMatrix || a.G % a.C1 != 0))
        return hipErrorInvalidConfiguration;
    // the four-step convolution row pass: rows k1 < N1 of N2 = N elements,
    // the N1 x N2 spectrum and the W_M table
    if (kind == KK_CONV_B && (!fixed || !a.spec || !a.tlo || !a.thi || a.N2 != a.N || a.N1 < 1 || a.C != a.N1 ||
                              a.M != a.N1 * a.N2))
        return hipErrorInvalidConfiguration;
    if (kind == KK_RADER_DIRECT && (a.TT != a.N || a.LS < a.N + 1 || a.N < 1 || !a.pin || !a.pout))
        return hipErrorInvalidConfiguration;
    if (kind == KK_RADER_FFT && (!a.pin || !a.pout || a.LS < a.N + ((a.N - 1) >> a.PS) + 1))
        return hipErrorInvalidConfiguration;
    // the direct runtime-shape kernels read (C2C, even R2C, even C2R with
    // KF_DYN_PRE) and write (C2C, even C2R) contiguous lines, with no radix-2
    // stage at a direct end
    if (!fixed && (a.flags & KF_DYN_DIRECT) &&
        !(kind == KK_PLAIN && a.in_es == 1 && a.out_es == 1 && a.nstages >= 2 && a.radix[0] != 2 &&
          a.radix[a.nstages - 1] != 2) &&
        !(kind == KK_R2C_HALF && a.in_es == 1 && a.nstages >= 1 && a.radix[0] != 2) &&
        !(kind == KK_C2R_HALF && a.out_es == 1 && a.nstages >= 1 && a.radix[a.nstages - 1] != 2 &&
          (!(a.flags & KF_DYN_PRE) || (a.in_es == 1 && a.nstages >= 2 && a.radix[0] != 2))))
        return hipErrorInvalidConfiguration;
    // boundary work runs in the runtime-shape C2C kernels only (staged, or
    // HBM-direct under the direct kernel's own conditions below)
    const bool fs_edge = kind == KK_FS_A_EDGE || kind == KK_FS_B_EDGE;
    const bool blue_edge = kind == KK_BLUE_1_EDGE;
    const bool real_edge = kind == KK_R2C_HALF_EDGE || kind == KK_C2R_HALF_EDGE;
    const bool plain_edge = kind == KK_PLAIN_EDGE;
    const bool side_edge = kind == KK_PLAIN_EDGE_IN || kind == KK_PLAIN_EDGE_OUT;
    if ((a.flags & (KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_IN | KF_ZERO_OUT)) && !(a.flags & KF_EDGE) && !fs_edge &&
        !blue_edge && !real_edge && !plain_edge && !side_edge)
        return hipErrorInvalidValue;
    // the first / last pass of a mixed-storage N-D chunk: fixed shapes, the
    // storage type on one side, no zero intervals
    if (side_edge && (!fixed || (a.flags & (KF_EDGE | KF_ZERO_IN | KF_ZERO_OUT)) ||
                      ((a.flags & KF_NARROW_IN) != 0) != (kind == KK_PLAIN_EDGE_IN) ||
                      ((a.flags & KF_NARROW_OUT) != 0) != (kind == KK_PLAIN_EDGE_OUT)))
        return hipErrorInvalidConfiguration;
    // the fixed one-upload rows of mixed-storage plans: narrow input and
    // output, zero intervals within the line's N elements
    if (plain_edge && (!fixed || (a.flags & KF_EDGE) || !(a.flags & KF_NARROW_IN) || !(a.flags & KF_NARROW_OUT) ||
                       ((a.flags & (KF_ZERO_IN | KF_ZERO_OUT)) && (a.zl < 0 || a.zl > a.zr || a.zr > a.N))))
        return hipErrorInvalidConfiguration;
    // the even-length real kernels with their boundary work: fixed shapes,
    // the zero interval on the real side (R2C input, C2R output) within the
    // line's 2N real elements
    if (real_edge &&
        (!fixed || (a.flags & KF_EDGE) ||
         (a.flags & (kind == KK_R2C_HALF_EDGE ? KF_ZERO_OUT : KF_ZERO_IN)) ||
         ((a.flags & (KF_ZERO_IN | KF_ZERO_OUT)) && (a.zl < 0 || a.zl > a.zr || a.zr > 2 * (long long)a.N))))
        return hipErrorInvalidConfiguration;
    // the one-upload Bluestein kernel with its boundary work: fixed shapes,
    // chirp and spectrum tables, zero intervals over the line's N elements
    if (blue_edge && (!fixed || (a.flags & KF_EDGE) || !a.chirp || !a.spec ||
                      ((a.flags & (KF_ZERO_IN | KF_ZERO_OUT)) &&
                       (a.zl < 0 || a.zl > a.zr || a.zr > a.nvalid || a.zr > a.nout))))
        return hipErrorInvalidConfiguration;
    // the mixed-storage four-step passes: fixed shapes, the first pass reads
    // the narrow input (and its zero interval), the last writes the narrow
    // output (and its zero interval), over line elements [0, M)
    if (fs_edge) {
        if (!fixed || (a.flags & KF_EDGE)) return hipErrorInvalidConfiguration;
        if (kind == KK_FS_A_EDGE &&
            (!(a.flags & KF_NARROW_IN) || (a.flags & (KF_NARROW_OUT | KF_ZERO_OUT)) || a.N2 < 1 || a.C != a.N2))
            return hipErrorInvalidConfiguration;
        if (kind == KK_FS_B_EDGE &&
            (!(a.flags & KF_NARROW_OUT) || (a.flags & (KF_NARROW_IN | KF_ZERO_IN)) || a.N1 < 1 || a.C != a.N1))
            return hipErrorInvalidConfiguration;
        if ((a.flags & (KF_ZERO_IN | KF_ZERO_OUT)) && (a.zl < 0 || a.zl > a.zr || a.zr > a.M))
            return hipErrorInvalidConfiguration;
    }
    if ((a.flags & KF_EDGE) && (fixed || kind != KK_PLAIN || (a.flags & KF_DYN_PRE) || a.zl > a.zr || a.zl < 0 ||
                                a.zr > a.N))
        return hipErrorInvalidConfiguration;
    // the register-exchange kernels address contiguous lines (element stride 1)
    if (fixed && fixed->table == FT_WAVE1024 && (a.in_es != 1 || a.out_es != 1 || !a.tw))
        return hipErrorInvalidConfiguration;
    if (fixed && fixed->table == FT_STAGE_PR && !a.tw) return hipErrorInvalidConfiguration;
    if (fixed) {
        // the fixed shape must be launched with exactly its own geometry
        if (fixed->kind != kind || fixed->prec != prec || fixed->dir != dir || fixed->N != a.N ||
            fixed->TT != a.TT || fixed->G != a.G || fixed->PS != a.PS || fixed->LS != a.LS ||
            fixed->nst != a.nstages)
            return hipErrorInvalidConfiguration;
        for (int i = 0; i < fixed->nst; ++i)
            if (fixed->radix[i] != a.radix[i]) return hipErrorInvalidConfiguration;
    }
    // Rader stages (a runtime radix above kMaxStockhamRadix) run only in the
    // staged runtime-shape kernel, which gives each line a second LDS region
    // of LS elements after the G lines: 2 G LS elements in all
    bool rader_stage = false;
    // (a fixed shape's radices are compile-time Stockham butterflies)
    for (int i = 0; i < a.nstages; ++i) rader_stage = rader_stage || (!fixed && a.radix[i] > kMaxStockhamRadix);
    if (rader_stage && !a.rtab) return hipErrorInvalidConfiguration;
    if (((a.flags & KF_RADER) != 0) != (a.rtab != nullptr)) return hipErrorInvalidConfiguration;
    if (a.rtab) {
        if (fixed || (a.flags & (KF_DYN_DIRECT | KF_EDGE)) || !rader_stage) return hipErrorInvalidConfiguration;
        if (lds_bytes < 2 * (size_t)a.G * (size_t)a.LS * (prec ? 16 : 8)) return hipErrorInvalidConfiguration;
    }
    return hipSuccess;
}

}  // namespace vkfx
