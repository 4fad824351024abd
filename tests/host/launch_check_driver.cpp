// Host-side checks of the launch validation (csrc/launch_check.cpp): each
// case builds the KArgs of one launch and compares check_launch's verdict
// with the expected one. Prints "ok <cases>" and exits 0 when all agree.
#include <cstdio>
#include <cstring>

#include "kernels.hpp"

using namespace vkfx;

static int fails = 0, cases = 0;

static void expect(const char* name, hipError_t got, hipError_t want) {
    ++cases;
    if (got != want) {
        ++fails;
        std::printf("FAIL %s: got %d, want %d\n", name, (int)got, (int)want);
    }
}

// A runtime-shape f32 line of N = 34 = 2 * 17 with a Rader stage for 17:
// G lines of LS elements, 34 threads per line.
static KArgs rader_args() {
    KArgs a;
    std::memset(&a, 0, sizeof a);
    a.N = 34;
    a.TT = 34;
    a.G = 2;
    a.LS = 37;
    a.PS = 4;
    a.nstages = 2;
    a.radix[0] = 2;
    a.radix[1] = 17;
    a.in_es = a.out_es = 1;
    static const int table = 0;
    a.rtab = &table;
    a.flags = KF_RADER;
    return a;
}

int main() {
    const size_t limit = 160 * 1024;
    const KArgs r = rader_args();
    const unsigned block = (unsigned)(r.G * r.TT);
    const size_t two = 2 * (size_t)r.G * r.LS * 8, one = (size_t)r.G * r.LS * 8;
    expect("rader staged, line + scratch region", check_launch(KK_PLAIN, 0, -1, r, block, two, limit, nullptr),
           hipSuccess);
    expect("rader staged, scratch region missing", check_launch(KK_PLAIN, 0, -1, r, block, one, limit, nullptr),
           hipErrorInvalidConfiguration);
    expect("rader f64 sized for f32", check_launch(KK_PLAIN, 1, -1, r, block, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs f = r;
    f.flags = 0;
    expect("rader stages without KF_RADER", check_launch(KK_PLAIN, 0, -1, f, block, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs d = r;
    d.flags |= KF_DYN_DIRECT;
    expect("rader with HBM-direct stages", check_launch(KK_PLAIN, 0, -1, d, block, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs e = r;
    e.flags |= KF_EDGE;
    e.zr = e.N;
    expect("rader with edge work", check_launch(KK_PLAIN, 0, -1, e, block, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    FixedKernel fx;
    std::memset(&fx, 0, sizeof fx);
    fx.kind = KK_PLAIN;
    fx.prec = 0;
    fx.dir = -1;
    fx.N = r.N;
    fx.TT = r.TT;
    fx.G = r.G;
    fx.PS = r.PS;
    fx.LS = r.LS;
    fx.nst = r.nstages;
    fx.radix[0] = 2;
    fx.radix[1] = 17;
    fx.lds_mult = 1;
    expect("rader on a fixed shape", check_launch(KK_PLAIN, 0, -1, r, block, two, limit, &fx),
           hipErrorInvalidConfiguration);
    KArgs n = r;
    n.rtab = nullptr;
    expect("rader radix without its table", check_launch(KK_PLAIN, 0, -1, n, block, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs s = r;
    s.radix[1] = 16;
    s.N = 32;
    s.TT = 16;
    expect("table without a rader radix", check_launch(KK_PLAIN, 0, -1, s, 32, two, limit, nullptr),
           hipErrorInvalidConfiguration);
    // ordinary launches around the new rules
    KArgs p = s;
    p.rtab = nullptr;
    p.flags = 0;
    expect("plain staged", check_launch(KK_PLAIN, 0, -1, p, 32, (size_t)p.G * p.LS * 8, limit, nullptr),
           hipSuccess);
    expect("plain, block != G * TT", check_launch(KK_PLAIN, 0, -1, p, 64, (size_t)p.G * p.LS * 8, limit, nullptr),
           hipErrorInvalidConfiguration);
    expect("plain, LDS beyond the limit", check_launch(KK_PLAIN, 0, -1, p, 32, limit + 8, limit, nullptr),
           hipErrorInvalidConfiguration);
    expect("plain, bad direction", check_launch(KK_PLAIN, 0, 0, p, 32, (size_t)p.G * p.LS * 8, limit, nullptr),
           hipErrorInvalidValue);
    // the four-step convolution row pass: rows of N2 = N, C = N1 rows per
    // transform, the spectrum and the W_M table present
    KArgs cb = p;
    static const float spec = 0, tw = 0;
    cb.C = cb.N1 = 4;
    cb.N2 = cb.N;
    cb.M = cb.N1 * cb.N2;
    cb.spec = &spec;
    cb.tlo = cb.thi = &tw;
    const size_t cb_lds = (size_t)cb.G * cb.LS * 8;
    FixedKernel fc;
    std::memset(&fc, 0, sizeof fc);
    fc.kind = KK_CONV_B;
    fc.dir = -1;
    fc.N = cb.N;
    fc.TT = cb.TT;
    fc.G = cb.G;
    fc.PS = cb.PS;
    fc.LS = cb.LS;
    fc.nst = cb.nstages;
    for (int i = 0; i < cb.nstages; ++i) fc.radix[i] = cb.radix[i];
    fc.lds_mult = 1;
    expect("conv rows", check_launch(KK_CONV_B, 0, -1, cb, 32, cb_lds, limit, &fc), hipSuccess);
    expect("conv rows on the runtime kernel", check_launch(KK_CONV_B, 0, -1, cb, 32, cb_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs cb1 = cb;
    cb1.spec = nullptr;
    expect("conv rows without the spectrum", check_launch(KK_CONV_B, 0, -1, cb1, 32, cb_lds, limit, &fc),
           hipErrorInvalidConfiguration);
    KArgs cb2 = cb;
    cb2.tlo = nullptr;
    expect("conv rows without the twiddle table", check_launch(KK_CONV_B, 0, -1, cb2, 32, cb_lds, limit, &fc),
           hipErrorInvalidConfiguration);
    KArgs cb3 = cb;
    cb3.N2 = cb.N / 2;
    cb3.M = cb3.N1 * cb3.N2;
    expect("conv rows, N2 != row length", check_launch(KK_CONV_B, 0, -1, cb3, 32, cb_lds, limit, &fc),
           hipErrorInvalidConfiguration);
    KArgs cb4 = cb;
    cb4.C = cb.N1 + 1;
    expect("conv rows, C != N1", check_launch(KK_CONV_B, 0, -1, cb4, 32, cb_lds, limit, &fc),
           hipErrorInvalidConfiguration);
    // the mixed-storage four-step passes: fixed shapes only, the column pass
    // with the narrow input, the row pass with the narrow output
    FixedKernel fe;
    std::memset(&fe, 0, sizeof fe);
    fe.kind = KK_FS_A_EDGE;
    fe.dir = -1;
    fe.N = p.N;
    fe.TT = p.TT;
    fe.G = p.G;
    fe.PS = p.PS;
    fe.LS = p.LS;
    fe.nst = p.nstages;
    fe.col = true;
    for (int i = 0; i < p.nstages; ++i) fe.radix[i] = p.radix[i];
    fe.lds_mult = 1;
    KArgs ea = p;
    ea.C = ea.N2 = 64;
    ea.N1 = ea.N;
    ea.M = ea.N1 * ea.N2;
    ea.flags = KF_NARROW_IN;
    const size_t e_lds = (size_t)ea.G * ea.LS * 8;
    expect("fs edge columns", check_launch(KK_FS_A_EDGE, 0, -1, ea, 32, e_lds, limit, &fe), hipSuccess);
    expect("fs edge columns on the runtime kernel", check_launch(KK_FS_A_EDGE, 0, -1, ea, 32, e_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs ea1 = ea;
    ea1.flags = 0;
    expect("fs edge columns without the narrow input", check_launch(KK_FS_A_EDGE, 0, -1, ea1, 32, e_lds, limit, &fe),
           hipErrorInvalidConfiguration);
    KArgs ea2 = ea;
    ea2.flags |= KF_ZERO_IN;
    ea2.zl = 10, ea2.zr = ea.M + 1;
    expect("fs edge columns, zero interval past the line", check_launch(KK_FS_A_EDGE, 0, -1, ea2, 32, e_lds, limit, &fe),
           hipErrorInvalidConfiguration);
    ea2.zr = ea.M;
    expect("fs edge columns, zero interval", check_launch(KK_FS_A_EDGE, 0, -1, ea2, 32, e_lds, limit, &fe), hipSuccess);
    KArgs ea3 = ea;
    ea3.flags |= KF_NARROW_OUT;
    expect("fs edge columns with a narrow output", check_launch(KK_FS_A_EDGE, 0, -1, ea3, 32, e_lds, limit, &fe),
           hipErrorInvalidConfiguration);
    FixedKernel fb = fe;
    fb.kind = KK_FS_B_EDGE;
    fb.col = false;
    KArgs eb = p;
    eb.C = eb.N1 = 64;
    eb.N2 = eb.N;
    eb.M = eb.N1 * eb.N2;
    eb.flags = KF_NARROW_OUT | KF_ZERO_OUT;
    eb.zl = 0, eb.zr = 5;
    expect("fs edge rows", check_launch(KK_FS_B_EDGE, 0, -1, eb, 32, e_lds, limit, &fb), hipSuccess);
    KArgs eb1 = eb;
    eb1.flags = KF_NARROW_OUT | KF_ZERO_IN;
    expect("fs edge rows with an input zero interval", check_launch(KK_FS_B_EDGE, 0, -1, eb1, 32, e_lds, limit, &fb),
           hipErrorInvalidConfiguration);
    KArgs eb2 = eb;
    eb2.C = eb.N1 - 1;
    expect("fs edge rows, C != N1", check_launch(KK_FS_B_EDGE, 0, -1, eb2, 32, e_lds, limit, &fb),
           hipErrorInvalidConfiguration);
    KArgs eb3 = eb;
    eb3.flags |= KF_EDGE;
    expect("fs edge rows with KF_EDGE", check_launch(KK_FS_B_EDGE, 0, -1, eb3, 32, e_lds, limit, &fb),
           hipErrorInvalidConfiguration);
    // the one-upload Bluestein kernel with its boundary work: fixed shapes
    // with chirp and spectrum, zero intervals within the line's N elements
    FixedKernel fbl = fe;
    fbl.kind = KK_BLUE_1_EDGE;
    fbl.col = false;
    static const float btab = 0;
    KArgs bl = p;
    bl.chirp = bl.spec = &btab;
    bl.nvalid = bl.nout = 100;
    bl.flags = KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_IN;
    bl.zl = 3, bl.zr = 100;
    expect("bluestein edges", check_launch(KK_BLUE_1_EDGE, 0, -1, bl, 32, e_lds, limit, &fbl), hipSuccess);
    expect("bluestein edges on the runtime kernel", check_launch(KK_BLUE_1_EDGE, 0, -1, bl, 32, e_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs bl1 = bl;
    bl1.zr = 101;
    expect("bluestein edges, zero interval past the line",
           check_launch(KK_BLUE_1_EDGE, 0, -1, bl1, 32, e_lds, limit, &fbl), hipErrorInvalidConfiguration);
    KArgs bl2 = bl;
    bl2.chirp = nullptr;
    expect("bluestein edges without a chirp", check_launch(KK_BLUE_1_EDGE, 0, -1, bl2, 32, e_lds, limit, &fbl),
           hipErrorInvalidConfiguration);
    KArgs bl3 = bl;
    bl3.flags |= KF_EDGE;
    expect("bluestein edges with KF_EDGE", check_launch(KK_BLUE_1_EDGE, 0, -1, bl3, 32, e_lds, limit, &fbl),
           hipErrorInvalidConfiguration);
    KArgs bl4 = bl;
    expect("narrow input on the plain Bluestein kernel", check_launch(KK_BLUE_1, 0, -1, bl4, 32, e_lds, limit, nullptr),
           hipErrorInvalidValue);
    // the even-length real kernels with their boundary work: the zero
    // interval on the real side only, within 2N reals
    FixedKernel fr = fe;
    fr.kind = KK_R2C_HALF_EDGE;
    fr.col = false;
    KArgs re = p;
    re.flags = KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_IN;
    re.zl = 1, re.zr = 2 * re.N;
    expect("real edges, R2C", check_launch(KK_R2C_HALF_EDGE, 0, -1, re, 32, e_lds, limit, &fr), hipSuccess);
    KArgs re1 = re;
    re1.zr = 2 * re.N + 1;
    expect("real edges, zero interval past the reals", check_launch(KK_R2C_HALF_EDGE, 0, -1, re1, 32, e_lds, limit, &fr),
           hipErrorInvalidConfiguration);
    KArgs re2 = re;
    re2.flags = KF_NARROW_IN | KF_ZERO_OUT;
    expect("real edges, R2C with an output zero interval",
           check_launch(KK_R2C_HALF_EDGE, 0, -1, re2, 32, e_lds, limit, &fr), hipErrorInvalidConfiguration);
    expect("real edges on the runtime kernel", check_launch(KK_R2C_HALF_EDGE, 0, -1, re, 32, e_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    FixedKernel fc2 = fr;
    fc2.kind = KK_C2R_HALF_EDGE;
    fc2.dir = 1;
    KArgs rc2 = re;
    rc2.flags = KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_OUT;
    expect("real edges, C2R", check_launch(KK_C2R_HALF_EDGE, 0, 1, rc2, 32, e_lds, limit, &fc2), hipSuccess);
    rc2.flags = KF_NARROW_IN | KF_ZERO_IN;
    expect("real edges, C2R with an input zero interval", check_launch(KK_C2R_HALF_EDGE, 0, 1, rc2, 32, e_lds, limit, &fc2),
           hipErrorInvalidConfiguration);
    // fixed one-upload rows with their boundary work
    FixedKernel fpl = fr;
    fpl.kind = KK_PLAIN_EDGE;
    KArgs pe = p;
    pe.flags = KF_NARROW_IN | KF_NARROW_OUT | KF_ZERO_OUT;
    pe.zl = 0, pe.zr = pe.N;
    expect("plain edges", check_launch(KK_PLAIN_EDGE, 0, -1, pe, 32, e_lds, limit, &fpl), hipSuccess);
    KArgs pe1 = pe;
    pe1.zr = pe.N + 1;
    expect("plain edges, zero interval past the line", check_launch(KK_PLAIN_EDGE, 0, -1, pe1, 32, e_lds, limit, &fpl),
           hipErrorInvalidConfiguration);
    KArgs pe2 = pe;
    pe2.flags |= KF_EDGE;
    expect("plain edges with KF_EDGE", check_launch(KK_PLAIN_EDGE, 0, -1, pe2, 32, e_lds, limit, &fpl),
           hipErrorInvalidConfiguration);
    expect("plain edges on the runtime kernel", check_launch(KK_PLAIN_EDGE, 0, -1, pe, 32, e_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    // the matrix convolution product: whole systems of C1 lines per block on
    // the runtime-shape kernel
    KArgs cm = p;
    static const float mspec = 0;
    cm.spec = &mspec;
    cm.C = 1;
    cm.C1 = 2;
    cm.flags = KF_CONV_MATRIX;
    const size_t cm_lds = (size_t)cm.G * cm.LS * 8;
    expect("conv matrix", check_launch(KK_CONV_1, 0, -1, cm, 32, cm_lds, limit, nullptr), hipSuccess);
    KArgs cm1 = cm;
    cm1.C1 = 3;
    expect("conv matrix, lines per block not whole systems", check_launch(KK_CONV_1, 0, -1, cm1, 32, cm_lds, limit,
                                                                         nullptr),
           hipErrorInvalidConfiguration);
    KArgs cm2 = cm;
    cm2.C1 = 4;
    cm2.G = 4;
    cm2.TT = 8;
    expect("conv matrix beyond 3 x 3", check_launch(KK_CONV_1, 0, -1, cm2, 32, (size_t)4 * cm.LS * 8, limit, nullptr),
           hipErrorInvalidConfiguration);
    KArgs cm3 = cm;
    cm3.flags = KF_CONV_SYM;
    expect("conv symmetric without the matrix flag", check_launch(KK_CONV_1, 0, -1, cm3, 32, cm_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    expect("conv matrix on a plain pass", check_launch(KK_PLAIN, 0, -1, cm, 32, cm_lds, limit, nullptr),
           hipErrorInvalidConfiguration);
    if (fails) return 1;
    std::printf("ok %d\n", cases);
    return 0;
}
