// runtime.cpp -- context, plans and the C ABI of the MI355X FFT path.
//
// A plan is a list of kernel launches (fft_kernels.hip) with their tables
// (twiddles, chirps, kernel spectra) uploaded once at plan time, mirroring
// what vkfft-rs's HIP runtime keeps in its module/LUT caches
// (src/backend/hip/runtime.rs:1422-1468, 2019-2039) but without any source
// generation or JIT step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <limits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "planner.hpp"
#include "vkfx.h"

using namespace vkfx;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(VKFX_ERR_NATIVE_RUNTIME, std::string(what) + ": " + hipGetErrorString(e));
}

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

typedef long double ld;
const ld kPi = 3.141592653589793238462643383279502884L;

// exp(-2 pi i k / n) with exact integer reduction of k.
void root(ld k, ld n, ld& c, ld& s) {
    ld a = -2.0L * kPi * k / n;
    c = cosl(a);
    s = sinl(a);
}

}  // namespace

// Pooled device / pinned host buffer. `ready` (optional) is recorded on the
// stream of its last user; the next user's stream waits on it, so reuse is
// stream-ordered.
struct PoolBuf {
    void* p = nullptr;
    size_t bytes = 0;
    hipEvent_t ready = nullptr;
};

struct vkfx_context {
    int device = 0;
    hipStream_t stream = nullptr;
    vkfx_device_profile profile{};
    std::vector<PoolBuf> dev_pool, host_pool;  // free buffers
    std::vector<hipStream_t> stream_pool;      // free streams for tickets
    void* scratch = nullptr;                   // this device's static scratch (vkfx_execute_noalloc)
    hipError_t scratch_err = hipSuccess;       // why `scratch` is null, if it is
    std::mutex mu;                             // guards the pools, `active` and `plans`
    int active = 0;                            // tickets submitted and not yet destroyed
    int plans = 0;                             // plans created and not yet destroyed
};

namespace {

// Buffers a launch reads or writes: the caller's input and output, the
// plan's workspace (per stream lane) and, for mixed storage/compute
// precisions, the compute-type copies of the input and output in the
// workspace; SEL_FULL is the N-point complex copy of a real transform run
// through a full-length C2C plan; SEL_AUX the compact spectrum between the
// complex axes and the real axis of an N-D C2R.
enum BufSel : int {
    SEL_IN = 0,
    SEL_OUT = 1,
    SEL_WORK = 2,
    SEL_STAGE_IN = 3,
    SEL_STAGE_OUT = 4,
    SEL_FULL = 5,
    SEL_AUX = 6,
    SEL_CONV_A = 7,  // real-application convolution: forward spectrum
    SEL_CONV_B = 8   // real-application convolution: multiplied spectrum
};

struct Launch {
    KernelKind kind;
    int dir;
    KArgs a;
    unsigned grid, block;
    size_t lds;
    int in_sel, out_sel;
    size_t in_off, out_off;  // byte offsets into the selected buffers
    std::string label;
    const FixedKernel* fixed;
    int chunk;  // batch chunk; chunks alternate between two stream lanes
    // boundary pass instead of an FFT kernel (type conversion, formatted
    // layouts, zero padding; convert.hip)
    bool boundary = false;
    // plain copy of copy_bytes (a transform of length 1; convert.hip)
    bool copy = false;
    size_t copy_bytes = 0;
    BoundaryArgs ba;
    // DCT / DST pre (1) or post (2) pass instead of an FFT kernel (r2r.hip)
    int r2r = 0;
    R2rArgs ra;
    // convolution multiply instead of an FFT kernel (conv.hip)
    bool conv = false;
    ConvArgs ca;
    const void* conv_kernel = nullptr;
};

// Line geometry of one FFT length inside a kernel.
struct Geometry {
    int N = 1, TT = 1, G = 1, LS = 1, PS = 4;
    std::vector<int> radix;
    size_t lds = 0;
    bool ok = false;
    bool wide = false;  // runtime-shape kernel with up to 32 elements per thread per stage
    bool rader = false;  // the radix list has Rader stages (lds holds a second region of G lines)
    int regions = 1;     // LDS regions of G lines (2 with Rader stages)
    const FixedKernel* fixed = nullptr;
};

// Stage radices: power-of-two part split into ceil(p/4) stages as evenly as
// possible (radix 16/8/4/2), pairs of 3 as radix 9, then one stage per
// remaining odd prime factor.
bool radix_schedule(size_t n, std::vector<int>& out) {
    out.clear();
    size_t m = n;
    int p = 0;
    while (m % 2 == 0) {
        m /= 2;
        ++p;
    }
    if (p > 0) {
        int s = (p + 3) / 4;
        int base = p / s, extra = p % s;
        for (int i = 0; i < s; ++i) out.push_back(1 << (base + (i < extra ? 1 : 0)));
    }
    int threes = 0;
    while (m % 3 == 0) {
        m /= 3;
        ++threes;
    }
    for (; threes >= 2; threes -= 2) out.push_back(9);
    if (threes) out.push_back(3);
    for (int q : {5, 7, 11, 13})
        while (m % q == 0) {
            m /= q;
            out.push_back(q);
        }
    return m == 1;
}

Geometry geometry(size_t n, int prec, int want_g, size_t lds_max, size_t lds_budget) {
    Geometry g;
    if (n == 0 || n > (1u << 20)) return g;
    if (!radix_schedule(n, g.radix)) return g;
    if ((int)g.radix.size() > kMaxStages) return g;
    g.N = (int)n;
    // threads per line: the narrow kernel (at most 16 elements per thread,
    // twice the resident waves) unless it would need more than 512 threads
    auto threads = [&](bool wide) {
        int tt = 1;
        for (int r : g.radix) {
            const int nb = (int)n / r, bpt = dyn_butterflies_per_thread(r, wide);
            tt = std::max(tt, (nb + bpt - 1) / bpt);
        }
        return tt;
    };
    int tt = threads(false);
    if (tt > 512) {
        g.wide = true;
        tt = threads(true);
    }
    if (tt > 512) return g;
    g.TT = tt;
    const size_t sz = prec ? 16 : 8;
    g.PS = prec ? 3 : 4;
    int ls = (int)n + ((int)n >> g.PS);
    if (ls % 2 == 0) ls += 1;
    g.LS = ls;
    const size_t line_bytes = (size_t)ls * sz;
    if (line_bytes > lds_max) return g;
    size_t budget = std::max(lds_budget, line_bytes);
    budget = std::min(budget, lds_max);
    int G = std::max(1, want_g);
    G = std::min(G, 512 / tt);
    G = std::min<int>(G, (int)(budget / line_bytes));
    G = std::min(G, kMaxLinesPerBlock);
    if (G < 1) return g;
    g.G = G;
    g.lds = (size_t)G * line_bytes;
    g.ok = true;
    return g;
}

// Radix list of a length whose prime factors above 13 run as Rader stages
// (the composite lengths the planner classifies as Rader, and the Rader
// convolutions of the recursive-Rader extension): the Stockham radices of
// the 2/3/5/7/11/13-smooth part, then one stage per larger prime factor.
bool radix_schedule_rader(size_t n, std::vector<int>& out) {
    size_t smooth = n;
    std::vector<int> rader;
    for (size_t q : prime_factorization(n))
        if (q > 13) {
            if (q > (size_t)std::numeric_limits<int>::max() / 2) return false;
            rader.push_back((int)q);
            smooth /= q;
        }
    if (!radix_schedule(smooth, out)) return false;
    if (smooth == 1) out.clear();
    out.insert(out.end(), rader.begin(), rader.end());
    return !out.empty() && (int)out.size() <= kMaxStages;
}

void host_fft(std::vector<ld>& re, std::vector<ld>& im);
struct Ctx;
void note_rader_stages(Ctx& c, const Geometry& g);

// Sub-radices of the length L = q - 1 FFTs of an FFT-mode Rader stage: the
// Stockham schedule of L's factors up to 13, then each prime factor in
// (13, kRaderSubPrimeMax] as a direct-multiplication stage.
bool rader_sub_schedule(size_t L, std::vector<int>& out) {
    out.clear();
    size_t smooth = L;
    std::vector<int> big;
    for (size_t f : prime_factorization(L))
        if (f > 13) {
            if (f > (size_t)kRaderSubPrimeMax) return false;
            big.push_back((int)f);
            smooth /= f;
        }
    if (smooth > 1 && !radix_schedule(smooth, out)) return false;
    if (smooth == 1) out.clear();
    out.insert(out.end(), big.begin(), big.end());
    return !out.empty() && out.size() <= 15;
}

// A Rader stage of prime q convolves by FFT (the reference's FFT-Rader node,
// rader_ir.rs:706-745) from kRaderFftStageMin on, as its direct
// multiplication costs q - 1 multiply-adds per output.
bool rader_stage_fft(size_t q) {
    std::vector<int> sub;
    return q >= (size_t)kRaderFftStageMin && rader_sub_schedule(q - 1, sub);
}

// Runtime-shape geometry of a radix list with Rader stages: the threads of a
// line cover its Stockham stages and at least min(N, 256) work items of the
// Rader stages; LDS holds the G lines and G scratch lines. `slot` adds one
// element after each line (the x0 slot of an FFT-mode Rader kernel).
Geometry geometry_rader(size_t n, int prec, int want_g, size_t lds_max, size_t lds_budget, bool slot = false) {
    Geometry g;
    if (n < 2 || n > (1u << 20)) return g;
    if (!radix_schedule_rader(n, g.radix)) return g;
    bool any = false;
    int tt = (int)std::min<size_t>(n, 256);
    for (int r : g.radix) {
        if (r > kMaxStockhamRadix) {
            any = true;
            continue;
        }
        const int nb = (int)n / r, bpt = dyn_butterflies_per_thread(r, false);
        tt = std::max(tt, (nb + bpt - 1) / bpt);
    }
    if (!any || tt > 512) return g;
    g.N = (int)n;
    g.TT = tt;
    const size_t sz = prec ? 16 : 8;
    g.PS = prec ? 3 : 4;
    int ls = (int)n + ((int)n >> g.PS) + (slot ? 2 : 0);
    if (ls % 2 == 0) ls += 1;
    g.LS = ls;
    g.regions = 2;  // line + scratch line
    const size_t line_bytes = (size_t)g.regions * (size_t)ls * sz;
    if (line_bytes > lds_max) return g;
    size_t budget = std::min(std::max(lds_budget, line_bytes), lds_max);
    int G = std::max(1, want_g);
    G = std::min(G, 512 / tt);
    G = std::min<int>(G, (int)(budget / line_bytes));
    G = std::min(G, kMaxLinesPerBlock);
    if (G < 1) return g;
    g.G = G;
    g.lds = (size_t)G * line_bytes;
    g.rader = true;
    g.ok = true;
    return g;
}

// Geometry of a kernel launch: the fixed-shape instantiation for
// (kind, precision, direction, length, lane mapping) when one is registered
// and fits, else the runtime-shape geometry.
Geometry kernel_geometry(KernelKind kind, int prec, int dir, size_t n, bool col, int want_g, size_t lds_max,
                         size_t lds_budget) {
    if (n <= (1u << 20)) {
        if (const FixedKernel* f = find_fixed(kind, prec, dir, (int)n, col)) {
            Geometry g;
            g.N = f->N;
            g.TT = f->TT;
            g.G = f->G;
            g.PS = f->PS;
            g.LS = f->LS;
            g.radix.assign(f->radix, f->radix + f->nst);
            g.lds = (size_t)g.G * g.LS * (prec ? 16 : 8) * f->lds_mult;
            g.fixed = f;
            g.ok = g.lds <= lds_max;
            if (g.ok) return g;
        }
    }
    return geometry(n, prec, want_g, lds_max, lds_budget);
}

}  // namespace

struct vkfx_plan {
    vkfx_context* ctx = nullptr;
    vkfx_plan_desc desc{};
    std::vector<Launch> launches;
    std::vector<std::unique_ptr<DevBuf>> tables;
    std::map<std::string, const void*> table_cache;
    DevBuf work;
    size_t work_bytes = 0;  // per lane while planning; total after plan_create
    size_t work_lane = 0;   // workspace bytes of one stream lane
    int lanes = 1;          // 2: chunks alternate between the caller's stream and the plan's aux stream
    bool serial = false;    // chunks depend on each other: one lane
    size_t stage_in_off = 0, stage_out_off = 0;  // dense compute-type copies behind boundary passes
    size_t stage_in_bytes = 0, stage_out_bytes = 0;
    bool stage_shared = false;  // C2C with both sides staged runs in place on one copy
    size_t full_off = 0, full_bytes = 0;  // SEL_FULL region (full-complex real transforms)
    size_t aux_off = 0, aux_bytes = 0;    // SEL_AUX region (N-D C2R compact spectrum)
    size_t conv_a_off = 0, conv_a_bytes = 0, conv_b_off = 0, conv_b_bytes = 0;  // SEL_CONV_A / SEL_CONV_B
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    hipStream_t aux = nullptr;  // the plan's second lane (two-lane plans; default priority)
    size_t in_bytes = 0, out_bytes = 0;
    bool real_out = false;    // output holds reals (C2R, DCT/DST, real-application convolution)
    int tickets = 0;          // live tickets of this plan (guarded by ctx->mu)
    std::string json;
    DevBuf host_in, host_out;  // staging for vkfx_execute_host
    // vkfx_plan_timing_start/stop: event pairs bound to FFT kernel dispatches
    struct {
        bool armed = false;
        std::vector<hipEvent_t> ev;  // begin/end of timed launch i at 2i, 2i+1
        std::vector<int> launch;     // index into launches of timed launch i
        size_t used = 0, cap = 0;
    } timing;
};

namespace {

// Bytes of one scalar of the caller-visible storage type.
size_t storage_scalar_bytes(int32_t precision) {
    return precision == VKFX_F64 ? 8 : precision == VKFX_F16_STORAGE_F32_COMPUTE ? 2 : 4;
}

// Dynamic LDS a plan may give one block: the device limit minus the kernels'
// static per-line bookkeeping (kMaxLinesPerBlock LineInfo records).
size_t lds_max_for(const vkfx_context* ctx) {
    size_t v = ctx->profile.shared_memory_bytes;
    if (!v) v = 65536;
    return v - 4096;
}

int upload(vkfx_plan* p, const std::string& key, const void* host, size_t bytes, const void** dev) {
    auto it = p->table_cache.find(key);
    if (it != p->table_cache.end()) {
        *dev = it->second;
        return VKFX_OK;
    }
    auto b = std::make_unique<DevBuf>();
    hipError_t e = hipMalloc(&b->p, bytes ? bytes : 16);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(table)");
    b->bytes = bytes;
    if (bytes) {
        e = hipMemcpy(b->p, host, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpy(table)");
    }
    *dev = b->p;
    p->table_cache[key] = b->p;
    p->tables.push_back(std::move(b));
    return VKFX_OK;
}

// Complex table of precision prec from long-double pairs.
std::vector<unsigned char> pack(const std::vector<ld>& re, const std::vector<ld>& im, int prec) {
    const size_t n = re.size();
    std::vector<unsigned char> bytes(n * (prec ? 16 : 8));
    if (prec) {
        double* d = (double*)bytes.data();
        for (size_t i = 0; i < n; ++i) {
            d[2 * i] = (double)re[i];
            d[2 * i + 1] = (double)im[i];
        }
    } else {
        float* f = (float*)bytes.data();
        for (size_t i = 0; i < n; ++i) {
            f[2 * i] = (float)re[i];
            f[2 * i + 1] = (float)im[i];
        }
    }
    return bytes;
}

// Stage twiddles exp(-2 pi i k/n), k < n.
int stage_table(vkfx_plan* p, size_t n, int prec, const void** dev) {
    std::string key = "tw:" + std::to_string(n) + ":" + std::to_string(prec);
    if (p->table_cache.count(key)) {
        *dev = p->table_cache[key];
        return VKFX_OK;
    }
    std::vector<ld> re(n), im(n);
    for (size_t k = 0; k < n; ++k) root((ld)k, (ld)n, re[k], im[k]);
    auto b = pack(re, im, prec);
    return upload(p, key, b.data(), b.size(), dev);
}

// Table of the register-exchange 1024-point kernel (fft_wave.hpp): the lane
// roots W1024^(l 2^j), j < 4, in [j][l] order (lane fastest), then W64^m,
// m < 4. Exponents are reduced in integers before the long-double
// evaluation.
int wave1024_table(vkfx_plan* p, int prec, const void** dev) {
    const std::string key = "wave1024:" + std::to_string(prec);
    if (p->table_cache.count(key)) {
        *dev = p->table_cache[key];
        return VKFX_OK;
    }
    std::vector<ld> re(kWave1024TableLen), im(kWave1024TableLen);
    for (int j = 0; j < 4; ++j)
        for (int l = 0; l < 64; ++l) root((ld)((l << j) % 1024), 1024.0L, re[j * 64 + l], im[j * 64 + l]);
    for (int m = 0; m < 4; ++m) root((ld)m, 64.0L, re[256 + m], im[256 + m]);
    auto b = pack(re, im, prec);
    return upload(p, key, b.data(), b.size(), dev);
}

// Per-stage twiddle blocks of a fixed shape (FT_STAGE_PR layout, kernels.hpp).
int stage_pr_table(vkfx_plan* p, const FixedKernel* f, int prec, const void** dev) {
    std::string key = "stage_pr:" + std::to_string(prec);
    for (int s = 0; s < f->nst; ++s) key += ":" + std::to_string(f->radix[s]);
    if (p->table_cache.count(key)) {
        *dev = p->table_cache[key];
        return VKFX_OK;
    }
    std::vector<ld> re, im;
    long long P = 1;
    for (int s = 0; s < f->nst; ++s) {
        const long long R = f->radix[s];
        if (P > 1)
            for (long long k = 0; k < P; ++k)
                for (long long i = 1; i < R; ++i) {
                    ld x, y;
                    root((ld)((k * i) % (P * R)), (ld)(P * R), x, y);
                    re.push_back(x);
                    im.push_back(y);
                }
        P *= R;
    }
    if (re.empty()) {
        re.push_back(1.0L);
        im.push_back(0.0L);
    }
    auto b = pack(re, im, prec);
    return upload(p, key, b.data(), b.size(), dev);
}

// Table block of a Rader stage for prime q (layout in kernels.hpp,
// rader_kernel_offset): slot and logq from the generator's powers, then the
// forward kernel exp(-2 pi i g^n / q) and its conjugate.
std::vector<unsigned char> rader_stage_block(size_t q, int prec) {
    const size_t L = q - 1, g = primitive_root(q);
    std::vector<size_t> pw(L);
    size_t r = 1;
    for (size_t e = 0; e < L; ++e) {
        pw[e] = r;
        r = (r * g) % q;
    }
    const size_t koff = (size_t)rader_kernel_offset((int)q), es = prec ? 16 : 8;
    std::vector<unsigned char> b(koff + 2 * L * es, 0);
    int* slot = (int*)b.data();
    int* logq = slot + q;
    slot[0] = (int)L;
    logq[0] = 0;
    for (size_t e = 0; e < L; ++e) {
        slot[pw[(L - e) % L]] = (int)e;  // g^-e
        logq[pw[e]] = (int)e;
    }
    std::vector<ld> re(2 * L), im(2 * L);
    for (size_t e = 0; e < L; ++e) {
        root((ld)pw[e], (ld)q, re[e], im[e]);
        re[L + e] = re[e];
        im[L + e] = -im[e];
    }
    auto k = pack(re, im, prec);
    std::memcpy(b.data() + koff, k.data(), k.size());
    return b;
}

// Table block of an FFT-mode Rader stage for prime q (layout in kernels.hpp,
// rader_fft_data_offset): the sub-radices of L = q - 1, slot, pw = g^m, the
// roots exp(-2 pi i k/L) and the spectra FFT_L(b)/L of the forward kernel
// b[n] = exp(-2 pi i g^n / q) and of its conjugate, in long double.
std::vector<unsigned char> rader_fft_stage_block(size_t q, int prec) {
    const size_t L = q - 1, g = primitive_root(q);
    std::vector<int> sub;
    rader_sub_schedule(L, sub);
    std::vector<size_t> pw(L);
    size_t r = 1;
    for (size_t e = 0; e < L; ++e) {
        pw[e] = r;
        r = (r * g) % q;
    }
    const size_t doff = (size_t)rader_fft_data_offset((int)q), es = prec ? 16 : 8;
    std::vector<unsigned char> b(doff + 3 * L * es, 0);
    int* hdr = (int*)b.data();
    hdr[0] = (int)sub.size();
    for (size_t i = 0; i < sub.size(); ++i) hdr[1 + i] = sub[i];
    int* slot = hdr + 16;
    int* pwi = slot + q;
    slot[0] = (int)L;
    for (size_t e = 0; e < L; ++e) {
        slot[pw[(L - e) % L]] = (int)e;  // g^-e
        pwi[e] = (int)pw[e];
    }
    std::vector<ld> re(3 * L), im(3 * L);
    for (size_t k = 0; k < L; ++k) root((ld)k, (ld)L, re[k], im[k]);
    for (int sgn = 0; sgn < 2; ++sgn) {
        std::vector<ld> br(L), bi(L);
        for (size_t n = 0; n < L; ++n) {
            root((ld)pw[n], (ld)q, br[n], bi[n]);
            if (sgn) bi[n] = -bi[n];
        }
        host_fft(br, bi);
        for (size_t k = 0; k < L; ++k) {
            re[(1 + sgn) * L + k] = br[k] / (ld)L;
            im[(1 + sgn) * L + k] = bi[k] / (ld)L;
        }
    }
    auto d = pack(re, im, prec);
    std::memcpy(b.data() + doff, d.data(), d.size());
    return b;
}

// Device table of every Rader stage of a radix list: rtab and per-stage byte
// offsets (distinct primes share a block; FFT-mode blocks carry
// kRaderFftStage in roff).
int rader_stage_tables(vkfx_plan* p, const std::vector<int>& radix, int prec, KArgs& a) {
    std::vector<unsigned char> all;
    std::map<int, size_t> at;
    std::string key = "rstages:" + std::to_string(prec);
    for (size_t s = 0; s < radix.size(); ++s) {
        if (radix[s] <= kMaxStockhamRadix) continue;
        const bool fft = rader_stage_fft((size_t)radix[s]);
        if (!at.count(radix[s])) {
            at[radix[s]] = all.size();
            auto b = fft ? rader_fft_stage_block((size_t)radix[s], prec) : rader_stage_block((size_t)radix[s], prec);
            all.insert(all.end(), b.begin(), b.end());
            all.resize((all.size() + 15) / 16 * 16, 0);
            key += std::string(fft ? ":f" : ":") + std::to_string(radix[s]);
        }
        if (at[radix[s]] >= (size_t)kRaderFftStage) return fail(VKFX_ERR_RESOURCE_LIMIT, "Rader stage tables too large");
        a.roff[s] = (int)at[radix[s]] | (fft ? kRaderFftStage : 0);
    }
    if (all.empty()) return VKFX_OK;
    return upload(p, key, all.data(), all.size(), &a.rtab);
}

// Two-level table for exp(-2 pi i k/L), k <= L: lo[j] = root(j), j < 2^s;
// hi[h] = root(h*2^s). The kernels form hi[k>>s]*lo[k&(2^s-1)].
int two_level(vkfx_plan* p, size_t L, int prec, const void** lo, const void** hi, int* shift) {
    int s = 0;
    while (((size_t)1 << (2 * s)) < L + 1) ++s;
    s = std::max(s, 1);
    const size_t nlo = (size_t)1 << s, nhi = (L >> s) + 2;
    std::string key = "tl:" + std::to_string(L) + ":" + std::to_string(prec);
    std::vector<ld> re(nlo), im(nlo);
    for (size_t j = 0; j < nlo; ++j) root((ld)j, (ld)L, re[j], im[j]);
    auto b = pack(re, im, prec);
    int rc = upload(p, key + ":lo", b.data(), b.size(), lo);
    if (rc) return rc;
    re.assign(nhi, 0);
    im.assign(nhi, 0);
    for (size_t h = 0; h < nhi; ++h) root((ld)(h << s), (ld)L, re[h], im[h]);
    b = pack(re, im, prec);
    rc = upload(p, key + ":hi", b.data(), b.size(), hi);
    *shift = s;
    return rc;
}

// Bluestein chirp c[n] = exp(sign * pi i n^2 / N) with n^2 reduced mod 2N
// (bluestein_ir.rs / lut.rs:295-304 define c[n] = exp(s*pi*i*n^2/N)).
std::vector<ld> chirp_angles(size_t N) {
    std::vector<ld> a(N);
    const unsigned __int128 twoN = 2 * (unsigned __int128)N;
    for (size_t n = 0; n < N; ++n) {
        unsigned __int128 sq = ((unsigned __int128)n * n) % twoN;
        a[n] = kPi * (ld)(unsigned long long)sq / (ld)N;
    }
    return a;
}

// In-place long-double FFT of smooth length (exp(-2 pi i jk/n)), recursive
// decimation in time; used once per plan for the Bluestein kernel spectrum.
void host_fft(std::vector<ld>& re, std::vector<ld>& im) {
    const size_t n = re.size();
    if (n <= 1) return;
    size_t r = 0;
    for (size_t q : {2, 3, 5, 7, 11, 13})
        if (n % q == 0) {
            r = q;
            break;
        }
    if (r == 0) {  // naive DFT for a prime remainder
        std::vector<ld> orr(n), oi(n);
        for (size_t k = 0; k < n; ++k) {
            ld sr = 0, si = 0;
            for (size_t j = 0; j < n; ++j) {
                ld c, s;
                root((ld)((j * k) % n), (ld)n, c, s);
                sr += re[j] * c - im[j] * s;
                si += re[j] * s + im[j] * c;
            }
            orr[k] = sr;
            oi[k] = si;
        }
        re.swap(orr);
        im.swap(oi);
        return;
    }
    const size_t m = n / r;
    std::vector<std::vector<ld>> sr(r, std::vector<ld>(m)), si(r, std::vector<ld>(m));
    for (size_t lane = 0; lane < r; ++lane) {
        for (size_t i = 0; i < m; ++i) {
            sr[lane][i] = re[lane + r * i];
            si[lane][i] = im[lane + r * i];
        }
        host_fft(sr[lane], si[lane]);
    }
    for (size_t k = 0; k < n; ++k) {
        ld ar = 0, ai = 0;
        for (size_t lane = 0; lane < r; ++lane) {
            ld c, s;
            root((ld)((lane * k) % n), (ld)n, c, s);
            const ld xr = sr[lane][k % m], xi = si[lane][k % m];
            ar += xr * c - xi * s;
            ai += xr * s + xi * c;
        }
        re[k] = ar;
        im[k] = ai;
    }
}

struct BlueTables {
    const void* chirp = nullptr;
    const void* spec = nullptr;
};

// chirp (length N, sign = transform direction) and the kernel spectrum
// FFT_M(b) / M with b[n] = conj(c[n]) mirrored (reference.rs:121-131). With
// n1 > 0 the spectrum is stored transposed for the four-step row pass.
int bluestein_tables(vkfx_plan* p, size_t N, size_t M, int sign, int prec, size_t n1, size_t n2, BlueTables* t) {
    std::vector<ld> ang = chirp_angles(N);
    std::vector<ld> cr(N), ci(N);
    for (size_t n = 0; n < N; ++n) {
        cr[n] = cosl(ang[n]);
        ci[n] = sign * sinl(ang[n]);
    }
    auto b = pack(cr, ci, prec);
    std::string key = "chirp:" + std::to_string(N) + ":" + std::to_string(sign) + ":" + std::to_string(prec);
    int rc = upload(p, key, b.data(), b.size(), &t->chirp);
    if (rc) return rc;
    std::vector<ld> br(M, 0), bi(M, 0);
    for (size_t n = 0; n < N; ++n) {
        br[n] = cr[n];
        bi[n] = -ci[n];
        if (n) {
            br[M - n] = cr[n];
            bi[M - n] = -ci[n];
        }
    }
    host_fft(br, bi);
    const ld inv = 1.0L / (ld)M;
    std::vector<ld> sr(M), si(M);
    for (size_t k = 0; k < M; ++k) {
        size_t dst = k;
        if (n1) {
            const size_t k1 = k % n1, k2 = k / n1;
            dst = k1 * n2 + k2;
        }
        sr[dst] = br[k] * inv;
        si[dst] = bi[k] * inv;
    }
    b = pack(sr, si, prec);
    key = "spec:" + std::to_string(N) + ":" + std::to_string(M) + ":" + std::to_string(sign) + ":" +
          std::to_string(prec) + ":" + std::to_string(n1);
    return upload(p, key, b.data(), b.size(), &t->spec);
}

size_t csize(int prec) { return prec ? 16 : 8; }
size_t rsize(int prec) { return prec ? 8 : 4; }

// Longest line planned as one upload (VKFX_MAX_UPLOAD, 0 = no cap beyond
// LDS): lets tests reach the multi-upload plans at small sizes.
size_t upload_cap() {
    const char* e = getenv("VKFX_MAX_UPLOAD");
    const long long v = e ? atoll(e) : 0;
    return v > 0 ? (size_t)v : SIZE_MAX;
}

// A length one kernel can hold (single upload), within the cap.
bool one_upload(size_t n, int prec, size_t lds_max) {
    return n <= upload_cap() && geometry(n, prec, 1, lds_max, lds_max).ok;
}

// Chooses M = N1 * N2 with both factors feasible single-upload lengths,
// minimising max(N1, N2) (N1 >= N2 on ties).
bool four_step_split(size_t M, int prec, size_t lds_max, size_t* n1, size_t* n2) {
    size_t best1 = 0, best2 = 0, bestmax = SIZE_MAX;
    for (size_t a = 2; a * a <= M; ++a) {
        if (M % a) continue;
        const size_t b = M / a;
        const size_t hi = std::max(a, b), lo = std::min(a, b);
        if (!one_upload(hi, prec, lds_max) || !one_upload(lo, prec, lds_max)) continue;
        if (hi < bestmax) {
            bestmax = hi;
            best1 = hi;
            best2 = lo;
        }
    }
    if (!best1) return false;
    *n1 = best1;
    *n2 = best2;
    return true;
}

// Three uploads for lengths with no two-upload split: M = N1 * (M1 * M2),
// N1 one upload (the first column pass over the whole line) and the rows of
// N2 = M1 * M2 a two-upload four-step of their own; minimises the largest
// of the three factors.
bool three_step_split(size_t M, int prec, size_t lds_max, size_t* n1, size_t* m1, size_t* m2) {
    size_t best = SIZE_MAX;
    for (size_t a = 2; a <= M / 4 && a <= (1u << 20); ++a) {
        if (M % a || !one_upload(a, prec, lds_max)) continue;
        size_t b1, b2;
        if (!four_step_split(M / a, prec, lds_max, &b1, &b2)) continue;
        const size_t hi = std::max(a, std::max(b1, b2));
        if (hi < best) {
            best = hi;
            *n1 = a, *m1 = b1, *m2 = b2;
        }
    }
    return best != SIZE_MAX;
}

PlannerTuning tuning_from(const vkfx_planner_tuning& t) {
    PlannerTuning p;
    p.min_rader_direct_prime = (size_t)t.min_rader_direct_prime;
    p.max_rader_direct_prime = (size_t)t.max_rader_direct_prime;
    p.min_rader_fft_prime = (size_t)t.min_rader_fft_prime;
    p.max_rader_fft_prime = (size_t)t.max_rader_fft_prime;
    p.allow_recursive_fft_rader = t.allow_recursive_fft_rader != 0;
    return p;
}

struct Ctx {
    vkfx_plan* p;
    int prec;
    size_t lds_max;
    PlannerTuning tuning;  // the plan's planner tuning (device default or FftConfig::with_tuning)
    size_t lds_budget = 80 * 1024;
    std::ostringstream js;
    bool first_pass = true;
    int cur_chunk = 0;
};

void note_pass(Ctx& c, const Launch& L) {
    if (!c.first_pass) c.js << ",";
    c.first_pass = false;
    if (L.r2r) {
        c.js << "{\"kernel\":\"" << L.label << "\",\"fft_len\":" << L.ra.L << ",\"len\":" << L.ra.n << "}";
        return;
    }
    if (L.copy) {
        c.js << "{\"kernel\":\"" << L.label << "\",\"bytes\":" << L.copy_bytes << "}";
        return;
    }
    if (L.conv) {
        c.js << "{\"kernel\":\"" << L.label << "\",\"tensor\":" << L.ca.T << ",\"coordinates\":" << L.ca.coords
             << ",\"systems\":" << L.ca.systems_out << ",\"planes\":" << L.ca.planes << "}";
        return;
    }
    if (L.boundary) {
        static const char* kType[] = {"f16", "f32", "f64"};
        bool zero = false, strided = false;
        for (int i = 0; i < L.ba.rank; ++i) zero |= L.ba.zero_right[i] > L.ba.zero_left[i];
        long long dense = 1;
        for (int i = L.ba.rank - 1; i >= 0; --i) {
            strided |= L.ba.src_stride[i] != dense || L.ba.dst_stride[i] != dense;
            dense *= L.ba.dims[i];
        }
        strided |= L.ba.src_batch != dense || L.ba.dst_batch != dense;
        c.js << "{\"kernel\":\"" << L.label << "\",\"from\":\"" << kType[L.ba.src_type] << "\",\"to\":\""
             << kType[L.ba.dst_type] << "\",\"elements\":" << L.ba.tensor_len * L.ba.batch
             << ",\"formatted\":" << (strided ? "true" : "false") << ",\"zero_padding\":" << (zero ? "true" : "false")
             << "}";
        return;
    }
    c.js << "{\"kernel\":\"" << L.label << "\",\"fft_len\":" << L.a.N << ",\"lines\":" << L.a.nlines
         << ",\"grid\":" << L.grid << ",\"block\":" << L.block << ",\"lines_per_block\":" << L.a.G
         << ",\"lds_bytes\":" << L.lds << ",\"fixed_shape\":" << (L.fixed ? "true" : "false")
         << ",\"twiddles\":\""
         << (!L.fixed                            ? "stage_roots"
             : L.fixed->table == FT_STAGE_PR     ? "per_stage_tables"
             : L.fixed->table == FT_WAVE1024     ? "lane_table"
                                                 : "stage_roots")
         << "\""
         << ",\"nontemporal\":[" << (L.fixed && L.fixed->nti ? "true" : "false") << ","
         << (L.fixed && L.fixed->nto ? "true" : "false") << "]"
         << ",\"runtime_variant\":{\"wide\":" << ((L.a.flags & KF_DYN_WIDE) ? "true" : "false")
         << ",\"hbm_direct\":" << ((L.a.flags & KF_DYN_DIRECT) ? "true" : "false")
         << ",\"direct_preprocess\":" << ((L.a.flags & KF_DYN_PRE) ? "true" : "false") << "}"
         << ",\"xcd_groups\":" << ((L.a.flags & KF_XCD_GROUPS) ? "true" : "false")
         << ",\"pair_loads\":" << ((L.a.flags & KF_PAIR_LOADS) ? "true" : "false")
         << ",\"radices\":[";
    for (int i = 0; i < L.a.nstages; ++i) c.js << (i ? "," : "") << L.a.radix[i];
    c.js << "]}";
}

// Launches whose blocks share HBM cache lines with their neighbours get their
// groups dealt to XCDs in contiguous ranges: the four-step passes that read
// or write the N/2+1-pitch real-transform spectra (unaligned 128-byte
// segments) and the Bluestein passes over pitch-N lines. Measured on C2: the
// C2R column pass reads 1.0x its bytes instead of 2.0x and the R2C row pass
// writes 1.0x instead of 1.19x. VKFX_XCD_GROUPS=0/1 forces it off/on for
// every launch of the plans built after it is set (tuning runs).
bool xcd_groups(KernelKind kind) {
    if (const char* e = getenv("VKFX_XCD_GROUPS")) return e[0] == '1';
    return kind == KK_FS_B_R2C || kind == KK_FS_A_C2R || kind == KK_FS_A_BLUE || kind == KK_BLUE_B ||
           kind == KK_FS_C_BLUE;
}

int add_launch(Ctx& c, KernelKind kind, int dir, const Geometry& g, KArgs a, long long nlines, unsigned grid,
               int in_sel, size_t in_off, int out_sel, size_t out_off, const char* label) {
    if (xcd_groups(kind)) a.flags |= KF_XCD_GROUPS;
    a.N = g.N;
    a.TT = g.TT;
    a.G = g.G;
    a.LS = g.LS;
    a.PS = g.PS;
    a.nstages = (int)g.radix.size();
    for (int i = 0; i < a.nstages; ++i) a.radix[i] = g.radix[i];
    a.nlines = nlines;
    if (!g.fixed && g.wide) a.flags |= KF_DYN_WIDE;
    if (g.rader) {
        // Rader stages run in the staged runtime-shape kernel only
        int rc = rader_stage_tables(c.p, g.radix, c.prec, a);
        if (rc) return rc;
        if (a.rtab) a.flags |= KF_RADER;
    }
    // runtime-shape C2C over contiguous lines: HBM-direct first and last stages
    if (!g.fixed && !g.rader && kind == KK_PLAIN && (a.flags & KF_IN_ROWMAJOR) && (a.flags & KF_OUT_ROWMAJOR) &&
        a.in_es == 1 && a.out_es == 1 && a.nstages >= 2 && a.radix[0] != 2 && a.radix[a.nstages - 1] != 2)
        a.flags |= KF_DYN_DIRECT;
    // runtime-shape even R2C: HBM-direct first stage, staged postprocess
    if (!g.fixed && !g.rader && kind == KK_R2C_HALF && (a.flags & KF_IN_ROWMAJOR) && a.in_es == 1 && a.nstages >= 1 &&
        a.radix[0] != 2)
        a.flags |= KF_DYN_DIRECT;
    // runtime-shape even C2R, HBM-direct last stage; KF_DYN_PRE: the first
    // stage also forms the preprocess from HBM when its loads span at least
    // 128 contiguous bytes per line (the preprocess twiddle of element
    // b + i N/R is w_b (w_(N/R))^i: one table lookup per butterfly). Measured
    // 8-30% over the staged preprocess in both precisions and every first
    // radix (f32 256, 2000, 6000, 12000, 200-9000; f64 2000-12000).
    if (!g.fixed && !g.rader && kind == KK_C2R_HALF && a.out_es == 1 && a.nstages >= 1 &&
        a.radix[a.nstages - 1] != 2) {
        a.flags |= KF_DYN_DIRECT;
        bool pre = a.in_es == 1 && a.nstages >= 2 && a.radix[0] != 2 &&
                   (long long)(g.N / a.radix[0]) * (c.prec ? 16 : 8) >= 128;
        // VKFX_C2R_PRE=0 keeps the staged preprocess (comparison runs)
        if (const char* e = getenv("VKFX_C2R_PRE")) pre = pre && e[0] != '0';
        if (pre) a.flags |= KF_DYN_PRE;
    }
    int rc = (g.fixed && g.fixed->table == FT_WAVE1024)   ? wave1024_table(c.p, c.prec, &a.tw)
             : (g.fixed && g.fixed->table == FT_STAGE_PR) ? stage_pr_table(c.p, g.fixed, c.prec, &a.tw)
                                                          : stage_table(c.p, g.N, c.prec, &a.tw);
    if (rc) return rc;
    rc = two_level(c.p, g.N, c.prec, &a.swlo, &a.swhi, &a.swshift);
    if (rc) return rc;
    Launch L{kind, dir, a, grid, (unsigned)(g.G * g.TT), g.lds, in_sel, out_sel, in_off, out_off, label, g.fixed,
             c.cur_chunk};
    c.p->launches.push_back(L);
    return VKFX_OK;
}

unsigned blocks_for(long long lines, int G) { return (unsigned)((lines + G - 1) / G); }

// Moves a KK_PLAIN launch onto the runtime-shape kernels (the only kernels
// that carry boundary work): a fixed shape is replaced by the runtime
// geometry of its length (rows: about 256 threads per block, columns: 8 / 16
// lines per block as for strided axes). Contiguous lines keep HBM-direct ends
// under the direct kernel's conditions; the others run staged.
Geometry edge_geometry(const Ctx& c, const KArgs& a) {
    const Geometry g0 = geometry((size_t)a.N, c.prec, 1, c.lds_max, c.lds_max);
    if (!g0.ok) return g0;
    const bool rows = (a.flags & KF_IN_ROWMAJOR) != 0;
    return geometry((size_t)a.N, c.prec, rows ? std::max(1, 256 / g0.TT) : (c.prec ? 8 : 16), c.lds_max,
                    c.lds_budget);
}

int to_edge_kernel(Ctx& c, Launch& L) {
    KArgs& a = L.a;
    if (L.fixed) {
        const Geometry g = edge_geometry(c, a);
        if (!g.ok)
            return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "no runtime geometry for length " + std::to_string(a.N));
        a.TT = g.TT;
        a.G = g.G;
        a.LS = g.LS;
        a.PS = g.PS;
        a.nstages = (int)g.radix.size();
        for (int i = 0; i < a.nstages; ++i) a.radix[i] = g.radix[i];
        a.flags &= ~KF_DYN_WIDE;
        if (g.wide) a.flags |= KF_DYN_WIDE;
        int rc = stage_table(c.p, g.N, c.prec, &a.tw);
        if (rc) return rc;
        L.grid = blocks_for(a.nlines, g.G);
        L.block = (unsigned)(g.G * g.TT);
        L.lds = g.lds;
        L.fixed = nullptr;
    }
    a.flags &= ~(KF_DYN_DIRECT | KF_DYN_PRE);
    const char* de = getenv("VKFX_EDGE_DIRECT");  // 0: staged ends only (comparison runs)
    const bool direct_on = !(de && de[0] == '0');
    if (direct_on && (a.flags & KF_IN_ROWMAJOR) && (a.flags & KF_OUT_ROWMAJOR) && a.in_es == 1 && a.out_es == 1 &&
        a.nstages >= 2 && a.radix[0] != 2 && a.radix[a.nstages - 1] != 2)
        a.flags |= KF_DYN_DIRECT;
    return VKFX_OK;
}

KArgs blank() {
    KArgs a;
    std::memset(&a, 0, sizeof(a));
    a.scale = 1.0;
    a.C = 1;
    a.C1 = 1;
    a.twdiv = 1;
    return a;
}

// Batch chunk of a 1-D multi-pass plan: `budget_mb` of workspace per chunk
// (measured: Bluestein three-pass C5b best at 96 MB; four-step plans at
// 64 MB: real 2^20 x 256 2.03 against 2.10 ms, C2C 2^18 x 512 1.10 against
// 1.28 ms at 96 MB).
size_t chunk_for(size_t batch, size_t per_batch_bytes, size_t budget_mb = 96) {
    size_t budget = budget_mb << 20;
    if (const char* e = getenv("VKFX_WORK_BUDGET_MB")) budget = (size_t)atoll(e) << 20;
    size_t c = std::max<size_t>(1, budget / std::max<size_t>(per_batch_bytes, 1));
    return std::min(c, batch);
}

// ---- Rader ---------------------------------------------------------------

struct RaderTables {
    const void* pin = nullptr;
    const void* pout = nullptr;
    const void* spec = nullptr;
    bool fft = false;
};

// Rader tables for a prime p with generator g (lut.rs:374-435): pin[s] =
// g^(-s) mod p (gather), pout[m] = g^m mod p (scatter) and the kernel
// b[n] = exp(dir 2 pi i g^n / p); in FFT mode the kernel is stored as
// FFT_{p-1}(b) / (p-1).
int rader_tables(vkfx_plan* p, size_t prime, int dir, int prec, bool fft, RaderTables* t) {
    const size_t L = prime - 1, g = primitive_root(prime);
    if (!g) return fail(VKFX_ERR_INVALID_ARGUMENT, "Rader length is not prime");
    std::vector<int> pw(L), pin(L), pout(L);
    size_t r = 1;
    for (size_t e = 0; e < L; ++e) {
        pw[e] = (int)r;
        r = (r * g) % prime;
    }
    for (size_t s = 0; s < L; ++s) {
        pin[s] = pw[(L - s) % L];
        pout[s] = pw[s];
    }
    std::string key = "rader:" + std::to_string(prime);
    int rc = upload(p, key + ":pin", pin.data(), L * sizeof(int), &t->pin);
    if (rc) return rc;
    rc = upload(p, key + ":pout", pout.data(), L * sizeof(int), &t->pout);
    if (rc) return rc;
    std::vector<ld> br(L), bi(L);
    for (size_t e = 0; e < L; ++e) {
        ld c, s;
        root((ld)pw[e], (ld)prime, c, s);  // exp(-2 pi i g^e / p)
        br[e] = c;
        bi[e] = dir < 0 ? s : -s;
    }
    if (fft) {
        host_fft(br, bi);
        const ld inv = 1.0L / (ld)L;
        for (size_t e = 0; e < L; ++e) {
            br[e] *= inv;
            bi[e] *= inv;
        }
    }
    auto b = pack(br, bi, prec);
    rc = upload(p, key + ":spec:" + std::to_string(dir) + ":" + std::to_string(prec) + (fft ? ":f" : ":d"), b.data(),
                b.size(), &t->spec);
    t->fft = fft;
    return rc;
}

bool is_prime(size_t n) { return n >= 2 && prime_factorization(n).size() == 1; }

// Adds one Rader launch over `lines` lines of a prime-length axis; false when
// this prime needs the recursive extension (executed through Bluestein).
int add_rader(Ctx& c, size_t prime, int dir, KArgs a, long long lines, int in_sel, size_t in_off, int out_sel,
              size_t out_off, bool* done) {
    *done = false;
    const size_t L = prime - 1;
    std::vector<int> rs;
    const bool smooth = radix_schedule(L, rs);
    bool fft = false;
    Geometry g;
    if (smooth) {
        g = geometry(L, c.prec, 1, c.lds_max, c.lds_max);
        fft = g.ok;
    }
    // a p-1 with prime factors above 13 (the recursive-Rader extension,
    // planner.rs:414-422): the length p-1 FFTs run those factors as Rader
    // stages themselves (direct multiplication inside the stage)
    bool nested = false;
    if (!fft && prime >= 89) {
        g = geometry_rader(L, c.prec, 1, c.lds_max, c.lds_max, true);
        if (!g.ok) return VKFX_OK;  // beyond one upload: the caller falls back
        fft = nested = true;
    }
    RaderTables t;
    int rc = rader_tables(c.p, prime, dir, c.prec, fft, &t);
    if (rc) return rc;
    a.pin = (const int*)t.pin, a.pout = (const int*)t.pout, a.spec = t.spec;
    if (fft) {
        g = nested ? geometry_rader(L, c.prec, std::max(1, 128 / g.TT), c.lds_max, c.lds_budget, true)
                   : geometry(L, c.prec, std::max(1, 128 / g.TT), c.lds_max, c.lds_budget);
        const int need = (int)L + (int)((L - 1) >> g.PS) + 2;  // x0 slot after the line
        if (g.LS < need) {
            g.LS = need | 1;
            g.lds = (size_t)g.G * g.LS * csize(c.prec) * (g.rader ? g.regions : 1);
        }
        c.js << "\"rader\":{\"prime\":" << prime << ",\"mode\":\"fft\",\"convolution_len\":" << L;
        if (nested) {
            c.js << ",\"nested_rader_primes\":[";
            bool first = true;
            for (int r : g.radix)
                if (r > kMaxStockhamRadix) {
                    c.js << (first ? "" : ",") << r;
                    first = false;
                }
            c.js << "],\"nested\":{";
            note_rader_stages(c, g);
            c.js << "}";
        }
        c.js << "},";
        rc = add_launch(c, KK_RADER_FFT, -1, g, a, lines, blocks_for(lines, g.G), in_sel, in_off, out_sel, out_off,
                        "rader_fft");
    } else {
        Geometry d;
        d.N = (int)L;
        d.TT = (int)L;
        d.G = std::max(1, std::min(kMaxLinesPerBlock, 256 / (int)L));
        d.LS = (int)L + 1;
        d.PS = 30;
        d.lds = (size_t)d.G * d.LS * csize(c.prec);
        d.ok = true;
        c.js << "\"rader\":{\"prime\":" << prime << ",\"mode\":\"direct\",\"convolution_len\":" << L << "},";
        rc = add_launch(c, KK_RADER_DIRECT, -1, d, a, lines, blocks_for(lines, d.G), in_sel, in_off, out_sel,
                        out_off, "rader_direct");
    }
    if (rc) return rc;
    *done = true;
    return VKFX_OK;
}

// Primes of the Rader stages of a radix list and, for FFT-mode stages, the
// sub-radices of their length p - 1 convolutions.
void note_rader_stages(Ctx& c, const Geometry& g) {
    c.js << "\"rader_primes\":[";
    bool first = true;
    for (int r : g.radix)
        if (r > kMaxStockhamRadix) {
            c.js << (first ? "" : ",") << r;
            first = false;
        }
    c.js << "],\"fft_convolution\":{";
    first = true;
    for (int r : g.radix)
        if (r > kMaxStockhamRadix && rader_stage_fft((size_t)r)) {
            std::vector<int> sub;
            rader_sub_schedule((size_t)r - 1, sub);
            c.js << (first ? "" : ",") << "\"" << r << "\":[";
            for (size_t i = 0; i < sub.size(); ++i) c.js << (i ? "," : "") << sub[i];
            c.js << "]";
            first = false;
        }
    c.js << "}";
}

void note_rader_mixed(Ctx& c, size_t n, const Geometry& g) {
    c.js << "\"rader_mixed\":{\"len\":" << n << ",";
    note_rader_stages(c, g);
    c.js << "},";
}

// ---- 1-D complex -----------------------------------------------------------

// Three-upload four-step of one 1-D axis (the reference's FourStepThreeUpload
// plans, recursive_ir.rs:756-893, kernel_ir.rs:1206-1236): a line of
// M = N1 * N2 is the matrix x[i1 * N2 + i2]; pass 1 transforms the N2 columns
// over i1 with the twiddle W_M^(i2 k1) (workspace, same layout); the rows of
// N2 = M1 * M2 are then a four-step of their own, in place on the workspace:
// pass 2 transforms each row's M2 columns over j1 (i2 = j2 + M2 j1) with
// W_N2^(j2 l1), pass 3 transforms the contiguous M2-runs over j2 and stores
// X[k1 + N1 (l1 + M1 l2)] (line (b, k1, l1): input b M + k1 N2 + l1 M2,
// output b M + k1 + l1 N1, element stride N1 M1).
int plan_c2c_three_upload(Ctx& c, size_t n, size_t batch, int dir, double sc) {
    vkfx_plan* p = c.p;
    const int prec = c.prec;
    const size_t cs = csize(prec);
    size_t n1, m1, m2;
    if (!three_step_split(n, prec, c.lds_max, &n1, &m1, &m2))
        return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "no three-upload four-step split for length " + std::to_string(n));
    const size_t n2 = m1 * m2;
    Geometry ga = kernel_geometry(KK_FS_A, prec, dir, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    Geometry gb = kernel_geometry(KK_FS_A, prec, dir, m1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    Geometry gc = kernel_geometry(KK_FS_B, prec, dir, m2, false, prec ? 8 : 16, c.lds_max, c.lds_budget);
    if (!ga.ok || !gb.ok || !gc.ok) return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "three-upload geometry");
    const size_t chunk = chunk_for(batch, n * cs, 64);
    p->work_bytes = std::max(p->work_bytes, chunk * n * cs);
    const void *alo, *ahi, *blo, *bhi;
    int ash, bsh;
    int rc = two_level(p, n, prec, &alo, &ahi, &ash);
    if (rc) return rc;
    rc = two_level(p, n2, prec, &blo, &bhi, &bsh);
    if (rc) return rc;
    c.js << "\"four_step\":{\"len\":" << n << ",\"uploads\":3,\"n1\":" << n1 << ",\"n2\":" << n2 << ",\"m1\":" << m1
         << ",\"m2\":" << m2 << ",\"chunk\":" << chunk << "},";
    for (size_t b0 = 0; b0 < batch; b0 += chunk) {
        c.cur_chunk = (int)(b0 / chunk);
        const size_t cb = std::min(chunk, batch - b0);
        KArgs a = blank();
        a.C = (long long)n2;
        a.in_es = (long long)n2, a.in_cs = 1, a.in_os = (long long)n;
        a.out_es = (long long)n2, a.out_cs = 1, a.out_os = (long long)n;
        a.tlo = alo, a.thi = ahi, a.tshift = ash;
        a.M = (long long)n, a.N1 = (long long)n1, a.N2 = (long long)n2;
        long long lines = (long long)(cb * n2);
        rc = add_launch(c, KK_FS_A, dir, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * n * cs, SEL_WORK, 0,
                        "three_upload_pass1");
        if (rc) return rc;
        KArgs b = blank();
        b.C = (long long)m2;
        b.in_es = (long long)m2, b.in_cs = 1, b.in_os = (long long)n2;
        b.out_es = (long long)m2, b.out_cs = 1, b.out_os = (long long)n2;
        b.tlo = blo, b.thi = bhi, b.tshift = bsh;
        b.M = (long long)n2, b.N1 = (long long)m1, b.N2 = (long long)m2;
        lines = (long long)(cb * n1 * m2);
        rc = add_launch(c, KK_FS_A, dir, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_WORK, 0,
                        "three_upload_pass2");
        if (rc) return rc;
        KArgs d = blank();
        d.C = (long long)m1;
        d.C1 = (long long)n1;
        d.in_es = 1, d.in_cs = (long long)m2, d.in_os1 = (long long)n2, d.in_os = (long long)n;
        d.out_es = (long long)(n1 * m1), d.out_cs = (long long)n1, d.out_os1 = 1, d.out_os = (long long)n;
        d.flags = KF_IN_ROWMAJOR;
        d.scale = sc;
        d.M = (long long)n2, d.N1 = (long long)m1, d.N2 = (long long)m2;
        lines = (long long)(cb * n1 * m1);
        rc = add_launch(c, KK_FS_B, dir, gc, d, lines, blocks_for(lines, gc.G), SEL_WORK, 0, SEL_OUT, b0 * n * cs,
                        "three_upload_pass3");
        if (rc) return rc;
    }
    return VKFX_OK;
}

int plan_c2c_1d(Ctx& c, size_t n, size_t batch, int dir, bool normalize, Algorithm alg, size_t conv_len) {
    vkfx_plan* p = c.p;
    const int prec = c.prec;
    const size_t cs = csize(prec);
    const double sc = (dir > 0 && normalize) ? 1.0 / (double)n : 1.0;
    if (n == 1) {
        // X[0] = x[0] (the scale of a normalized inverse is 1/1): one copy
        Launch L{};
        L.copy = true;
        L.copy_bytes = batch * cs;
        L.in_sel = SEL_IN, L.out_sel = SEL_OUT;
        L.label = "copy";
        p->launches.push_back(L);
        return VKFX_OK;
    }
    if (alg == Algorithm::Stockham) {
        Geometry g = geometry(n, prec, 256, c.lds_max, c.lds_budget);
        if (g.ok && n <= upload_cap()) {
            g = kernel_geometry(KK_PLAIN, prec, dir, n, false, std::max(1, 256 / g.TT), c.lds_max, c.lds_budget);
            // one launch by default (VKFX_SPLIT=k splits the batch for tuning runs)
            size_t parts = 1;
            if (const char* e = getenv("VKFX_SPLIT")) parts = std::max(1, std::min(atoi(e), 64));
            const size_t per = (batch + parts - 1) / parts;
            for (size_t b0 = 0; b0 < batch; b0 += per) {
                c.cur_chunk = (int)(b0 / per);
                const size_t cb = std::min(per, batch - b0);
                KArgs a = blank();
                a.in_es = a.out_es = 1;
                a.in_os = a.out_os = (long long)n;
                a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
                a.scale = sc;
                int rc = add_launch(c, KK_PLAIN, dir, g, a, (long long)cb, blocks_for(cb, g.G), SEL_IN, b0 * n * cs,
                                    SEL_OUT, b0 * n * cs, "stockham");
                if (rc) return rc;
            }
            return VKFX_OK;
        }
        size_t n1, n2;
        if (!four_step_split(n, prec, c.lds_max, &n1, &n2)) return plan_c2c_three_upload(c, n, batch, dir, sc);
        Geometry ga = kernel_geometry(KK_FS_A, prec, dir, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
        Geometry gb = kernel_geometry(KK_FS_B, prec, dir, n2, false, prec ? 8 : 16, c.lds_max, c.lds_budget);
        if (!ga.ok || !gb.ok) return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "four-step geometry");
        const size_t chunk = chunk_for(batch, n * cs, 64);
        p->work_bytes = std::max(p->work_bytes, chunk * n * cs);
        const void *tlo, *thi;
        int tsh;
        int rc = two_level(p, n, prec, &tlo, &thi, &tsh);
        if (rc) return rc;
        c.js << "\"four_step\":{\"len\":" << n << ",\"n1\":" << n1 << ",\"n2\":" << n2 << ",\"chunk\":" << chunk
             << "},";
        for (size_t b0 = 0; b0 < batch; b0 += chunk) {
        c.cur_chunk = (int)(b0 / chunk);
            const size_t cb = std::min(chunk, batch - b0);
            KArgs a = blank();
            a.C = (long long)n2;
            a.in_es = (long long)n2, a.in_cs = 1, a.in_os = (long long)n;
            a.out_es = (long long)n2, a.out_cs = 1, a.out_os = (long long)n;
            a.tlo = tlo, a.thi = thi, a.tshift = tsh;
            a.M = (long long)n, a.N1 = (long long)n1, a.N2 = (long long)n2;
            long long lines = (long long)(cb * n2);
            rc = add_launch(c, KK_FS_A, dir, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * n * cs, SEL_WORK, 0,
                            "four_step_columns");
            if (rc) return rc;
            KArgs b = blank();
            b.C = (long long)n1;
            b.in_es = 1, b.in_cs = (long long)n2, b.in_os = (long long)n;
            b.out_es = (long long)n1, b.out_cs = 1, b.out_os = (long long)n;
            b.flags = KF_IN_ROWMAJOR;
            b.scale = sc;
            b.M = (long long)n, b.N1 = (long long)n1, b.N2 = (long long)n2;
            lines = (long long)(cb * n1);
            rc = add_launch(c, KK_FS_B, dir, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_OUT, b0 * n * cs,
                            "four_step_rows");
            if (rc) return rc;
        }
        return VKFX_OK;
    }
    if (alg == Algorithm::Rader && is_prime(n) && n > 2) {
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = a.out_os = (long long)n;
        a.scale = sc;
        bool done = false;
        int rc = add_rader(c, n, dir, a, (long long)batch, SEL_IN, 0, SEL_OUT, 0, &done);
        if (rc || done) return rc;
    }
    if (alg == Algorithm::Rader && !is_prime(n)) {
        // composite length with Rader prime factors: one upload of Stockham
        // stages plus a Rader stage per such factor (mixed_ir.rs)
        Geometry g0 = geometry_rader(n, prec, 1, c.lds_max, c.lds_max);
        if (g0.ok) {
            Geometry g = geometry_rader(n, prec, std::max(1, 256 / g0.TT), c.lds_max, c.lds_budget);
            KArgs a = blank();
            a.in_es = a.out_es = 1;
            a.in_os = a.out_os = (long long)n;
            a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
            a.scale = sc;
            note_rader_mixed(c, n, g);
            return add_launch(c, KK_PLAIN, dir, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                              "rader_mixed");
        }
    }
    if (alg == Algorithm::Rader) c.js << "\"rader_fallback\":\"bluestein\",";
    // Bluestein (also Rader axes beyond one upload).
    const size_t M = conv_len ? conv_len : next_smooth_at_least(2 * n - 1, {2, 3, 5, 7});
    if (M < 2 * n - 1) return fail(VKFX_ERR_INVALID_ARGUMENT, "Bluestein convolution length below 2N-1");
    Geometry g = kernel_geometry(KK_BLUE_1, prec, -1, M, false, 1, c.lds_max, c.lds_max);
    if (g.ok) {
        BlueTables t;
        int rc = bluestein_tables(p, n, M, dir, prec, 0, 0, &t);
        if (rc) return rc;
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = a.out_os = (long long)n;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        a.scale = sc;
        a.chirp = t.chirp, a.spec = t.spec;
        a.nvalid = (long long)n, a.nout = (long long)n, a.M = (long long)M;
        c.js << "\"bluestein\":{\"len\":" << n << ",\"m\":" << M << ",\"uploads\":1},";
        return add_launch(c, KK_BLUE_1, -1, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                          "bluestein_single");
    }
    size_t n1, n2;
    if (!four_step_split(M, prec, c.lds_max, &n1, &n2))
        return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "no four-step split for Bluestein M " + std::to_string(M));
    Geometry ga = kernel_geometry(KK_FS_A_BLUE, prec, -1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    Geometry gc = kernel_geometry(KK_FS_C_BLUE, prec, 1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    Geometry gb = kernel_geometry(KK_BLUE_B, prec, -1, n2, false,
                                  std::max(1, 256 / std::max(1, geometry(n2, prec, 1, c.lds_max, c.lds_max).TT)),
                                  c.lds_max, c.lds_budget);
    if (!ga.ok || !gb.ok || !gc.ok) return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "Bluestein four-step geometry");
    BlueTables t;
    int rc = bluestein_tables(p, n, M, dir, prec, n1, n2, &t);
    if (rc) return rc;
    const void *tlo, *thi;
    int tsh;
    rc = two_level(p, M, prec, &tlo, &thi, &tsh);
    if (rc) return rc;
    const size_t chunk = chunk_for(batch, M * cs);
    p->work_bytes = std::max(p->work_bytes, chunk * M * cs);
    c.js << "\"bluestein\":{\"len\":" << n << ",\"m\":" << M << ",\"uploads\":2,\"n1\":" << n1 << ",\"n2\":" << n2
         << ",\"chunk\":" << chunk << "},";
    for (size_t b0 = 0; b0 < batch; b0 += chunk) {
        c.cur_chunk = (int)(b0 / chunk);
        const size_t cb = std::min(chunk, batch - b0);
        KArgs a = blank();
        a.C = (long long)n2;
        a.in_es = (long long)n2, a.in_cs = 1, a.in_os = (long long)n;
        a.out_es = (long long)n2, a.out_cs = 1, a.out_os = (long long)M;
        a.tlo = tlo, a.thi = thi, a.tshift = tsh;
        a.chirp = t.chirp;
        a.nvalid = (long long)n, a.M = (long long)M, a.N1 = (long long)n1, a.N2 = (long long)n2;
        long long lines = (long long)(cb * n2);
        rc = add_launch(c, KK_FS_A_BLUE, -1, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * n * cs, SEL_WORK, 0,
                        "bluestein_columns");
        if (rc) return rc;
        KArgs b = blank();
        b.C = (long long)n1;
        b.in_es = 1, b.in_cs = (long long)n2, b.in_os = (long long)M;
        b.out_es = 1, b.out_cs = (long long)n2, b.out_os = (long long)M;
        b.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        b.spec = t.spec;
        b.tlo = tlo, b.thi = thi, b.tshift = tsh;
        b.M = (long long)M, b.N1 = (long long)n1, b.N2 = (long long)n2;
        lines = (long long)(cb * n1);
        rc = add_launch(c, KK_BLUE_B, -1, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_WORK, 0,
                        "bluestein_rows");
        if (rc) return rc;
        KArgs d = blank();
        d.C = (long long)n2;
        d.in_es = (long long)n2, d.in_cs = 1, d.in_os = (long long)M;
        d.out_es = (long long)n2, d.out_cs = 1, d.out_os = (long long)n;
        d.chirp = t.chirp;
        d.scale = sc;
        d.nout = (long long)n, d.M = (long long)M, d.N1 = (long long)n1, d.N2 = (long long)n2;
        lines = (long long)(cb * n2);
        rc = add_launch(c, KK_FS_C_BLUE, 1, gc, d, lines, blocks_for(lines, gc.G), SEL_WORK, 0, SEL_OUT, b0 * n * cs,
                        "bluestein_columns_out");
        if (rc) return rc;
    }
    return VKFX_OK;
}

// ---- N-D complex -----------------------------------------------------------

// A strided axis whose single-upload kernel could hold only a few adjacent
// columns per block (narrow HBM segments, one block per CU) is split into two
// passes of length L1 x L2 = len over 32-column tiles: FFT over n1 with the
// W_len^(n2*k1) twiddle, then FFT over n2 with a natural-order store.
bool split_strided_axis(size_t len, int prec, size_t lds_budget, size_t* l1, size_t* l2) {
    const size_t cs = csize(prec);
    const size_t want_cols = prec ? 8 : 16;
    if (len * want_cols * cs <= lds_budget) return false;
    size_t best1 = 0, best2 = 0, bestmax = SIZE_MAX;
    for (size_t a = 2; a * a <= len; ++a) {
        if (len % a) continue;
        const size_t b = len / a, hi = std::max(a, b), lo = std::min(a, b);
        std::vector<int> rs;
        if (!radix_schedule(hi, rs) || !radix_schedule(lo, rs)) continue;
        if (hi < bestmax) {
            bestmax = hi;
            best1 = hi;
            best2 = lo;
        }
    }
    if (!best1 || best1 * want_cols * cs > lds_budget) return false;
    *l1 = best1;
    *l2 = best2;
    return true;
}

// Axes whose bit is set in `omit` are left untransformed (the real axis of an
// N-D real transform).
int plan_c2c_nd(Ctx& c, const vkfx_plan_desc& d, uint32_t omit) {
    const int prec = c.prec;
    const int dir = d.direction;
    const size_t cs = csize(prec);
    size_t per_batch = 1;
    for (uint32_t i = 0; i < d.rank; ++i) per_batch *= d.dims[i];
    // Batch chunks small enough for the Infinity Cache to keep a chunk's
    // intermediate between its axis passes.
    size_t chunk = d.batch;
    bool any_split = false;
    auto active = [&](uint32_t ax) { return d.dims[ax] > 1 && !(omit >> ax & 1u); };
    for (uint32_t ax = 0; ax + 1 < d.rank; ++ax) {
        size_t l1, l2;
        if (d.axis_algorithm[ax] == VKFX_ALG_STOCKHAM && active(ax) &&
            split_strided_axis(d.dims[ax], prec, c.lds_budget, &l1, &l2))
            any_split = true;
    }
    // batch chunks of 128 MB (C3: one 4096^2 f32 image in flight, 2.04 ms per
    // step against 2.40 ms with 256 MB); slab chunks of 256 MB (C4: 2.32 ms
    // against 2.40 ms at 128 MB and 2.47-2.54 ms at 384 MB and above)
    size_t chunk_budget = 128ull << 20, slab_budget = 256ull << 20;
    if (const char* e = getenv("VKFX_ND_CHUNK_MB")) chunk_budget = slab_budget = (size_t)atoll(e) << 20;
    chunk = std::max<size_t>(1, std::min(d.batch, chunk_budget / std::max<size_t>(per_batch * cs, 1)));
    if (any_split) c.p->work_bytes = std::max(c.p->work_bytes, chunk * per_batch * cs);
    // A volume larger than the chunk budget runs its axes 1.. (which stay
    // inside one slab of fixed index along axis 0) slab chunk by slab chunk,
    // then axis 0 over the whole volume.
    const size_t slab = per_batch / d.dims[0];
    int slab_axes = 0;
    for (uint32_t ax = 1; ax < d.rank; ++ax) slab_axes += active(ax);
    size_t slabs = 0;
    if (chunk == 1 && per_batch * cs > chunk_budget && active(0) && slab_axes >= 2)
        slabs = std::max<size_t>(1, slab_budget / (slab * cs));
    c.js << "\"nd\":{\"chunk\":" << chunk << ",\"slabs_per_chunk\":" << slabs << "},";

    // Launches of one axis over `total` elements at byte offset `off`.
    auto axis_pass = [&](int ax, size_t total, size_t off, int in_sel) -> int {
        const size_t len = d.dims[ax];
        size_t inner = 1;
        for (uint32_t j = ax + 1; j < d.rank; ++j) inner *= d.dims[j];
        const size_t outer = total / (len * inner);
        const double sc = (dir > 0 && d.normalize) ? 1.0 / (double)len : 1.0;
        const bool contiguous = inner == 1;
        const int alg = d.axis_algorithm[ax];
        int rc;
        size_t l1 = 0, l2 = 0;
        if (alg == VKFX_ALG_STOCKHAM && !contiguous && split_strided_axis(len, prec, c.lds_budget, &l1, &l2)) {
            // pass A: lines (o, n2, c), FFT over n1 at stride L2*inner, twiddle, store in place pattern
            Geometry ga = kernel_geometry(KK_FS_A, prec, dir, l1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
            Geometry gb = kernel_geometry(KK_PLAIN, prec, dir, l2, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
            if (!ga.ok || !gb.ok) return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "split axis geometry");
            const void *tlo, *thi;
            int tsh;
            rc = two_level(c.p, len, prec, &tlo, &thi, &tsh);
            if (rc) return rc;
            KArgs a = blank();
            a.C = (long long)(l2 * inner);
            a.in_cs = a.out_cs = 1;
            a.in_es = a.out_es = (long long)(l2 * inner);
            a.in_os = a.out_os = (long long)(len * inner);
            a.twdiv = (long long)inner;
            a.tlo = tlo, a.thi = thi, a.tshift = tsh;
            long long lines = (long long)(outer * l2 * inner);
            rc = add_launch(c, KK_FS_A, dir, ga, a, lines, blocks_for(lines, ga.G), in_sel, off, SEL_WORK, 0,
                            "split_axis_pass1");
            if (rc) return rc;
            // pass B: lines (o, k1, c), FFT over n2 at stride inner, store k1 + L1*k2
            KArgs b = blank();
            b.C = (long long)inner;
            b.C1 = (long long)l1;
            b.in_cs = b.out_cs = 1;
            b.in_es = (long long)inner, b.in_os1 = (long long)(l2 * inner), b.in_os = (long long)(len * inner);
            b.out_es = (long long)(l1 * inner), b.out_os1 = (long long)inner, b.out_os = (long long)(len * inner);
            b.scale = sc;
            lines = (long long)(outer * l1 * inner);
            rc = add_launch(c, KK_PLAIN, dir, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_OUT, off,
                            "split_axis_pass2");
            return rc;
        }
        KArgs a = blank();
        a.C = (long long)inner;
        a.in_es = a.out_es = (long long)inner;
        a.in_cs = a.out_cs = 1;
        a.in_os = a.out_os = (long long)(len * inner);
        a.flags = contiguous ? (KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR) : 0;
        a.scale = sc;
        const long long lines = (long long)(outer * inner);
        if (alg == VKFX_ALG_STOCKHAM) {
            Geometry g0 = geometry(len, prec, 1, c.lds_max, c.lds_max);
            if (!g0.ok)
                return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                            "N-D axis length " + std::to_string(len) + " exceeds one upload");
            const int want = contiguous ? std::max(1, 256 / g0.TT) : (prec ? 8 : 16);
            Geometry g = kernel_geometry(KK_PLAIN, prec, dir, len, !contiguous, want, c.lds_max, c.lds_budget);
            rc = add_launch(c, KK_PLAIN, dir, g, a, lines, blocks_for(lines, g.G), in_sel, off, SEL_OUT, off,
                            contiguous ? "stockham_rows" : "stockham_columns");
        } else {
            if (alg == VKFX_ALG_RADER && is_prime(len) && len > 2) {
                bool done = false;
                rc = add_rader(c, len, dir, a, lines, in_sel, off, SEL_OUT, off, &done);
                if (rc) return rc;
                if (done) return VKFX_OK;
            }
            if (alg == VKFX_ALG_RADER && !is_prime(len)) {
                Geometry g0 = geometry_rader(len, prec, 1, c.lds_max, c.lds_max);
                if (g0.ok) {
                    const int want = contiguous ? std::max(1, 256 / g0.TT) : (prec ? 8 : 16);
                    Geometry g = geometry_rader(len, prec, want, c.lds_max, c.lds_budget);
                    note_rader_mixed(c, len, g);
                    return add_launch(c, KK_PLAIN, dir, g, a, lines, blocks_for(lines, g.G), in_sel, off, SEL_OUT,
                                      off, "rader_mixed_axis");
                }
            }
            const size_t M = d.convolution_len[ax] ? d.convolution_len[ax]
                                                   : next_smooth_at_least(2 * len - 1, {2, 3, 5, 7});
            Geometry g = geometry(M, prec, contiguous ? 1 : 4, c.lds_max, c.lds_max);
            if (!g.ok)
                return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                            "N-D Bluestein axis needs more than one upload (M=" + std::to_string(M) + ")");
            BlueTables t;
            rc = bluestein_tables(c.p, len, M, dir, prec, 0, 0, &t);
            if (rc) return rc;
            a.chirp = t.chirp, a.spec = t.spec;
            a.nvalid = (long long)len, a.nout = (long long)len, a.M = (long long)M;
            rc = add_launch(c, KK_BLUE_1, -1, g, a, lines, blocks_for(lines, g.G), in_sel, off, SEL_OUT, off,
                            "bluestein_axis");
        }
        return rc;
    };
    auto copy_pass = [&](size_t total, size_t off) -> int {
        // every axis has length 1: the transform is a copy
        Geometry g = geometry(1, prec, 64, c.lds_max, c.lds_budget);
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = a.out_os = 1;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        return add_launch(c, KK_PLAIN, dir, g, a, (long long)total, blocks_for(total, g.G), SEL_IN, off, SEL_OUT, off,
                          "copy");
    };

    int next_chunk = 0;
    for (size_t b0 = 0; b0 < d.batch; b0 += chunk) {
        const size_t cb = std::min(chunk, d.batch - b0);
        const size_t off = b0 * per_batch * cs;
        const size_t total = cb * per_batch;
        if (slabs) {
            for (size_t s0 = 0; s0 < d.dims[0]; s0 += slabs) {
                c.cur_chunk = next_chunk++;
                const size_t ns = std::min(slabs, d.dims[0] - s0);
                bool sfirst = true;
                for (int ax = (int)d.rank - 1; ax >= 1; --ax) {
                    if (!active(ax)) continue;
                    int rc = axis_pass(ax, ns * slab, off + s0 * slab * cs, sfirst ? SEL_IN : SEL_OUT);
                    if (rc) return rc;
                    sfirst = false;
                }
            }
            c.cur_chunk = next_chunk++;
            int rc = axis_pass(0, total, off, SEL_OUT);
            if (rc) return rc;
            continue;
        }
        c.cur_chunk = next_chunk++;
        bool first = true;
        for (int ax = (int)d.rank - 1; ax >= 0; --ax) {
            if (!active(ax)) continue;
            int rc = axis_pass(ax, total, off, first ? SEL_IN : SEL_OUT);
            if (rc) return rc;
            first = false;
        }
        if (first) {
            int rc = copy_pass(total, off);
            if (rc) return rc;
        }
    }
    // One stream lane: slab chunks feed the axis-0 pass of their volume, and
    // a single chunk in flight keeps its intermediate in the Infinity Cache.
    c.p->serial = true;
    return VKFX_OK;
}

// ---- real ------------------------------------------------------------------

PlannerDevice planner_device(uint64_t shared) {
    PlannerDevice d;
    if (shared) {
        d.shared_memory_bytes = shared;
        size_t p2 = 1;
        while (p2 * 2 <= shared) p2 *= 2;
        d.shared_memory_pow2_bytes = p2;
    }
    return d;
}

// Real transform through a full-length C2C plan (the FullComplex shape,
// src/real_ir.rs:935-946, 1038-1053, 1124-1213), for lengths whose half-size
// or odd-length FFT has no Stockham geometry: R2C promotes x to complex,
// runs the N-point C2C (Stockham, Rader or Bluestein as the planner decides)
// and keeps N/2+1 bins; C2R expands the Hermitian bins to N, runs the
// inverse C2C and keeps the real part.
int plan_real_full_complex(Ctx& c, size_t n, size_t batch, bool r2c, bool normalize) {
    vkfx_plan* p = c.p;
    const size_t h = n / 2 + 1;
    const bool f64 = c.prec == 1;
    AxisDecision ad = plan_c2c_axis(n, batch, f64, false, c.tuning, planner_device(c.p->ctx->profile.shared_memory_bytes));
    p->full_bytes = batch * n * csize(c.prec);
    p->serial = true;
    c.js << "\"real\":{\"len\":" << n << ",\"algorithm\":\"full_complex\",\"c2c\":\""
         << (ad.algorithm == Algorithm::Stockham ? "stockham" : ad.algorithm == Algorithm::Rader ? "rader" : "bluestein")
         << "\"},";
    auto boundary = [&](int in_sel, int out_sel, long long len, long long src_batch, long long dst_batch, int ss, int ds,
                        int mode, const char* label) {
        Launch L{};
        L.boundary = true;
        L.label = label;
        L.in_sel = in_sel, L.out_sel = out_sel;
        BoundaryArgs& a = L.ba;
        a.rank = 1;
        a.dims[0] = len;
        a.src_stride[0] = a.dst_stride[0] = 1;
        a.tensor_len = len;
        a.batch = (long long)batch;
        a.src_batch = src_batch, a.dst_batch = dst_batch;
        a.src_scalars = ss, a.dst_scalars = ds;
        a.mode = mode;
        a.src_type = a.dst_type = c.prec ? 2 : 1;
        p->launches.push_back(L);
    };
    const long long N = (long long)n, H = (long long)h;
    if (r2c)
        boundary(SEL_IN, SEL_FULL, N, N, N, 1, 2, 0, "real_promote");
    else
        boundary(SEL_IN, SEL_FULL, N, H, N, 2, 2, 1, "hermitian_expand");
    const size_t first = p->launches.size();
    int rc = plan_c2c_1d(c, n, batch, r2c ? -1 : 1, !r2c && normalize, ad.algorithm,
                         ad.algorithm == Algorithm::Bluestein ? ad.convolution_len : 0);
    if (rc) return rc;
    for (size_t i = first; i < p->launches.size(); ++i) {
        Launch& L = p->launches[i];
        if (L.in_sel == SEL_IN || L.in_sel == SEL_OUT) L.in_sel = SEL_FULL;
        if (L.out_sel == SEL_IN || L.out_sel == SEL_OUT) L.out_sel = SEL_FULL;
    }
    if (r2c)
        boundary(SEL_FULL, SEL_OUT, H, N, H, 2, 2, 0, "truncate");
    else
        boundary(SEL_FULL, SEL_OUT, N, N, N, 2, 1, 0, "real_part");
    return VKFX_OK;
}

int plan_r2c(Ctx& c, size_t n, size_t batch);
int plan_c2r(Ctx& c, size_t n, size_t batch, bool normalize);

// N-D real transform (NdRealFftIr, src/nd_real_ir.rs:754-870): the real
// axis (the fastest) as a 1-D R2C/C2R over every row, the other axes as
// C2C over the compact [.., N/2+1] spectrum. R2C runs the real axis into
// the output and the complex axes in place there; C2R runs the complex axes
// from the (read-only) input into the SEL_AUX copy and the real axis from
// there into the output. The inverse normalizes every axis by its length.
int plan_real_nd(Ctx& c, const vkfx_plan_desc& d, bool r2c) {
    vkfx_plan* p = c.p;
    const uint32_t r = d.rank;
    const size_t n = d.dims[r - 1], h = n / 2 + 1;
    size_t outer = 1;
    for (uint32_t i = 0; i + 1 < r; ++i) outer *= d.dims[i];
    const size_t rows = d.batch * outer;
    vkfx_plan_desc e = d;
    e.transform = VKFX_C2C;
    e.dims[r - 1] = h;
    e.direction = r2c ? VKFX_FORWARD : VKFX_INVERSE;
    e.normalize = r2c ? 0 : d.normalize;
    const uint32_t omit = d.omit_dimension | 1u << (r - 1);
    int rc;
    if (r2c) {
        rc = plan_r2c(c, n, rows);
        if (rc) return rc;
        const size_t first = p->launches.size();
        rc = plan_c2c_nd(c, e, omit);
        if (rc) return rc;
        for (size_t i = first; i < p->launches.size(); ++i)
            if (p->launches[i].in_sel == SEL_IN) p->launches[i].in_sel = SEL_OUT;
    } else {
        p->aux_bytes = rows * h * csize(c.prec);
        const size_t first = p->launches.size();
        rc = plan_c2c_nd(c, e, omit);
        if (rc) return rc;
        for (size_t i = first; i < p->launches.size(); ++i) {
            Launch& L = p->launches[i];
            if (L.in_sel == SEL_OUT) L.in_sel = SEL_AUX;
            if (L.out_sel == SEL_OUT) L.out_sel = SEL_AUX;
        }
        const size_t mid = p->launches.size();
        rc = plan_c2r(c, n, rows, d.normalize != 0);
        if (rc) return rc;
        for (size_t i = mid; i < p->launches.size(); ++i)
            if (p->launches[i].in_sel == SEL_IN) p->launches[i].in_sel = SEL_AUX;
    }
    p->serial = true;
    c.js << "\"real_nd\":{\"real_axis\":" << n << ",\"rows\":" << rows << "},";
    return VKFX_OK;
}

// Real-application convolution (NdRealConvolutionIr, execute_nd_real_convolution_ir,
// src/convolution_ir.rs:3884-4251): the N-D R2C of the `coords` input
// tensors into SEL_CONV_A, the kernel-spectrum multiply over the compact
// spectra into SEL_CONV_B (K * coords systems), the normalized N-D C2R of
// those into the output.
int plan_convolution_real(Ctx& c, const vkfx_plan_desc& d, size_t coords, size_t kernels, const ConvArgs& ca,
                          const void* kernel) {
    vkfx_plan* p = c.p;
    const size_t T = (size_t)ca.T;
    p->conv_a_bytes = coords * T * csize(c.prec);
    p->conv_b_bytes = kernels * coords * T * csize(c.prec);
    vkfx_plan_desc e = d;
    e.perform_convolution = 0;
    e.batch = coords;
    e.transform = VKFX_R2C;
    e.direction = VKFX_FORWARD;
    e.normalize = 0;
    size_t first = p->launches.size();
    int rc = plan_real_nd(c, e, true);
    if (rc) return rc;
    for (size_t i = first; i < p->launches.size(); ++i) {
        Launch& L = p->launches[i];
        if (L.in_sel == SEL_OUT) L.in_sel = SEL_CONV_A;
        if (L.out_sel == SEL_OUT) L.out_sel = SEL_CONV_A;
    }
    Launch m{};
    m.conv = true;
    m.ca = ca;
    m.conv_kernel = kernel;
    m.label = "convolution_multiply";
    m.in_sel = SEL_CONV_A, m.out_sel = SEL_CONV_B;
    p->launches.push_back(m);
    vkfx_plan_desc f = e;
    f.batch = kernels * coords;
    f.transform = VKFX_C2R;
    f.direction = VKFX_INVERSE;
    f.normalize = 1;  // the inverse child is always normalized
    first = p->launches.size();
    rc = plan_real_nd(c, f, false);
    if (rc) return rc;
    for (size_t i = first; i < p->launches.size(); ++i)
        if (p->launches[i].in_sel == SEL_IN) p->launches[i].in_sel = SEL_CONV_B;
    c.js << "\"convolution\":{\"real\":true,\"coordinates\":" << coords << ",\"kernels\":" << kernels
         << ",\"matrix\":" << ca.matrix << ",\"symmetric\":" << (ca.symmetric ? "true" : "false")
         << ",\"conjugate_sequence\":" << (ca.conj_seq ? "true" : "false") << ",\"cross_power_normalize\":"
         << (ca.cross_norm ? "true" : "false") << "},";
    return VKFX_OK;
}

// Convolution (performConvolution, src/convolution_ir.rs:4252-4344): forward
// C2C of every [batch][coordinate] tensor into the SEL_FULL copy, the
// frequency-domain multiply into the output, normalized inverse C2C in place.
int plan_c2c_nd(Ctx& c, const vkfx_plan_desc& d, uint32_t omit = 0);
int plan_convolution(Ctx& c, const vkfx_plan_desc& d, size_t coords, size_t out_systems, const ConvArgs& ca,
                     const void* kernel) {
    vkfx_plan* p = c.p;
    size_t T = 1;
    for (uint32_t i = 0; i < d.rank; ++i) T *= d.dims[i];
    const size_t cs = csize(c.prec);
    p->full_bytes = d.batch * coords * T * cs;
    p->serial = true;
    auto transform = [&](size_t batch, int dir, bool normalize, int in_to, int out_to, uint32_t omit = 0) -> int {
        const size_t first = p->launches.size();
        int rc;
        if (d.rank == 1) {
            const int alg = d.axis_algorithm[0];
            Algorithm a = alg == VKFX_ALG_STOCKHAM ? Algorithm::Stockham
                          : alg == VKFX_ALG_RADER  ? Algorithm::Rader
                                                   : Algorithm::Bluestein;
            rc = plan_c2c_1d(c, d.dims[0], batch, dir, normalize, a, alg == VKFX_ALG_RADER ? 0 : d.convolution_len[0]);
        } else {
            vkfx_plan_desc e = d;
            e.batch = batch;
            e.direction = dir;
            e.normalize = normalize ? 1 : 0;
            rc = plan_c2c_nd(c, e, omit);
        }
        if (rc) return rc;
        for (size_t i = first; i < p->launches.size(); ++i) {
            Launch& L = p->launches[i];
            if (L.in_sel == SEL_IN) L.in_sel = in_to;
            else if (L.in_sel == SEL_OUT) L.in_sel = out_to;
            if (L.out_sel == SEL_OUT) L.out_sel = out_to;
        }
        return VKFX_OK;
    };
    c.js << "\"convolution\":{\"coordinates\":" << coords << ",\"kernels\":" << ca.kernel_count << ",\"matrix\":"
         << ca.matrix << ",\"symmetric\":" << (ca.symmetric ? "true" : "false") << ",\"independent\":"
         << (ca.independent ? "true" : "false") << ",\"conjugate_sequence\":" << (ca.conj_seq ? "true" : "false")
         << ",\"cross_power_normalize\":" << (ca.cross_norm ? "true" : "false");
    // one line per tensor, no coordinate mixing, one upload: the forward FFT,
    // the multiply and the normalized inverse FFT in one kernel, one HBM pass
    // (the reference fuses the multiply into its last forward / first inverse
    // upload, convolution_ir.rs:4252-4440)
    // The fan-out over kernels and coordinates without coordinate mixing
    // rides on the same kernel: output line (s, o) of system s (kernel s when
    // there are several kernels, whose input is system 0) reads input line
    // (s_in, o) and multiplies by plane kid * planes + (independent ? o : 0)
    // (conv.hip states the rule), one HBM read and write per output line.
    // A matrix convolution runs the runtime-shape kernel with whole systems
    // of M coordinate lines per block, whose product mixes the coordinates.
    if (d.rank == 1 && d.axis_algorithm[0] == VKFX_ALG_STOCKHAM) {
        const size_t n = d.dims[0];
        Geometry g0 = geometry(n, c.prec, 1, c.lds_max, c.lds_max);
        const int Mx = ca.matrix;
        Geometry g;
        if (g0.ok && Mx) {
            const int want = std::max(1, 256 / g0.TT) / Mx * Mx;
            g = geometry(n, c.prec, std::max(want, Mx), c.lds_max, c.lds_budget);
            if (g.ok && g.G % Mx) g = geometry(n, c.prec, Mx, c.lds_max, c.lds_max);
            if (g.G % Mx) g.ok = false;
        } else if (g0.ok) {
            g = kernel_geometry(KK_CONV_1, c.prec, -1, n, false, std::max(1, 256 / g0.TT), c.lds_max, c.lds_budget);
        }
        if (g0.ok && g.ok) {
            const bool fan = ca.kernel_count > 1;
            const long long M = (long long)coords, ln = (long long)n;
            KArgs a = blank();
            a.in_es = a.out_es = 1;
            a.C1 = M;
            a.in_os = fan ? 0 : M * ln, a.in_os1 = ln;
            a.out_os = M * ln, a.out_os1 = ln;
            a.spec_os = fan ? (long long)ca.planes * ln : 0;
            a.spec_os1 = ca.independent ? ln : 0;
            a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR | (ca.conj_seq ? KF_CONV_CONJ : 0) |
                      (ca.cross_norm ? KF_CONV_CROSS : 0) | (Mx ? KF_CONV_MATRIX : 0) |
                      (Mx && ca.symmetric ? KF_CONV_SYM : 0);
            a.scale = 1.0 / (double)n;
            a.spec = kernel;
            a.N2 = 1;
            p->full_bytes = 0;
            p->serial = false;
            c.js << ",\"fused\":true},";
            const long long lines = (long long)(out_systems * coords);
            return add_launch(c, KK_CONV_1, -1, g, a, lines, blocks_for(lines, g.G), SEL_IN, 0, SEL_OUT, 0,
                              "convolution_fused");
        }
        // two uploads (N = N1 * N2), scalar convolutions only (one
        // coordinate, one kernel): the forward column pass (FFT over n1,
        // W_N^(n2*k1)) into the workspace, one row pass (FFT over n2, multiply,
        // inverse FFT, W_N^(-k1*m2)) in place, and the inverse column pass
        // into the output, whose twiddle row c / N2 is 0 (no twiddle): three
        // HBM passes per chunk instead of five
        size_t n1 = 0, n2 = 0;
        const bool scalar = !Mx && ca.kernel_count <= 1 && coords == 1;
        if (!g0.ok && scalar && four_step_split(n, c.prec, c.lds_max, &n1, &n2)) {
            const int prec = c.prec;
            Geometry ga = kernel_geometry(KK_FS_A, prec, -1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
            Geometry gc = kernel_geometry(KK_FS_A, prec, 1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
            Geometry gb = kernel_geometry(KK_CONV_B, prec, -1, n2, false,
                                          std::max(1, 256 / std::max(1, geometry(n2, prec, 1, c.lds_max, c.lds_max).TT)),
                                          c.lds_max, c.lds_budget);
            // only with a fixed-shape row pass: on the runtime-shape kernel
            // the three passes are no faster than the five of fixed shapes
            // (10^5 = 400 x 250 f32 before its row shape: 0.32 ms fused
            // against 0.25 ms for the forward and inverse transforms alone)
            if (ga.ok && gb.ok && gc.ok && gb.fixed) {
                const void *tlo, *thi;
                int tsh;
                int rc = two_level(p, n, prec, &tlo, &thi, &tsh);
                if (rc) return rc;
                const size_t chunk = chunk_for(d.batch, n * cs, 64);
                p->work_bytes = std::max(p->work_bytes, chunk * n * cs);
                p->full_bytes = 0;
                p->serial = false;
                c.js << ",\"fused\":true,\"n1\":" << n1 << ",\"n2\":" << n2 << ",\"chunk\":" << chunk << "},";
                for (size_t b0 = 0; b0 < d.batch; b0 += chunk) {
                    c.cur_chunk = (int)(b0 / chunk);
                    const size_t cb = std::min(chunk, d.batch - b0);
                    KArgs a = blank();
                    a.C = (long long)n2;
                    a.in_es = a.out_es = (long long)n2;
                    a.in_cs = a.out_cs = 1;
                    a.in_os = a.out_os = (long long)n;
                    a.tlo = tlo, a.thi = thi, a.tshift = tsh;
                    a.M = (long long)n, a.N1 = (long long)n1, a.N2 = (long long)n2;
                    long long lines = (long long)(cb * n2);
                    rc = add_launch(c, KK_FS_A, -1, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * n * cs,
                                    SEL_WORK, 0, "convolution_columns");
                    if (rc) return rc;
                    KArgs b = blank();
                    b.C = (long long)n1;
                    b.in_es = b.out_es = 1;
                    b.in_cs = b.out_cs = (long long)n2;
                    b.in_os = b.out_os = (long long)n;
                    b.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR | (ca.conj_seq ? KF_CONV_CONJ : 0) |
                              (ca.cross_norm ? KF_CONV_CROSS : 0);
                    b.spec = kernel;
                    b.scale = 1.0 / (double)n;
                    b.tlo = tlo, b.thi = thi, b.tshift = tsh;
                    b.M = (long long)n, b.N1 = (long long)n1, b.N2 = (long long)n2;
                    lines = (long long)(cb * n1);
                    rc = add_launch(c, KK_CONV_B, -1, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_WORK,
                                    0, "convolution_rows");
                    if (rc) return rc;
                    KArgs e = a;
                    e.twdiv = (long long)n2;
                    lines = (long long)(cb * n2);
                    rc = add_launch(c, KK_FS_A, 1, gc, e, lines, blocks_for(lines, gc.G), SEL_WORK, 0, SEL_OUT,
                                    b0 * n * cs, "convolution_columns_out");
                    if (rc) return rc;
                }
                return VKFX_OK;
            }
        }
    }
    // N-D scalar convolution over Stockham axes: the forward FFT of every
    // axis but axis 0 into the workspace, one kernel per axis-0 line (forward
    // FFT, multiply, inverse FFT normalized by 1/N0) into the output, and the
    // normalized inverse of the other axes in place, 2D - 1 passes over the
    // data instead of 2D + 1 (the multiply folded into the last forward /
    // first inverse axis, as the reference folds it into its uploads), or
    // 2D - 1 instead of 2D + 3 where the plain plan splits axis 0 into two
    // passes per direction. Taken with a fixed-shape column kernel for N0, or
    // where axis 0 would be split (its runtime-shape column kernel then still
    // wins); an axis 0 of one pass without a fixed-shape kernel keeps the
    // separate multiply, since its fixed-shape FFT column passes beat the
    // runtime-shape fused kernel ([128, 128, 128] x 4 f32 before the fixed
    // column kernel: 192 us unfused, 201 us fused).
    size_t sl1 = 0, sl2 = 0;
    bool nd_fused = d.rank >= 2 && !ca.matrix && ca.kernel_count <= 1 && coords == 1 && d.dims[0] > 1;
    for (uint32_t i = 0; nd_fused && i < d.rank; ++i) nd_fused = d.axis_algorithm[i] == VKFX_ALG_STOCKHAM;
    if (nd_fused) {
        const size_t n0 = d.dims[0], rest = T / n0;
        const bool split = split_strided_axis(n0, c.prec, c.lds_budget, &sl1, &sl2);
        Geometry g = kernel_geometry(KK_CONV_1, c.prec, -1, n0, true, c.prec ? 8 : 16, c.lds_max, c.lds_budget);
        // strided columns: at least 8 adjacent columns per block, so each
        // HBM access moves 64 bytes or more
        if (g.ok && g.G >= 8 && (g.fixed || split)) {
            c.js << ",\"fused\":true,\"fused_axis\":0},";
            int rc = transform(d.batch, -1, false, SEL_IN, SEL_FULL, 1u);
            if (rc) return rc;
            KArgs a = blank();
            a.C = (long long)rest;
            a.in_cs = a.out_cs = 1;
            a.in_es = a.out_es = (long long)rest;
            a.in_os = a.out_os = (long long)T;
            a.N2 = (long long)rest;
            a.flags = (ca.conj_seq ? KF_CONV_CONJ : 0) | (ca.cross_norm ? KF_CONV_CROSS : 0);
            a.scale = 1.0 / (double)n0;
            a.spec = kernel;
            const long long lines = (long long)(d.batch * rest);
            rc = add_launch(c, KK_CONV_1, -1, g, a, lines, blocks_for(lines, g.G), SEL_FULL, 0, SEL_OUT, 0,
                            "convolution_fused_axis0");
            if (rc) return rc;
            return transform(d.batch, 1, true, SEL_OUT, SEL_OUT, 1u);
        }
    }
    c.js << ",\"fused\":false},";
    int rc = transform(d.batch * coords, -1, false, SEL_IN, SEL_FULL);
    if (rc) return rc;
    Launch m{};
    m.conv = true;
    m.ca = ca;
    m.conv_kernel = kernel;
    m.label = "convolution_multiply";
    m.in_sel = SEL_FULL, m.out_sel = SEL_OUT;
    p->launches.push_back(m);
    // the inverse child is always normalized (convolution_ir.rs:4449-4451)
    rc = transform(out_systems * coords, 1, true, SEL_OUT, SEL_OUT);
    if (rc) return rc;
    return VKFX_OK;
}

// DCT / DST of length n as one complex FFT of length L between a pre and a
// post pass (r2r.hip, which states the algebra of each reduction):
//   DCT-I   L = 2(n-1): even extension (w = 1 at the ends, 2 inside), Re
//   DST-I   L = 2(n+1): odd extension, -2 Im
//   DCT-II  L = n:      Makhoul reordering, 2 Re(e^{-i pi k/2n} V_k)
//   DCT-III L = n:      V_j = e^{i pi j/2n} (x_j - i x_{n-j}), inverse FFT, un-reorder
//   DCT-IV  L = n/2 (even n): z_j = (x_2j + i x_{n-1-2j}) e^{-i pi (4j+1)/4n},
//           outputs 2 Re / -2 Im of e^{-i pi j/n} Z_j; odd n: L = 2n extension
//   DST-II/III/IV: the DCT forms with the input sign or reversal and the
//           output reversal or sign (DST-II_k = DCT-II((-1)^j x)_{n-1-k},
//           DST-III_k = (-1)^k DCT-III(reversed x)_k, same for type IV)
// The inverse direction runs the type's inverse partner (II <-> III,
// r2r_ir.rs:2308-2316), scaled when normalized (inverse_pair_scale,
// r2r_ir.rs:2318-2346).
int plan_r2r(Ctx& c, size_t n, size_t batch, int kind, int dir, bool normalize, size_t inner = 1,
             int in_sel = SEL_IN) {
    vkfx_plan* p = c.p;
    // kind: 0..3 DCT-I..IV, 4..7 DST-I..IV
    int eff = kind;
    if (dir > 0) {
        if (kind == 1) eff = 2;
        else if (kind == 2) eff = 1;
        else if (kind == 5) eff = 6;
        else if (kind == 6) eff = 5;
    }
    double scale = 1.0;
    if (dir > 0 && normalize) {
        const double den = kind == 0 ? 2.0 * (double)(n - 1) : kind == 4 ? 2.0 * (double)(n + 1) : 2.0 * (double)n;
        scale = 1.0 / den;
    }
    R2rArgs a;
    a.n = (long long)n;
    a.batch = (long long)batch;
    a.inner = (long long)inner;
    // FFT lengths of the reference's reductions (r2r_ir.rs:76-110): 2(N-1)
    // for DCT-I, 2(N+1) for DST-I, N for types II and III, N/2 for even type
    // IV (2N for odd type IV)
    int fft_dir = -1;
    switch (eff) {
        case 0: a.L = 2 * (a.n - 1); a.wmode = 1; break;
        case 1: a.L = a.n; a.op = R2R_REORDER; break;
        case 2: a.L = a.n; a.op = R2R_SPECTRUM; fft_dir = 1; break;
        case 3:
            if (a.n % 2 == 0) {
                a.L = a.n / 2; a.op = R2R_HALF;
            } else {
                a.L = 2 * a.n; a.ph = 1; a.pq = 1; a.q2 = 1; a.s = 2.0;
            }
            break;
        case 4: a.L = 2 * (a.n + 1); a.off = 1; a.r = 1; a.im = 1; a.s = 2.0; break;
        case 5: a.L = a.n; a.op = R2R_REORDER; a.flip = 1; break;
        case 6: a.L = a.n; a.op = R2R_SPECTRUM; a.flip = 1; fft_dir = 1; break;
        default:
            if (a.n % 2 == 0) {
                a.L = a.n / 2; a.op = R2R_HALF; a.flip = 1;
            } else {
                a.L = 2 * a.n; a.ph = 1; a.pq = 1; a.q2 = 1; a.im = 1; a.s = 2.0;
            }
            break;
    }
    a.s *= scale;
    const size_t L = (size_t)a.L;
    const bool f64 = c.prec == 1;
    AxisDecision ad = plan_c2c_axis(L, batch, f64, false, c.tuning,
                                    planner_device(p->ctx->profile.shared_memory_bytes));
    p->full_bytes = std::max(p->full_bytes, batch * L * csize(c.prec));
    p->serial = true;
    static const char* kNames[] = {"dct1", "dct2", "dct3", "dct4", "dst1", "dst2", "dst3", "dst4"};
    c.js << "\"r2r\":{\"type\":\"" << kNames[kind] << "\",\"runs\":\"" << kNames[eff] << "\",\"fft_len\":" << L
         << ",\"c2c\":\""
         << (ad.algorithm == Algorithm::Stockham ? "stockham" : ad.algorithm == Algorithm::Rader ? "rader" : "bluestein")
         << "\"},";
    Launch pre{};
    pre.r2r = 1;
    pre.ra = a;
    pre.label = "r2r_pre";
    pre.in_sel = in_sel, pre.out_sel = SEL_FULL;
    p->launches.push_back(pre);
    const size_t first = p->launches.size();
    int rc = plan_c2c_1d(c, L, batch, fft_dir, false, ad.algorithm,
                         ad.algorithm == Algorithm::Bluestein ? ad.convolution_len : 0);
    if (rc) return rc;
    for (size_t i = first; i < p->launches.size(); ++i) {
        Launch& L2 = p->launches[i];
        if (L2.in_sel == SEL_IN || L2.in_sel == SEL_OUT) L2.in_sel = SEL_FULL;
        if (L2.out_sel == SEL_IN || L2.out_sel == SEL_OUT) L2.out_sel = SEL_FULL;
    }
    Launch post = pre;
    post.r2r = 2;
    post.label = "r2r_post";
    post.in_sel = SEL_FULL, post.out_sel = SEL_OUT;
    p->launches.push_back(post);
    return VKFX_OK;
}

// N-D DCT / DST (NdR2rIr, src/r2r_ir.rs:1769-1990, execute_nd_r2r_ir
// :2216-2300): the same type along every active axis, fastest first; each
// axis is the 1-D pre pass / C2C / post pass over its lines, read and written
// in place with the axis stride. Axes of length 1 and omitted axes are left
// as they are; the inverse normalizes each axis by its own factor.
int plan_r2r_nd(Ctx& c, const vkfx_plan_desc& d) {
    vkfx_plan* p = c.p;
    size_t per = 1;
    for (uint32_t i = 0; i < d.rank; ++i) per *= d.dims[i];
    bool first = true;
    for (int ax = (int)d.rank - 1; ax >= 0; --ax) {
        const size_t n = d.dims[ax];
        if (n == 1 || (d.omit_dimension >> ax & 1u)) continue;
        if (d.transform == VKFX_DCT_I && n < 2)
            return fail(VKFX_ERR_INVALID_ARGUMENT, "InvalidTransformLength: DCT-I axis of length 1");
        size_t inner = 1;
        for (uint32_t j = ax + 1; j < d.rank; ++j) inner *= d.dims[j];
        const int rc = plan_r2r(c, n, d.batch * (per / n), d.transform - VKFX_DCT_I, d.direction, d.normalize != 0,
                                inner, first ? SEL_IN : SEL_OUT);
        if (rc) return rc;
        first = false;
    }
    if (first) {
        // no active axis: the transform is a copy
        Launch L{};
        L.boundary = true;
        L.label = "copy";
        L.in_sel = SEL_IN, L.out_sel = SEL_OUT;
        BoundaryArgs& a = L.ba;
        a.rank = 1;
        a.dims[0] = (long long)per;
        a.src_stride[0] = a.dst_stride[0] = 1;
        a.tensor_len = (long long)per;
        a.batch = (long long)d.batch;
        a.src_batch = a.dst_batch = (long long)per;
        a.src_scalars = a.dst_scalars = 1;
        a.src_type = a.dst_type = c.prec ? 2 : 1;
        p->launches.push_back(L);
    }
    p->serial = true;
    return VKFX_OK;
}

int plan_r2c(Ctx& c, size_t n, size_t batch) {
    vkfx_plan* p = c.p;
    const int prec = c.prec;
    const size_t cs = csize(prec), rs = rsize(prec);
    const size_t h = n / 2 + 1;
    if (n % 2) {
        Geometry g0 = geometry(n, prec, 1, c.lds_max, c.lds_max);
        if (!g0.ok) return plan_real_full_complex(c, n, batch, true, false);
        Geometry g = geometry(n, prec, std::max(1, 256 / g0.TT), c.lds_max, c.lds_budget);
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = (long long)n, a.out_os = (long long)h;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        a.nout = (long long)h;
        return add_launch(c, KK_R2C_FULL, -1, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                          "r2c_full");
    }
    const size_t M = n / 2;
    const void *rlo, *rhi;
    int rsh;
    int rc = two_level(p, n, prec, &rlo, &rhi, &rsh);
    if (rc) return rc;
    // one upload when the half length has a runtime geometry or a fixed shape
    // (a fixed shape without padding can hold a line the runtime one cannot)
    Geometry g0 = geometry(M, prec, 1, c.lds_max, c.lds_max);
    const Geometry gh = kernel_geometry(KK_R2C_HALF, prec, -1, M, false, g0.ok ? std::max(1, 256 / g0.TT) : 1,
                                        c.lds_max, c.lds_budget);
    if (g0.ok || (gh.ok && gh.fixed)) {
        const Geometry& g = gh;
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = (long long)M, a.out_os = (long long)h;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        a.rlo = rlo, a.rhi = rhi, a.rshift = rsh;
        c.js << "\"real\":{\"len\":" << n << ",\"half\":" << M << ",\"uploads\":1},";
        return add_launch(c, KK_R2C_HALF, -1, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                          "r2c_even_half");
    }
    size_t n1, n2;
    if (!four_step_split(M, prec, c.lds_max, &n1, &n2)) return plan_real_full_complex(c, n, batch, true, false);
    // the shorter factor goes to the column pass when both passes have fixed
    // shapes that way round: more columns per block, wider row segments
    // (M = 2^19: 32 columns of 512, 256-byte segments, instead of 16 of 1024)
    if (n1 != n2 && kernel_geometry(KK_FS_A, prec, -1, n2, true, 1, c.lds_max, c.lds_budget).fixed &&
        kernel_geometry(KK_FS_B_R2C, prec, -1, n1, false, 1, c.lds_max, c.lds_max).fixed)
        std::swap(n1, n2);
    // the mirror-row pass needs N1 divisible by 2H; H lines + H mirrors per block
    if (n1 % 2 != 0 && n2 % 2 == 0) std::swap(n1, n2);
    // both factors odd (M odd, e.g. 9009): the full-length complex plan
    if (n1 % 2 != 0) return plan_real_full_complex(c, n, batch, true, false);
    Geometry gb1 = geometry(n2, prec, 1, c.lds_max, c.lds_max);
    int H = prec ? 4 : 8;
    while (H > 1 && (n1 % (2 * H) != 0)) H /= 2;
    Geometry gb = kernel_geometry(KK_FS_B_R2C, prec, -1, n2, false, 2 * H, c.lds_max, c.lds_max);
    if (gb.fixed && n1 % gb.G == 0) H = gb.G / 2;
    if (!gb1.ok || gb.G != 2 * H) return plan_real_full_complex(c, n, batch, true, false);
    Geometry ga = kernel_geometry(KK_FS_A, prec, -1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    const void *tlo, *thi;
    int tsh;
    rc = two_level(p, M, prec, &tlo, &thi, &tsh);
    if (rc) return rc;
    const size_t chunk = chunk_for(batch, M * cs, 64);
    p->work_bytes = std::max(p->work_bytes, chunk * M * cs);
    c.js << "\"real\":{\"len\":" << n << ",\"half\":" << M << ",\"uploads\":2,\"n1\":" << n1 << ",\"n2\":" << n2
         << ",\"chunk\":" << chunk << "},";
    for (size_t b0 = 0; b0 < batch; b0 += chunk) {
        c.cur_chunk = (int)(b0 / chunk);
        const size_t cb = std::min(chunk, batch - b0);
        KArgs a = blank();
        a.C = (long long)n2;
        a.in_es = (long long)n2, a.in_cs = 1, a.in_os = (long long)M;
        a.out_es = (long long)n2, a.out_cs = 1, a.out_os = (long long)M;
        a.tlo = tlo, a.thi = thi, a.tshift = tsh;
        a.M = (long long)M, a.N1 = (long long)n1, a.N2 = (long long)n2;
        long long lines = (long long)(cb * n2);
        rc = add_launch(c, KK_FS_A, -1, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * n * rs, SEL_WORK, 0,
                        "r2c_columns");
        if (rc) return rc;
        KArgs b = blank();
        b.C = (long long)n1;
        b.in_es = 1, b.in_cs = (long long)n2, b.in_os = (long long)M;
        b.out_os = (long long)h;
        b.flags = KF_IN_ROWMAJOR;
        b.rlo = rlo, b.rhi = rhi, b.rshift = rsh;
        b.M = (long long)M, b.N1 = (long long)n1, b.N2 = (long long)n2;
        lines = (long long)(cb * n1);
        const unsigned grid = (unsigned)(cb * (n1 / (2 * H)));
        rc = add_launch(c, KK_FS_B_R2C, -1, gb, b, lines, grid, SEL_WORK, 0, SEL_OUT, b0 * h * cs, "r2c_rows_post");
        if (rc) return rc;
    }
    return VKFX_OK;
}

int plan_c2r(Ctx& c, size_t n, size_t batch, bool normalize) {
    vkfx_plan* p = c.p;
    const int prec = c.prec;
    const size_t cs = csize(prec), rs = rsize(prec);
    const size_t h = n / 2 + 1;
    const double sc = normalize ? 1.0 / (double)n : 1.0;
    if (n % 2) {
        Geometry g0 = geometry(n, prec, 1, c.lds_max, c.lds_max);
        if (!g0.ok) return plan_real_full_complex(c, n, batch, false, normalize);
        Geometry g = geometry(n, prec, std::max(1, 256 / g0.TT), c.lds_max, c.lds_budget);
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = (long long)h, a.out_os = (long long)n;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        a.scale = sc;
        return add_launch(c, KK_C2R_FULL, 1, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                          "c2r_full");
    }
    const size_t M = n / 2;
    const void *rlo, *rhi;
    int rsh;
    int rc = two_level(p, n, prec, &rlo, &rhi, &rsh);
    if (rc) return rc;
    // one upload when the half length has a runtime geometry or a fixed shape
    // (a fixed shape without padding can hold a line the runtime one cannot)
    Geometry g0 = geometry(M, prec, 1, c.lds_max, c.lds_max);
    const Geometry gh = kernel_geometry(KK_C2R_HALF, prec, 1, M, false, g0.ok ? std::max(1, 256 / g0.TT) : 1,
                                        c.lds_max, c.lds_budget);
    if (g0.ok || (gh.ok && gh.fixed)) {
        const Geometry& g = gh;
        KArgs a = blank();
        a.in_es = a.out_es = 1;
        a.in_os = (long long)h, a.out_os = (long long)M;
        a.flags = KF_IN_ROWMAJOR | KF_OUT_ROWMAJOR;
        a.rlo = rlo, a.rhi = rhi, a.rshift = rsh;
        a.scale = sc;
        c.js << "\"real\":{\"len\":" << n << ",\"half\":" << M << ",\"uploads\":1},";
        return add_launch(c, KK_C2R_HALF, 1, g, a, (long long)batch, blocks_for(batch, g.G), SEL_IN, 0, SEL_OUT, 0,
                          "c2r_even_half");
    }
    size_t n1, n2;
    if (!four_step_split(M, prec, c.lds_max, &n1, &n2)) return plan_real_full_complex(c, n, batch, false, normalize);
    // take the orientation whose two passes have fixed shapes registered
    if (!find_fixed(KK_FS_A_C2R, prec, 1, (int)n1, true) && find_fixed(KK_FS_A_C2R, prec, 1, (int)n2, true) &&
        find_fixed(KK_FS_B, prec, 1, (int)n1, false))
        std::swap(n1, n2);
    Geometry ga = kernel_geometry(KK_FS_A_C2R, prec, 1, n1, true, prec ? 8 : 16, c.lds_max, c.lds_budget);
    Geometry gb = kernel_geometry(KK_FS_B, prec, 1, n2, false, prec ? 8 : 16, c.lds_max, c.lds_budget);
    if (!ga.ok || !gb.ok) return plan_real_full_complex(c, n, batch, false, normalize);
    // columns beside their mirrors in one block when the groups tile N2 evenly
    const bool pairs = ga.G % 2 == 0 && n2 % 2 == 0 && n2 % (size_t)ga.G == 0;
    // fixed shapes whose first stage can take the pair loads use them
    // (VKFX_C2R_PAIR_LOADS=0: every element reads X[k] and X[M-k] itself)
    const char* pe = getenv("VKFX_C2R_PAIR_LOADS");
    const bool pair_loads = !(pe && pe[0] == '0');
    const void *tlo, *thi;
    int tsh;
    rc = two_level(p, M, prec, &tlo, &thi, &tsh);
    if (rc) return rc;
    const size_t chunk = chunk_for(batch, M * cs, 64);
    p->work_bytes = std::max(p->work_bytes, chunk * M * cs);
    c.js << "\"real\":{\"len\":" << n << ",\"half\":" << M << ",\"uploads\":2,\"n1\":" << n1 << ",\"n2\":" << n2
         << ",\"chunk\":" << chunk << ",\"mirror_pairs\":" << (pairs ? "true" : "false") << "},";
    for (size_t b0 = 0; b0 < batch; b0 += chunk) {
        c.cur_chunk = (int)(b0 / chunk);
        const size_t cb = std::min(chunk, batch - b0);
        KArgs a = blank();
        a.C = (long long)n2;
        a.in_es = (long long)n2, a.in_cs = 1, a.in_os = (long long)h;
        a.out_es = (long long)n2, a.out_cs = 1, a.out_os = (long long)M;
        a.tlo = tlo, a.thi = thi, a.tshift = tsh;
        a.rlo = rlo, a.rhi = rhi, a.rshift = rsh;
        a.M = (long long)M, a.N1 = (long long)n1, a.N2 = (long long)n2;
        if (pairs) a.flags |= KF_MIRROR_PAIRS | (pair_loads ? KF_PAIR_LOADS : 0);
        long long lines = (long long)(cb * n2);
        rc = add_launch(c, KK_FS_A_C2R, 1, ga, a, lines, blocks_for(lines, ga.G), SEL_IN, b0 * h * cs, SEL_WORK, 0,
                        "c2r_columns_pre");
        if (rc) return rc;
        KArgs b = blank();
        b.C = (long long)n1;
        b.in_es = 1, b.in_cs = (long long)n2, b.in_os = (long long)M;
        b.out_es = (long long)n1, b.out_cs = 1, b.out_os = (long long)M;
        b.flags = KF_IN_ROWMAJOR;
        b.scale = sc;
        b.M = (long long)M, b.N1 = (long long)n1, b.N2 = (long long)n2;
        lines = (long long)(cb * n1);
        rc = add_launch(c, KK_FS_B, 1, gb, b, lines, blocks_for(lines, gb.G), SEL_WORK, 0, SEL_OUT, b0 * n * rs,
                        "c2r_rows");
        if (rc) return rc;
    }
    return VKFX_OK;
}

}  // namespace

// ============================================================== C ABI

extern "C" {

const char* vkfx_last_error(void) { return g_err.c_str(); }

#ifdef VKFX_INDEX_TEST
const char* vkfx_version(void) { return "vkfx-mi355x 0.1.0 (gfx950, index-map test build)"; }
#else
const char* vkfx_version(void) { return "vkfx-mi355x 0.1.0 (gfx950)"; }
#endif

int vkfx_context_create(int device_index, vkfx_context** out) {
    if (!out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null output pointer");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(VKFX_ERR_NATIVE_UNAVAILABLE, "HIP runtime has no usable device");
    if (device_index < 0 || device_index >= count)
        return fail(VKFX_ERR_NATIVE_UNAVAILABLE, "HIP device index out of range");
    e = hipSetDevice(device_index);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device_index);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    auto* ctx = new vkfx_context();
    ctx->device = device_index;
    // once per device, with the device current: the address of its copy of
    // the static scratch (a failure only disables vkfx_execute_noalloc)
    ctx->scratch_err = vkfx::static_scratch_address(device_index, &ctx->scratch);
    e = hipStreamCreate(&ctx->stream);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipStreamCreate");
    }
    vkfx_device_profile& pr = ctx->profile;
    pr.shared_memory_bytes = prop.sharedMemPerBlock;
    size_t p2 = 1;
    while (p2 * 2 <= pr.shared_memory_bytes) p2 *= 2;
    pr.shared_memory_pow2_bytes = p2;
    pr.max_threads_per_block = prop.maxThreadsPerBlock;
    pr.warp_size = prop.warpSize;
    pr.compute_units = prop.multiProcessorCount;
    pr.global_memory_bytes = prop.totalGlobalMem;
    std::snprintf(pr.name, sizeof(pr.name), "%s", prop.name[0] ? prop.name : prop.gcnArchName);
    std::snprintf(pr.arch, sizeof(pr.arch), "%s", prop.gcnArchName);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return fail(VKFX_ERR_NATIVE_UNAVAILABLE, std::string("library built for gfx950, device is ") + prop.gcnArchName);
    }
    *out = ctx;
    return VKFX_OK;
}

int vkfx_context_destroy(vkfx_context* ctx) {
    if (!ctx) return VKFX_OK;
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        if (ctx->active || ctx->plans)
            return fail(VKFX_ERR_NATIVE_RUNTIME, "cannot destroy a context with " + std::to_string(ctx->plans) +
                                                     " live plan(s) and " + std::to_string(ctx->active) +
                                                     " live ticket(s); destroy them first");
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (hipStream_t s : ctx->stream_pool) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
    for (PoolBuf& b : ctx->dev_pool) {
        if (b.ready) (void)hipEventDestroy(b.ready);
        (void)hipFree(b.p);
    }
    for (PoolBuf& b : ctx->host_pool) {
        if (b.ready) (void)hipEventDestroy(b.ready);
        (void)hipHostFree(b.p);
    }
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return VKFX_OK;
}

int vkfx_context_profile(const vkfx_context* ctx, vkfx_device_profile* out) {
    if (!ctx || !out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    *out = ctx->profile;
    return VKFX_OK;
}

int vkfx_context_synchronize(vkfx_context* ctx) {
    if (!ctx) return fail(VKFX_ERR_INVALID_ARGUMENT, "null context");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? VKFX_OK : hip_fail(e, "hipStreamSynchronize");
}

int vkfx_plan_create(vkfx_context* ctx, const vkfx_plan_desc* desc_in, vkfx_plan** out) {
    if (!ctx || !desc_in || !out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    vkfx_plan_desc d = *desc_in;
    if (d.rank < 1 || d.rank > VKFX_MAX_RANK) return fail(VKFX_ERR_INVALID_ARGUMENT, "rank must be 1..4");
    if (d.batch == 0) return fail(VKFX_ERR_INVALID_ARGUMENT, "batch count must be >= 1");
    for (uint32_t i = 0; i < d.rank; ++i)
        if (d.dims[i] == 0) return fail(VKFX_ERR_INVALID_ARGUMENT, "ZeroLength: axis " + std::to_string(i));
    if (d.precision < VKFX_F32 || d.precision > VKFX_F64_COMPUTE_F32_STORAGE)
        return fail(VKFX_ERR_UNSUPPORTED_PRECISION,
                    "precision must be F32, F64, F16StorageF32Compute or F64ComputeF32Storage");
    if (d.direction != VKFX_FORWARD && d.direction != VKFX_INVERSE)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "direction must be -1 or +1");
    if (d.transform == VKFX_R2C && d.direction != VKFX_FORWARD)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "R2C requires Direction::Forward");
    if (d.transform == VKFX_C2R && d.direction != VKFX_INVERSE)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "C2R requires Direction::Inverse");
    if (d.transform < VKFX_C2C || d.transform > VKFX_DST_IV) return fail(VKFX_ERR_INVALID_ARGUMENT, "unknown transform");
    const bool r2r = d.transform >= VKFX_DCT_I;
    // omitDimension (config.rs:1053-1067)
    if (d.omit_dimension >> d.rank)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "omitDimension metadata must match the FFT dimensionality");
    if (d.omit_dimension && d.rank == 1)
        return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "omitDimension currently supports multidimensional transforms only");
    if ((d.transform == VKFX_R2C || d.transform == VKFX_C2R) && (d.omit_dimension >> (d.rank - 1) & 1u))
        return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "omitDimension cannot disable the contiguous R2C/C2R axis");
    if (d.omit_dimension && d.perform_convolution)
        return fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                    "performConvolution currently requires active dimensions without omitDimension");
    if (d.transform == VKFX_DCT_I && d.rank == 1 && d.dims[0] < 2)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "InvalidTransformLength { axis: 0, transform: DCT-I, length: 1 }");
    // storage and compute scalar types (0 f16, 1 f32, 2 f64)
    const bool f64 = d.precision == VKFX_F64 || d.precision == VKFX_F64_COMPUTE_F32_STORAGE;
    const int store_t = d.precision == VKFX_F16_STORAGE_F32_COMPUTE ? 0 : d.precision == VKFX_F64 ? 2 : 1;
    const int comp_t = f64 ? 2 : 1;
    size_t total = d.batch;
    for (uint32_t i = 0; i < d.rank; ++i) {
        if (d.dims[i] > (size_t)1 << 40 || total > ((size_t)1 << 46) / d.dims[i])
            return fail(VKFX_ERR_ARITHMETIC_OVERFLOW, "tensor element count overflow");
        total *= d.dims[i];
    }
    PlannerDevice pdev = planner_device(ctx->profile.shared_memory_bytes);
    PlannerTuning tuning = tuning_for_amd(f64);
    if (d.custom_tuning) tuning = tuning_from(d.tuning);
    try {
        if (d.use_library_planner) {
            for (uint32_t i = 0; i < d.rank; ++i) {
                AxisDecision ad;
                if (d.transform == VKFX_C2C)
                    ad = plan_c2c_axis(d.dims[i], d.batch, f64, i + 1 != d.rank, tuning, pdev);
                else
                    ad = plan_axis_portable(d.dims[i], tuning);
                d.axis_algorithm[i] = (int32_t)ad.algorithm;
                d.convolution_len[i] = ad.convolution_len;
            }
        }
    } catch (const std::exception& ex) {
        return fail(VKFX_ERR_INVALID_ARGUMENT, std::string("planner: ") + ex.what());
    }
    (void)hipSetDevice(ctx->device);
    auto* p = new vkfx_plan();
    p->ctx = ctx;
    p->desc = d;
    Ctx c{p, f64 ? 1 : 0, lds_max_for(ctx), tuning};
    if (const char* e = getenv("VKFX_LDS_BUDGET_KB")) c.lds_budget = (size_t)atoll(e) << 10;

    const size_t cs = csize(c.prec), rs = rsize(c.prec);
    c.js << "{\"rank\":" << d.rank << ",\"dims\":[";
    for (uint32_t i = 0; i < d.rank; ++i) c.js << (i ? "," : "") << d.dims[i];
    static const char* kPrecName[] = {"f32", "f64", "f16_storage_f32_compute", "f64_compute_f32_storage"};
    c.js << "],\"batch\":" << d.batch << ",\"precision\":\"" << kPrecName[d.precision] << "\",\"transform\":\""
         << (d.transform == VKFX_C2C ? "c2c" : d.transform == VKFX_R2C ? "r2c" : d.transform == VKFX_C2R ? "c2r" : "r2r")
         << "\",\"axes\":[";
    for (uint32_t i = 0; i < d.rank; ++i) {
        const int alg = d.axis_algorithm[i];
        c.js << (i ? "," : "") << "{\"len\":" << d.dims[i] << ",\"algorithm\":\""
             << (alg == VKFX_ALG_STOCKHAM ? "stockham" : alg == VKFX_ALG_RADER ? "rader" : "bluestein") << "\"";
        if (d.convolution_len[i]) c.js << ",\"convolution_len\":" << d.convolution_len[i];
        c.js << "}";
    }
    c.js << "],";
    int rc = VKFX_OK;
    // convolution geometry (validated before any planning)
    size_t conv_coords = 1, conv_out_systems = d.batch;
    ConvArgs conv_args;
    const void* conv_kernel = nullptr;
    const bool conv_real = d.perform_convolution && d.transform == VKFX_R2C && d.rank > 1;
    if (d.perform_convolution) {
        if (d.transform != VKFX_C2C && !conv_real)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "performConvolution supports C2C plus multidimensional R2C application transforms");
        if (!rc && conv_real && d.batch != 1)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "multidimensional real performConvolution supports batch1 independent-coordinate or matrix "
                      "K=1/K>1 layouts");
        const int M = d.matrix_convolution > 1 ? (int)d.matrix_convolution : 0;
        if (!rc && M && M != 2 && M != 3)
            rc = fail(VKFX_ERR_INVALID_ARGUMENT, "matrix convolution IR requires a 2x2 or 3x3 matrix");
        if (!rc && M == 3 && d.symmetric_kernel)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "3x3 symmetric-kernel matrix convolution is not executable (convolution_ir.rs:112-117)");
        if (!rc && d.symmetric_kernel && !M)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "symmetricKernel requires matrixConvolution > 1");
        conv_coords = M ? (size_t)M : std::max<uint32_t>(1, d.coordinate_features);
        const size_t K = std::max<uint32_t>(1, d.kernel_count);
        // ownership rules of FftConfig::validate for C2C (config.rs:1156-1300)
        if (!rc && K > 1 && d.batch != 1)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "numberKernels is a one-input fan-out: multi-kernel convolution takes batch 1");
        if (!rc && !conv_real && !M && conv_coords != 1)
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "coordinateFeatures > 1 without matrixConvolution is only materialized for real application "
                      "convolution");
        if (!rc && M && (size_t)std::max<uint32_t>(1, d.coordinate_features) != (size_t)M)
            rc = fail(VKFX_ERR_INVALID_ARGUMENT, "matrix convolution coordinate count must equal its matrix size");
        if (!rc && !conv_real && d.rank > 1 && M && (d.batch != 1 || K != 1))
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "multidimensional performConvolution supports scalar K=1/K>1 layouts or a batch1/K1 matrix "
                      "layout");
        bool formatted = d.in_batch_stride || d.out_batch_stride, padded = false;
        for (uint32_t i = 0; i < d.rank; ++i) {
            formatted = formatted || d.in_axis_stride[i] || d.out_axis_stride[i];
            padded = padded || d.zero_left[i] != d.zero_right[i];
        }
        // formatted: scalar batch1 K1 real ownership; zero padding: real with
        // a nonsymmetric matrix or no matrix (config.rs:1273-1300)
        if (!rc && formatted && !(conv_real && conv_coords == 1 && K == 1 && !M))
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      conv_real ? "multidimensional real formatted performConvolution currently requires scalar batch1 K1"
                                : "formatted performConvolution requires a real application");
        if (!rc && padded && !(conv_real && !(M && d.symmetric_kernel)))
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      conv_real ? "multidimensional real performConvolution zero padding requires batch1/K1 "
                                  "nonsymmetric matrix ownership"
                                : "performConvolution zero padding requires a multidimensional real application");
        const bool mixed = d.precision == VKFX_F16_STORAGE_F32_COMPUTE || d.precision == VKFX_F64_COMPUTE_F32_STORAGE;
        if (!rc && mixed && !conv_real &&
            (d.rank != 1 || d.batch != 1 || conv_coords != 1 || K != 1 || d.conjugate_sequence ||
             d.cross_power_normalize))
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "mixed-storage performConvolution requires dense default-policy 1D C2C batch1 scalar K1");
        // config.rs:1244-1272: unformatted real ownership (scalar, independent K>1 fan-out, 3x3 matrix)
        if (!rc && mixed && conv_real &&
            !((conv_coords == 1 && !M) || (conv_coords > 1 && !M && K > 1) || (M == 3 && conv_coords == 3)))
            rc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH,
                      "mixed-storage real performConvolution requires scalar, independent-coordinate K>1 or 3x3 "
                      "matrix ownership");
        conv_out_systems = K > 1 ? K : d.batch;
        size_t T = 1;  // tensor length of the spectra: compact for the real application
        for (uint32_t i = 0; i < d.rank; ++i) T *= (conv_real && i + 1 == d.rank) ? d.dims[i] / 2 + 1 : d.dims[i];
        const bool independent = conv_real ? !M : d.independent_coordinates != 0;
        const size_t planes = M ? (d.symmetric_kernel ? (size_t)(M * (M + 1) / 2) : (size_t)(M * M))
                                : (independent ? conv_coords : 1);
        const size_t need = K * planes * T * (f64 ? 16 : 8);
        if (!rc && (!d.kernel_spectrum || d.kernel_spectrum_bytes != need))
            rc = fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "convolution kernel spectrum: expected " + std::to_string(need) +
                                                          " bytes, got " + std::to_string(d.kernel_spectrum_bytes));
        if (!rc) {
            // non-finite kernel values are rejected (convolution_ir.rs:347-355)
            bool finite = true;
            const size_t nv = need / (f64 ? 8 : 4);
            for (size_t i = 0; i < nv && finite; ++i)
                finite = f64 ? std::isfinite(((const double*)d.kernel_spectrum)[i])
                             : std::isfinite(((const float*)d.kernel_spectrum)[i]);
            if (!finite) rc = fail(VKFX_ERR_INVALID_ARGUMENT, "convolution kernel spectrum contains non-finite values");
        }
        if (!rc) rc = upload(p, "conv_kernel", d.kernel_spectrum, need, &conv_kernel);
        conv_args.T = (long long)T;
        conv_args.systems_out = (long long)conv_out_systems;
        conv_args.coords = (int)conv_coords;
        conv_args.planes = (int)planes;
        conv_args.kernel_count = (int)K;
        conv_args.matrix = M;
        conv_args.symmetric = d.symmetric_kernel ? 1 : 0;
        conv_args.independent = independent ? 1 : 0;
        conv_args.conj_seq = d.conjugate_sequence ? 1 : 0;
        conv_args.cross_norm = d.cross_power_normalize ? 1 : 0;
        if (rc) {
            delete p;
            return rc;
        }
    }
    try {
        if (conv_real) {
            p->in_bytes = conv_coords * total * rs;
            p->out_bytes = conv_out_systems * conv_coords * total * rs;
            rc = plan_convolution_real(c, d, conv_coords, conv_out_systems, conv_args, conv_kernel);
        } else if (d.perform_convolution) {
            size_t T = 1;
            for (uint32_t i = 0; i < d.rank; ++i) T *= d.dims[i];
            p->in_bytes = d.batch * conv_coords * T * cs;
            p->out_bytes = conv_out_systems * conv_coords * T * cs;
            rc = plan_convolution(c, d, conv_coords, conv_out_systems, conv_args, conv_kernel);
        } else if (d.transform == VKFX_C2C) {
            p->in_bytes = p->out_bytes = total * cs;
            if (d.rank == 1) {
                const int alg = d.axis_algorithm[0];
                Algorithm a = alg == VKFX_ALG_STOCKHAM ? Algorithm::Stockham
                              : alg == VKFX_ALG_RADER  ? Algorithm::Rader
                                                       : Algorithm::Bluestein;
                size_t conv = d.convolution_len[0];
                if (alg == VKFX_ALG_RADER) conv = 0;  // Bluestein fallback uses M = next smooth >= 2N-1
                rc = plan_c2c_1d(c, d.dims[0], d.batch, d.direction, d.normalize != 0, a, conv);
            } else {
                rc = plan_c2c_nd(c, d, d.omit_dimension);
            }
        } else if (r2r) {
            p->in_bytes = p->out_bytes = total * rs;
            if (d.rank == 1)
                rc = plan_r2r(c, d.dims[0], d.batch, d.transform - VKFX_DCT_I, d.direction, d.normalize != 0);
            else
                rc = plan_r2r_nd(c, d);
        } else {
            const size_t n = d.dims[d.rank - 1];
            const size_t real_elems = total, compact_elems = total / n * (n / 2 + 1);
            const bool r2c_kind = d.transform == VKFX_R2C;
            p->in_bytes = r2c_kind ? real_elems * rs : compact_elems * cs;
            p->out_bytes = r2c_kind ? compact_elems * cs : real_elems * rs;
            if (d.rank > 1)
                rc = plan_real_nd(c, d, r2c_kind);
            else
                rc = r2c_kind ? plan_r2c(c, n, d.batch) : plan_c2r(c, n, d.batch, d.normalize != 0);
        }
    } catch (const std::exception& ex) {
        rc = fail(VKFX_ERR_INVALID_ARGUMENT, std::string("plan: ") + ex.what());
    }
    if (rc) {
        delete p;
        return rc;
    }
    {
        // Boundary passes: type conversion (mixed precisions), formatted
        // layouts and zero padding sit between the caller's buffers and dense
        // compute-type copies in the workspace that the FFT passes use.
        const bool real_in = d.transform == VKFX_R2C || r2r,
                   real_out = d.transform == VKFX_C2R || r2r || conv_real;
        p->real_out = real_out;
        const size_t rank = d.rank;
        long long in_dims[VKFX_MAX_RANK], out_dims[VKFX_MAX_RANK];
        for (size_t i = 0; i < rank; ++i) in_dims[i] = out_dims[i] = (long long)d.dims[i];
        if (d.transform == VKFX_R2C && !conv_real) out_dims[rank - 1] = (long long)(d.dims[rank - 1] / 2 + 1);
        if (d.transform == VKFX_C2R) in_dims[rank - 1] = (long long)(d.dims[rank - 1] / 2 + 1);
        // resolve_formatted_axis_strides / _batch_stride (config.rs:1463-1522)
        auto resolve = [&](const long long* dims, const uint64_t* over, uint64_t batch_over, long long* st,
                           long long* bst, bool* formatted, const char* side) -> int {
            *formatted = false;
            st[rank - 1] = 1;
            if (over[rank - 1] && over[rank - 1] != 1)
                return fail(VKFX_ERR_INVALID_ARGUMENT,
                            std::string(side) + ": formatted fastest-axis stride must remain one stored element");
            for (int ax = (int)rank - 2; ax >= 0; --ax) {
                const long long minimum = st[ax + 1] * dims[ax + 1];
                st[ax] = over[ax] ? (long long)over[ax] : minimum;
                if (st[ax] < minimum)
                    return fail(VKFX_ERR_INVALID_ARGUMENT,
                                std::string(side) + ": formatted axis stride overlaps the next faster logical axis");
                *formatted |= st[ax] != minimum;
            }
            const long long minimum = st[0] * dims[0];
            *bst = batch_over ? (long long)batch_over : minimum;
            if (*bst < minimum)
                return fail(VKFX_ERR_INVALID_ARGUMENT, std::string(side) + ": formatted batch stride overlaps the logical tensor");
            *formatted |= *bst != minimum;
            return VKFX_OK;
        };
        long long in_st[VKFX_MAX_RANK], out_st[VKFX_MAX_RANK], in_bst = 0, out_bst = 0;
        bool fmt_in = false, fmt_out = false;
        int brc = resolve(in_dims, d.in_axis_stride, d.in_batch_stride, in_st, &in_bst, &fmt_in, "input");
        if (!brc) brc = resolve(out_dims, d.out_axis_stride, d.out_batch_stride, out_st, &out_bst, &fmt_out, "output");
        // zero padding ranges and the boundary that owns them (zero_pad_ir.rs:38-46)
        bool any_zero = false;
        for (size_t i = 0; i < rank && !brc; ++i) {
            if (d.zero_left[i] > d.zero_right[i] || d.zero_right[i] > d.dims[i])
                brc = fail(VKFX_ERR_INVALID_ARGUMENT, "InvalidZeroPaddingRange on axis " + std::to_string(i));
            any_zero |= d.zero_right[i] > d.zero_left[i];
        }
        if (!brc && any_zero && d.zero_frequency && d.transform != VKFX_C2C)
            brc = fail(VKFX_ERR_UNSUPPORTED_KERNEL_PATH, "frequency-domain zero padding is C2C only");
        for (size_t i = 0; i < rank && !brc; ++i)
            if (d.grouped_batch[i] > d.batch)
                brc = fail(VKFX_ERR_INVALID_ARGUMENT, "groupedBatch exceeds the batch count");
        if (brc) {
            delete p;
            return brc;
        }
        const bool fwd = d.direction == VKFX_FORWARD;
        // a real-application convolution masks its input (forward R2C) and
        // its output (inverse C2R): spatial padding on both children
        const bool zp_in = any_zero && (conv_real || (d.zero_frequency ? !fwd : fwd));
        const bool zp_out = any_zero && (conv_real || !zp_in);
        const bool mixed = store_t != comp_t;
        // 1-D C2C whose only boundary work is a formatted batch stride: the
        // passes that read the caller's input or write its output take that
        // stride as their per-transform stride, so no boundary pass runs
        // (the reference keeps layouts inside its passes). Every such pass
        // must address transform b at b * n (in_os / out_os = n, chunk
        // offsets multiples of n elements).
        auto fuse_batch_stride = [&](bool in_side, long long bst) {
            const long long n = (long long)d.dims[0];
            const size_t unit = (size_t)n * csize(c.prec);
            for (const Launch& L : p->launches) {
                if (L.boundary || L.r2r || L.copy) return false;
                if (in_side && L.in_sel == SEL_IN && (L.a.in_os != n || L.in_off % unit)) return false;
                if (!in_side && L.out_sel == SEL_OUT && (L.a.out_os != n || L.out_off % unit)) return false;
            }
            for (Launch& L : p->launches) {
                if (in_side && L.in_sel == SEL_IN) {
                    L.a.in_os = bst;
                    L.in_off = L.in_off / unit * (size_t)bst * csize(c.prec);
                }
                if (!in_side && L.out_sel == SEL_OUT) {
                    L.a.out_os = bst;
                    L.out_off = L.out_off / unit * (size_t)bst * csize(c.prec);
                }
            }
            return true;
        };
        const bool plain_1d = d.transform == VKFX_C2C && !d.perform_convolution && rank == 1 && !mixed && !any_zero;
        bool fused_in = false, fused_out = false;
        if (plain_1d && fmt_in) fused_in = fuse_batch_stride(true, in_bst);
        if (plain_1d && fmt_out) fused_out = fuse_batch_stride(false, out_bst);
        // C2C plans in chunks of the form: the first pass (a plain one-upload
        // line pass) reads the caller's input, the passes between run in
        // place on the output and the workspace, the last (a plain one-upload
        // line pass) leaves the result in the output. The boundary work then
        // happens inside the first pass's loads and the last pass's stores,
        // and no boundary pass runs (the reference keeps it inside its
        // passes, src/zero_pad_ir.rs:607-617):
        //  - rank 1, one pass per chunk: storage conversion and the zero
        //    interval (a line is the whole axis) on runtime-shape kernels
        //    with KF_EDGE;
        //  - formatted layouts of rank <= 3 with every axis active and one
        //    pass per axis: the first pass's lines (batch, axis 0, axis 1)
        //    and the last pass's lines (batch, axis 1, axis 2) take the
        //    caller's strides (three line levels), on any kernel.
        // When the output is narrower or formatted, the passes between the
        // first and the last run on a compute-type copy in the workspace.
        // VKFX_FUSED_EDGES=0 keeps the boundary passes (comparison runs).
        const char* fe = getenv("VKFX_FUSED_EDGES");
        const bool fuse_on = !(fe && fe[0] == '0');
        // mixed-storage one-pass chunks keep a fixed row shape that has an
        // edge variant (VKFX_FIXED_EDGES=0: the runtime-shape edge kernels);
        // the first and last passes of a multi-pass chunk (N-D) keep theirs
        // when both have input / output variants and there is no zero interval
        const char* fxe = getenv("VKFX_FIXED_EDGES");
        const bool fixed_edges = mixed && !(fxe && fxe[0] == '0');
        auto end_variant = [&](const Launch& L, bool first, bool last) -> const FixedKernel* {
            if (!fixed_edges || !L.fixed) return nullptr;
            if (first && last) return kind_variant(L.fixed, KK_PLAIN_EDGE);
            if (any_zero) return nullptr;
            return kind_variant(L.fixed, first ? KK_PLAIN_EDGE_IN : KK_PLAIN_EDGE_OUT);
        };
        bool all_active = true;
        for (size_t i = 0; i < rank; ++i) all_active &= d.dims[i] > 1 && !(d.omit_dimension >> i & 1u);
        // the first and last passes of a chunk are plain one-upload line
        // passes; the passes between (split-axis and Bluestein axis passes
        // included) touch only the output, in place, and the workspace
        auto chunks_fusable = [&]() {
            if (d.transform != VKFX_C2C || d.perform_convolution || p->launches.empty()) return false;
            int prev_chunk = -1;
            for (size_t i = 0; i < p->launches.size(); ++i) {
                const Launch& L = p->launches[i];
                if (L.boundary || L.copy || L.r2r || L.conv || L.chunk < prev_chunk) return false;
                const bool first = L.chunk != prev_chunk;
                const bool last = i + 1 == p->launches.size() || p->launches[i + 1].chunk != L.chunk;
                const bool plain = L.kind == KK_PLAIN && !L.a.rtab;
                if ((first || last) && !plain) return false;
                // a fixed shape that would carry edges needs an edge variant (one-pass
                // chunks) or a runtime geometry of its length
                if ((first || last) && (mixed || any_zero) && L.fixed && !end_variant(L, first, last) &&
                    !edge_geometry(c, L.a).ok)
                    return false;
                if ((L.in_sel == SEL_IN) != first || (first && L.out_sel != SEL_OUT && !last)) return false;
                if (last && L.out_sel != SEL_OUT) return false;
                if ((L.in_sel != SEL_IN && L.in_sel != SEL_OUT && L.in_sel != SEL_WORK) ||
                    (L.out_sel != SEL_OUT && L.out_sel != SEL_WORK))
                    return false;
                prev_chunk = L.chunk;
            }
            return true;
        };
        // one launch per active axis and chunk, rows first and axis 0 last
        auto layout_fusable = [&]() {
            if (rank > 3 || !all_active) return false;
            size_t run = 0;
            for (size_t i = 0; i < p->launches.size(); ++i) {
                ++run;
                if (i + 1 == p->launches.size() || p->launches[i + 1].chunk != p->launches[i].chunk) {
                    if (run != rank) return false;
                    run = 0;
                }
            }
            return true;
        };
        const bool shape_ok = fuse_on && chunks_fusable();
        const bool want_layout = (fmt_in && !fused_in) || (fmt_out && !fused_out);
        const bool layout_ok = want_layout && shape_ok && layout_fusable();
        // Edges ride on runtime-shape kernels, which pay where a 1-D line is
        // the whole transform (mixed 1024 x 8192: 33.5 us against 94.8 with
        // boundary passes) but not on N-D column passes (F16 2048^2 x 4: the
        // runtime-shape column pass with the conversion 145 us against 35 us
        // for the fixed shape plus 40 us for a flat conversion pass).
        // Mixed-storage 1-D two-upload C2C: per chunk the column pass (the
        // caller's input into the workspace) and the row pass (the workspace
        // into the caller's output) on fixed shapes, whose edge kinds read and
        // write the storage type and apply the zero intervals; no boundary
        // pass and no compute-type copy (F64ComputeF32Storage 2^20 x 8: two
        // passes of 24 bytes per element instead of four passes of 112 bytes
        // per element in all).
        auto four_step_edges = [&]() {
            if (!fuse_on || !mixed || rank != 1 || want_layout || d.transform != VKFX_C2C ||
                d.perform_convolution || p->launches.empty() || p->launches.size() % 2)
                return false;
            for (size_t i = 0; i < p->launches.size(); i += 2) {
                const Launch& A = p->launches[i];
                const Launch& B = p->launches[i + 1];
                if (A.boundary || A.copy || A.r2r || A.conv || B.boundary || B.copy || B.r2r || B.conv) return false;
                if (A.kind != KK_FS_A || B.kind != KK_FS_B || A.chunk != B.chunk || A.a.rtab || B.a.rtab) return false;
                if (A.in_sel != SEL_IN || A.out_sel != SEL_WORK || B.in_sel != SEL_WORK || B.out_sel != SEL_OUT)
                    return false;
                if (!kind_variant(A.fixed, KK_FS_A_EDGE) || !kind_variant(B.fixed, KK_FS_B_EDGE)) return false;
            }
            return true;
        };
        const bool fs_edges = four_step_edges();
        if (fs_edges) {
            const size_t cs = csize(c.prec);
            const size_t scs = (store_t == 0 ? 2 : store_t == 1 ? 4 : 8) * 2;  // storage bytes per complex element
            for (size_t i = 0; i < p->launches.size(); i += 2) {
                Launch& A = p->launches[i];
                Launch& B = p->launches[i + 1];
                A.kind = KK_FS_A_EDGE;
                A.fixed = kind_variant(A.fixed, KK_FS_A_EDGE);
                A.a.flags |= KF_NARROW_IN | (zp_in ? KF_ZERO_IN : 0);
                A.in_off = A.in_off / cs * scs;
                B.kind = KK_FS_B_EDGE;
                B.fixed = kind_variant(B.fixed, KK_FS_B_EDGE);
                B.a.flags |= KF_NARROW_OUT | (zp_out ? KF_ZERO_OUT : 0);
                B.out_off = B.out_off / cs * scs;
                if (any_zero) {
                    A.a.zl = B.a.zl = (long long)d.zero_left[0];
                    A.a.zr = B.a.zr = (long long)d.zero_right[0];
                }
            }
        }
        // 1-D one-upload Bluestein: the single kernel reads the caller's input
        // and writes the caller's output in the storage type, with the zero
        // intervals, on the edge variant of its fixed shape
        auto bluestein_edges = [&]() {
            if (!fuse_on || !(mixed || any_zero) || rank != 1 || want_layout || d.transform != VKFX_C2C ||
                d.perform_convolution || p->launches.empty())
                return false;
            for (const Launch& L : p->launches)
                if (L.boundary || L.copy || L.r2r || L.conv || L.kind != KK_BLUE_1 || L.in_sel != SEL_IN ||
                    L.out_sel != SEL_OUT || L.a.rtab || !kind_variant(L.fixed, KK_BLUE_1_EDGE))
                    return false;
            return true;
        };
        const bool bl_edges = !fs_edges && bluestein_edges();
        if (bl_edges) {
            const size_t cs = csize(c.prec);
            const size_t scs = (store_t == 0 ? 2 : store_t == 1 ? 4 : 8) * 2;  // storage bytes per complex element
            for (Launch& L : p->launches) {
                L.kind = KK_BLUE_1_EDGE;
                L.fixed = kind_variant(L.fixed, KK_BLUE_1_EDGE);
                if (mixed) {
                    L.a.flags |= KF_NARROW_IN | KF_NARROW_OUT;
                    L.in_off = L.in_off / cs * scs;
                    L.out_off = L.out_off / cs * scs;
                }
                if (zp_in) L.a.flags |= KF_ZERO_IN;
                if (zp_out) L.a.flags |= KF_ZERO_OUT;
                if (any_zero) {
                    L.a.zl = (long long)d.zero_left[0];
                    L.a.zr = (long long)d.zero_right[0];
                }
            }
        }
        // 1-D even-length real transforms of one upload: the R2C or C2R kernel
        // reads and writes the caller's buffers in the storage type, with the
        // zero interval of the real side, on the edge variant of its fixed shape
        auto real_edges = [&]() {
            if (!fuse_on || !(mixed || any_zero) || rank != 1 || want_layout || d.perform_convolution ||
                (d.transform != VKFX_R2C && d.transform != VKFX_C2R) || p->launches.empty())
                return false;
            const KernelKind k = d.transform == VKFX_R2C ? KK_R2C_HALF : KK_C2R_HALF;
            const KernelKind ke = d.transform == VKFX_R2C ? KK_R2C_HALF_EDGE : KK_C2R_HALF_EDGE;
            for (const Launch& L : p->launches)
                if (L.boundary || L.copy || L.r2r || L.conv || L.kind != k || L.in_sel != SEL_IN ||
                    L.out_sel != SEL_OUT || L.a.rtab || !kind_variant(L.fixed, ke))
                    return false;
            return true;
        };
        const bool re_edges = !fs_edges && !bl_edges && real_edges();
        if (re_edges) {
            const size_t cs = csize(c.prec);
            const size_t scs = (store_t == 0 ? 2 : store_t == 1 ? 4 : 8) * 2;  // storage bytes per complex element
            const KernelKind ke = d.transform == VKFX_R2C ? KK_R2C_HALF_EDGE : KK_C2R_HALF_EDGE;
            for (Launch& L : p->launches) {
                L.kind = ke;
                L.fixed = kind_variant(L.fixed, ke);
                if (mixed) {
                    L.a.flags |= KF_NARROW_IN | KF_NARROW_OUT;
                    L.in_off = L.in_off / cs * scs;
                    L.out_off = L.out_off / cs * scs;
                }
                if (zp_in) L.a.flags |= KF_ZERO_IN;
                if (zp_out) L.a.flags |= KF_ZERO_OUT;
                if (any_zero) {
                    L.a.zl = (long long)d.zero_left[0];
                    L.a.zr = (long long)d.zero_right[0];
                }
            }
        }
        // N-D: every chunk's first and last pass on a fixed shape with its variant
        auto nd_ends_fixed = [&]() {
            if (rank < 2 || !mixed || any_zero || want_layout) return false;
            int prev_chunk = -1;
            for (size_t i = 0; i < p->launches.size(); ++i) {
                const Launch& L = p->launches[i];
                const bool first = L.chunk != prev_chunk;
                const bool last = i + 1 == p->launches.size() || p->launches[i + 1].chunk != L.chunk;
                prev_chunk = L.chunk;
                if ((first || last) && (first == last || !end_variant(L, first, last))) return false;
            }
            return true;
        };
        const bool fused_edges = !fs_edges && !bl_edges && !re_edges && shape_ok && (mixed || any_zero) &&
                                 (rank == 1 || nd_ends_fixed()) && (!want_layout || layout_ok);
        const bool fused_layout = layout_ok && (fused_edges || !(mixed || any_zero));
        bool edge_stage = false;  // passes between the first and the last run on a compute-type copy
        if (fused_edges || fused_layout) {
            const bool stage_mid = mixed || (fmt_out && !fused_out);
            const size_t cs = csize(c.prec);
            const size_t scs = (store_t == 0 ? 2 : store_t == 1 ? 4 : 8) * 2;  // storage bytes per complex element
            long long per_batch = 1;
            for (size_t i = 0; i < rank; ++i) per_batch *= (long long)d.dims[i];
            const long long* dm = in_dims;
            int prev_chunk = -1;
            for (size_t i = 0; i < p->launches.size(); ++i) {
                Launch& L = p->launches[i];
                const bool first = L.chunk != prev_chunk;
                const bool last = i + 1 == p->launches.size() || p->launches[i + 1].chunk != L.chunk;
                prev_chunk = L.chunk;
                if (fused_edges && (first || last)) {
                    // a one-pass chunk on a fixed row shape with an edge
                    // variant keeps its shape; the others move to the
                    // runtime-shape edge kernels
                    const FixedKernel* fe = end_variant(L, first, last);
                    if (fe) {
                        L.kind = first && last ? KK_PLAIN_EDGE : first ? KK_PLAIN_EDGE_IN : KK_PLAIN_EDGE_OUT;
                        L.fixed = fe;
                    } else {
                        int rc = to_edge_kernel(c, L);
                        if (rc) {
                            delete p;
                            return rc;
                        }
                        L.a.flags |= KF_EDGE;
                    }
                    if (any_zero) L.a.zl = (long long)d.zero_left[0], L.a.zr = (long long)d.zero_right[0];
                    if (first && mixed) L.a.flags |= KF_NARROW_IN;
                    if (first && zp_in) L.a.flags |= KF_ZERO_IN;
                    if (last && mixed) L.a.flags |= KF_NARROW_OUT;
                    if (last && zp_out) L.a.flags |= KF_ZERO_OUT;
                }
                KArgs& a = L.a;
                if (first) {
                    const long long b0 = (long long)(L.in_off / ((size_t)per_batch * cs));
                    const bool fmt = fmt_in && fused_layout;
                    const long long bst = fmt ? in_bst : per_batch;
                    // dense: the same element offset in the storage type
                    L.in_off = fmt ? (size_t)(b0 * bst) * (mixed ? scs : cs) : L.in_off / cs * (mixed ? scs : cs);
                    if (fmt && rank == 1) {
                        a.in_os = bst;
                    } else if (fmt) {
                        // rows: lines (batch, i0[, i1]) at the caller's strides; dense on the output side
                        a.C = rank == 3 ? dm[1] : 1;
                        a.in_cs = rank == 3 ? in_st[1] : 1;
                        a.out_cs = rank == 3 ? dm[2] : 1;
                        a.C1 = dm[0];
                        a.in_os1 = in_st[0];
                        a.out_os1 = rank == 3 ? dm[1] * dm[2] : dm[1];
                        a.in_os = bst;
                        a.out_os = per_batch;
                    }
                } else if (stage_mid && L.in_sel == SEL_OUT) {
                    L.in_sel = SEL_STAGE_OUT;
                }
                if (last) {
                    const long long b0 = (long long)(L.out_off / ((size_t)per_batch * cs));
                    const bool fmt = fmt_out && fused_layout;
                    const long long bst = fmt ? out_bst : per_batch;
                    L.out_off = fmt ? (size_t)(b0 * bst) * (mixed ? scs : cs) : L.out_off / cs * (mixed ? scs : cs);
                    if (fmt && rank == 1) {
                        a.out_os = bst;
                    } else if (fmt) {
                        // axis 0 columns: lines (batch, i1[, i2]) at the caller's strides; dense input
                        a.C = rank == 3 ? dm[2] : dm[1];
                        a.in_cs = a.out_cs = 1;
                        a.C1 = rank == 3 ? dm[1] : 1;
                        a.in_os1 = rank == 3 ? dm[2] : 0;
                        a.out_os1 = rank == 3 ? out_st[1] : 0;
                        a.out_es = out_st[0];
                        a.in_os = per_batch;
                        a.out_os = bst;
                    }
                } else if (stage_mid && L.out_sel == SEL_OUT) {
                    L.out_sel = SEL_STAGE_OUT;
                    edge_stage = true;
                }
            }
        }
        const bool fused_all = fused_edges || fused_layout || fs_edges || bl_edges || re_edges;
        const bool need_in = !fused_all && (mixed || (fmt_in && !fused_in) || zp_in);
        const bool need_out = !fused_all && (mixed || (fmt_out && !fused_out) || zp_out);
        const size_t ssz = store_t == 0 ? 2 : store_t == 1 ? 4 : 8;
        const size_t cin = p->in_bytes, cout = p->out_bytes;  // dense compute-type bytes
        const int in_scal = real_in ? 1 : 2, out_scal = real_out ? 1 : 2;
        auto make = [&](bool in_side) {
            Launch L{};
            L.boundary = true;
            BoundaryArgs& a = L.ba;
            a.rank = (int)rank;
            a.batch = (long long)((in_side ? d.batch : conv_out_systems) * conv_coords);
            const long long* dims = in_side ? in_dims : out_dims;
            long long dense = 1;
            for (int ax = (int)rank - 1; ax >= 0; --ax) {
                a.dims[ax] = dims[ax];
                const long long phys = in_side ? in_st[ax] : out_st[ax];
                a.src_stride[ax] = in_side ? phys : dense;
                a.dst_stride[ax] = in_side ? dense : phys;
                dense *= dims[ax];
                if (in_side ? zp_in : zp_out) {
                    a.zero_left[ax] = (long long)d.zero_left[ax];
                    a.zero_right[ax] = (long long)d.zero_right[ax];
                }
            }
            a.tensor_len = dense;
            a.src_batch = in_side ? in_bst : dense;
            a.dst_batch = in_side ? dense : out_bst;
            a.src_scalars = a.dst_scalars = in_side ? in_scal : out_scal;
            a.src_type = in_side ? store_t : comp_t;
            a.dst_type = in_side ? comp_t : store_t;
            L.label = in_side ? "boundary_in" : "boundary_out";
            L.in_sel = in_side ? SEL_IN : SEL_STAGE_OUT;
            L.out_sel = in_side ? SEL_STAGE_IN : SEL_OUT;
            return L;
        };
        for (Launch& L : p->launches) {
            auto remap = [&](int s) {
                return (need_in && s == SEL_IN) ? (int)SEL_STAGE_IN : (need_out && s == SEL_OUT) ? (int)SEL_STAGE_OUT : s;
            };
            L.in_sel = remap(L.in_sel);
            L.out_sel = remap(L.out_sel);
        }
        if (need_in) p->launches.insert(p->launches.begin(), make(true));
        if (need_out) p->launches.push_back(make(false));
        p->in_bytes = (size_t)in_bst * d.batch * conv_coords * in_scal * ssz;
        p->out_bytes = (size_t)out_bst * conv_out_systems * conv_coords * out_scal * ssz;
        if (need_in || need_out) p->serial = true;  // the boundary passes bracket every chunk
        p->stage_in_bytes = need_in ? cin : 0;
        // C2C runs in place on one copy when both sides are staged
        p->stage_shared = need_out && need_in && d.transform == VKFX_C2C;
        p->stage_out_bytes = (need_out && !p->stage_shared) || edge_stage ? cout : 0;
        c.js << "\"boundary\":{\"input\":" << (need_in ? "true" : "false") << ",\"output\":"
             << (need_out ? "true" : "false") << ",\"fused_batch_stride\":[" << (fused_in ? "true" : "false")
             << "," << (fused_out ? "true" : "false") << "],\"fused_edges\":" << (fused_edges || fs_edges || bl_edges || re_edges ? "true" : "false")
             << ",\"four_step_edges\":" << (fs_edges ? "true" : "false")
             << ",\"bluestein_edges\":" << (bl_edges ? "true" : "false")
             << ",\"real_edges\":" << (re_edges ? "true" : "false")
             << ",\"fused_layout\":" << (fused_layout ? "true" : "false")
             << ",\"zero_padding\":\""
             << (!any_zero ? "none" : d.zero_frequency ? "frequency" : "spatial") << "\",\"grouped_batch\":[";
        for (size_t i = 0; i < rank; ++i) c.js << (i ? "," : "") << d.grouped_batch[i];
        c.js << "]},";
    }
    int nchunks = 1;
    for (const Launch& L : p->launches) nchunks = std::max(nchunks, L.chunk + 1);
    // Nontemporal roles of the fixed-shape passes: a pass reading the
    // caller's input streams it (nontemporal loads), the last pass of a chunk
    // streams the caller's output (nontemporal stores), and every other access
    // stays cached so that a chunk's intermediate is served from the Infinity
    // Cache by the next pass. VKFX_NT_ROLES=0 keeps each shape's first
    // registered variant.
    const char* ne = getenv("VKFX_NT_ROLES");
    const bool nt_roles = !(ne && ne[0] == '0');
    for (size_t i = 0; nt_roles && i < p->launches.size(); ++i) {
        Launch& L = p->launches[i];
        if (!L.fixed) continue;
        bool last = true;
        for (size_t j = i + 1; j < p->launches.size() && last; ++j) last = p->launches[j].chunk != L.chunk;
        L.fixed = fixed_variant(L.fixed, L.in_sel == SEL_IN, L.out_sel == SEL_OUT && last);
    }
    // two lanes pay a fork/join (two events, ~10 us) per execute, so only
    // plans with several chunks use them
    p->lanes = nchunks >= 4 && !p->serial ? 2 : 1;
    if (const char* e = getenv("VKFX_LANES")) p->lanes = (atoi(e) == 1 || p->serial) ? 1 : p->lanes;
    p->work_lane = p->work_bytes;
    p->work_bytes = p->work_lane * p->lanes;
    if (p->full_bytes) {
        p->full_off = (p->work_bytes + 255) / 256 * 256;
        p->work_bytes = p->full_off + p->full_bytes;
    }
    if (p->aux_bytes) {
        p->aux_off = (p->work_bytes + 255) / 256 * 256;
        p->work_bytes = p->aux_off + p->aux_bytes;
    }
    if (p->conv_a_bytes) {
        p->conv_a_off = (p->work_bytes + 255) / 256 * 256;
        p->conv_b_off = (p->conv_a_off + p->conv_a_bytes + 255) / 256 * 256;
        p->work_bytes = p->conv_b_off + p->conv_b_bytes;
    }
    if (p->stage_in_bytes || p->stage_out_bytes) {
        // workspace: [lane work][full complex][aux][conv a][conv b][stage in][stage out]
        auto align = [](size_t v) { return (v + 255) / 256 * 256; };
        const bool shared = p->stage_shared;
        p->stage_in_off = align(p->work_bytes);
        p->stage_out_off = shared ? p->stage_in_off : p->stage_in_off + align(p->stage_in_bytes);
        p->work_bytes = shared ? p->stage_in_off + p->stage_in_bytes : p->stage_out_off + p->stage_out_bytes;
    }
    if (p->lanes == 2) {
        // each two-lane plan forks onto a stream of its own, so plans on
        // different caller streams do not serialize their odd chunks
        hipError_t e = hipEventCreateWithFlags(&p->ev_fork, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&p->ev_join, hipEventDisableTiming);
        if (e == hipSuccess) e = hipStreamCreate(&p->aux);
        if (e != hipSuccess) {
            if (p->ev_fork) (void)hipEventDestroy(p->ev_fork);
            if (p->ev_join) (void)hipEventDestroy(p->ev_join);
            delete p;
            return hip_fail(e, "plan stream lane");
        }
    }
    c.js << "\"lanes\":" << p->lanes << ",\"workspace_bytes\":" << p->work_bytes << ",\"passes\":[";
    for (const Launch& L : p->launches) note_pass(c, L);
    c.js << "]}";
    p->json = c.js.str();
    if (p->work_bytes) {
        hipError_t e = hipMalloc(&p->work.p, p->work_bytes);
        if (e != hipSuccess) {
            delete p;
            return hip_fail(e, "hipMalloc(workspace)");
        }
        p->work.bytes = p->work_bytes;
    }
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        ++ctx->plans;
    }
    *out = p;
    return VKFX_OK;
}

int vkfx_plan_destroy(vkfx_plan* plan) {
    if (!plan) return VKFX_OK;
    {
        std::lock_guard<std::mutex> lock(plan->ctx->mu);
        if (plan->tickets)
            return fail(VKFX_ERR_NATIVE_RUNTIME, "cannot destroy a plan while " + std::to_string(plan->tickets) +
                                                     " of its ticket(s) are alive; destroy them first");
        --plan->ctx->plans;
    }
    (void)hipSetDevice(plan->ctx->device);
    (void)hipStreamSynchronize(plan->ctx->stream);
    if (plan->aux) {
        (void)hipStreamSynchronize(plan->aux);
        (void)hipStreamDestroy(plan->aux);
    }
    if (plan->ev_fork) (void)hipEventDestroy(plan->ev_fork);
    if (plan->ev_join) (void)hipEventDestroy(plan->ev_join);
    for (hipEvent_t e : plan->timing.ev) (void)hipEventDestroy(e);
    delete plan;
    return VKFX_OK;
}

int vkfx_plan_resources(const vkfx_plan* plan, vkfx_pass_resources* out, uint32_t capacity, uint32_t* count) {
    if (!plan || !count || (capacity && !out)) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    (void)hipSetDevice(plan->ctx->device);
    const int prec =
        (plan->desc.precision == VKFX_F64 || plan->desc.precision == VKFX_F64_COMPUTE_F32_STORAGE) ? 1 : 0;
    std::vector<std::pair<std::string, const void*>> seen;
    uint32_t n = 0;
    for (const Launch& L : plan->launches) {
        const void* fn = nullptr;
        unsigned block = 256;
        size_t lds = 0;
        if (L.boundary) {
            fn = boundary_kernel_fn(L.ba.src_type, L.ba.dst_type);
        } else if (L.r2r) {
            fn = r2r_kernel_fn(L.r2r == 1, prec);
        } else if (L.conv) {
            fn = conv_kernel_fn(prec);
        } else if (L.copy) {
            fn = copy_kernel_fn();
        } else {
            fn = fft_kernel_fn(L.kind, prec, L.dir, L.fixed, L.a.flags);
            block = L.block;
            lds = L.lds;
        }
        if (!fn) return fail(VKFX_ERR_NATIVE_RUNTIME, "no device function for pass " + L.label);
        bool dup = false;
        for (const auto& s : seen) dup = dup || (s.first == L.label && s.second == fn);
        if (dup) continue;
        seen.emplace_back(L.label, fn);
        if (n < capacity) {
            hipFuncAttributes attr{};
            hipError_t e = hipFuncGetAttributes(&attr, fn);
            if (e != hipSuccess) return hip_fail(e, "hipFuncGetAttributes");
            if (lds > 65536) {
                e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute");
            }
            int blocks = 0;
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, (int)block, lds);
            if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
            vkfx_pass_resources& r = out[n];
            std::memset(&r, 0, sizeof r);
            std::snprintf(r.pass, sizeof r.pass, "%s", L.label.c_str());
            r.registers_per_thread = (uint32_t)attr.numRegs;
            r.static_shared_bytes = (uint32_t)attr.sharedSizeBytes;
            r.dynamic_shared_bytes = (uint32_t)lds;
            r.local_bytes_per_thread = (uint32_t)attr.localSizeBytes;
            r.max_threads_per_block = (uint32_t)attr.maxThreadsPerBlock;
            r.block_threads = block;
            r.resident_blocks_per_cu = (uint32_t)blocks;
            r.waves_per_cu = (uint32_t)blocks * ((block + 63) / 64);
        }
        ++n;
    }
    *count = n;
    return VKFX_OK;
}

int vkfx_plan_timing_start(vkfx_plan* plan, uint32_t max_launches) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (max_launches == 0 || max_launches > (1u << 20))
        return fail(VKFX_ERR_INVALID_ARGUMENT, "max_launches must be in [1, 2^20]");
    (void)hipSetDevice(plan->ctx->device);
    auto& tm = plan->timing;
    while (tm.ev.size() < 2 * (size_t)max_launches) {
        hipEvent_t e = nullptr;
        hipError_t r = hipEventCreate(&e);  // default flags: timing enabled
        if (r != hipSuccess) return hip_fail(r, "hipEventCreate(timing)");
        tm.ev.push_back(e);
    }
    tm.launch.assign(max_launches, -1);
    tm.cap = max_launches;
    tm.used = 0;
    tm.armed = true;
    return VKFX_OK;
}

int vkfx_plan_timing_stop(vkfx_plan* plan, vkfx_pass_timing* out, uint32_t capacity, uint32_t* count) {
    if (!plan || !count || (capacity && !out)) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    auto& tm = plan->timing;
    if (!tm.armed) return fail(VKFX_ERR_INVALID_ARGUMENT, "plan timing was not started");
    tm.armed = false;
    (void)hipSetDevice(plan->ctx->device);
    std::vector<vkfx_pass_timing> recs;
    for (size_t i = 0; i < tm.used; ++i) {
        hipError_t r = hipEventSynchronize(tm.ev[2 * i + 1]);
        float ms = 0.f;
        if (r == hipSuccess) r = hipEventElapsedTime(&ms, tm.ev[2 * i], tm.ev[2 * i + 1]);
        if (r != hipSuccess) return hip_fail(r, "hipEventElapsedTime(timing)");
        const Launch& L = plan->launches[(size_t)tm.launch[i]];
        vkfx_pass_timing* rec = nullptr;
        for (auto& x : recs)
            if (L.label == x.pass && (uint32_t)L.a.N == x.fft_len && (uint64_t)L.a.nlines == x.lines) rec = &x;
        if (!rec) {
            recs.emplace_back();
            rec = &recs.back();
            std::memset(rec, 0, sizeof *rec);
            std::snprintf(rec->pass, sizeof rec->pass, "%s", L.label.c_str());
            rec->fft_len = (uint32_t)L.a.N;
            rec->lines = (uint64_t)L.a.nlines;
            rec->min_ms = ms;
            rec->max_ms = ms;
        }
        rec->launches += 1;
        rec->total_ms += ms;
        rec->min_ms = std::min(rec->min_ms, (double)ms);
        rec->max_ms = std::max(rec->max_ms, (double)ms);
    }
    tm.used = 0;
    for (size_t i = 0; i < recs.size() && i < capacity; ++i) out[i] = recs[i];
    *count = (uint32_t)recs.size();
    return VKFX_OK;
}

int vkfx_plan_output_info(const vkfx_plan* plan, int32_t* real_output, uint64_t* widened_bytes) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (real_output) *real_output = plan->real_out ? 1 : 0;
    if (widened_bytes) *widened_bytes = plan->real_out ? 2 * plan->out_bytes : plan->out_bytes;
    return VKFX_OK;
}

int vkfx_plan_io_bytes(const vkfx_plan* plan, uint64_t* in_bytes, uint64_t* out_bytes) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (in_bytes) *in_bytes = plan->in_bytes;
    if (out_bytes) *out_bytes = plan->out_bytes;
    return VKFX_OK;
}

int vkfx_plan_workspace_bytes(const vkfx_plan* plan, uint64_t* out) {
    if (!plan || !out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    *out = plan->work_bytes;
    return VKFX_OK;
}

int vkfx_plan_describe(const vkfx_plan* plan, char* buf, size_t cap) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (buf && cap) {
        const size_t n = std::min(cap - 1, plan->json.size());
        std::memcpy(buf, plan->json.data(), n);
        buf[n] = 0;
    }
    return (int)plan->json.size();
}

int vkfx_execute(vkfx_plan* plan, const void* d_in, void* d_out, void* d_work, void* stream) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (!d_in || !d_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null device buffer");
    if ((plan->desc.transform == VKFX_R2C || plan->desc.transform == VKFX_C2R) && d_in == d_out)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "R2C/C2R cannot run in place");
    if (d_in == d_out && plan->in_bytes != plan->out_bytes)
        return fail(VKFX_ERR_INVALID_ARGUMENT, "in-place execution needs equal input and output sizes");
    void* work = d_work ? d_work : plan->work.p;
    if (plan->work_bytes && !work) return fail(VKFX_ERR_INVALID_ARGUMENT, "plan needs a workspace");
    hipStream_t s = stream ? (hipStream_t)stream : plan->ctx->stream;
    (void)hipSetDevice(plan->ctx->device);
    const int prec =
        (plan->desc.precision == VKFX_F64 || plan->desc.precision == VKFX_F64_COMPUTE_F32_STORAGE) ? 1 : 0;
    hipStream_t lane_stream[2] = {s, plan->aux};
    if (plan->lanes == 2) {
        // fork: the aux lane starts after everything already queued on s
        hipError_t e = hipEventRecord(plan->ev_fork, s);
        if (e == hipSuccess) e = hipStreamWaitEvent(plan->aux, plan->ev_fork, 0);
        if (e != hipSuccess) return hip_fail(e, "stream fork");
    }
    for (size_t li = 0; li < plan->launches.size(); ++li) {
        const Launch& L = plan->launches[li];
        const int lane = plan->lanes == 2 ? (L.chunk & 1) : 0;
        KArgs a = L.a;
        auto sel = [&](int which, size_t off) -> char* {
            char* base = which == SEL_IN             ? (char*)d_in
                         : which == SEL_OUT          ? (char*)d_out
                         : which == SEL_STAGE_IN     ? (char*)work + plan->stage_in_off
                         : which == SEL_STAGE_OUT    ? (char*)work + plan->stage_out_off
                         : which == SEL_FULL         ? (char*)work + plan->full_off
                         : which == SEL_AUX          ? (char*)work + plan->aux_off
                         : which == SEL_CONV_A       ? (char*)work + plan->conv_a_off
                         : which == SEL_CONV_B       ? (char*)work + plan->conv_b_off
                                                     : (char*)work + (size_t)lane * plan->work_lane;
            return base + off;
        };
        if (L.conv) {
            int e = launch_conv(prec, L.ca, sel(L.in_sel, 0), L.conv_kernel, sel(L.out_sel, 0), lane_stream[lane]);
            if (e != hipSuccess) return hip_fail((hipError_t)e, ("launch " + L.label).c_str());
            continue;
        }
        if (L.r2r) {
            int e = launch_r2r(L.r2r == 1, prec, L.ra, sel(L.in_sel, 0), sel(L.out_sel, 0), lane_stream[lane]);
            if (e != hipSuccess) return hip_fail((hipError_t)e, ("launch " + L.label).c_str());
            continue;
        }
        if (L.boundary) {
            int e = launch_boundary(L.ba, sel(L.in_sel, 0), sel(L.out_sel, 0), lane_stream[lane]);
            if (e != hipSuccess) return hip_fail((hipError_t)e, ("launch " + L.label).c_str());
            continue;
        }
        if (L.copy) {
            int e = launch_copy(sel(L.in_sel, L.in_off), sel(L.out_sel, L.out_off), L.copy_bytes, lane_stream[lane]);
            if (e != hipSuccess) return hip_fail((hipError_t)e, ("launch " + L.label).c_str());
            continue;
        }
        a.in = sel(L.in_sel, L.in_off);
        a.out = sel(L.out_sel, L.out_off);
        hipEvent_t t0 = nullptr, t1 = nullptr;
        auto& tm = plan->timing;
        if (tm.armed && tm.used < tm.cap) {
            t0 = tm.ev[2 * tm.used];
            t1 = tm.ev[2 * tm.used + 1];
            tm.launch[tm.used++] = (int)li;
        }
        int e = launch(L.kind, prec, L.dir, a, L.grid, L.block, L.lds, lane_stream[lane], L.fixed, t0, t1);
        if (e != hipSuccess) return hip_fail((hipError_t)e, ("launch " + L.label).c_str());
    }
    if (plan->lanes == 2) {
        // join: s continues only after the aux lane's work
        hipError_t e = hipEventRecord(plan->ev_join, plan->aux);
        if (e == hipSuccess) e = hipStreamWaitEvent(s, plan->ev_join, 0);
        if (e != hipSuccess) return hip_fail(e, "stream join");
    }
    return VKFX_OK;
}

int vkfx_execute_noalloc(vkfx_plan* plan, const void* d_in, void* d_out, void* stream) {
    if (!plan) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan");
    if (plan->work_bytes > vkfx::kStaticScratchBytes)
        return fail(VKFX_ERR_RESOURCE_LIMIT, "plan workspace of " + std::to_string(plan->work_bytes) +
                                                 " bytes exceeds the static scratch of " +
                                                 std::to_string(vkfx::kStaticScratchBytes) +
                                                 " bytes; use vkfx_execute with a workspace");
    if (plan->work_bytes && !plan->ctx->scratch)
        return hip_fail(plan->ctx->scratch_err, "hipGetSymbolAddress(static scratch)");
    // the plan's passes write every scratch element before reading it, so
    // the array needs no clearing between calls
    return vkfx_execute(plan, d_in, d_out, plan->work_bytes ? plan->ctx->scratch : nullptr, stream);
}

int vkfx_execute_host(vkfx_plan* plan, const void* h_in, uint64_t in_bytes, void* h_out, uint64_t out_bytes) {
    if (!plan || !h_in || !h_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    if (in_bytes != plan->in_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "InputLengthMismatch: expected " + std::to_string(plan->in_bytes) +
                                                        " bytes, got " + std::to_string(in_bytes));
    if (out_bytes != plan->out_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "output buffer: expected " + std::to_string(plan->out_bytes) +
                                                        " bytes, got " + std::to_string(out_bytes));
    (void)hipSetDevice(plan->ctx->device);
    hipStream_t s = plan->ctx->stream;
    auto ensure = [&](DevBuf& b, size_t bytes) -> int {
        if (b.bytes >= bytes && b.p) return VKFX_OK;
        if (b.p) (void)hipFree(b.p);
        b.p = nullptr;
        b.bytes = 0;
        hipError_t e = hipMalloc(&b.p, bytes ? bytes : 16);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(staging)");
        b.bytes = bytes;
        return VKFX_OK;
    };
    int rc = ensure(plan->host_in, plan->in_bytes);
    if (!rc) rc = ensure(plan->host_out, plan->out_bytes);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(plan->host_in.p, h_in, in_bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(H2D)");
    rc = vkfx_execute(plan, plan->host_in.p, plan->host_out.p, nullptr, s);
    if (rc) return rc;
    e = hipMemcpyAsync(h_out, plan->host_out.p, out_bytes, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(D2H)");
    e = hipStreamSynchronize(s);
    return e == hipSuccess ? VKFX_OK : hip_fail(e, "hipStreamSynchronize");
}

int vkfx_planner_axis(uint64_t len, uint64_t batch, int32_t precision, int32_t axis_is_strided,
                      int32_t allow_recursive_rader, uint64_t shared_memory_bytes, int32_t* algorithm,
                      uint64_t* convolution_len) {
    if (!algorithm || !convolution_len) return fail(VKFX_ERR_INVALID_ARGUMENT, "null output");
    if (len == 0) return fail(VKFX_ERR_INVALID_ARGUMENT, "ZeroLength");
    try {
        const bool f64 = precision == VKFX_F64 || precision == VKFX_F64_COMPUTE_F32_STORAGE;
        AxisDecision d = plan_c2c_axis(len, batch ? batch : 1, f64, axis_is_strided != 0,
                                       tuning_for_amd(f64, allow_recursive_rader != 0),
                                       planner_device(shared_memory_bytes));
        *algorithm = (int32_t)d.algorithm;
        *convolution_len = d.convolution_len;
    } catch (const std::exception& ex) {
        return fail(VKFX_ERR_INVALID_ARGUMENT, ex.what());
    }
    return VKFX_OK;
}

int vkfx_planner_axis_tuned(uint64_t len, uint64_t batch, int32_t precision, int32_t axis_is_strided,
                            const vkfx_planner_tuning* tuning, uint64_t shared_memory_bytes, int32_t* algorithm,
                            uint64_t* convolution_len) {
    if (!algorithm || !convolution_len) return fail(VKFX_ERR_INVALID_ARGUMENT, "null output");
    if (len == 0) return fail(VKFX_ERR_INVALID_ARGUMENT, "ZeroLength");
    try {
        const bool f64 = precision == VKFX_F64 || precision == VKFX_F64_COMPUTE_F32_STORAGE;
        const PlannerTuning t = tuning ? tuning_from(*tuning) : tuning_for_amd(f64);
        AxisDecision d = plan_c2c_axis(len, batch ? batch : 1, f64, axis_is_strided != 0, t,
                                       planner_device(shared_memory_bytes));
        *algorithm = (int32_t)d.algorithm;
        *convolution_len = d.convolution_len;
    } catch (const std::exception& ex) {
        return fail(VKFX_ERR_INVALID_ARGUMENT, ex.what());
    }
    return VKFX_OK;
}

int vkfx_planner_bluestein_padding(uint64_t len, uint64_t batch, int32_t precision, uint64_t shared_memory_bytes,
                                   uint64_t* padded) {
    if (!padded) return fail(VKFX_ERR_INVALID_ARGUMENT, "null output");
    if (len < 2) return fail(VKFX_ERR_INVALID_ARGUMENT, "Bluestein length must be >= 2");
    try {
        *padded = bluestein_auto_padding(len, batch ? batch : 1,
                                         precision == VKFX_F64 || precision == VKFX_F64_COMPUTE_F32_STORAGE,
                                         planner_device(shared_memory_bytes));
    } catch (const std::exception& ex) {
        return fail(VKFX_ERR_INVALID_ARGUMENT, ex.what());
    }
    return VKFX_OK;
}

uint64_t vkfx_planner_next_smooth(uint64_t target) {
    try {
        return next_smooth_at_least(target, {2, 3, 5, 7});
    } catch (...) {
        return 0;
    }
}

}  // extern "C"

// ---- async tickets and device-resident chains -------------------------------

namespace {

// Takes a pooled buffer of exactly `bytes` (device or pinned host), or
// allocates one. When `s` is given and the buffer carries a release event,
// s waits on it before the buffer is touched.
int pool_take(vkfx_context* ctx, bool host, size_t bytes, hipStream_t s, PoolBuf* out) {
    std::lock_guard<std::mutex> lock(ctx->mu);
    std::vector<PoolBuf>& pool = host ? ctx->host_pool : ctx->dev_pool;
    for (size_t i = 0; i < pool.size(); ++i) {
        if (pool[i].bytes != bytes) continue;
        *out = pool[i];
        pool.erase(pool.begin() + (long)i);
        if (out->ready) {
            hipError_t e = s ? hipStreamWaitEvent(s, out->ready, 0) : hipEventSynchronize(out->ready);
            if (e != hipSuccess) return hip_fail(e, "pool buffer wait");
        }
        return VKFX_OK;
    }
    PoolBuf b;
    b.bytes = bytes;
    hipError_t e = host ? hipHostMalloc(&b.p, bytes ? bytes : 16, hipHostMallocDefault)
                        : hipMalloc(&b.p, bytes ? bytes : 16);
    if (e != hipSuccess) return hip_fail(e, host ? "hipHostMalloc" : "hipMalloc");
    *out = b;
    return VKFX_OK;
}

// Returns a buffer to its pool; with a stream, its release event is recorded
// there so the next user waits for the work already queued on it.
void pool_give(vkfx_context* ctx, bool host, PoolBuf b, hipStream_t s) {
    if (!b.p) return;
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (s) {
        if (!b.ready && hipEventCreateWithFlags(&b.ready, hipEventDisableTiming) != hipSuccess) b.ready = nullptr;
        if (b.ready && hipEventRecord(b.ready, s) != hipSuccess) {
            (void)hipStreamSynchronize(s);
        }
        if (!b.ready) (void)hipStreamSynchronize(s);
    }
    (host ? ctx->host_pool : ctx->dev_pool).push_back(b);
}

int chain_check(vkfx_plan* const* plans, uint32_t count) {
    if (!plans || count == 0) return fail(VKFX_ERR_INVALID_ARGUMENT, "resident chain requires at least one plan");
    for (uint32_t i = 0; i < count; ++i) {
        if (!plans[i]) return fail(VKFX_ERR_INVALID_ARGUMENT, "null plan in chain");
        if (plans[i]->ctx != plans[0]->ctx) return fail(VKFX_ERR_INVALID_ARGUMENT, "chain plans span contexts");
        if (i + 1 < count && plans[i]->out_bytes != plans[i + 1]->in_bytes)
            return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH,
                        "resident chain transition " + std::to_string(i) + ": output " +
                            std::to_string(plans[i]->out_bytes) + " bytes, next input " +
                            std::to_string(plans[i + 1]->in_bytes) + " bytes");
    }
    return VKFX_OK;
}

// Runs the chain on s; intermediates come from the device pool and go back
// with release events recorded on s.
int chain_run(vkfx_plan* const* plans, uint32_t count, const void* d_in, void* d_out, hipStream_t s) {
    vkfx_context* ctx = plans[0]->ctx;
    PoolBuf tmp[2];
    const void* cur = d_in;
    int rc = VKFX_OK;
    for (uint32_t i = 0; i < count && !rc; ++i) {
        void* dst = d_out;
        if (i + 1 < count) {
            PoolBuf& t = tmp[i & 1];
            if (t.p && t.bytes != plans[i]->out_bytes) {
                pool_give(ctx, false, t, s);
                t = PoolBuf();
            }
            if (!t.p) rc = pool_take(ctx, false, plans[i]->out_bytes, s, &t);
            if (rc) break;
            dst = t.p;
        }
        rc = vkfx_execute(plans[i], cur, dst, nullptr, s);
        cur = dst;
    }
    for (PoolBuf& t : tmp) pool_give(ctx, false, t, s);
    return rc;
}

}  // namespace

struct vkfx_ticket {
    vkfx_plan* plan = nullptr;
    vkfx_context* ctx = nullptr;
    size_t out_bytes = 0;   // the plan's output bytes, copied at submit
    bool real_out = false;  // the plan's output holds reals
    size_t scalar_bytes = 0;
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;
    PoolBuf d_in, d_out, d_work, h_in, h_out;
};

int vkfx_submit_host(vkfx_plan* plan, const void* h_in, uint64_t in_bytes, vkfx_ticket** out) {
    if (!plan || !h_in || !out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (in_bytes != plan->in_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "InputLengthMismatch: expected " + std::to_string(plan->in_bytes) +
                                                        " bytes, got " + std::to_string(in_bytes));
    vkfx_context* ctx = plan->ctx;
    (void)hipSetDevice(ctx->device);
    auto* t = new vkfx_ticket();
    t->plan = plan;
    t->ctx = ctx;
    t->out_bytes = plan->out_bytes;
    t->real_out = plan->real_out;
    t->scalar_bytes = storage_scalar_bytes(plan->desc.precision);
    auto cleanup = [&](int rc) {
        if (t->stream) (void)hipStreamSynchronize(t->stream);
        pool_give(ctx, false, t->d_in, nullptr);
        pool_give(ctx, false, t->d_out, nullptr);
        pool_give(ctx, false, t->d_work, nullptr);
        pool_give(ctx, true, t->h_in, nullptr);
        pool_give(ctx, true, t->h_out, nullptr);
        if (t->stream) {
            std::lock_guard<std::mutex> lock(ctx->mu);
            ctx->stream_pool.push_back(t->stream);
        }
        if (t->done) (void)hipEventDestroy(t->done);
        delete t;
        return rc;
    };
    hipError_t e = hipSuccess;
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        if (!ctx->stream_pool.empty()) {
            t->stream = ctx->stream_pool.back();
            ctx->stream_pool.pop_back();
        }
    }
    if (!t->stream) {
        e = hipStreamCreate(&t->stream);  // default priority
        if (e != hipSuccess) {
            t->stream = nullptr;
            return cleanup(hip_fail(e, "hipStreamCreate"));
        }
    }
    e = hipEventCreateWithFlags(&t->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        t->done = nullptr;
        return cleanup(hip_fail(e, "hipEventCreate"));
    }
    int rc = pool_take(ctx, false, plan->in_bytes, t->stream, &t->d_in);
    if (!rc) rc = pool_take(ctx, false, plan->out_bytes, t->stream, &t->d_out);
    if (!rc && plan->work_bytes) rc = pool_take(ctx, false, plan->work_bytes, t->stream, &t->d_work);
    if (!rc) rc = pool_take(ctx, true, plan->in_bytes, nullptr, &t->h_in);
    if (!rc) rc = pool_take(ctx, true, plan->out_bytes, nullptr, &t->h_out);
    if (rc) return cleanup(rc);
    std::memcpy(t->h_in.p, h_in, in_bytes);
    e = hipMemcpyAsync(t->d_in.p, t->h_in.p, in_bytes, hipMemcpyHostToDevice, t->stream);
    if (e != hipSuccess) return cleanup(hip_fail(e, "hipMemcpyAsync(H2D)"));
    rc = vkfx_execute(plan, t->d_in.p, t->d_out.p, t->d_work.p, t->stream);
    if (rc) return cleanup(rc);
    e = hipMemcpyAsync(t->h_out.p, t->d_out.p, plan->out_bytes, hipMemcpyDeviceToHost, t->stream);
    if (e == hipSuccess) e = hipEventRecord(t->done, t->stream);
    if (e != hipSuccess) return cleanup(hip_fail(e, "ticket enqueue"));
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        ++ctx->active;
        ++plan->tickets;
    }
    *out = t;
    return VKFX_OK;
}

int vkfx_ticket_ready(const vkfx_ticket* t, int32_t* ready) {
    if (!t || !ready) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    hipError_t e = hipEventQuery(t->done);
    if (e == hipSuccess) {
        *ready = 1;
        return VKFX_OK;
    }
    if (e == hipErrorNotReady) {
        *ready = 0;
        return VKFX_OK;
    }
    return hip_fail(e, "hipEventQuery");
}

int vkfx_ticket_wait(vkfx_ticket* t, void* h_out, uint64_t out_bytes) {
    if (!t || !h_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    if (out_bytes != t->out_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "output buffer: expected " + std::to_string(t->out_bytes) +
                                                        " bytes, got " + std::to_string(out_bytes));
    hipError_t e = hipEventSynchronize(t->done);
    if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    std::memcpy(h_out, t->h_out.p, out_bytes);
    return VKFX_OK;
}

int vkfx_ticket_wait_complex(vkfx_ticket* t, void* h_out, uint64_t out_bytes) {
    if (!t || !h_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    if (!t->real_out) return vkfx_ticket_wait(t, h_out, out_bytes);
    if (out_bytes != 2 * t->out_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "complex-widened output buffer: expected " +
                                                        std::to_string(2 * t->out_bytes) + " bytes, got " +
                                                        std::to_string(out_bytes));
    hipError_t e = hipEventSynchronize(t->done);
    if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    // {v, 0} per real value, in the storage scalar type
    const size_t sb = t->scalar_bytes, n = t->out_bytes / sb;
    const unsigned char* src = (const unsigned char*)t->h_out.p;
    unsigned char* dst = (unsigned char*)h_out;
    for (size_t i = 0; i < n; ++i) {
        std::memcpy(dst + 2 * i * sb, src + i * sb, sb);
        std::memset(dst + (2 * i + 1) * sb, 0, sb);
    }
    return VKFX_OK;
}

int vkfx_ticket_destroy(vkfx_ticket* t) {
    if (!t) return VKFX_OK;
    vkfx_context* ctx = t->ctx;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(t->stream);
    pool_give(ctx, false, t->d_in, nullptr);
    pool_give(ctx, false, t->d_out, nullptr);
    pool_give(ctx, false, t->d_work, nullptr);
    pool_give(ctx, true, t->h_in, nullptr);
    pool_give(ctx, true, t->h_out, nullptr);
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        ctx->stream_pool.push_back(t->stream);
        --ctx->active;
        --t->plan->tickets;
    }
    (void)hipEventDestroy(t->done);
    delete t;
    return e == hipSuccess ? VKFX_OK : hip_fail(e, "hipStreamSynchronize");
}

int vkfx_context_cache_stats(vkfx_context* ctx, uint64_t* transient_buffers, uint64_t* pooled_streams,
                             uint64_t* in_flight) {
    if (!ctx) return fail(VKFX_ERR_INVALID_ARGUMENT, "null context");
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (transient_buffers) *transient_buffers = ctx->dev_pool.size() + ctx->host_pool.size();
    if (pooled_streams) *pooled_streams = ctx->stream_pool.size();
    if (in_flight) *in_flight = (uint64_t)ctx->active;
    return VKFX_OK;
}

int vkfx_context_clear_caches(vkfx_context* ctx) {
    if (!ctx) return fail(VKFX_ERR_INVALID_ARGUMENT, "null context");
    std::lock_guard<std::mutex> lock(ctx->mu);
    if (ctx->active)
        return fail(VKFX_ERR_NATIVE_RUNTIME, "cannot clear HIP runtime caches while " + std::to_string(ctx->active) +
                                                 " submission(s) are in flight");
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    for (PoolBuf& b : ctx->dev_pool) {
        if (b.ready) (void)hipEventDestroy(b.ready);
        e = hipFree(b.p);
        if (e != hipSuccess) return hip_fail(e, "hipFree");
    }
    ctx->dev_pool.clear();
    for (PoolBuf& b : ctx->host_pool) {
        if (b.ready) (void)hipEventDestroy(b.ready);
        e = hipHostFree(b.p);
        if (e != hipSuccess) return hip_fail(e, "hipHostFree");
    }
    ctx->host_pool.clear();
    for (hipStream_t s : ctx->stream_pool) {
        (void)hipStreamSynchronize(s);
        (void)hipStreamDestroy(s);
    }
    ctx->stream_pool.clear();
    return VKFX_OK;
}

int vkfx_execute_chain(vkfx_plan* const* plans, uint32_t count, const void* d_in, void* d_out, void* stream) {
    int rc = chain_check(plans, count);
    if (rc) return rc;
    if (!d_in || !d_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null device buffer");
    vkfx_context* ctx = plans[0]->ctx;
    (void)hipSetDevice(ctx->device);
    return chain_run(plans, count, d_in, d_out, stream ? (hipStream_t)stream : ctx->stream);
}

int vkfx_execute_chain_host(vkfx_plan* const* plans, uint32_t count, const void* h_in, uint64_t in_bytes,
                            void* h_out, uint64_t out_bytes) {
    int rc = chain_check(plans, count);
    if (rc) return rc;
    if (!h_in || !h_out) return fail(VKFX_ERR_INVALID_ARGUMENT, "null argument");
    if (in_bytes != plans[0]->in_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "InputLengthMismatch: expected " +
                                                        std::to_string(plans[0]->in_bytes) + " bytes, got " +
                                                        std::to_string(in_bytes));
    if (out_bytes != plans[count - 1]->out_bytes)
        return fail(VKFX_ERR_INPUT_LENGTH_MISMATCH, "output buffer: expected " +
                                                        std::to_string(plans[count - 1]->out_bytes) +
                                                        " bytes, got " + std::to_string(out_bytes));
    vkfx_context* ctx = plans[0]->ctx;
    (void)hipSetDevice(ctx->device);
    hipStream_t s = ctx->stream;
    PoolBuf din, dout;
    rc = pool_take(ctx, false, in_bytes, s, &din);
    if (!rc) rc = pool_take(ctx, false, out_bytes, s, &dout);
    hipError_t e = hipSuccess;
    if (!rc) {
        e = hipMemcpyAsync(din.p, h_in, in_bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(H2D)");
    }
    if (!rc) rc = chain_run(plans, count, din.p, dout.p, s);
    if (!rc) {
        e = hipMemcpyAsync(h_out, dout.p, out_bytes, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(D2H)");
    }
    e = hipStreamSynchronize(s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    pool_give(ctx, false, din, nullptr);
    pool_give(ctx, false, dout, nullptr);
    return rc;
}
