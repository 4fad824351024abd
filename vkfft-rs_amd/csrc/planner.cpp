// planner.cpp -- restatement of the vkfft-rs planner decisions this path
// consumes (paths relative to the vkfft-rs repository root). The Bluestein
// padding tables are data of the reference planner and must stay identical.
#include "planner.hpp"

#include <algorithm>
#include <climits>
#include <stdexcept>

namespace vkfx {

std::vector<size_t> prime_factorization(size_t value) {
    std::vector<size_t> f;
    if (value < 2) return f;
    while (value % 2 == 0) {
        f.push_back(2);
        value /= 2;
    }
    for (size_t d = 3; d <= value / d; d += 2)
        while (value % d == 0) {
            f.push_back(d);
            value /= d;
        }
    if (value > 1) f.push_back(value);
    return f;
}

bool is_smooth(size_t value, const std::vector<size_t>& primes) {
    if (value == 0) return false;
    for (size_t p : primes)
        while (value % p == 0) value /= p;
    return value == 1;
}

static void smooth_visit(const std::vector<size_t>& p, size_t idx, size_t cur, size_t target, size_t& best) {
    if (cur >= best) return;
    if (idx == p.size()) {
        if (cur >= target) best = cur;
        return;
    }
    size_t value = cur;
    for (;;) {
        smooth_visit(p, idx + 1, value, target, best);
        if (value > SIZE_MAX / p[idx]) break;
        size_t next = value * p[idx];
        if (next < best)
            value = next;
        else
            break;
    }
}

size_t next_smooth_at_least(size_t target, const std::vector<size_t>& primes) {
    if (target <= 1) return 1;
    std::vector<size_t> ord = primes;
    std::sort(ord.begin(), ord.end());
    ord.erase(std::unique(ord.begin(), ord.end()), ord.end());
    if (ord.empty() || ord[0] < 2) throw std::invalid_argument("smooth-number prime set must contain values >= 2");
    size_t best = SIZE_MAX;
    if (ord[0] == 2) {
        size_t p2 = 1;
        while (p2 < target && p2 <= SIZE_MAX / 2) p2 <<= 1;
        if (p2 >= target) best = p2;
    }
    smooth_visit(ord, 0, 1, target, best);
    if (best == SIZE_MAX) throw std::overflow_error("smooth convolution length");
    return best;
}

static size_t mod_pow(size_t base, size_t e, size_t m) {
    unsigned __int128 r = 1, b = base % m;
    while (e) {
        if (e & 1) r = (r * b) % m;
        b = (b * b) % m;
        e >>= 1;
    }
    return (size_t)r;
}

size_t primitive_root(size_t prime) {
    if (prime == 2) return 1;
    if (prime < 2 || prime_factorization(prime).size() != 1) return 0;
    size_t phi = prime - 1;
    std::vector<size_t> u = prime_factorization(phi);
    u.erase(std::unique(u.begin(), u.end()), u.end());
    for (size_t g = 2; g < prime; ++g) {
        bool ok = true;
        for (size_t f : u)
            if (mod_pow(g, phi / f, prime) == 1) {
                ok = false;
                break;
            }
        if (ok) return g;
    }
    return 0;
}

PlannerTuning tuning_for_amd(bool f64, bool allow_recursive_rader) {
    // PlannerTuning::for_device (src/config.rs:395-420), AMD vendor branch.
    PlannerTuning t;
    t.max_rader_direct_prime = 89;
    t.min_rader_fft_prime = f64 ? 29 : 17;
    t.allow_recursive_fft_rader = allow_recursive_rader;
    return t;
}

// ------------------------------------------------ register-schedule quality

namespace {
constexpr int kRadixTable = 33;  // VKFFT_RADIX_TABLE_LEN
using Table = size_t[kRadixTable];

// optimize_radix_kernels with register_boost = 1 (scheduler.rs:10639-10798).
void optimize_radix_kernels(Table& reg, Table& mul) {
    if ((reg[32] > 0 || reg[2] % 32 == 0) && reg[32] % 32 == 0 && mul[2] >= 5) {
        mul[32] = mul[2] / 5;
        mul[2] -= mul[32] * 5;
        if (reg[2] % 32 == 0) reg[32] = reg[2];
    }
    if ((reg[16] > 0 || reg[2] % 16 == 0) && reg[16] % 16 == 0 && mul[2] >= 4) {
        mul[16] = mul[2] / 4;
        mul[2] -= mul[16] * 4;
        if (reg[2] % 16 == 0) reg[16] = reg[2];
    }
    if (reg[15] > 0 && reg[15] % 15 == 0 && mul[3] >= 1 && mul[5] >= 1) {
        mul[15] = std::min(mul[3], mul[5]);
        mul[3] -= mul[15];
        mul[5] -= mul[15];
    }
    if (reg[14] > 0 && reg[14] % 14 == 0 && mul[2] >= 1 && mul[7] >= 1) {
        mul[14] = std::min(mul[2], mul[7]);
        mul[2] -= mul[14];
        mul[7] -= mul[14];
    }
    if (reg[12] > 0 && reg[12] % 12 == 0 && mul[2] >= 2 && mul[3] >= 1) {
        mul[12] = std::min(mul[3], mul[2] / 2);
        mul[2] -= 2 * mul[12];
        mul[3] -= mul[12];
    }
    if (reg[10] > 0 && reg[10] % 10 == 0 && mul[2] >= 1 && mul[5] >= 1) {
        mul[10] = std::min(mul[2], mul[5]);
        mul[2] -= mul[10];
        mul[5] -= mul[10];
    }
    if (reg[9] > 0 && reg[9] % 9 == 0 && mul[3] >= 2) {
        mul[9] = mul[3] / 2;
        mul[3] -= mul[9] * 2;
    }
    if ((reg[8] > 0 || reg[2] % 8 == 0) && reg[8] % 8 == 0 && mul[2] >= 3) {
        mul[8] = mul[2] / 3;
        mul[2] -= mul[8] * 3;
        if (reg[2] % 8 == 0) reg[8] = reg[2];
    }
    if (reg[6] > 0 && reg[6] % 6 == 0 && mul[2] >= 1 && mul[3] >= 1) {
        mul[6] = std::min(mul[2], mul[3]);
        mul[2] -= mul[6];
        mul[3] -= mul[6];
    }
    if ((reg[4] > 0 || reg[2] % 4 == 0) && reg[4] % 4 == 0 && mul[2] >= 2) {
        mul[4] = mul[2] / 2;
        mul[2] -= mul[4] * 2;
        if (reg[2] % 4 == 0) reg[4] = reg[2];
    }
}

// derive_vkfft_composite_registers (scheduler.rs:10440-10478).
void derive_composites(Table& r) {
    r[32] = r[2] % 32 == 0 ? r[2] : 0;
    r[16] = r[2] % 16 == 0 ? r[2] : 0;
    r[8] = r[2] % 8 == 0 ? r[2] : 0;
    r[4] = r[2] % 4 == 0 ? r[2] : 0;
    if (r[2] >= 12 && r[3] >= 12) {
        size_t v = std::min(r[2], r[3]);
        r[12] = v % 12 == 0 ? v : 0;
    } else {
        r[12] = 0;
    }
    r[6] = std::min(r[2], r[3]);
    r[9] = r[3] % 9 == 0 ? r[3] : 0;
    r[10] = std::min(r[2], r[5]);
    r[14] = std::min(r[2], r[7]);
    r[15] = std::min(r[3], r[5]);
}

// The shared tail: optimize, list stages, min/max register demand
// (finalize_mixed_radix_register_schedule, min_max_stage_registers).
bool finalize_is_good(Table& reg, Table& mul) {
    optimize_radix_kernels(reg, mul);
    size_t mx = 0, mn = SIZE_MAX;
    for (int radix = kRadixTable - 1; radix >= 2; --radix)
        if (mul[radix] > 0 && reg[radix] > 0) {
            mx = std::max(mx, reg[radix]);
            mn = std::min(mn, reg[radix]);
        }
    if (mx == 0) throw std::logic_error("mixed-radix scheduler produced no executable stages");
    return !(mx > 16 || mx >= 2 * mn);
}
}  // namespace

bool radix_sequence_is_good(size_t fft_len, size_t rhs) {
    (void)rhs;  // the power-of-two table always yields equal min/max <= 8 registers
    if (fft_len == 0) throw std::invalid_argument("zero length");
    if ((fft_len & (fft_len - 1)) == 0) return true;  // power_of_two_register_table
    const size_t primes[6] = {2, 3, 5, 7, 11, 13};
    size_t ex[6] = {0, 0, 0, 0, 0, 0}, rem = fft_len;
    for (int i = 0; i < 6; ++i)
        while (rem % primes[i] == 0) {
            rem /= primes[i];
            ex[i]++;
        }
    if (rem != 1) throw std::invalid_argument("register schedule needs 2/3/5/7/11/13-smooth length");
    Table reg = {0}, mul = {0};
    for (int i = 0; i < 6; ++i) mul[primes[i]] = ex[i];
    unsigned mask = 0;
    for (int i = 0; i < 6; ++i)
        if (ex[i]) mask |= 1u << i;
    auto is = [&](std::initializer_list<int> idx) {
        unsigned m = 0;
        for (int i : idx) m |= 1u << i;
        return m == mask;
    };
    if (is({0, 1})) {
        // plan_nvidia_vulkan_two_three_radix_registers (scheduler.rs:9882-9988)
        size_t p = (ex[0] == ex[1] || ex[0] == 1) ? 6 : 12;
        reg[2] = reg[3] = p;
        reg[32] = reg[2] % 32 == 0 ? reg[2] : 0;
        reg[16] = reg[2] % 16 == 0 ? reg[2] : 0;
        reg[8] = reg[2] % 8 == 0 ? reg[2] : 0;
        reg[4] = reg[2] % 4 == 0 ? reg[2] : 0;
        if (reg[2] >= 12 && reg[3] >= 12) {
            reg[12] = std::min(reg[2], reg[3]);
            if (reg[12] % 12) reg[12] = 0;
        }
        reg[6] = std::min(reg[2], reg[3]);
        reg[9] = reg[3] % 9 == 0 ? reg[3] : 0;
        return finalize_is_good(reg, mul);
    }
    // plan_nvidia_vulkan_small_mixed_radix_registers (scheduler.rs:10006-10395),
    // the branches reachable by 2/3/5/7/11/13-smooth lengths.
    const size_t e2 = ex[0], e3 = ex[1];
    if (is({1})) reg[3] = e3 == 1 ? 3 : 9;
    else if (is({2})) reg[5] = 5;
    else if (is({3})) reg[7] = 7;
    else if (is({4})) reg[11] = 11;
    else if (is({5})) reg[13] = 13;
    else if (is({0, 2})) { reg[2] = e2 <= 2 ? 10 : 8; reg[5] = 10; }
    else if (is({0, 3})) { if (e2 <= 2) { reg[2] = 14; reg[7] = 14; } else { reg[2] = 8; reg[7] = 7; } }
    else if (is({0, 4})) { reg[2] = e2 == 1 ? 10 : 8; reg[11] = 11; }
    else if (is({0, 5})) { reg[2] = e2 <= 2 ? 12 : 8; reg[13] = 13; }
    else if (is({1, 2})) { reg[3] = 15; reg[5] = 15; }
    else if (is({1, 3})) { reg[3] = e3 == 1 ? 6 : 9; reg[7] = 7; }
    else if (is({1, 4})) { reg[3] = 9; reg[11] = 11; }
    else if (is({1, 5})) { reg[3] = e3 == 1 ? 12 : 9; reg[13] = 13; }
    else if (is({0, 2, 4}) || is({0, 2, 5}) || is({0, 2, 4, 5})) {
        reg[2] = e2 <= 2 ? 10 : 8; reg[5] = 10;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 3, 4}) || is({0, 3, 5}) || is({0, 3, 4, 5})) {
        reg[2] = (e2 == 1 || e2 == 2) ? 14 : e2 == 3 ? 8 : 16; reg[7] = 14;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 4, 5})) {
        reg[2] = e2 <= 2 ? 12 : 8; reg[11] = 11; reg[13] = 13;
    } else if (is({0, 2, 3, 4}) || is({0, 2, 3, 5}) || is({0, 2, 3, 4, 5})) {
        reg[2] = (e2 == 1 || e2 == 2) ? 10 : e2 == 3 ? 8 : 16; reg[5] = 10; reg[7] = 14;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({1, 2, 4}) || is({1, 2, 5}) || is({1, 2, 4, 5})) {
        reg[3] = 15; reg[5] = 15;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({1, 3, 4}) || is({1, 3, 5}) || is({1, 3, 4, 5})) {
        if (e3 == 1) { reg[3] = 12; reg[7] = 14; } else { reg[3] = 9; reg[7] = 7; }
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({1, 4, 5})) {
        reg[3] = e3 == 1 ? 12 : 9; reg[11] = 11; reg[13] = 13;
    } else if (is({1, 2, 3, 4}) || is({1, 2, 3, 5}) || is({1, 2, 3, 4, 5})) {
        reg[3] = 15; reg[5] = 15; reg[7] = 14;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 1, 4, 5})) {
        if (e2 == 1) { reg[2] = 6; reg[3] = 6; } else { reg[2] = 12; reg[3] = 12; }
        reg[11] = 11; reg[13] = 13;
    } else if (is({0, 1, 2, 4}) || is({0, 1, 2, 5}) || is({0, 1, 2, 4, 5})) {
        if (e2 == 1) { reg[2] = 10; reg[3] = 15; } else { reg[2] = 12; reg[3] = 12; }
        reg[5] = 10;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 1, 3, 4}) || is({0, 1, 3, 5}) || is({0, 1, 3, 4, 5})) {
        reg[2] = 12; reg[3] = 12; reg[7] = 14;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 1, 2, 3, 4}) || is({0, 1, 2, 3, 5}) || is({0, 1, 2, 3, 4, 5})) {
        if (e2 == 1) { reg[2] = 14; reg[3] = 15; }
        else if (e2 == 2 || e2 == 3) { reg[2] = 12; reg[3] = 12; }
        else { reg[2] = 16; reg[3] = 12; }
        reg[5] = 15; reg[7] = 14;
        if (ex[4]) reg[11] = 11;
        if (ex[5]) reg[13] = 13;
    } else if (is({0, 1, 2})) {
        if (e2 == 1) { reg[2] = 6; reg[3] = 6; reg[5] = 5; } else { reg[2] = 12; reg[3] = 12; reg[5] = 10; }
    } else if (is({0, 1, 3})) {
        if (e2 <= 2) { reg[2] = 6; reg[3] = 6; reg[7] = 7; } else { reg[2] = 8; reg[3] = 6; reg[7] = 7; }
    } else if (is({0, 1, 4})) {
        if (e2 == 1) { reg[2] = 6; reg[3] = 6; } else { reg[2] = 12; reg[3] = 12; }
        reg[11] = 11;
    } else if (is({0, 1, 5})) {
        if (e2 == 1) { reg[2] = 6; reg[3] = 6; } else { reg[2] = 12; reg[3] = 12; }
        reg[13] = 13;
    } else if (is({0, 2, 3})) {
        reg[2] = e2 <= 2 ? 10 : 8; reg[5] = 10; reg[7] = 7;
    } else if (is({1, 2, 3})) {
        reg[3] = 15; reg[5] = 15; reg[7] = 14;
    } else if (is({0, 1, 2, 3})) {
        if (e2 == 1) { reg[2] = 14; reg[3] = 15; }
        else if (e2 == 2 || e2 == 3) { reg[2] = 12; reg[3] = 12; }
        else { reg[2] = 16; reg[3] = 12; }
        reg[5] = 15; reg[7] = 14;
    } else if ((mask & 1u) == 0 && (mask & 2u) == 0) {
        // every factor index >= 2: one register slot per prime radix
        for (int i = 2; i < 6; ++i)
            if (ex[i]) reg[primes[i]] = primes[i];
    } else {
        throw std::logic_error("register-table dispatch missed a factor subset");
    }
    derive_composites(reg);
    return finalize_is_good(reg, mul);
}

// ------------------------------------------------------------ Bluestein pad

namespace {
struct PadRow {
    size_t threshold, padded;
};
// OTHER_WIDE_BLUESTEIN_AUTO_PADDING (scheduler.rs:121-176): F64 on AMD.
const PadRow kWide[] = {
    {17, 36},     {19, 40},     {23, 56},     {29, 64},     {34, 70},     {37, 78},     {41, 81},
    {43, 90},     {46, 125},    {67, 150},    {76, 175},    {89, 189},    {97, 198},    {101, 243},
    {123, 256},   {129, 270},   {136, 512},   {257, 625},   {314, 640},   {321, 702},   {353, 750},
    {376, 756},   {379, 768},   {386, 875},   {439, 1024},  {513, 1296},  {649, 1300},  {651, 1323},
    {663, 1344},  {673, 1512},  {757, 1792},  {897, 2016},  {1009, 2048}, {1025, 2187}, {1095, 3136},
    {1569, 3159}, {1581, 3430}, {1717, 3584}, {1793, 4096}, {2049, 4224}, {2113, 4375}, {2189, 4480},
    {2241, 4704}, {2353, 4928}, {2465, 4992}, {2497, 5005}, {2504, 5103}, {2553, 5376}, {2689, 5632},
    {2817, 5824}, {2913, 6048}, {3026, 6144}, {3073, 6875}, {3439, 8192},
};
// OTHER_F32_BLUESTEIN_AUTO_PADDING (scheduler.rs:178-208): F32 on AMD.
const PadRow kF32[] = {
    {17, 36},     {19, 42},     {23, 64},     {34, 81},     {43, 88},     {46, 125},    {67, 150},
    {76, 162},    {82, 175},    {89, 256},    {129, 512},   {257, 625},   {314, 768},   {386, 1024},
    {513, 1296},  {649, 2048},  {1025, 2187}, {1095, 2304}, {1153, 2500}, {1251, 2592}, {1297, 3072},
    {1537, 3125}, {1564, 3136}, {1569, 4096}, {2049, 4375}, {2189, 4608}, {2305, 5184}, {2593, 6561},
    {3282, 8192},
};

// upstream_bluestein_auto_padding_from_table (scheduler.rs:244-272).
size_t padding_from_table(size_t len, bool f64) {
    const PadRow* t = f64 ? kWide : kF32;
    const size_t n = f64 ? sizeof(kWide) / sizeof(PadRow) : sizeof(kF32) / sizeof(PadRow);
    const size_t required = len * 2 - 1;
    for (size_t i = 0; i < n; ++i) {
        if (len < t[i].threshold) break;
        if (i + 1 == n || len < t[i + 1].threshold) return required <= t[i].padded ? t[i].padded : 0;
    }
    return 0;
}

size_t next_pow2(size_t v) {
    size_t p = 1;
    while (p < v) p <<= 1;
    return p;
}
}  // namespace

size_t bluestein_auto_padding(size_t len, size_t batch, bool f64, const PlannerDevice& dev) {
    if (size_t p = padding_from_table(len, f64)) return p;
    // upstream_bluestein_generic_padding (scheduler.rs:283-357)
    const size_t required = len * 2 - 1;
    const size_t max_rhs = len * batch;
    const size_t complex_bytes = f64 ? 16 : 8;
    const size_t used = (len & (len - 1)) == 0 ? dev.shared_memory_pow2_bytes : dev.shared_memory_bytes;
    const size_t max_shared = used / complex_bytes;
    size_t cand = required;
    for (;;) {
        const size_t np = next_pow2(cand);
        const bool three_quarters = (unsigned __int128)np * 3 <= (unsigned __int128)cand * 4;
        const bool fits = np <= max_shared || required > max_shared;
        if (len < 128 || (three_quarters && fits)) cand = np;
        if (is_smooth(cand, {2, 3, 5, 7})) {
            const size_t rhs = std::max<size_t>(max_rhs / cand, 1);
            if (radix_sequence_is_good(cand, rhs)) return cand;
        }
        cand += 1;
    }
}

// ---------------------------------------------------------- axis decisions

namespace {
bool rader_safe_prime(size_t p, const PlannerTuning& t) {
    // rader_fft_passes_upstream_safe_prime_gate (planner.rs:498-503)
    if (p <= 2) return false;
    for (size_t f : prime_factorization(p - 1))
        if (f >= t.min_rader_direct_prime) return false;
    return true;
}

bool is_stockham_prime(size_t p) { return p == 2 || p == 3 || p == 5 || p == 7 || p == 11 || p == 13; }

RaderModeKind rader_mode_portable(size_t p, const PlannerTuning& t);

bool recursively_plannable(size_t len, const PlannerTuning& t) {
    // rader_convolution_is_recursively_plannable (planner.rs:521-533)
    for (size_t q : prime_factorization(len))
        if (!is_stockham_prime(q) && rader_mode_portable(q, t) == RaderModeKind::None) return false;
    return true;
}

RaderModeKind rader_mode_portable(size_t p, const PlannerTuning& t) {
    // rader_mode_with_stockham_primes (planner.rs:470-496)
    const bool fft_ok = p >= t.min_rader_fft_prime && p < t.max_rader_fft_prime;
    if (fft_ok && rader_safe_prime(p, t)) return RaderModeKind::Fft;
    if (p >= t.min_rader_direct_prime && p < t.max_rader_direct_prime) return RaderModeKind::Direct;
    if (t.allow_recursive_fft_rader && fft_ok && recursively_plannable(p - 1, t)) return RaderModeKind::Fft;
    return RaderModeKind::None;
}

template <class Sel>
AxisDecision classify(size_t len, Sel&& select) {
    // plan_axis_algorithm_with_rader_selector (planner.rs:282-347)
    AxisDecision d;
    if (len == 0) throw std::invalid_argument("zero-length axis");
    if (len == 1) return d;
    std::vector<size_t> f = prime_factorization(len);
    size_t i = 0;
    while (i < f.size()) {
        size_t p = f[i], mult = 1;
        while (i + mult < f.size() && f[i + mult] == p) ++mult;
        if (is_stockham_prime(p)) {
            for (size_t k = 0; k < mult; ++k) d.stockham_factors.push_back(p);
        } else {
            RaderModeKind m = select(p);
            if (m == RaderModeKind::None) {
                AxisDecision b;
                b.algorithm = Algorithm::Bluestein;
                return b;
            }
            d.rader.push_back({p, mult, primitive_root(p), m});
        }
        i += mult;
    }
    d.algorithm = d.rader.empty() ? Algorithm::Stockham : Algorithm::Rader;
    return d;
}

size_t rader_fft_shared_limit(size_t avail, size_t len, bool strided, size_t cb, size_t coal, size_t cfg) {
    // c2c_rader_fft_shared_limit (planner.rs:442-463)
    const size_t max_shared = avail / cb;
    const size_t max_strided = coal > cb ? avail / coal : max_shared;
    const size_t dev = (!strided && len <= max_shared) ? max_shared : max_strided;
    return std::min(dev, cfg);
}
}  // namespace

AxisDecision plan_axis_portable(size_t len, const PlannerTuning& t) {
    AxisDecision d = classify(len, [&](size_t p) { return rader_mode_portable(p, t); });
    if (d.algorithm == Algorithm::Bluestein)  // plan_bluestein (planner.rs:535-545)
        d.convolution_len = next_smooth_at_least(len * 2 - 1, {2, 3, 5, 7});
    return d;
}

AxisDecision plan_c2c_axis(size_t len, size_t batch, bool f64, bool strided, const PlannerTuning& tuning,
                           const PlannerDevice& dev) {
    const size_t cb = f64 ? 16 : 8;
    const size_t coal = dev.coalesced_memory_bytes;
    const size_t used = (len & (len - 1)) == 0 ? dev.shared_memory_pow2_bytes : dev.shared_memory_bytes;
    size_t fft_limit = rader_fft_shared_limit(used, len, strided, cb, coal, tuning.max_rader_fft_prime);
    // upstream_effective_rader_tuning (config.rs:348-358)
    PlannerTuning eff = tuning;
    const size_t per_coal = std::max<size_t>(coal / cb, 1);
    const size_t cap = (dev.max_threads_per_block / per_coal) * 2 - 1;
    eff.max_rader_direct_prime = std::max(std::min(eff.max_rader_direct_prime, cap), eff.min_rader_direct_prime);
    AxisDecision d = classify(len, [&](size_t p) {
        const bool in_scan = p >= tuning.min_rader_direct_prime && p >= tuning.min_rader_fft_prime && p < fft_limit;
        if (in_scan) {
            if (rader_safe_prime(p, tuning)) return RaderModeKind::Fft;
            const size_t reserve = (p - 1) * cb;
            fft_limit = rader_fft_shared_limit(used > reserve ? used - reserve : 0, len, strided, cb, coal,
                                               tuning.max_rader_fft_prime);
        }
        if (p >= tuning.min_rader_direct_prime && p < eff.max_rader_direct_prime) return RaderModeKind::Direct;
        const bool fft_ok = p >= tuning.min_rader_fft_prime && p < tuning.max_rader_fft_prime;
        if (tuning.allow_recursive_fft_rader && fft_ok && recursively_plannable(p - 1, eff)) return RaderModeKind::Fft;
        return RaderModeKind::None;
    });
    if (d.algorithm == Algorithm::Bluestein) d.convolution_len = bluestein_auto_padding(len, batch, f64, dev);
    return d;
}

}  // namespace vkfx
