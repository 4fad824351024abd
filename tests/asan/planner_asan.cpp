// Host-side sanitizer run of the planner restatement (planner.cpp): the
// decision procedure over every length up to 20000 and a sample of larger
// ones, both precisions, contiguous and strided axes, default and recursive
// Rader tuning and three shared-memory sizes, built with AddressSanitizer and
// UndefinedBehaviorSanitizer. Besides memory and UB errors it checks the
// invariants every caller relies on; it prints "ok <cases>" and exits 0.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "planner.hpp"

using namespace vkfx;

static int fails = 0;
#define CHECK(c, ...)                                  \
    do {                                               \
        if (!(c)) {                                    \
            if (++fails < 20) std::printf(__VA_ARGS__); \
        }                                              \
    } while (0)

static bool is_prime(size_t n) {
    if (n < 2) return false;
    for (size_t d = 2; d * d <= n; ++d)
        if (n % d == 0) return false;
    return true;
}

int main() {
    size_t cases = 0;
    std::vector<size_t> lens;
    for (size_t n = 1; n <= 20000; ++n) lens.push_back(n);
    for (size_t n = 20001; n < 5000000; n = n * 5 / 4 + 7) lens.push_back(n);
    for (size_t n : {65537ul, 131071ul, 1048576ul, 4194304ul, 16777216ul, 268435456ul, 536870912ul}) lens.push_back(n);
    const size_t lds[] = {32 * 1024, 64 * 1024, 160 * 1024};
    for (size_t n : lens) {
        const auto f = prime_factorization(n);
        size_t prod = 1;
        for (size_t p : f) {
            CHECK(is_prime(p), "factor %zu of %zu not prime\n", p, n);
            prod *= p;
        }
        CHECK(n < 2 || prod == n, "factorization of %zu multiplies to %zu\n", n, prod);
        for (int f64 = 0; f64 < 2; ++f64)
            for (int strided = 0; strided < 2; ++strided)
                for (int rec = 0; rec < 2; ++rec)
                    for (size_t l : lds) {
                        if (n > 20000 && (l != 160 * 1024 || rec)) continue;
                        PlannerDevice dev;
                        dev.shared_memory_bytes = l;
                        size_t p2 = 1;
                        while (p2 * 2 <= l) p2 *= 2;
                        dev.shared_memory_pow2_bytes = p2;
                        const PlannerTuning t = tuning_for_amd(f64 != 0, rec != 0);
                        const size_t batch = 1 + (n * 7 + l) % 97;
                        const AxisDecision d = plan_c2c_axis(n, batch, f64 != 0, strided != 0, t, dev);
                        ++cases;
                        if (d.algorithm == Algorithm::Bluestein) {
                            CHECK(d.convolution_len + 1 >= 2 * n, "Bluestein M %zu < 2N-1 for N %zu\n",
                                  d.convolution_len, n);
                            // table entries (scheduler.rs:178-208) may carry 11 and 13
                            CHECK(is_smooth(d.convolution_len, {2, 3, 5, 7, 11, 13}), "M %zu not 13-smooth\n",
                                  d.convolution_len);
                        }
                        if (d.algorithm == Algorithm::Rader)
                            for (const RaderPrime& r : d.rader) {
                                CHECK(is_prime(r.prime) && n % r.prime == 0, "Rader prime %zu of %zu\n", r.prime, n);
                                CHECK(r.generator == primitive_root(r.prime), "generator of %zu\n", r.prime);
                            }
                        if (d.algorithm == Algorithm::Stockham && !d.stockham_factors.empty()) {
                            size_t q = 1;
                            for (size_t s : d.stockham_factors) q *= s;
                            CHECK(q == n, "Stockham factors of %zu multiply to %zu\n", n, q);
                        }
                    }
        const AxisDecision r = plan_axis_portable(n, tuning_for_amd(false));
        (void)r;
        if (n >= 2 && n <= 4096) {
            const size_t m = bluestein_auto_padding(n, 1 + n % 13, n % 2 == 0, PlannerDevice{});
            CHECK(m + 1 >= 2 * n, "auto padding %zu < 2N-1 for %zu\n", m, n);
        }
        if (is_prime(n) && n > 2 && n < 70000) {
            const size_t g = primitive_root(n);
            size_t x = 1, order = 0;
            do {
                x = (x * g) % n;
                ++order;
            } while (x != 1 && order <= n);
            CHECK(order == n - 1, "primitive root %zu of %zu has order %zu\n", g, n, order);
        }
    }
    for (size_t t = 2; t < 300000; t = t * 3 / 2 + 1) {
        const size_t s = next_smooth_at_least(t, {2, 3, 5, 7});
        CHECK(s >= t && is_smooth(s, {2, 3, 5, 7}), "next smooth of %zu: %zu\n", t, s);
        (void)radix_sequence_is_good(s, 1);
    }
    if (fails) {
        std::printf("%d failures\n", fails);
        return 1;
    }
    std::printf("ok %zu\n", cases);
    return 0;
}
