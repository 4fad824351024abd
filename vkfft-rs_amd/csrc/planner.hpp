// planner.hpp -- the subset of vkfft-rs's planner this path consumes,
// restated in C++ so the library can plan on its own when no Rust caller
// hands it a decision. Rust callers pass the decision they already made.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace vkfx {

enum class Algorithm : int { Stockham = 0, Rader = 1, Bluestein = 2 };
enum class RaderModeKind : int { None = 0, Direct = 1, Fft = 2 };

// DeviceProfile fields the planner reads (src/config.rs:250-265).
struct PlannerDevice {
    size_t shared_memory_bytes = 160 * 1024;
    size_t shared_memory_pow2_bytes = 128 * 1024;
    size_t max_threads_per_block = 1024;
    size_t coalesced_memory_bytes = 32;  // upstream_coalesced_memory_bytes, HIP (src/config.rs:304-317)
};

// PlannerTuning (src/config.rs:366-420).
struct PlannerTuning {
    size_t min_rader_direct_prime = 17;
    size_t max_rader_direct_prime = 89;
    size_t min_rader_fft_prime = 17;
    size_t max_rader_fft_prime = 16384;
    bool allow_recursive_fft_rader = false;
};

struct RaderPrime {
    size_t prime, multiplicity, generator;
    RaderModeKind mode;
};

struct AxisDecision {
    Algorithm algorithm = Algorithm::Stockham;
    size_t convolution_len = 0;        // Bluestein M
    std::vector<size_t> stockham_factors;
    std::vector<RaderPrime> rader;
};

std::vector<size_t> prime_factorization(size_t value);                 // planner.rs:581-604
bool is_smooth(size_t value, const std::vector<size_t>& primes);        // planner.rs:606-617
size_t next_smooth_at_least(size_t target, const std::vector<size_t>& primes);  // planner.rs:684-733
size_t primitive_root(size_t prime);                                   // planner.rs:645-667

// PlannerTuning::for_device for an AMD GPU (src/config.rs:395-420); f64 = true for F64.
PlannerTuning tuning_for_amd(bool f64, bool allow_recursive_rader = false);

// Register-schedule quality used by the Bluestein padding search
// (scheduler.rs:9882-9988, 9990-10424, 10425-10636, 10639-10818).
bool radix_sequence_is_good(size_t fft_len, size_t rhs_transform_count);

// upstream_bluestein_auto_padding for HIP/AMD (scheduler.rs:225-373).
size_t bluestein_auto_padding(size_t len, size_t batch, bool f64, const PlannerDevice& dev);

// plan_c2c_axis_algorithm_for_device for HIP/AMD (planner.rs:349-440).
// strided = the axis is not the contiguous (last) tensor dimension.
AxisDecision plan_c2c_axis(size_t len, size_t batch, bool f64, bool strided, const PlannerTuning& tuning,
                           const PlannerDevice& dev);

// plan_axis_algorithm, the portable classifier used for R2C/C2R axes
// (planner.rs:276-347, 535-545).
AxisDecision plan_axis_portable(size_t len, const PlannerTuning& tuning);

}  // namespace vkfx
