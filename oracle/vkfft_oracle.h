/*
 * vkfft_oracle.h -- CPU restatement of vkfft-rs's reference transforms.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the MI355X
 * execution path: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path never links or calls it.
 *
 * All complex buffers are interleaved double pairs {re, im}, the layout of
 * vkfft-rs `Complex64` (src/complex.rs:4-9). `sign` is the exponent sign of
 * `Direction::exponent_sign` (src/config.rs:10-15): -1 forward, +1 inverse.
 */
#ifndef VKFFT_ORACLE_H
#define VKFFT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference::dft (src/reference.rs:14-23, 44-58): naive O(n^2) DFT. */
int vko_dft(const double *in, double *out, size_t n, int sign, int normalize);

/* reference::fft (src/reference.rs:25-42, 60-153): recursive prime-radix
 * decimation over STOCKHAM_PRIMES {2,3,5,7,11,13}, Bluestein for anything else. */
int vko_fft(const double *in, double *out, size_t n, int sign, int normalize);

/* Batched vko_fft over `batch` contiguous transforms of length n, split over
 * `threads` pthreads (transforms are independent, so the split is exact). */
int vko_fft_batch(const double *in, double *out, size_t n, size_t batch, int sign,
                  int normalize, int threads);

/* R2C as the full-complex FFT truncated to n/2+1 bins
 * (src/real_ir.rs:935-946). in: batch*n reals, out: batch*(n/2+1) complex. */
int vko_r2c_batch(const double *in, double *out, size_t n, size_t batch, int threads);

/* C2R by Hermitian expansion then inverse FFT, real part kept
 * (src/real_ir.rs:1038-1053). in: batch*(n/2+1) complex, out: batch*n reals. */
int vko_c2r_batch(const double *in, double *out, size_t n, size_t batch, int normalize,
                  int threads);

/* Separable N-D C2C (src/nd_ir.rs:1303-1337): axes processed last to first,
 * each line packed, transformed with vko_fft and scattered back. dims are in
 * vkfft-rs order (slowest to fastest). */
/* Direct DCT/DST bins, FFTW REDFT00/10/01/11 and RODFT00/10/01/11
 * (src/r2r_ir.rs:2351-2434 evaluate_bin), unnormalized; kind 0..3 = DCT-I..IV,
 * 4..7 = DST-I..IV. O(N^2) per line, batch lines back to back, threads > 1
 * splits the batch. */
int vko_r2r_batch(const double *in, double *out, size_t n, size_t batch, int kind, int threads);

int vko_fft_nd(const double *in, double *out, const size_t *dims, size_t rank, size_t batch,
               int sign, int normalize, int threads);

/* planner::next_smooth_at_least (src/planner.rs:684-733). Returns 0 on error. */
size_t vko_next_smooth_at_least(size_t target, const size_t *primes, size_t nprimes);

/* planner::prime_factorization (src/planner.rs:581-604). Returns count written. */
size_t vko_prime_factorization(size_t value, size_t *factors, size_t cap);

/* planner::primitive_root (src/planner.rs:657-682). 0 = none. */
size_t vko_primitive_root(size_t prime);

/* Seeded inputs shared by tests and bench: splitmix64 seeding xoshiro256**.
 * uniform: (u53 * 2^-53) * 2 - 1 in [-1, 1); normal: Box-Muller in f64. */
void vko_fill_uniform(double *out, size_t count, uint64_t seed);
void vko_fill_normal(double *out, size_t count, uint64_t seed);
void vko_fill_uniform_f32(float *out, size_t count, uint64_t seed);
void vko_fill_normal_f32(float *out, size_t count, uint64_t seed);

/* Input formulas of the committed FFTW fixtures, evaluated in C exactly as
 * vkfft-rs tools/generate_fftw_golden.c:8-31 defines them (complex-v1,
 * real-v1 in double; complex-f32-v1, real-f32-v1 in float). */
void vko_fixture_complex_v1(size_t n, double *out);
void vko_fixture_real_v1(size_t n, double *out);
void vko_fixture_complex_f32_v1(size_t n, float *out);
void vko_fixture_real_f32_v1(size_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif
