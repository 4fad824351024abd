/*
 * vkfft_oracle.c -- CPU restatement of vkfft-rs's reference transforms in C.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product path). Each
 * function cites the vkfft-rs source it restates (paths relative to the
 * vkfft-rs repository root).
 *
 * The arithmetic follows src/reference.rs operation by operation: the same
 * recursion order over STOCKHAM_PRIMES, the same angle expression
 * `sign * 2.0 * PI * lane * k / n` evaluated left to right, the same
 * Bluestein chirp `sign * PI * i * i / n`, and Complex64's textbook multiply
 * (src/complex.rs).
 */
#include "vkfft_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    double re, im;
} cplx;

static const double VKO_PI = 3.14159265358979323846264338327950288;
static const size_t STOCKHAM_PRIMES[6] = {2, 3, 5, 7, 11, 13};   /* src/planner.rs:10 */
static const size_t BLUESTEIN_PRIMES[4] = {2, 3, 5, 7};          /* src/planner.rs:17 */

static inline cplx c_mul(cplx a, cplx b) {
    cplx r = {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
    return r;
}
static inline cplx c_add(cplx a, cplx b) {
    cplx r = {a.re + b.re, a.im + b.im};
    return r;
}
static inline cplx exp_i(double angle) { /* Complex64::exp_i, src/complex.rs:96-98 */
    cplx r = {cos(angle), sin(angle)};
    return r;
}

/* ---------------------------------------------------------------- planner */

size_t vko_prime_factorization(size_t value, size_t *factors, size_t cap) {
    /* src/planner.rs:581-604 */
    size_t count = 0;
    if (value < 2) return 0;
    while (value % 2 == 0) {
        if (count < cap) factors[count] = 2;
        count++;
        value /= 2;
    }
    for (size_t d = 3; d <= value / d; d += 2) {
        while (value % d == 0) {
            if (count < cap) factors[count] = d;
            count++;
            value /= d;
        }
    }
    if (value > 1) {
        if (count < cap) factors[count] = value;
        count++;
    }
    return count;
}

static size_t mod_pow(size_t base, size_t exponent, size_t modulus) {
    /* src/planner.rs:669-682 */
    unsigned __int128 result = 1, b = base % modulus;
    while (exponent > 0) {
        if (exponent & 1) result = (result * b) % modulus;
        b = (b * b) % modulus;
        exponent >>= 1;
    }
    return (size_t)result;
}

size_t vko_primitive_root(size_t prime) {
    /* src/planner.rs:645-667 */
    size_t f[64];
    if (prime == 2) return 1;
    if (prime < 2 || vko_prime_factorization(prime, f, 64) != 1) return 0;
    size_t phi = prime - 1;
    size_t nf = vko_prime_factorization(phi, f, 64);
    size_t uniq[64], nu = 0;
    for (size_t i = 0; i < nf; ++i)
        if (nu == 0 || uniq[nu - 1] != f[i]) uniq[nu++] = f[i];
    for (size_t g = 2; g < prime; ++g) {
        int ok = 1;
        for (size_t i = 0; i < nu; ++i)
            if (mod_pow(g, phi / uniq[i], prime) == 1) {
                ok = 0;
                break;
            }
        if (ok) return g;
    }
    return 0;
}

static void smooth_visit(const size_t *p, size_t np, size_t idx, size_t cur, size_t target,
                         size_t *best) {
    /* inner `visit` of src/planner.rs:708-724 */
    if (cur >= *best) return;
    if (idx == np) {
        if (cur >= target) *best = cur;
        return;
    }
    size_t value = cur;
    for (;;) {
        smooth_visit(p, np, idx + 1, value, target, best);
        if (value > SIZE_MAX / p[idx]) break;
        size_t next = value * p[idx];
        if (next < *best)
            value = next;
        else
            break;
    }
}

size_t vko_next_smooth_at_least(size_t target, const size_t *primes, size_t nprimes) {
    /* src/planner.rs:684-733 */
    if (target <= 1) return 1;
    if (nprimes == 0 || nprimes > 16) return 0;
    size_t ord[16];
    size_t n = 0;
    for (size_t i = 0; i < nprimes; ++i) {
        if (primes[i] < 2) return 0;
        ord[n++] = primes[i];
    }
    for (size_t i = 1; i < n; ++i) /* sort_unstable + dedup */
        for (size_t j = i; j > 0 && ord[j - 1] > ord[j]; --j) {
            size_t t = ord[j];
            ord[j] = ord[j - 1];
            ord[j - 1] = t;
        }
    size_t m = 0;
    for (size_t i = 0; i < n; ++i)
        if (m == 0 || ord[m - 1] != ord[i]) ord[m++] = ord[i];
    size_t best = SIZE_MAX;
    if (ord[0] == 2) {
        size_t p2 = 1;
        while (p2 < target && p2 <= SIZE_MAX / 2) p2 <<= 1;
        if (p2 >= target) best = p2;
    }
    smooth_visit(ord, m, 0, 1, target, &best);
    return best == SIZE_MAX ? 0 : best;
}

/* ------------------------------------------------------------------ FFTs */

int vko_dft(const double *in, double *out, size_t n, int sign, int normalize) {
    /* src/reference.rs:14-23 and dft_unscaled :44-58 */
    const cplx *x = (const cplx *)in;
    cplx *y = (cplx *)malloc(sizeof(cplx) * (n ? n : 1));
    if (!y) return -1;
    double s = (double)sign;
    for (size_t k = 0; k < n; ++k) {
        cplx sum = {0.0, 0.0};
        for (size_t i = 0; i < n; ++i) {
            double angle = s * 2.0 * VKO_PI * (double)i * (double)k / (double)n;
            sum = c_add(sum, c_mul(x[i], exp_i(angle)));
        }
        y[k] = sum;
    }
    if (sign > 0 && normalize && n) {
        double scale = 1.0 / (double)n;
        for (size_t k = 0; k < n; ++k) {
            y[k].re *= scale;
            y[k].im *= scale;
        }
    }
    memcpy(out, y, sizeof(cplx) * n);
    free(y);
    return 0;
}

static int fft_unscaled(const cplx *in, cplx *out, size_t n, int sign);

static int mixed_radix_unscaled(const cplx *in, cplx *out, size_t n, int sign, size_t radix) {
    /* src/reference.rs:76-105 */
    size_t inner_len = n / radix;
    cplx *seq = (cplx *)malloc(sizeof(cplx) * inner_len);
    cplx *inner = (cplx *)malloc(sizeof(cplx) * n); /* radix blocks of inner_len */
    if (!seq || !inner) {
        free(seq);
        free(inner);
        return -1;
    }
    for (size_t lane = 0; lane < radix; ++lane) {
        for (size_t index = 0; index < inner_len; ++index) seq[index] = in[lane + radix * index];
        if (fft_unscaled(seq, inner + lane * inner_len, inner_len, sign)) {
            free(seq);
            free(inner);
            return -1;
        }
    }
    double s = (double)sign;
    for (size_t k = 0; k < n; ++k) {
        size_t inner_index = k % inner_len;
        cplx sum = {0.0, 0.0};
        for (size_t lane = 0; lane < radix; ++lane) {
            double angle = s * 2.0 * VKO_PI * (double)lane * (double)k / (double)n;
            sum = c_add(sum, c_mul(inner[lane * inner_len + inner_index], exp_i(angle)));
        }
        out[k] = sum;
    }
    free(seq);
    free(inner);
    return 0;
}

static int bluestein_unscaled(const cplx *in, cplx *out, size_t n, int sign) {
    /* src/reference.rs:107-153 */
    size_t m = vko_next_smooth_at_least(2 * n - 1, BLUESTEIN_PRIMES, 4);
    if (m == 0) return -1;
    double s = (double)sign;
    cplx *a = (cplx *)calloc(m, sizeof(cplx));
    cplx *b = (cplx *)calloc(m, sizeof(cplx));
    cplx *af = (cplx *)malloc(sizeof(cplx) * m);
    cplx *bf = (cplx *)malloc(sizeof(cplx) * m);
    int rc = -1;
    if (!a || !b || !af || !bf) goto done;
    for (size_t i = 0; i < n; ++i) {
        double fi = (double)i;
        double angle = s * VKO_PI * fi * fi / (double)n;
        cplx chirp = exp_i(angle);
        cplx inv = exp_i(-angle);
        a[i] = c_mul(in[i], chirp);
        b[i] = inv;
        if (i != 0) b[m - i] = inv;
    }
    if (fft_unscaled(a, af, m, -1) || fft_unscaled(b, bf, m, -1)) goto done;
    for (size_t i = 0; i < m; ++i) a[i] = c_mul(af[i], bf[i]);
    if (fft_unscaled(a, af, m, 1)) goto done;
    {
        double cs = 1.0 / (double)m;
        for (size_t i = 0; i < n; ++i) {
            cplx v = {af[i].re * cs, af[i].im * cs};
            double fi = (double)i;
            double angle = s * VKO_PI * fi * fi / (double)n;
            out[i] = c_mul(v, exp_i(angle));
        }
    }
    rc = 0;
done:
    free(a);
    free(b);
    free(af);
    free(bf);
    return rc;
}

static int fft_unscaled(const cplx *in, cplx *out, size_t n, int sign) {
    /* src/reference.rs:60-74 */
    if (n <= 1) {
        if (n == 1) out[0] = in[0];
        return 0;
    }
    for (int i = 0; i < 6; ++i)
        if (n % STOCKHAM_PRIMES[i] == 0) return mixed_radix_unscaled(in, out, n, sign, STOCKHAM_PRIMES[i]);
    return bluestein_unscaled(in, out, n, sign);
}

int vko_fft(const double *in, double *out, size_t n, int sign, int normalize) {
    /* src/reference.rs:25-42 */
    if (n == 0) return 0;
    cplx *tmp = (cplx *)malloc(sizeof(cplx) * n);
    if (!tmp) return -1;
    if (fft_unscaled((const cplx *)in, tmp, n, sign)) {
        free(tmp);
        return -1;
    }
    if (sign > 0 && normalize) {
        double scale = 1.0 / (double)n;
        for (size_t i = 0; i < n; ++i) {
            tmp[i].re *= scale;
            tmp[i].im *= scale;
        }
    }
    memcpy(out, tmp, sizeof(cplx) * n);
    free(tmp);
    return 0;
}

/* ------------------------------------------------------- batch drivers */

typedef struct {
    int kind; /* 0 c2c, 1 r2c, 2 c2r, 3 r2r (sign = DCT/DST kind) */
    const double *in;
    double *out;
    size_t n, first, last;
    int sign, normalize, rc;
} job_t;

/* One DCT/DST bin, FFTW's unnormalized definitions (src/r2r_ir.rs:2351-2434).
 * kind 0..3 DCT-I..IV (REDFT00/10/01/11), 4..7 DST-I..IV (RODFT00/10/01/11). */
static double r2r_bin(int kind, const double *x, size_t n, size_t k) {
    double sum = 0.0;
    const double dk = (double)k;
    switch (kind) {
        case 0: /* REDFT00 */
            sum = x[0] + ((k % 2 == 0) ? x[n - 1] : -x[n - 1]);
            for (size_t j = 1; j + 1 < n; ++j) sum += 2.0 * x[j] * cos(VKO_PI * (double)j * dk / (double)(n - 1));
            return sum;
        case 1: /* REDFT10 */
            for (size_t j = 0; j < n; ++j) sum += 2.0 * x[j] * cos(VKO_PI * ((double)j + 0.5) * dk / (double)n);
            return sum;
        case 2: /* REDFT01 */
            sum = x[0];
            for (size_t j = 1; j < n; ++j) sum += 2.0 * x[j] * cos(VKO_PI * (double)j * (dk + 0.5) / (double)n);
            return sum;
        case 3: /* REDFT11 */
            for (size_t j = 0; j < n; ++j)
                sum += 2.0 * x[j] * cos(VKO_PI * ((double)j + 0.5) * (dk + 0.5) / (double)n);
            return sum;
        case 4: /* RODFT00 */
            for (size_t j = 0; j < n; ++j)
                sum += 2.0 * x[j] * sin(VKO_PI * (double)(j + 1) * (double)(k + 1) / (double)(n + 1));
            return sum;
        case 5: /* RODFT10 */
            for (size_t j = 0; j < n; ++j)
                sum += 2.0 * x[j] * sin(VKO_PI * ((double)j + 0.5) * (double)(k + 1) / (double)n);
            return sum;
        case 6: /* RODFT01 */
            sum = (k % 2 == 0) ? x[n - 1] : -x[n - 1];
            for (size_t j = 0; j + 1 < n; ++j)
                sum += 2.0 * x[j] * sin(VKO_PI * (double)(j + 1) * (dk + 0.5) / (double)n);
            return sum;
        default: /* RODFT11 */
            for (size_t j = 0; j < n; ++j)
                sum += 2.0 * x[j] * sin(VKO_PI * ((double)j + 0.5) * (dk + 0.5) / (double)n);
            return sum;
    }
}

static int run_one(job_t *j, size_t t) {
    size_t n = j->n, h = n / 2 + 1;
    if (j->kind == 0) return vko_fft(j->in + 2 * n * t, j->out + 2 * n * t, n, j->sign, j->normalize);
    if (j->kind == 3) {
        for (size_t k = 0; k < n; ++k) j->out[n * t + k] = r2r_bin(j->sign, j->in + n * t, n, k);
        return 0;
    }
    cplx *buf = (cplx *)calloc(n * 2, sizeof(cplx));
    if (!buf) return -1;
    cplx *full = buf, *res = buf + n;
    int rc;
    if (j->kind == 1) {
        /* RealFftAlgorithm::FullComplex forward, src/real_ir.rs:935-946 */
        for (size_t i = 0; i < n; ++i) {
            full[i].re = j->in[n * t + i];
            full[i].im = 0.0;
        }
        rc = vko_fft((double *)full, (double *)res, n, -1, 0);
        if (!rc) memcpy(j->out + 2 * h * t, res, sizeof(cplx) * h);
    } else {
        /* RealFftAlgorithm::FullComplex inverse, src/real_ir.rs:1038-1053 */
        const cplx *x = (const cplx *)(j->in + 2 * h * t);
        for (size_t k = 0; k < n; ++k) {
            if (k < h)
                full[k] = x[k];
            else {
                full[k].re = x[n - k].re;
                full[k].im = -x[n - k].im;
            }
        }
        rc = vko_fft((double *)full, (double *)res, n, 1, j->normalize);
        if (!rc)
            for (size_t i = 0; i < n; ++i) j->out[n * t + i] = res[i].re;
    }
    free(buf);
    return rc;
}

static void *job_main(void *arg) {
    job_t *j = (job_t *)arg;
    j->rc = 0;
    for (size_t t = j->first; t < j->last && !j->rc; ++t) j->rc = run_one(j, t);
    return NULL;
}

static int run_batch(int kind, const double *in, double *out, size_t n, size_t batch, int sign,
                     int normalize, int threads) {
    if (n == 0 || batch == 0) return 0;
    if (threads < 1) threads = 1;
    if ((size_t)threads > batch) threads = (int)batch;
    job_t *jobs = (job_t *)calloc((size_t)threads, sizeof(job_t));
    pthread_t *tids = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        return -1;
    }
    size_t per = batch / (size_t)threads, extra = batch % (size_t)threads, cur = 0;
    for (int i = 0; i < threads; ++i) {
        size_t cnt = per + ((size_t)i < extra ? 1 : 0);
        job_t jj = {kind, in, out, n, cur, cur + cnt, sign, normalize, 0};
        jobs[i] = jj;
        cur += cnt;
    }
    int rc = 0;
    if (threads == 1) {
        job_main(&jobs[0]);
        rc = jobs[0].rc;
    } else {
        for (int i = 0; i < threads; ++i) pthread_create(&tids[i], NULL, job_main, &jobs[i]);
        for (int i = 0; i < threads; ++i) {
            pthread_join(tids[i], NULL);
            if (jobs[i].rc) rc = jobs[i].rc;
        }
    }
    free(jobs);
    free(tids);
    return rc;
}

int vko_fft_batch(const double *in, double *out, size_t n, size_t batch, int sign, int normalize,
                  int threads) {
    return run_batch(0, in, out, n, batch, sign, normalize, threads);
}

int vko_r2r_batch(const double *in, double *out, size_t n, size_t batch, int kind, int threads) {
    if (kind < 0 || kind > 7) return -1;
    if (kind == 0 && n < 2) return -1; /* DCT-I needs two points */
    return run_batch(3, in, out, n, batch, kind, 0, threads);
}

int vko_r2c_batch(const double *in, double *out, size_t n, size_t batch, int threads) {
    return run_batch(1, in, out, n, batch, -1, 0, threads);
}

int vko_c2r_batch(const double *in, double *out, size_t n, size_t batch, int normalize,
                  int threads) {
    return run_batch(2, in, out, n, batch, 1, normalize, threads);
}

int vko_fft_nd(const double *in, double *out, const size_t *dims, size_t rank, size_t batch,
               int sign, int normalize, int threads) {
    /* src/nd_ir.rs:1303-1337: for each axis from last to first, pack every
     * line of that axis into a contiguous batch, run the 1-D transform, and
     * scatter the results back in place. */
    size_t total = batch;
    for (size_t a = 0; a < rank; ++a) total *= dims[a];
    if (total == 0) return 0;
    memmove(out, in, sizeof(double) * 2 * total);
    for (size_t ax = rank; ax-- > 0;) {
        size_t len = dims[ax], inner = 1, outer = batch;
        for (size_t a = ax + 1; a < rank; ++a) inner *= dims[a];
        for (size_t a = 0; a < ax; ++a) outer *= dims[a];
        size_t lines = outer * inner;
        double *pack = (double *)malloc(sizeof(double) * 2 * total);
        double *res = (double *)malloc(sizeof(double) * 2 * total);
        if (!pack || !res) {
            free(pack);
            free(res);
            return -1;
        }
        for (size_t o = 0; o < outer; ++o)
            for (size_t i = 0; i < inner; ++i)
                for (size_t e = 0; e < len; ++e) {
                    size_t src = (o * len + e) * inner + i, dst = (o * inner + i) * len + e;
                    pack[2 * dst] = out[2 * src];
                    pack[2 * dst + 1] = out[2 * src + 1];
                }
        int rc = vko_fft_batch(pack, res, len, lines, sign, normalize, threads);
        if (!rc)
            for (size_t o = 0; o < outer; ++o)
                for (size_t i = 0; i < inner; ++i)
                    for (size_t e = 0; e < len; ++e) {
                        size_t dst = (o * len + e) * inner + i, src = (o * inner + i) * len + e;
                        out[2 * dst] = res[2 * src];
                        out[2 * dst + 1] = res[2 * src + 1];
                    }
        free(pack);
        free(res);
        if (rc) return rc;
    }
    return 0;
}

/* ----------------------------------------------------------- seeded RNG */

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
typedef struct {
    uint64_t s[4];
} xoshiro;
static void xo_seed(xoshiro *x, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) x->s[i] = splitmix64(&sm);
}
static uint64_t xo_next(xoshiro *x) { /* xoshiro256** */
    uint64_t *s = x->s;
    uint64_t result = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
}
static double xo_unit(xoshiro *x) { return (double)(xo_next(x) >> 11) * 0x1.0p-53; }

void vko_fill_uniform(double *out, size_t count, uint64_t seed) {
    xoshiro x;
    xo_seed(&x, seed);
    for (size_t i = 0; i < count; ++i) out[i] = xo_unit(&x) * 2.0 - 1.0;
}
void vko_fill_normal(double *out, size_t count, uint64_t seed) {
    xoshiro x;
    xo_seed(&x, seed);
    for (size_t i = 0; i < count; i += 2) {
        double u1 = xo_unit(&x), u2 = xo_unit(&x);
        if (u1 < 0x1.0p-60) u1 = 0x1.0p-60;
        double r = sqrt(-2.0 * log(u1)), th = 2.0 * VKO_PI * u2;
        out[i] = r * cos(th);
        if (i + 1 < count) out[i + 1] = r * sin(th);
    }
}
void vko_fill_uniform_f32(float *out, size_t count, uint64_t seed) {
    xoshiro x;
    xo_seed(&x, seed);
    for (size_t i = 0; i < count; ++i) out[i] = (float)(xo_unit(&x) * 2.0 - 1.0);
}
void vko_fill_normal_f32(float *out, size_t count, uint64_t seed) {
    xoshiro x;
    xo_seed(&x, seed);
    for (size_t i = 0; i < count; i += 2) {
        double u1 = xo_unit(&x), u2 = xo_unit(&x);
        if (u1 < 0x1.0p-60) u1 = 0x1.0p-60;
        double r = sqrt(-2.0 * log(u1)), th = 2.0 * VKO_PI * u2;
        out[i] = (float)(r * cos(th));
        if (i + 1 < count) out[i + 1] = (float)(r * sin(th));
    }
}

/* ------------------------------------------------------ fixture inputs */

void vko_fixture_complex_v1(size_t n, double *out) {
    for (size_t i = 0; i < n; ++i) {
        double x = (double)i;
        out[2 * i] = sin(0.137 * x) + 0.0013 * x;
        out[2 * i + 1] = cos(0.071 * x) - 0.0009 * x;
    }
}
void vko_fixture_real_v1(size_t n, double *out) {
    for (size_t i = 0; i < n; ++i) {
        double x = (double)i;
        out[i] = sin(0.173 * x) + 0.003 * x - 0.27 * cos(0.071 * x);
    }
}
void vko_fixture_complex_f32_v1(size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        float x = (float)i;
        out[2 * i] = sinf(0.137f * x) + 0.0013f * x;
        out[2 * i + 1] = cosf(0.071f * x) - 0.0009f * x;
    }
}
void vko_fixture_real_f32_v1(size_t n, float *out) {
    for (size_t i = 0; i < n; ++i) {
        float x = (float)i;
        out[i] = sinf(0.173f * x) + 0.003f * x - 0.27f * cosf(0.071f * x);
    }
}
