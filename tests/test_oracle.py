"""Pins the CPU oracle (oracle/vkfft_oracle.c, a restatement of vkfft-rs
src/reference.rs) against the FFTW 3.3.9 fixtures the reference commits
(tests/fixtures/*.txt), the reference's own known-answer tests
(src/reference.rs:178-200), brute-force DFTs, closed forms and numpy's
pocketfft. The oracle is the checker for every GPU parity test."""
import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import oracle as o


def _corpus(name):
    return o.parse_fixture(os.path.join(GOLDEN, name))


def _max_err(a, b):
    return float(np.max(np.abs(np.asarray(a) - np.asarray(b))))


# -------------------------------------------------- FFTW golden fixtures

def test_fftw_c2c_n47_inputs_and_outputs():
    case = _corpus("fftw_precision_v1.txt")["cases"]["c2c-n47"]
    rows = np.array(case["rows"])
    x = rows[:, 0] + 1j * rows[:, 1]
    expected = rows[:, 2] + 1j * rows[:, 3]
    # the committed inputs are exactly the complex-v1 formula
    assert np.array_equal(x, o.fixture_input("complex-v1", 47))
    # reference tolerance for CPU executors: 2e-10 * N (tests/fftw_golden.rs)
    assert _max_err(o.fft(x), expected) <= 2e-10 * 47


def test_fftw_r2c_n45():
    case = _corpus("fftw_precision_v1.txt")["cases"]["r2c-n45"]
    split = case["meta"]["_split"]
    x = np.array([r[0] for r in case["rows"][:split]])
    out = np.array(case["rows"][split:])
    expected = out[:, 0] + 1j * out[:, 1]
    assert np.array_equal(x, o.fixture_input("real-v1", 45))
    assert _max_err(o.r2c_batch(x, 45), expected) <= 2e-10 * 45


@pytest.mark.parametrize("corpus", ["fftw_precision_medium_v1.txt", "fftw_precision_medium_f32_v1.txt"])
@pytest.mark.parametrize("case", ["c2c-bluestein-n103", "c2c-rader-n257", "c2c-smooth-n1536",
                                  "c2c-large-smooth-n4096"])
def test_fftw_medium_c2c(corpus, case):
    c = _corpus(corpus)["cases"][case]
    n = int(c["meta"]["shape"])
    x = o.fixture_input(c["meta"]["input"], n).astype(np.complex128)
    rows = np.array(c["rows"])
    expected = rows[:, 0] + 1j * rows[:, 1]
    assert _max_err(o.fft(x), expected) <= 2e-10 * n


@pytest.mark.parametrize("corpus", ["fftw_precision_medium_v1.txt", "fftw_precision_medium_f32_v1.txt"])
@pytest.mark.parametrize("case", ["r2c-nd-17x34", "r2c-nd-64x64"])
def test_fftw_medium_r2c_nd(corpus, case):
    """2-D R2C = separable complex N-D transform (nd_ir.rs:1303-1337) of the
    real input, truncated to cols/2+1 on the last axis."""
    c = _corpus(corpus)["cases"][case]
    rows_, cols = (int(v) for v in c["meta"]["shape"].split())
    x = o.fixture_input(c["meta"]["input"], rows_ * cols).astype(np.complex128)
    full = o.fft_nd(x, [rows_, cols]).reshape(rows_, cols)
    got = full[:, : cols // 2 + 1].reshape(-1)
    rows = np.array(c["rows"])
    expected = rows[:, 0] + 1j * rows[:, 1]
    assert _max_err(got, expected) <= 2e-10 * rows_ * cols


# ------------------------------------------------ reference.rs known answers

def _sample(n):
    # src/reference.rs:159-166
    x = np.arange(n, dtype=np.float64)
    return np.sin(0.37 * x) + x * 0.01 + 1j * (np.cos(0.19 * x) - x * 0.02)


@pytest.mark.parametrize("n", [2, 3, 4, 6, 7, 11, 13, 17, 19, 31, 47, 77])
def test_mixed_radix_and_bluestein_match_naive_dft(n):
    x = _sample(n)
    assert _max_err(o.fft(x), o.dft(x)) <= 5e-10 * n


@pytest.mark.parametrize("n", [8, 17, 47, 64])
def test_normalized_inverse_round_trips(n):
    x = _sample(n)
    assert _max_err(o.fft(o.fft(x), "inverse", True), x) < 5e-10 * n


# ------------------------------------------------------ closed forms

@pytest.mark.parametrize("n", [1, 2, 5, 16, 30, 97, 1024, 4099])
def test_impulse_is_all_ones(n):
    x = np.zeros(n, dtype=np.complex128)
    x[0] = 1
    assert _max_err(o.fft(x), np.ones(n)) < 1e-12 * max(n, 1)


@pytest.mark.parametrize("n,k0", [(64, 5), (360, 7), (4099, 123), (103, 1)])
def test_single_tone_is_a_delta(n, k0):
    idx = np.arange(n)
    x = np.exp(2j * np.pi * k0 * idx / n)
    y = o.fft(x)
    expected = np.zeros(n, dtype=np.complex128)
    expected[k0] = n
    assert _max_err(y, expected) < 1e-9 * n


def test_inverse_sign_convention():
    # inverse uses exp(+2 pi i jk/n): a forward tone at +k0 appears at -k0
    n, k0 = 32, 3
    x = np.exp(2j * np.pi * k0 * np.arange(n) / n)
    y = o.fft(x, "inverse")
    assert abs(y[(n - k0) % n] - n) < 1e-9 and abs(y[k0]) < 1e-9


@pytest.mark.parametrize("n", [12, 210, 1000, 4099])
def test_linearity_and_parseval(n):
    a = o.complex_uniform(n, 11, np.complex128)
    b = o.complex_uniform(n, 12, np.complex128)
    fa, fb = o.fft(a), o.fft(b)
    assert _max_err(o.fft(2.5 * a - 1j * b), 2.5 * fa - 1j * fb) < 1e-10 * n
    assert abs(np.vdot(fa, fa).real - n * np.vdot(a, a).real) < 1e-9 * n * np.vdot(a, a).real


@pytest.mark.parametrize("n", [24, 1024, 4099, 6561])
def test_matches_pocketfft(n):
    x = o.complex_uniform(n, n, np.complex128)
    assert o.rel_l2(o.fft(x), np.fft.fft(x)) < 1e-12
    assert o.rel_l2(o.fft(x, "inverse", True), np.fft.ifft(x)) < 1e-12


def test_batch_threads_match_single():
    x = o.complex_uniform(8 * 96, 3, np.complex128)
    one = o.fft_batch(x, 96, threads=1)
    many = o.fft_batch(x, 96, threads=4)
    assert np.array_equal(one, many)
    assert np.array_equal(one[96:192], o.fft(x[96:192]))


@pytest.mark.parametrize("n", [16, 45, 1024])
def test_r2c_c2r_round_trip_and_hermitian(n):
    x = o.uniform(3 * n, 5)
    X = o.r2c_batch(x, n)
    full = np.fft.fft(x.reshape(3, n), axis=1)
    assert o.rel_l2(X.reshape(3, -1), full[:, : n // 2 + 1]) < 1e-12
    back = o.c2r_batch(X, n, normalize=True)
    assert _max_err(back, x) < 1e-12 * n


def test_nd_is_separable():
    dims = [6, 10, 8]
    x = o.complex_uniform(2 * 480, 9, np.complex128)
    got = o.fft_nd(x, dims, batch=2).reshape(2, *dims)
    assert o.rel_l2(got, np.fft.fftn(x.reshape(2, *dims), axes=(1, 2, 3))) < 1e-12


def test_planner_helpers():
    # src/planner.rs:1119 pins next_smooth_at_least(2061) over {2,3,5,7}
    assert o.next_smooth_at_least(2061) == 2100
    assert o.next_smooth_at_least(8197) == 8232
    assert o.next_smooth_at_least(131073) == 131220
    assert o.prime_factorization(4098) == [2, 3, 683]
    assert o.primitive_root(4099) == 2 and o.primitive_root(17) == 3 and o.primitive_root(257) == 3


def test_seeded_rng_is_deterministic_and_uniform():
    a = o.uniform(100000, 42)
    assert np.array_equal(a, o.uniform(100000, 42))
    assert a.min() >= -1 and a.max() < 1 and abs(a.mean()) < 0.01
    z = o.normal(100000, 7)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    assert np.array_equal(o.uniform(10, 42, np.float32), a[:10].astype(np.float32))


def test_precision_metrics_follow_reference_definition():
    # src/precision.rs:31-101
    m = o.precision_metrics([1 + 0j, 2, 0], [1 + 0j, 1, 0])
    assert m["max_difference"] == 1 and m["avg_difference"] == pytest.approx(1 / 3)
    assert m["max_eps"] == 1 and m["avg_eps"] == pytest.approx(1 / 3)


@pytest.mark.parametrize("kind", ["dct1", "dct2", "dct3", "dct4", "dst1", "dst2", "dst3", "dst4"])
@pytest.mark.parametrize("n", [2, 3, 7, 16, 33, 100])
def test_r2r_matches_scipy(kind, n):
    """The oracle's DCT/DST bins (r2r_ir.rs:2351-2434, FFTW REDFT/RODFT) against
    scipy.fft (pocketfft, FFTW's unnormalized conventions), a library routine."""
    import scipy.fft as sf
    if kind == "dct1" and n < 2:
        pytest.skip("DCT-I needs two points")
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n))
    t = int(kind[-1])
    ref = (sf.dct if kind.startswith("dct") else sf.dst)(x, type=t, axis=1)
    got = o.r2r_batch(x, n, kind, threads=2).reshape(3, n)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12 * n)


def test_r2r_inverse_pairs_and_closed_forms():
    """DCT-II/III and DST-II/III are inverse pairs up to 2N; DCT-I, DCT-IV,
    DST-I, DST-IV are their own inverses up to 2(N-1), 2N, 2(N+1), 2N
    (inverse_pair_scale, r2r_ir.rs:2318-2346); a constant input has DCT-II
    2N at bin 0 and zero elsewhere."""
    n = 12
    x = np.random.default_rng(1).standard_normal(n)
    for fwd, inv, den in [("dct2", "dct3", 2 * n), ("dct3", "dct2", 2 * n), ("dst2", "dst3", 2 * n),
                          ("dst3", "dst2", 2 * n), ("dct1", "dct1", 2 * (n - 1)), ("dct4", "dct4", 2 * n),
                          ("dst1", "dst1", 2 * (n + 1)), ("dst4", "dst4", 2 * n)]:
        y = o.r2r_batch(o.r2r_batch(x, n, fwd), n, inv) / den
        np.testing.assert_allclose(y, x, rtol=0, atol=1e-12)
    c = o.r2r_batch(np.ones(n), n, "dct2")
    assert abs(c[0] - 2 * n) < 1e-12 and np.max(np.abs(c[1:])) < 1e-12


def _circ_conv(x, h):
    """Brute-force circular convolution y[n] = sum_m x[m] h[(n-m) mod N]."""
    n = x.size
    return np.array([sum(x[m] * h[(j - m) % n] for m in range(n)) for j in range(n)])


def test_convolution_is_circular_convolution():
    """performConvolution with kernel spectrum DFT(h) convolves with h; the
    conjugated sequence gives the circular correlation sum_m conj(x[m]) h[n+m]."""
    n, batch = 12, 2
    rng = np.random.default_rng(5)
    x = rng.standard_normal(n * batch) + 1j * rng.standard_normal(n * batch)
    h = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    y = o.convolution(x, np.fft.fft(h), [n], batch).reshape(batch, n)
    for b in range(batch):
        assert np.allclose(y[b], _circ_conv(x[b * n:(b + 1) * n], h), atol=1e-12)
    yc = o.convolution(x, np.fft.fft(h), [n], batch, conj_sequence=True).reshape(batch, n)
    xb = x[:n]
    corr = np.array([sum(np.conj(xb[m]) * h[(j + m) % n] for m in range(n)) for j in range(n)])
    assert np.allclose(yc[0], corr, atol=1e-12)


def test_convolution_kernels_and_matrix_layouts():
    n = 10
    rng = np.random.default_rng(6)
    c = lambda k: rng.standard_normal(k) + 1j * rng.standard_normal(k)
    x = c(n)
    hs = [c(n) for _ in range(3)]
    # multi-kernel fan-out: output system k is x convolved with h_k
    y = o.convolution(x, np.concatenate([np.fft.fft(h) for h in hs]), [n], 1, kernel_count=3).reshape(3, n)
    for k in range(3):
        assert np.allclose(y[k], _circ_conv(x, hs[k]), atol=1e-12)
    # 2x2 matrix: y_o = sum_i x_i * h_(o,i), planes row-major
    xs = [c(n), c(n)]
    hm = [[c(n), c(n)], [c(n), c(n)]]
    spec = np.concatenate([np.fft.fft(hm[a][b]) for a in range(2) for b in range(2)])
    y = o.convolution(np.concatenate(xs), spec, [n], 1, matrix=2).reshape(2, n)
    for a in range(2):
        assert np.allclose(y[a], _circ_conv(xs[0], hm[a][0]) + _circ_conv(xs[1], hm[a][1]), atol=1e-12)
    # symmetric 2x2 planes [xx, xy, yy]: (0,1) and (1,0) share plane 1
    assert [o.conv_plane_index(2, True, a, b) for a in range(2) for b in range(2)] == [0, 1, 1, 2]
    hs3 = [c(n) for _ in range(3)]
    y = o.convolution(np.concatenate(xs), np.concatenate([np.fft.fft(h) for h in hs3]), [n], 1, matrix=2,
                      symmetric=True).reshape(2, n)
    assert np.allclose(y[0], _circ_conv(xs[0], hs3[0]) + _circ_conv(xs[1], hs3[1]), atol=1e-12)
    assert np.allclose(y[1], _circ_conv(xs[0], hs3[1]) + _circ_conv(xs[1], hs3[2]), atol=1e-12)
    # the 3x3 symmetric index aliases yz and zz (why that layout is rejected)
    assert o.conv_plane_index(3, True, 1, 2) == o.conv_plane_index(3, True, 2, 2) == 4


def test_cross_power_spectrum_is_phase_correlation():
    """conj(X) * FFT(roll(x, s)) normalized to unit modulus transforms back to
    a delta at the shift s (2-D as well)."""
    rng = np.random.default_rng(7)
    n, s = 64, 13
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    y = o.convolution(x, np.fft.fft(np.roll(x, s)), [n], 1, conj_sequence=True, cross_power=True)
    e = np.zeros(n)
    e[s] = 1
    assert np.allclose(y, e, atol=1e-12)
    dims = [16, 24]
    x2 = rng.standard_normal(16 * 24) + 1j * rng.standard_normal(16 * 24)
    sh = np.roll(x2.reshape(dims), (3, 5), axis=(0, 1))
    y2 = o.convolution(x2, np.fft.fft2(sh), dims, 1, conj_sequence=True, cross_power=True).reshape(dims)
    e2 = np.zeros(dims)
    e2[3, 5] = 1
    assert np.allclose(y2, e2, atol=1e-12)


def test_convolution_backends_agree():
    rng = np.random.default_rng(8)
    for dims, batch in (([1009], 2), ([12, 10], 3)):
        t = int(np.prod(dims))
        x = rng.standard_normal(t * batch) + 1j * rng.standard_normal(t * batch)
        k = rng.standard_normal(t) + 1j * rng.standard_normal(t)
        a = o.convolution(x, k, dims, batch, conj_sequence=True, cross_power=True)
        b = o.convolution(x, k, dims, batch, conj_sequence=True, cross_power=True, backend="numpy")
        assert o.rel_l2(a, b) <= 1e-12


def _circ_conv2(x, h):
    """Brute-force 2-D circular convolution."""
    n0, n1 = x.shape
    y = np.zeros_like(x)
    for a in range(n0):
        for b in range(n1):
            y[a, b] = sum(x[p, q] * h[(a - p) % n0, (b - q) % n1] for p in range(n0) for q in range(n1))
    return y


def test_real_convolution_is_circular_convolution():
    """The real-application convolution with kernel spectra rfftn(h) convolves
    each coordinate (independent: plane (k, c)) or sums a matrix row."""
    rng = np.random.default_rng(9)
    dims = [5, 6]
    xs = rng.standard_normal((2, 5, 6))
    hs = rng.standard_normal((2, 2, 5, 6))  # [kernel][coordinate]
    spec = np.fft.rfftn(hs, axes=(2, 3)).reshape(-1)
    y = o.convolution_real(xs, spec, dims, coords=2, kernel_count=2).reshape(2, 2, 5, 6)
    for k in range(2):
        for c in range(2):
            assert np.allclose(y[k, c], _circ_conv2(xs[c], hs[k, c]), atol=1e-12)
    hm = rng.standard_normal((4, 5, 6))  # 2x2 matrix planes, row-major
    ym = o.convolution_real(xs, np.fft.rfftn(hm, axes=(1, 2)).reshape(-1), dims, coords=2, matrix=2).reshape(2, 5, 6)
    for oc in range(2):
        ref = _circ_conv2(xs[0], hm[2 * oc]) + _circ_conv2(xs[1], hm[2 * oc + 1])
        assert np.allclose(ym[oc], ref, atol=1e-12)


# ------------------------------------------- mixed-storage FFTW corpora

@pytest.mark.parametrize("corpus", ["fftw_precision_medium_f16_storage_v1.txt",
                                    "fftw_precision_medium_f64_f32_storage_v1.txt"])
def test_mixed_storage_corpora_pin_the_oracle(corpus):
    """As the reference's CPU half of these corpora
    (fftw_medium_f16_storage_golden.rs:264-300, ..._f64_f32_storage_golden.rs:
    264-300): the f64 oracle on the storage-rounded inputs, rounded to the
    storage type, reproduces FFTW's committed bits. Exact for all but values
    within the oracle's f64 error of a rounding boundary: at most 1 ulp apart
    (or, for the bins FFTW returns as exact zeros, within the oracle's f64
    error of 2e-10 * N, the reference's CPU fixture tolerance) and at least
    99.5% identical over the corpus."""
    import golden_bits as gb
    width, cases = gb.parse(os.path.join(GOLDEN, corpus))
    total = exact = 0
    for name, case in cases.items():
        x = gb.storage_input(case, width)
        got = gb.to_bits(gb.scalars(gb.oracle_output(case, x), case["kind"]), width)
        d = gb.ulps(got, case["bits"], width)
        n = int(np.prod(case["shape"]))
        near = np.abs(gb.from_bits(got, width) - gb.from_bits(case["bits"], width)) <= 2e-10 * n
        assert np.all((d <= 1) | near), (name, int(d.max()))
        total += d.size
        exact += int(np.sum(d == 0))
    assert exact >= 0.995 * total, (exact, total)
