"""Pins of the CPU index maps (oracle/index_maps.py) used by the bit-exact
GPU addressing tests: closed forms (digit reversal), and the same maps with
real butterflies and twiddles reproducing numpy.fft (pocketfft)."""
import numpy as np
import pytest

from oracle import index_maps as im


def digit_reversal(radices):
    """Mixed-radix digit reversal: i = d0 + r0*(d1 + r1*(d2 + ...)) maps to
    the number whose most significant digit is d0."""
    out = []
    for i in range(int(np.prod(radices))):
        t, v = i, 0
        for r in radices:
            v = v * r + t % r
            t //= r
        out.append(v)
    return np.array(out)


@pytest.mark.parametrize("radices", [[2] * 9, [16, 8, 8], [8, 3, 7, 7, 7], [9, 9, 5], [4, 9, 9], [3, 5, 7],
                                     [16, 16, 16], [13, 11, 2]])
def test_identity_stockham_is_digit_reversal(radices):
    n = int(np.prod(radices))
    p = im.stockham_perm(n, radices)
    assert np.array_equal(p, digit_reversal(radices))
    assert np.array_equal(np.sort(p), np.arange(n))


@pytest.mark.parametrize("radices", [[16, 8, 8], [8, 3, 7, 7, 7], [9, 9, 5], [4, 9, 9], [16, 16, 4], [7, 11, 13],
                                     [2, 2, 2, 3]])
def test_stage_maps_compute_the_dft(radices):
    n = int(np.prod(radices))
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n) + 1j * rng.standard_normal(n)
    np.testing.assert_allclose(im.stockham_fft(x, radices), np.fft.fft(x), rtol=0, atol=1e-9 * np.sqrt(n))
    np.testing.assert_allclose(im.stockham_fft(x, radices, +1), np.fft.ifft(x) * n, rtol=0, atol=1e-9 * np.sqrt(n))


@pytest.mark.parametrize("n1,rad1,n2,rad2", [(16, [4, 4], 8, [8]), (27, [3, 9], 20, [4, 5]), (64, [8, 8], 64, [8, 8])])
def test_four_step_map_computes_the_dft(n1, rad1, n2, rad2):
    """Four-step with real math on the same placement as four_step_perm:
    column FFTs over n1, twiddle exp(-2 pi i k1 n2 / M), row FFTs over n2,
    output at k1 + n1*k2."""
    m = n1 * n2
    rng = np.random.default_rng(m)
    x = rng.standard_normal(m) + 1j * rng.standard_normal(m)
    w = x.reshape(n1, n2).astype(np.complex128)
    cols = np.stack([im.stockham_fft(w[:, c], rad1) for c in range(n2)], axis=1)
    k1 = np.arange(n1)[:, None]
    c = np.arange(n2)[None, :]
    cols = cols * np.exp(-2j * np.pi * k1 * c / m)
    out = np.empty(m, dtype=np.complex128)
    for r in range(n1):
        out[r + n1 * np.arange(n2)] = im.stockham_fft(cols[r], rad2)
    np.testing.assert_allclose(out, np.fft.fft(x), rtol=0, atol=1e-9 * np.sqrt(m))
    # and the identity-butterfly placement is the permutation four_step_perm describes
    src = im.four_step_perm(n1, rad1, n2, rad2)
    sa, sb = im.stockham_perm(n1, rad1), im.stockham_perm(n2, rad2)
    for kk1 in range(n1):
        for kk2 in range(n2):
            assert src[kk1 + n1 * kk2] == sa[kk1] * n2 + sb[kk2]


def _four_step_fft(x, n1, rad1, n2, rad2, row_fft=None):
    m = n1 * n2
    w = x.reshape(n1, n2).astype(np.complex128)
    cols = np.stack([im.stockham_fft(w[:, c], rad1) for c in range(n2)], axis=1)
    cols = cols * np.exp(-2j * np.pi * np.arange(n1)[:, None] * np.arange(n2)[None, :] / m)
    out = np.empty(m, dtype=np.complex128)
    for r in range(n1):
        out[r + n1 * np.arange(n2)] = row_fft(cols[r]) if row_fft else im.stockham_fft(cols[r], rad2)
    return out


@pytest.mark.parametrize("n1,rad1,m1,rad2,m2,rad3", [(16, [4, 4], 16, [16], 16, [4, 4]), (27, [3, 9], 9, [9], 9, [3, 3]),
                                                     (12, [3, 4], 8, [8], 4, [4])])
def test_three_pass_map_computes_the_dft(n1, rad1, m1, rad2, m2, rad3):
    """Three uploads with real math on the placement of three_pass_perm: a
    four-step over n1 x n2 whose row FFTs are four-steps over m1 x m2."""
    n2 = m1 * m2
    m = n1 * n2
    rng = np.random.default_rng(m)
    x = rng.standard_normal(m) + 1j * rng.standard_normal(m)
    out = _four_step_fft(x, n1, rad1, n2, None, row_fft=lambda r: _four_step_fft(r, m1, rad2, m2, rad3))
    np.testing.assert_allclose(out, np.fft.fft(x), rtol=0, atol=1e-9 * np.sqrt(m))
    src = im.three_pass_perm(n1, rad1, m1, rad2, m2, rad3)
    assert np.array_equal(np.sort(src), np.arange(m))
    sa, sub = im.stockham_perm(n1, rad1), im.four_step_perm(m1, rad2, m2, rad3)
    for kk1 in range(0, n1, 3):
        for kk2 in range(0, n2, 5):
            assert src[kk1 + n1 * kk2] == sa[kk1] * n2 + sub[kk2]


def test_bluestein_maps_zero_fill_and_truncate():
    n, m = 11, 24
    src = im.bluestein_single_perm(n, m, [2, 3, 4])
    assert src.shape == (n,)
    s = im.stockham_perm(m, [2, 3, 4])
    for k in range(n):
        v = s[s[k]]
        assert src[k] == (v if v < n else -1)
    src3 = im.bluestein_three_pass_perm(n, 6, [2, 3], 4, [4], [3, 2])
    assert src3.shape == (n,)
    assert ((src3 >= -1) & (src3 < n)).all()


# ------------------------------------------- Bluestein maps by brute force

def _stage_moves(line, radices):
    """One identity-butterfly Stockham pass over a list of tags, element by
    element: the butterfly b of a radix-R stage after radices multiplying to
    P reads in[b + i*N/R] and writes its i-th input to out[j + (b - j)*R + i*P],
    j = b mod P (kernel_ir.rs:1486-1727)."""
    n = len(line)
    p = 1
    for r in radices:
        out = [None] * n
        for b in range(n // r):
            j = b % p
            for i in range(r):
                out[j + (b - j) * r + i * p] = line[b + i * (n // r)]
        assert None not in out
        line = out
        p *= r
    return line


def _bluestein_single_sim(n, m, radices):
    """x zero-padded to M (tag -1), forward FFT_M, spectrum multiply (in
    place), inverse FFT_M with the same radices, truncation to N
    (bluestein_ir.rs:933-1089), all by explicit moves."""
    a = list(range(n)) + [-1] * (m - n)
    a = _stage_moves(a, radices)
    a = _stage_moves(a, radices)
    return np.array(a[:n])


def _bluestein_three_pass_sim(n, n1, rad1, n2, rad2, rad3):
    """The same over M = n1 * n2 in three passes on the matrix a[e*n2 + c]:
    columns (length n1, rad1) in place, rows (length n2: forward rad2,
    multiply, inverse rad2) in place, inverse columns (rad3) in place,
    truncation to N."""
    m = n1 * n2
    a = list(range(n)) + [-1] * (m - n)
    for c in range(n2):
        col = _stage_moves([a[e * n2 + c] for e in range(n1)], rad1)
        for e in range(n1):
            a[e * n2 + c] = col[e]
    for e in range(n1):
        row = _stage_moves(_stage_moves(a[e * n2:(e + 1) * n2], rad2), rad2)
        a[e * n2:(e + 1) * n2] = row
    for c in range(n2):
        col = _stage_moves([a[e * n2 + c] for e in range(n1)], rad3)
        for e in range(n1):
            a[e * n2 + c] = col[e]
    return np.array(a[:n])


@pytest.mark.parametrize("n,m,radices", [(11, 24, [2, 3, 4]), (11, 24, [4, 3, 2]), (5, 9, [3, 3]),
                                         (13, 32, [2, 4, 4]), (7, 16, [16]), (17, 45, [5, 3, 3])])
def test_bluestein_single_map_by_simulation(n, m, radices):
    assert np.array_equal(im.bluestein_single_perm(n, m, radices), _bluestein_single_sim(n, m, radices))


@pytest.mark.parametrize("n,n1,rad1,n2,rad2,rad3", [(11, 6, [2, 3], 4, [4], [3, 2]),
                                                    (13, 4, [4], 8, [2, 4], [2, 2]),
                                                    (23, 9, [3, 3], 6, [3, 2], [3, 3]),
                                                    (29, 10, [5, 2], 6, [2, 3], [2, 5])])
def test_bluestein_three_pass_map_by_simulation(n, n1, rad1, n2, rad2, rad3):
    got = im.bluestein_three_pass_perm(n, n1, rad1, n2, rad2, rad3)
    assert np.array_equal(got, _bluestein_three_pass_sim(n, n1, rad1, n2, rad2, rad3))


RADER_PRIMES = [17, 19, 23, 29, 31, 47, 83, 89, 97, 113, 193, 257]


@pytest.mark.parametrize("p", RADER_PRIMES)
def test_rader_butterfly_is_the_dft(p):
    """The Rader butterfly's gather (a[s] = x[g^-s]), kernel and scatter
    (X[g^m] = x0 + conv[m], X[0] = x0 + sum a) with the planner's generator
    compute the p-point DFT: pins the maps the identity forms reuse."""
    from oracle import oracle as orc
    rng = np.random.default_rng(p)
    x = rng.standard_normal((3, p)) + 1j * rng.standard_normal((3, p))
    y = im.rader_butterfly(x, p, orc.primitive_root(p))
    assert np.max(np.abs(y - np.fft.fft(x, axis=-1))) <= 1e-12 * p


@pytest.mark.parametrize("p", RADER_PRIMES)
def test_rader_identity_forms(p):
    """Closed forms of the identity Rader butterflies: with the unit impulse
    X[k] = x0 + x[k^-1 mod p] (k >= 1) and X[0] = x0 + x[1]; with the
    convolution's identity Stockham maps (FFT mode) and an identity sub-map,
    the same."""
    from oracle import oracle as orc
    g = orc.primitive_root(p)
    x = np.arange(p, dtype=np.float64) * 1000 + 7
    y = im.rader_butterfly(x, p, g, "impulse")
    inv = np.array([pow(int(k), p - 2, p) for k in range(1, p)])
    assert y[0] == x[0] + x[1]
    assert np.array_equal(y[1:], x[0] + x[inv])
    assert np.array_equal(im.rader_butterfly(x, p, g, "maps", np.arange(p - 1)), y)


@pytest.mark.parametrize("radices", [[2, 17], [17, 4], [3, 17, 17], [29, 31, 2], [89, 4], [8, 97], [257, 2, 2]])
def test_stockham_identity_maps(radices):
    """stockham_identity: without Rader radices it is the identity-butterfly
    Stockham permutation; with them, replacing every identity Rader
    butterfly by the real one (a DFT, as pinned above) gives the plain
    stage maps with real butterflies, i.e. numpy.fft."""
    from oracle import oracle as orc
    n = int(np.prod(radices))
    rng = np.random.default_rng(n)
    x = rng.standard_normal((2, n)) + 1j * rng.standard_normal((2, n))
    plain = [r for r in radices if r <= 16]
    if plain:
        m = int(np.prod(plain))
        xs = x[:, :m]
        assert np.array_equal(im.stockham_identity(xs, plain), xs[:, im.stockham_perm(m, plain)])
    # the same stage loop with real butterflies and twiddles is stockham_fft
    assert np.max(np.abs(im.stockham_fft(x[0], radices) - np.fft.fft(x[0]))) <= 1e-10 * n
    rader = {r: (orc.primitive_root(r), None) for r in radices if r > 16}
    y = im.stockham_identity(x, radices, rader)
    # every output is x0 of its butterfly plus one named input: integer tags stay exact
    t = np.arange(2 * n, dtype=np.float64).reshape(2, n)
    yt = im.stockham_identity(t, radices, rader)
    assert np.array_equal(yt, np.round(yt)) and y.shape == x.shape
