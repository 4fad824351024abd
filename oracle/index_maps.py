"""CPU index maps of the Stockham, four-step and Bluestein data movement.

Test infrastructure only: tests/ compare the index-map test build of the GPU
library (identity butterflies, twiddles, chirps and spectra) with these maps
bit for bit. Each map says where every output element comes from:
out[k] = in[src[k]] (src = -1: a zero of Bluestein padding).

- Stockham stage (src/kernel_ir.rs:1486-1727, math 4565-4608,
  docs/KERNEL_IR.md:20-37): for radix R after radices multiplying to P,
  butterfly b reads in(i) = b + i*N/R and writes out(q) = j + (b-j)*R + q*P
  with j = b mod P. With an identity butterfly, output q is input i = q.
- Four-step (FourStepMapping / StockhamIoMapping, src/kernel_ir.rs:201-227,
  826-864, 1042-1238): a line of M = N1*N2 is the matrix x[n1*N2 + n2]; the
  column pass transforms over n1 for each n2 and keeps the layout, the row
  pass transforms over n2 for each k1 and stores X[k1 + N1*k2].
- Three uploads (FourStepThreeUpload, src/kernel_ir.rs:1206-1236): the same
  four-step with each row of N2 = M1*M2 transformed by a four-step of its own.
- Bluestein (src/bluestein_ir.rs:933-1089): a = x zero-padded to M, FFT_M,
  spectrum multiply, inverse FFT_M, truncation to N.
- Rader butterfly of a prime p with generator g (src/rader_ir.rs:1957-2101,
  lut.rs:374-435): a[s] = x[g^-s], a length p-1 cyclic convolution with the
  kernel b[n] = exp(-2 pi i g^n / p), X[g^m] = x[0] + conv[m] and
  X[0] = x[0] + sum(a). Under identity arithmetic the index-map build
  replaces the kernel by the unit impulse and the sum by a[0] (direct
  multiplication), or runs the convolution's two length p-1 FFTs as their
  identity Stockham maps (FFT mode), so each output is x[0] plus one named
  input and the gather and scatter show bit for bit.

`stockham_fft` runs the same stage maps with real butterflies and twiddles;
tests pin the maps by checking it against numpy.fft (pocketfft) and the
closed form of radix-2 (bit reversal composed to natural order).
"""
from __future__ import annotations

import numpy as np


def stockham_perm(n: int, radices) -> np.ndarray:
    """src of an identity-butterfly Stockham pass over one line of length n."""
    assert int(np.prod(radices)) == n, (n, radices)
    cur = np.arange(n, dtype=np.int64)
    p = 1
    for r in radices:
        nb = n // r
        b = np.arange(nb, dtype=np.int64)
        j = b % p
        nxt = np.empty(n, dtype=np.int64)
        base = j + (b - j) * r
        for q in range(r):
            nxt[base + q * p] = cur[b + q * nb]
        cur = nxt
        p *= r
    return cur


def stockham_fft(x: np.ndarray, radices, sign: int = -1) -> np.ndarray:
    """The same stage maps with DFT butterflies and stage twiddles
    exp(sign*2*pi*i*j*i/(P*R)); natural-order DFT of x (pins the maps)."""
    n = x.size
    cur = x.astype(np.complex128)
    p = 1
    for r in radices:
        nb = n // r
        b = np.arange(nb)
        j = b % p
        v = np.stack([cur[b + i * nb] * np.exp(sign * 2j * np.pi * j * i / (p * r)) for i in range(r)])
        k = np.arange(r)
        w = np.exp(sign * 2j * np.pi * np.outer(k, k) / r)
        out = w @ v
        nxt = np.empty(n, dtype=np.complex128)
        base = j + (b - j) * r
        for q in range(r):
            nxt[base + q * p] = out[q]
        cur = nxt
        p *= r
    return cur


def rader_butterfly(x: np.ndarray, p: int, g: int, kernel=None, sub_perm=None) -> np.ndarray:
    """Rader butterflies of prime p over x[..., i], i = 0..p-1 (generator g).
    kernel None: the DFT's kernel exp(-2 pi i g^n / p) (the result is the
    p-point DFT); kernel "impulse": the identity-arithmetic form of the direct
    multiplication (conv[m] = a[m], a[0] for the sum); kernel "maps": the
    identity-arithmetic FFT form with the convolution's Stockham map
    sub_perm (f = a[sub_perm] for the sum, conv = f[sub_perm])."""
    L = p - 1
    pw = np.array([pow(g, e, p) for e in range(L)], dtype=np.int64)
    a = x[..., pw[(L - np.arange(L)) % L]]          # a[s] = x[g^-s]
    if kernel is None:
        b = np.exp(-2j * np.pi * pw / p)
        conv = np.fft.ifft(np.fft.fft(a, axis=-1) * np.fft.fft(b), axis=-1)
        dc = a.sum(axis=-1)
    elif kernel == "impulse":
        conv, dc = a, a[..., 0]
    else:
        f = a[..., sub_perm]
        conv, dc = f[..., sub_perm], f[..., 0]
    out = np.empty(x.shape, dtype=np.result_type(x, conv))
    out[..., 0] = x[..., 0] + dc
    out[..., pw] = x[..., :1] + conv
    return out


def stockham_identity(x: np.ndarray, radices, rader=None) -> np.ndarray:
    """The identity-arithmetic pass of a runtime radix list over lines
    x[batch, n]: the Stockham stage maps with identity butterflies, and for a
    prime radix above 16 the identity Rader butterfly. rader[p] = (g, None)
    for a direct-multiplication stage, (g, sub_perm) for an FFT-mode stage."""
    n = x.shape[-1]
    assert int(np.prod(radices)) == n, (n, radices)
    cur = x.copy()
    p = 1
    for r in radices:
        nb = n // r
        b = np.arange(nb, dtype=np.int64)
        j = b % p
        v = np.stack([cur[..., b + i * nb] for i in range(r)], axis=-1)  # [..., nb, r]
        if r > 16:
            g, sub = rader[r]
            v = rader_butterfly(v, r, g, "impulse" if sub is None else "maps", sub)
        nxt = np.empty_like(cur)
        base = j + (b - j) * r
        for q in range(r):
            nxt[..., base + q * p] = v[..., q]
        cur = nxt
        p *= r
    return cur


def four_step_perm(n1: int, rad1, n2: int, rad2) -> np.ndarray:
    """src of a two-pass line of M = n1*n2: X[k1 + n1*k2] = x[sa[k1]*n2 + sb[k2]]."""
    sa = stockham_perm(n1, rad1)
    sb = stockham_perm(n2, rad2)
    k1 = np.arange(n1)[:, None]
    k2 = np.arange(n2)[None, :]
    src = np.empty(n1 * n2, dtype=np.int64)
    src[(k1 + n1 * k2).reshape(-1)] = (sa[k1] * n2 + sb[k2]).reshape(-1)
    return src


def three_pass_perm(n1: int, rad1, m1: int, rad2, m2: int, rad3) -> np.ndarray:
    """src of a three-upload line of M = n1*n2, n2 = m1*m2 (FourStepThreeUpload,
    src/kernel_ir.rs:1206-1236, as a four-step whose rows are four-steps):
    X[k1 + n1*k2] = x[sa[k1]*n2 + sub[k2]], sub = four_step_perm(m1, m2)."""
    n2 = m1 * m2
    sa = stockham_perm(n1, rad1)
    sub = four_step_perm(m1, rad2, m2, rad3)
    k1 = np.arange(n1)[:, None]
    k2 = np.arange(n2)[None, :]
    src = np.empty(n1 * n2, dtype=np.int64)
    src[(k1 + n1 * k2).reshape(-1)] = (sa[k1] * n2 + sub[k2]).reshape(-1)
    return src


def bluestein_single_perm(n: int, m: int, radices) -> np.ndarray:
    """Whole Bluestein transform in one pass: forward and inverse FFT_M with
    the same radices; out[k] = a[s[s[k]]] for k < n, a = x zero-padded."""
    s = stockham_perm(m, radices)
    src = s[s[:n]]
    return np.where(src < n, src, -1)


def bluestein_three_pass_perm(n: int, n1: int, rad1, n2: int, rad2, rad3) -> np.ndarray:
    """Bluestein over M = n1*n2 in three passes: column pass (rad1) on the
    zero-padded input, row pass with forward and inverse FFTs (rad2), inverse
    column pass (rad3) with truncation: out[c + n2*e] = a[sa[sc[e]]*n2 + sb[sb[c]]]."""
    sa = stockham_perm(n1, rad1)
    sb = stockham_perm(n2, rad2)
    sc = stockham_perm(n1, rad3)
    e = np.arange(n1)[:, None]
    c = np.arange(n2)[None, :]
    m_idx = (c + n2 * e).reshape(-1)
    src_full = (sa[sc[e]] * n2 + sb[sb[c]]).reshape(-1)
    src = np.full(n1 * n2, -1, dtype=np.int64)
    src[m_idx] = src_full
    src = src[:n]
    return np.where(src < n, src, -1)


def apply_line_map(x: np.ndarray, dims, batch: int, axis_maps) -> np.ndarray:
    """Applies per-axis line maps (src arrays, axis order slowest..fastest)
    to a batch of row-major volumes; maps along distinct axes commute."""
    v = x.reshape((batch,) + tuple(dims))
    for ax, src in enumerate(axis_maps):
        if src is None:
            continue
        v = np.take(v, src, axis=ax + 1)
    return v.reshape(-1)


def gather(x: np.ndarray, src: np.ndarray, n: int, batch: int, out_len: int) -> np.ndarray:
    """Batched 1-D gather with zero fill: out[b, k] = x[b, src[k]] (0 where src < 0)."""
    xb = x.reshape(batch, n)
    safe = np.where(src >= 0, src, 0)
    out = xb[:, safe]
    out[:, src < 0] = 0
    assert out.shape[1] == out_len
    return out.reshape(-1)
