"""ctypes binding of the CPU oracle (liboracle.so built from vkfft_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the MI355X path. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

Every transform restates vkfft-rs `src/reference.rs` (f64, recursive
prime-radix decimation with Bluestein fallback); see vkfft_oracle.c for the
per-function citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_c_double_p = ctypes.POINTER(ctypes.c_double)
_c_size_p = ctypes.POINTER(ctypes.c_size_t)


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sz = ctypes.c_size_t
        L.vko_dft.argtypes = [_c_double_p, _c_double_p, sz, ctypes.c_int, ctypes.c_int]
        L.vko_fft.argtypes = [_c_double_p, _c_double_p, sz, ctypes.c_int, ctypes.c_int]
        L.vko_fft_batch.argtypes = [_c_double_p, _c_double_p, sz, sz, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int]
        L.vko_r2c_batch.argtypes = [_c_double_p, _c_double_p, sz, sz, ctypes.c_int]
        L.vko_c2r_batch.argtypes = [_c_double_p, _c_double_p, sz, sz, ctypes.c_int, ctypes.c_int]
        L.vko_r2r_batch.argtypes = [_c_double_p, _c_double_p, sz, sz, ctypes.c_int, ctypes.c_int]
        L.vko_fft_nd.argtypes = [_c_double_p, _c_double_p, _c_size_p, sz, sz, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int]
        L.vko_next_smooth_at_least.argtypes = [sz, _c_size_p, sz]
        L.vko_next_smooth_at_least.restype = sz
        L.vko_prime_factorization.argtypes = [sz, _c_size_p, sz]
        L.vko_prime_factorization.restype = sz
        L.vko_primitive_root.argtypes = [sz]
        L.vko_primitive_root.restype = sz
        for name in ("vko_fill_uniform", "vko_fill_normal"):
            getattr(L, name).argtypes = [_c_double_p, sz, ctypes.c_uint64]
        for name in ("vko_fill_uniform_f32", "vko_fill_normal_f32"):
            getattr(L, name).argtypes = [ctypes.POINTER(ctypes.c_float), sz, ctypes.c_uint64]
        L.vko_fixture_complex_v1.argtypes = [sz, _c_double_p]
        L.vko_fixture_real_v1.argtypes = [sz, _c_double_p]
        L.vko_fixture_complex_f32_v1.argtypes = [sz, ctypes.POINTER(ctypes.c_float)]
        L.vko_fixture_real_f32_v1.argtypes = [sz, ctypes.POINTER(ctypes.c_float)]
        for name in ("vko_dft", "vko_fft", "vko_fft_batch", "vko_r2c_batch", "vko_c2r_batch",
                     "vko_fft_nd"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _dp(a: np.ndarray):
    return a.ctypes.data_as(_c_double_p)


def _as_c128(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.complex128))


def _sign(direction: str) -> int:
    if direction not in ("forward", "inverse"):
        raise ValueError(f"direction must be 'forward' or 'inverse', got {direction!r}")
    return -1 if direction == "forward" else 1


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed (rc={rc})")


def dft(x, direction="forward", normalize=False) -> np.ndarray:
    """reference::dft (src/reference.rs:14-23)."""
    x = _as_c128(x)
    out = np.empty_like(x)
    _check(lib().vko_dft(_dp(x), _dp(out), x.size, _sign(direction), int(normalize)), "dft")
    return out


def fft(x, direction="forward", normalize=False) -> np.ndarray:
    """reference::fft on one sequence (src/reference.rs:25-42)."""
    x = _as_c128(x)
    out = np.empty_like(x)
    _check(lib().vko_fft(_dp(x), _dp(out), x.size, _sign(direction), int(normalize)), "fft")
    return out


def fft_batch(x, n: int, direction="forward", normalize=False, threads=1) -> np.ndarray:
    """reference::fft over batch*n contiguous values, batch split over threads."""
    x = _as_c128(x).reshape(-1)
    if n == 0 or x.size % n:
        raise ValueError("input size must be a multiple of n")
    out = np.empty_like(x)
    _check(lib().vko_fft_batch(_dp(x), _dp(out), n, x.size // n, _sign(direction),
                               int(normalize), int(threads)), "fft_batch")
    return out


def r2c_batch(x, n: int, threads=1) -> np.ndarray:
    """Full-complex R2C truncated to n/2+1 (src/real_ir.rs:935-946)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float64)).reshape(-1)
    batch = x.size // n
    out = np.empty(batch * (n // 2 + 1), dtype=np.complex128)
    _check(lib().vko_r2c_batch(_dp(x), _dp(out), n, batch, int(threads)), "r2c")
    return out


def c2r_batch(x, n: int, normalize=False, threads=1) -> np.ndarray:
    """Hermitian-expansion C2R (src/real_ir.rs:1038-1053)."""
    x = _as_c128(x).reshape(-1)
    h = n // 2 + 1
    batch = x.size // h
    out = np.empty(batch * n, dtype=np.float64)
    _check(lib().vko_c2r_batch(_dp(x), _dp(out), n, batch, int(normalize), int(threads)), "c2r")
    return out


R2R_KINDS = {"dct1": 0, "dct2": 1, "dct3": 2, "dct4": 3, "dst1": 4, "dst2": 5, "dst3": 6, "dst4": 7}


def r2r_batch(x, n: int, kind: str, threads=1) -> np.ndarray:
    """Direct DCT/DST (FFTW REDFT/RODFT, unnormalized; src/r2r_ir.rs:2351-2434)."""
    x = np.ascontiguousarray(x, dtype=np.float64).reshape(-1)
    batch = x.size // n
    out = np.empty(batch * n, dtype=np.float64)
    _check(lib().vko_r2r_batch(_dp(x), _dp(out), n, batch, R2R_KINDS[kind], int(threads)), "r2r")
    return out


def fft_nd(x, dims, batch=1, direction="forward", normalize=False, threads=1) -> np.ndarray:
    """Separable N-D C2C, axes last to first (src/nd_ir.rs:1303-1337)."""
    x = _as_c128(x).reshape(-1)
    d = (ctypes.c_size_t * len(dims))(*dims)
    out = np.empty_like(x)
    _check(lib().vko_fft_nd(_dp(x), _dp(out), d, len(dims), batch, _sign(direction),
                            int(normalize), int(threads)), "fft_nd")
    return out


def conv_plane_index(m: int, symmetric: bool, out_coord: int, in_coord: int) -> int:
    """ConvolutionMatrixLayout::kernel_plane_index (src/convolution_ir.rs:128-147):
    row-major M*M planes, or the upper triangle row by row when symmetric."""
    if not symmetric:
        return out_coord * m + in_coord
    j, l = out_coord, in_coord
    return l * m - l * l + j if l < j else j * m - j * j + l


def convolution(x, spectrum, dims, batch=1, matrix=0, symmetric=False, kernel_count=1,
                conj_sequence=False, cross_power=False, threads=1, backend="oracle") -> np.ndarray:
    """performConvolution (execute_convolution_ir / execute_nd_convolution_ir,
    src/convolution_ir.rs:4252-4440): forward FFT of every [system][coordinate]
    tensor, multiply by the kernel spectrum [kernel][plane][tensor]
    (ConvolutionMultiplyPolicy::apply, :58-80: conj of the sequence, then
    division by the modulus with no zero guard), normalized inverse FFT.
    A matrix layout sums over input coordinates and normalizes the row sum.
    backend "numpy" runs the two transforms with numpy.fft (pocketfft) instead
    of the oracle's restatement, for f64 checks below the oracle's own error."""
    dims = list(dims)
    t = int(np.prod(dims))
    coords = matrix if matrix else 1
    x = _as_c128(x).reshape(-1)
    k = _as_c128(spectrum).reshape(-1)
    nd = len(dims) > 1

    def transform(v, systems, direction, normalize):
        if backend == "numpy":
            a = v.reshape((systems,) + tuple(dims))
            axes = tuple(range(1, len(dims) + 1))
            r = np.fft.fftn(a, axes=axes) if direction == "forward" else np.fft.ifftn(a, axes=axes)
            return r.reshape(-1)
        if nd:
            return fft_nd(v, dims, systems, direction, normalize, threads)
        return fft_batch(v, dims[0], direction, normalize, threads)

    spec = transform(x, batch * coords, "forward", False).reshape(batch, coords, t)
    out_systems = kernel_count if kernel_count > 1 else batch
    planes = (matrix * (matrix + 1) // 2 if symmetric else matrix * matrix) if matrix else 1
    kern = k.reshape(kernel_count, planes, t)
    seq = np.conj(spec) if conj_sequence else spec
    prod = np.zeros((out_systems, coords, t), dtype=np.complex128)
    for s in range(out_systems):
        s_in, kid = (0, s) if kernel_count > 1 else (s, 0)
        for o in range(coords):
            if matrix:
                acc = np.zeros(t, dtype=np.complex128)
                for i in range(coords):
                    acc += seq[s_in, i] * kern[kid, conv_plane_index(matrix, symmetric, o, i)]
            else:
                acc = seq[s_in, o] * kern[kid, 0]
            if cross_power:
                acc = acc * (1.0 / np.sqrt(acc.real ** 2 + acc.imag ** 2))
            prod[s, o] = acc
    return transform(prod.reshape(-1), out_systems * coords, "inverse", True)


def convolution_real(x, spectrum, dims, coords=1, matrix=0, symmetric=False, kernel_count=1,
                     conj_sequence=False, cross_power=False) -> np.ndarray:
    """Real-application performConvolution (execute_nd_real_convolution_ir,
    src/convolution_ir.rs:4185-4251), batch 1: rfftn of the `coords` real
    tensors, multiply over the compact [.., N/2+1] spectra (matrix: output
    (k, o) sums input i with plane (k, plane(o, i)); otherwise output (k, c)
    uses plane (k, c)), normalized irfftn of the K * coords products. The
    transforms are numpy's (pocketfft); the kernel spectrum must be Hermitian
    (the rfftn of real kernels) for the inverse to be well defined."""
    dims = list(dims)
    axes = tuple(range(1, len(dims) + 1))
    h = dims[-1] // 2 + 1
    t = int(np.prod(dims[:-1])) * h
    xs = np.asarray(x, dtype=np.float64).reshape((coords,) + tuple(dims))
    spec = np.fft.rfftn(xs, axes=axes).reshape(coords, t)
    seq = np.conj(spec) if conj_sequence else spec
    planes = (matrix * (matrix + 1) // 2 if symmetric else matrix * matrix) if matrix else coords
    kern = np.asarray(spectrum, dtype=np.complex128).reshape(kernel_count, planes, t)
    prod = np.zeros((kernel_count, coords, t), dtype=np.complex128)
    for kid in range(kernel_count):
        for o in range(coords):
            if matrix:
                acc = np.zeros(t, dtype=np.complex128)
                for i in range(coords):
                    acc += seq[i] * kern[kid, conv_plane_index(matrix, symmetric, o, i)]
            else:
                acc = seq[o] * kern[kid, o]
            if cross_power:
                acc = acc * (1.0 / np.sqrt(acc.real ** 2 + acc.imag ** 2))
            prod[kid, o] = acc
    shaped = prod.reshape((kernel_count * coords,) + tuple(dims[:-1]) + (h,))
    return np.fft.irfftn(shaped, s=dims, axes=axes).reshape(-1)


def next_smooth_at_least(target: int, primes=(2, 3, 5, 7)) -> int:
    p = (ctypes.c_size_t * len(primes))(*primes)
    return int(lib().vko_next_smooth_at_least(target, p, len(primes)))


def prime_factorization(value: int):
    buf = (ctypes.c_size_t * 64)()
    n = lib().vko_prime_factorization(value, buf, 64)
    return [int(buf[i]) for i in range(n)]


def primitive_root(prime: int):
    g = int(lib().vko_primitive_root(prime))
    return g if g else None


def uniform(count: int, seed: int, dtype=np.float64) -> np.ndarray:
    """Seeded uniform[-1,1): splitmix64 -> xoshiro256**, u53*2^-53*2-1."""
    if np.dtype(dtype) == np.float32:
        out = np.empty(count, dtype=np.float32)
        lib().vko_fill_uniform_f32(out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), count, seed)
    else:
        out = np.empty(count, dtype=np.float64)
        lib().vko_fill_uniform(_dp(out), count, seed)
    return out


def normal(count: int, seed: int, dtype=np.float64) -> np.ndarray:
    """Seeded normal(0,1) by Box-Muller in f64 (then rounded for f32)."""
    if np.dtype(dtype) == np.float32:
        out = np.empty(count, dtype=np.float32)
        lib().vko_fill_normal_f32(out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), count, seed)
    else:
        out = np.empty(count, dtype=np.float64)
        lib().vko_fill_normal(_dp(out), count, seed)
    return out


def complex_uniform(count: int, seed: int, dtype=np.complex64) -> np.ndarray:
    """count complex values with re/im i.i.d. uniform[-1,1), interleaved draw order."""
    real_dtype = np.float32 if np.dtype(dtype) == np.complex64 else np.float64
    return uniform(2 * count, seed, real_dtype).view(dtype)


def rel_l2(actual, expected) -> float:
    """||a - e||_2 / ||e||_2 accumulated in f64."""
    a = np.asarray(actual).astype(np.complex128 if np.iscomplexobj(actual) else np.float64).ravel()
    e = np.asarray(expected).astype(np.complex128 if np.iscomplexobj(expected) else np.float64).ravel()
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


def precision_metrics(actual, expected) -> dict:
    """Sample-11 metrics of src/precision.rs:31-101 (avg/max abs difference and
    avg/max per-bin relative eps; eps falls back to the difference when the
    reference magnitude is below f64::MIN_POSITIVE)."""
    a = np.asarray(actual).astype(np.complex128).ravel()
    e = np.asarray(expected).astype(np.complex128).ravel()
    if a.size != e.size or a.size == 0:
        raise ValueError("precision metrics need equal, non-empty inputs")
    diff = np.abs(a - e)
    ref = np.abs(e)
    tiny = np.finfo(np.float64).tiny
    eps = np.where(ref > tiny, diff / np.where(ref > tiny, ref, 1.0), diff)
    return {"avg_difference": float(diff.mean()), "max_difference": float(diff.max()),
            "avg_eps": float(eps.mean()), "max_eps": float(eps.max())}


def fixture_input(formula: str, count: int) -> np.ndarray:
    """Inputs of the FFTW fixtures (generate_fftw_golden.c:8-31): complex-v1 and
    real-v1 in f64, complex-f32-v1 and real-f32-v1 computed in C float."""
    L = lib()
    fp = ctypes.POINTER(ctypes.c_float)
    if formula == "complex-v1":
        out = np.empty(count, dtype=np.complex128)
        L.vko_fixture_complex_v1(count, out.ctypes.data_as(_c_double_p))
    elif formula == "real-v1":
        out = np.empty(count, dtype=np.float64)
        L.vko_fixture_real_v1(count, _dp(out))
    elif formula == "complex-f32-v1":
        out = np.empty(count, dtype=np.complex64)
        L.vko_fixture_complex_f32_v1(count, out.ctypes.data_as(fp))
    elif formula == "real-f32-v1":
        out = np.empty(count, dtype=np.float32)
        L.vko_fixture_real_f32_v1(count, out.ctypes.data_as(fp))
    else:
        raise ValueError(f"unknown fixture input formula {formula!r}")
    return out


def parse_fixture(path: str) -> dict:
    """Parses a vkfft-rs FFTW fixture corpus (tests/fixtures/*.txt format)."""
    cases = {}
    lines = open(path).read().splitlines()
    i = 0
    header = {}
    while i < len(lines) and not lines[i].startswith("case "):
        k, _, v = lines[i].partition(" ")
        header[k] = v
        i += 1
    while i < len(lines):
        name = lines[i].split()[1]
        i += 1
        meta = {}
        while i < len(lines) and lines[i].split()[0] in ("kind", "length", "shape", "input", "output"):
            k, _, v = lines[i].partition(" ")
            meta[k] = v
            i += 1
            if k == "output" and "length" not in meta:
                break
        rows = []
        while i < len(lines) and not lines[i].startswith("case "):
            if lines[i].startswith("output "):
                meta["output"] = lines[i].split()[1]
                meta["_split"] = len(rows)
            else:
                rows.append([float(t) for t in lines[i].split()])
            i += 1
        cases[name] = {"meta": meta, "rows": rows}
    return {"header": header, "cases": cases}
