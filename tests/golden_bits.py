"""Parser and ulp helpers for the reference's mixed-storage FFTW corpora
(tests/golden/fftw_precision_medium_f16_storage_v1.txt and
..._f64_f32_storage_v1.txt, copied from vkfft-rs tests/fixtures/): FFTW 3.3.9
outputs rounded to the storage type, one hex bit pattern per scalar
(vkfft-rs tests/fftw_medium_f16_storage_golden.rs:21-89,
tests/fftw_medium_f64_f32_storage_golden.rs:21-89)."""
import numpy as np

from oracle import oracle as o

CASES = ["c2c-bluestein-n103", "c2c-rader-n257", "c2c-smooth-n1536", "c2c-large-smooth-n4096",
         "r2c-nd-17x34", "r2c-nd-64x64", "dct2-nd-17x34"]


def parse(path):
    lines = open(path).read().splitlines()
    assert lines[0] == "schema 1" and lines[1] == "source fftw-3.3.9"
    storage = lines[3].split()[1]
    width = {"binary16-rne-from-f32-v1": 16, "binary32-rne-from-f64-v1": 32}[storage]
    i, cases = 5, {}
    while i < len(lines):
        name = lines[i].split()[1]
        kind = lines[i + 1].split()[1]
        shape = [int(v) for v in lines[i + 2].split()[1:]]
        formula = lines[i + 3].split()[1]
        count = int(lines[i + 4].split()[1])
        rows = lines[i + 5:i + 5 + count]
        bits = np.array([int(t, 16) for r in rows for t in r.split()],
                        dtype=np.uint16 if width == 16 else np.uint32)
        assert bits.size == count * (1 if kind == "dct2" else 2)
        cases[name] = {"kind": kind, "shape": shape, "input": formula, "count": count, "bits": bits}
        i += 5 + count
    assert list(cases) == CASES, list(cases)
    return width, cases


def ordered(bits, width):
    """Sign-magnitude bit patterns -> integers ordered like the values
    (half_ordered / f32_ordered of the reference tests)."""
    b = bits.astype(np.int64)
    sign = 1 << (width - 1)
    return np.where(b & sign, sign - (b & (sign - 1)), sign + b)


def ulps(a_bits, b_bits, width):
    return np.abs(ordered(a_bits, width) - ordered(b_bits, width))


def to_bits(values, width):
    """f64 results -> storage bits: Binary16::from_f32(v as f32) (round to
    nearest even twice) or (v as f32).to_bits()."""
    v = np.asarray(values, dtype=np.float64).astype(np.float32)
    return v.astype(np.float16).view(np.uint16) if width == 16 else v.view(np.uint32)


def from_bits(bits, width):
    return (bits.view(np.float16) if width == 16 else bits.view(np.float32)).astype(np.float32)


def storage_input(case, width):
    """The case's input as the device buffer holds it: the f32 formula
    (complex-f32-v1 / real-f32-v1, computed in C float), rounded to binary16
    for the F16-storage corpus (complex/real-f16-storage-v1)."""
    n = int(np.prod(case["shape"]))
    formula = "complex-f32-v1" if case["kind"] == "c2c" else "real-f32-v1"
    x = o.fixture_input(formula, n)
    if width == 16:
        s = x.view(np.float32) if np.iscomplexobj(x) else x
        s = s.astype(np.float16).astype(np.float32)
        x = s.view(np.complex64) if np.iscomplexobj(x) else s
    return x


def oracle_output(case, x):
    """The oracle (C restatement of reference.rs, f64) on the storage input,
    in the corpus's output order: full spectrum for C2C, the compact
    [rows][cols/2+1] spectrum for R2C, DCT-II along every axis for dct2."""
    shape = case["shape"]
    if case["kind"] == "c2c":
        return o.fft(x.astype(np.complex128))
    if case["kind"] == "r2c":
        full = o.fft_nd(x.astype(np.complex128), shape).reshape(shape)
        return full[:, : shape[1] // 2 + 1].reshape(-1)
    r, c = shape
    a = o.r2r_batch(x.astype(np.float64), c, "dct2").reshape(r, c)
    return o.r2r_batch(np.ascontiguousarray(a.T).reshape(-1), r, "dct2").reshape(c, r).T.reshape(-1)


def scalars(values, kind):
    v = np.asarray(values)
    return v.reshape(-1) if kind == "dct2" else np.stack([v.real, v.imag], axis=-1).reshape(-1)
