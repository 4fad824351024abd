"""A seeded random corpus of 1-D C2C transforms with boundary work: the four
storage / compute precisions, 1-D zero padding (spatial or frequency domain,
src/zero_pad_ir.rs:38-46, 607-617) and formatted batch strides, over lengths
whose plans carry that work in different places (one-upload Stockham, the
edge passes of two-upload lengths with fixed edge shapes, boundary passes
around other four-steps, Bluestein and Rader plans), in both directions with
and without normalization, against pocketfft's float64 FFT of the
storage-rounded, masked input. The corpus is fixed by its seed; a case's id
names it."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
SPATIAL, FREQ = vk.ZeroPaddingDomain.Spatial, vk.ZeroPaddingDomain.Frequency
LENGTHS = [64, 360, 1000, 1024, 4096, 97, 4099, 1 << 16, 1 << 18, 3 << 16, 100000]
TOL = {F32: 2e-5, F64: 2e-13, F16S: 1e-3, F64C: 1e-7}


def corpus(seed=31, count=100):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        n = int(rng.choice(LENGTHS))
        batch = int(rng.integers(1, 4))
        prec = [F32, F64, F16S, F64C][int(rng.integers(4))]
        direction = FWD if rng.random() < 0.5 else INV
        normalize = bool(rng.random() < 0.5)
        zero = None
        if rng.random() < 0.5:
            left = int(rng.integers(0, n))
            right = int(rng.integers(left + 1, n + 1))
            zero = (left, right, SPATIAL if rng.random() < 0.6 else FREQ)
        # a formatted batch stride (a few padding elements between transforms)
        # on plain precisions without zero padding
        stride = int(rng.integers(1, 9)) if (zero is None and prec in (F32, F64) and rng.random() < 0.5) else 0
        if prec in (F64, F64C) and n * batch > 1 << 18:
            continue  # keep the f64 reference quick
        cases.append((n, batch, prec, direction, normalize, zero, stride))
    return cases


def case_id(c):
    n, batch, prec, direction, normalize, zero, stride = c
    name = {F32: "f32", F64: "f64", F16S: "f16s", F64C: "f64c"}[prec]
    z = "" if zero is None else "-z{}:{}{}".format(zero[0], zero[1], "s" if zero[2] == SPATIAL else "f")
    return "{}-b{}-{}-{}{}{}{}".format(n, batch, name, "fwd" if direction == FWD else "inv",
                                       "-norm" if normalize else "", z, f"-bs+{stride}" if stride else "")


CASES = corpus()


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_edge_corpus(hip_ctx, case):
    n, batch, prec, direction, normalize, zero, stride = case
    cdt = np.complex128 if prec == F64 else np.complex64
    x = o.complex_uniform(n * batch, n % 991 + batch, cdt)
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(normalize)
    if zero is not None:
        c = c.with_zero_padding(0, zero[0], zero[1]).with_zero_padding_domain(zero[2])
    if stride:
        c = c.with_input_buffer_batch_stride(n + stride).with_output_buffer_batch_stride(n + stride + 1)
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, direction), x)
    xin = x.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64) if prec == F16S else x
    mask = np.zeros((batch, n), dtype=bool)
    if zero is not None:
        mask[:, zero[0]:zero[1]] = True
    mask = mask.reshape(-1)
    input_side = zero is not None and (direction == FWD) == (zero[2] == SPATIAL)
    if input_side:
        xin = np.where(mask, 0, xin)
    v = xin.astype(np.complex128).reshape(batch, n)
    ref = (np.fft.fft(v, axis=1) if direction == FWD else
           np.fft.ifft(v, axis=1) * (1 if normalize else n)).reshape(-1)
    if zero is not None and not input_side:
        ref = np.where(mask, 0, ref)
        assert (y[mask] == 0).all()
    if not np.any(ref):
        assert not np.any(y)  # the whole line is zero on one side
        return
    assert o.rel_l2(y, ref) <= TOL[prec]
