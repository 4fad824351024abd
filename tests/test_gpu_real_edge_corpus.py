"""A seeded random corpus of 1-D real transforms with boundary work: R2C
and normalized C2R in the four storage / compute precisions, with and
without a spatial zero interval over real elements (src/zero_pad_ir.rs:38-46;
an odd end splits a packed pair), over lengths whose plans carry that work
in different places (the edge variants of the one-upload even-length real
shapes, boundary passes around runtime-shape, odd-length and two-upload
plans), against pocketfft's float64 rfft / irfft of the storage-rounded
input. The corpus is fixed by its seed; a case's id names it."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
R2C, C2R = vk.TransformKind.RealToComplex, vk.TransformKind.ComplexToReal
LENGTHS = [64, 96, 100, 194, 360, 1000, 1001, 1024, 1536, 4096, 6144, 8198, 16384, 1 << 20]
TOL = {F32: 2e-5, F64: 2e-13, F16S: 2e-3, F64C: 1e-7}


def corpus(seed=13, count=60):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        n = int(rng.choice(LENGTHS))
        batch = int(rng.integers(1, 4))
        prec = [F32, F64, F16S, F64C][int(rng.integers(4))]
        kind = "r2c" if rng.random() < 0.5 else "c2r"
        zero = None
        if rng.random() < 0.5:
            left = int(rng.integers(0, n))
            zero = (left, int(rng.integers(left + 1, n + 1)))
        if n * batch > (1 << 20) and prec in (F64, F64C):
            continue  # keep the f64 reference quick
        cases.append((n, batch, prec, kind, zero))
    return cases


def case_id(c):
    n, batch, prec, kind, zero = c
    name = {F32: "f32", F64: "f64", F16S: "f16s", F64C: "f64c"}[prec]
    return "{}-b{}-{}-{}{}".format(n, batch, name, kind, "" if zero is None else "-z{}:{}".format(*zero))


CASES = corpus()


def f16_real(v):
    return v.astype(np.float16).astype(np.float32)


def f16_cpx(v):
    return v.astype(np.complex64).view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_real_edge_corpus(hip_ctx, case):
    n, batch, prec, kind, zero = case
    rdt = np.float64 if prec == F64 else np.float32
    mask = np.zeros((batch, n), dtype=bool)
    if zero is not None:
        mask[:, zero[0]:zero[1]] = True
    x = o.normal(n * batch, n % 977 + batch, rdt)
    xin = (f16_real(x) if prec == F16S else x).astype(np.float64).reshape(batch, n)
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
    if zero is not None:
        c = c.with_zero_padding(0, zero[0], zero[1])
    if kind == "r2c":
        y = hip_ctx.execute_transform(vk.TransformIr.build(c.with_transform(R2C), FWD), x)
        ref = np.fft.rfft(np.where(mask, 0, xin), axis=1).reshape(-1)
        if not np.any(ref):
            assert not np.any(y)
            return
        assert o.rel_l2(y, ref) <= TOL[prec]
        return
    S = np.fft.rfft(xin, axis=1)
    Sin = f16_cpx(S) if prec == F16S else S.astype(np.complex128 if prec == F64 else np.complex64)
    ir = vk.TransformIr.build(c.with_transform(C2R).with_inverse_normalization(True), INV)
    z = hip_ctx.execute_transform(ir, Sin.reshape(-1))
    expect = np.where(mask, 0, np.fft.irfft(Sin.astype(np.complex128), n, axis=1)).reshape(-1)
    m = mask.reshape(-1)
    assert (z[m] == 0).all()
    if not np.any(expect):
        assert not np.any(z)
        return
    assert o.rel_l2(z, expect) <= TOL[prec]
