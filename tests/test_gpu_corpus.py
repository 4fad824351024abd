"""A seeded random corpus of transforms across the planner's paths: rank 1 to
3, axis lengths drawn from sizes that select every axis algorithm (registered
and runtime-shape Stockham, split strided axes, Rader by FFT and by direct
multiplication, Rader stages inside mixed-radix lengths, Bluestein), C2C in
both directions with and without normalization (also in the two mixed
storage precisions), and R2C followed by C2R, against pocketfft's float64
transforms. The corpus is fixed by its seed; a case's id names its shape so
that a failure reproduces on its own."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
R2C, C2R = vk.TransformKind.RealToComplex, vk.TransformKind.ComplexToReal

# 1: copy axis; 2-16, 64-2048: registered shapes; 12, 30, 48, 100, 210, 360,
# 1000: smooth runtime or rule-built rows; 17, 31, 97: Rader (direct, FFT);
# 34, 226: Rader stages in mixed-radix lengths; 4099-sized primes stay out of
# N-D (their Bluestein axis needs more than one upload)
SIZES = [1, 2, 3, 5, 7, 8, 12, 16, 17, 30, 31, 34, 48, 64, 97, 100, 128, 210, 226, 256, 360, 512, 1000, 1024,
         2048]
MAX_ELEMS = 1 << 19


def corpus(seed=2026, count=200):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        rank = int(rng.integers(1, 4))
        dims = [int(rng.choice(SIZES)) for _ in range(rank)]
        if int(np.prod(dims)) > MAX_ELEMS or (rank == 1 and dims[0] == 1):
            continue
        batch = int(rng.integers(1, 4))
        prec = F32 if rng.random() < 0.6 else F64
        kind = "c2c" if rng.random() < 0.65 else "real"
        if kind == "real" and dims[-1] < 2:
            continue
        direction = FWD if rng.random() < 0.5 else INV
        normalize = bool(rng.random() < 0.5)
        if kind == "c2c" and rng.random() < 0.25:
            prec = F16S if prec == F32 else F64C
        cases.append((dims, batch, prec, kind, direction, normalize))
    return cases


def case_id(c):
    dims, batch, prec, kind, direction, normalize = c
    name = {F32: "f32", F64: "f64", F16S: "f16s", F64C: "f64c"}[prec]
    return "{}-b{}-{}-{}{}".format("x".join(map(str, dims)), batch, name, kind,
                                   "" if kind == "real" else ("-fwd" if direction == FWD else "-inv")
                                   + ("-norm" if normalize else ""))


CASES = corpus()


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_corpus(hip_ctx, case):
    dims, batch, prec, kind, direction, normalize = case
    axes = tuple(range(1, len(dims) + 1))
    shape = (batch,) + tuple(dims)
    # the transform bars, with room for the longest sums of the corpus
    # (binary16 storage: the rounding of the output; f32 storage of f64
    # passes: the rounding of input and output)
    tol = {F32: 2e-5, F64: 2e-13, F16S: 1e-3, F64C: 1e-7}[prec]
    seed = int(np.prod(dims)) * 7 + batch
    if kind == "c2c":
        cdt = np.complex128 if prec == F64 else np.complex64
        x = o.complex_uniform(batch * int(np.prod(dims)), seed, cdt)
        cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec) \
            .with_inverse_normalization(normalize)
        y = hip_ctx.execute_transform(vk.TransformIr.build(cfg, direction), x)
        if prec == F16S:  # the library computes on the binary16-rounded input
            x = x.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)
        v = x.astype(np.complex128).reshape(shape)
        if direction == FWD:
            ref = np.fft.fftn(v, axes=axes)
        else:
            ref = np.fft.ifftn(v, axes=axes) * (1 if normalize else int(np.prod(dims)))
        assert o.rel_l2(y, ref.reshape(-1)) <= tol
        return
    rdt = np.float32 if prec == F32 else np.float64
    x = o.uniform(batch * int(np.prod(dims)), seed, rdt)
    cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(R2C)
    X = hip_ctx.execute_transform(vk.TransformIr.build(cfg, FWD), x)
    ref = np.fft.rfftn(x.astype(np.float64).reshape(shape), axes=axes)
    assert o.rel_l2(X, ref.reshape(-1)) <= tol
    # C2R of the exact (Hermitian) spectrum, normalized: the input back
    cdt = np.complex64 if prec == F32 else np.complex128
    cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(C2R) \
        .with_inverse_normalization(True)
    z = hip_ctx.execute_transform(vk.TransformIr.build(cfg, INV), ref.astype(cdt).reshape(-1))
    assert o.rel_l2(z, x.astype(np.float64)) <= tol
