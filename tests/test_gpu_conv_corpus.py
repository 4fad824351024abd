"""A seeded random corpus of convolutions (performConvolution) across the
planner's convolution paths: one-upload 1-D lengths (fixed and runtime
shapes), two-upload lengths with and without a fixed-shape row pass, Rader
and Bluestein axes, N-D tensors whose axis 0 has a fixed-shape column
kernel, is split, or neither; scalar, multi-kernel and 2x2 / 3x3 (and
symmetric 2x2) matrix convolutions, with sequence conjugation and cross-power
normalization, in f32 and f64, within the ownership rules of
FftConfig::validate (src/config.rs:1156-1300): several kernels need batch 1,
N-D matrices need batch 1 and one kernel, 3x3 symmetric is rejected. Each
case is checked against the oracle's restatement (pinned to brute-force
circular convolution)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
TOL = {F32: 1e-5, F64: 2e-13}
ONE_D = [64, 256, 360, 1024, 1536, 2048, 4096, 97, 4099, 1 << 16, 100000, 3 << 16]
N_D = [[64, 48], [256, 20], [1024, 24], [48, 30], [128, 12, 3], [16, 12, 10], [768, 10, 3], [97, 16]]


def planes(matrix, symmetric):
    if matrix <= 1:
        return 1
    return matrix * (matrix + 1) // 2 if symmetric else matrix * matrix


def corpus(seed=77, count=120):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        dims = [int(rng.choice(ONE_D))] if rng.random() < 0.6 else list(N_D[int(rng.integers(len(N_D)))])
        prec = F32 if rng.random() < 0.7 else F64
        r = rng.random()
        matrix = 0 if r < 0.6 else (2 if r < 0.85 else 3)
        symmetric = matrix == 2 and rng.random() < 0.4
        kernels = int(rng.integers(2, 4)) if rng.random() < 0.3 else 1
        if len(dims) > 1 and matrix:
            kernels = 1
        batch = 1 if (kernels > 1 or (len(dims) > 1 and matrix)) else int(rng.integers(1, 4))
        conj = bool(rng.random() < 0.3)
        cross = bool(rng.random() < 0.2)
        if prec == F64 and int(np.prod(dims)) > 1 << 16:
            continue  # keep the f64 oracle reference quick
        cases.append((dims, batch, prec, matrix, symmetric, kernels, conj, cross))
    return cases


def case_id(c):
    dims, batch, prec, matrix, symmetric, kernels, conj, cross = c
    return "{}-b{}-{}-m{}{}-k{}{}{}".format("x".join(map(str, dims)), batch, "f32" if prec == F32 else "f64",
                                           matrix, "s" if symmetric else "", kernels, "-conj" if conj else "",
                                           "-cross" if cross else "")


CASES = corpus()


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_convolution_corpus(hip_ctx, case):
    dims, batch, prec, matrix, symmetric, kernels, conj, cross = case
    t = int(np.prod(dims))
    coords = matrix if matrix > 1 else 1
    dt = np.complex64 if prec == F32 else np.complex128
    x = o.complex_uniform(batch * coords * t, 300 + t % 97, dt)
    k = o.complex_uniform(kernels * planes(matrix, symmetric) * t, 400 + t % 89, dt)
    c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_convolution(True) \
        .with_convolution_kernel_count(kernels)
    if matrix > 1:
        c = c.with_matrix_convolution(matrix).with_symmetric_convolution_kernel(symmetric)
    if conj:
        c = c.with_convolution_conjugation(vk.ConvolutionConjugation.Sequence)
    if cross:
        c = c.with_cross_power_spectrum_normalization(True)
    conv = vk.ConvolutionIr.build(c, k)
    y = hip_ctx.execute_convolution(conv, x)
    ref = o.convolution(x, k, dims, batch, matrix if matrix > 1 else 0, symmetric, kernels, conj, cross, threads=8,
                        backend="numpy" if prec == F64 else "oracle")
    assert y.size == ref.size
    assert o.rel_l2(y, ref) <= TOL[prec]
