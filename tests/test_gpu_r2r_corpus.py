"""A seeded random corpus of DCT / DST types I-IV (TransformKind::Dct/Dst,
src/r2r_ir.rs:2351-2434): 1-D and N-D (NdR2rIr, :1769-2300) over lengths
whose reductions land on different C2C plans (even and odd lengths, powers of
two, smooth and prime lengths: Stockham, Rader, Bluestein; the N/2 reduction
of even type IV, the 2N extension of odd type IV), f32 and f64, forward and
the normalized inverse round trip, against scipy.fft (pocketfft) in float64.
The corpus is fixed by its seed; a case's id names it."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
KINDS = ["dct1", "dct2", "dct3", "dct4", "dst1", "dst2", "dst3", "dst4"]
LENGTHS = [2, 3, 5, 8, 9, 16, 17, 31, 48, 64, 97, 100, 127, 128, 257, 360, 500, 1000, 1024, 2047, 4096]
TOL = {F32: 2e-5, F64: 2e-13}


def corpus(seed=5, count=80):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        name = KINDS[int(rng.integers(len(KINDS)))]
        rank = 1 if rng.random() < 0.6 else int(rng.integers(2, 4))
        dims = [int(rng.choice(LENGTHS)) for _ in range(rank)]
        if name == "dct1" and min(dims) < 2:
            continue
        if int(np.prod(dims)) > 1 << 17:
            continue
        batch = int(rng.integers(1, 4))
        prec = F32 if rng.random() < 0.6 else F64
        cases.append((name, dims, batch, prec))
    return cases


def case_id(c):
    name, dims, batch, prec = c
    return "{}-{}-b{}-{}".format(name, "x".join(map(str, dims)), batch, "f32" if prec == F32 else "f64")


CASES = corpus()


def kind_of(name):
    t = int(name[-1])
    return vk.TransformKind.dct(t) if name.startswith("dct") else vk.TransformKind.dst(t)


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_r2r_corpus(hip_ctx, case):
    import scipy.fft as sf
    name, dims, batch, prec = case
    rd = np.float32 if prec == F32 else np.float64
    x = o.uniform(batch * int(np.prod(dims)), int(np.prod(dims)) % 983 + batch, rd)
    c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind_of(name))
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    axes = tuple(range(1, len(dims) + 1))
    v = x.astype(np.float64).reshape((batch,) + tuple(dims))
    fn = sf.dctn if name.startswith("dct") else sf.dstn
    ref = fn(v, type=int(name[-1]), axes=axes).reshape(-1)
    assert o.rel_l2(y, ref) <= TOL[prec]
    # the normalized inverse restores the input
    ci = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind_of(name)) \
        .with_inverse_normalization(True)
    z = hip_ctx.execute_transform(vk.TransformIr.build(ci, INV), ref.astype(rd))
    assert o.rel_l2(z, x.astype(np.float64)) <= 2 * TOL[prec]
