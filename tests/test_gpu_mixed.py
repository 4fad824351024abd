"""Mixed storage/compute precisions through the C ABI: F16StorageF32Compute
(binary16 buffers, f32 passes) and F64ComputeF32Storage (f32 buffers, f64
passes), src/config.rs:108-145. The first two tests restate the reference's
HIP tests (src/backend/hip/runtime.rs:3345-3448) with their tolerances."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse


def ir_for(dims, batch, prec, direction=FWD, kind=vk.TransformKind.ComplexToComplex, normalize=False):
    cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind) \
        .with_inverse_normalization(normalize)
    return vk.TransformIr.build(cfg, direction)


def ref_input(n):
    x = np.arange(n, dtype=np.float32)
    return (np.sin(0.15 * x) + 1j * np.cos(0.09 * x)).astype(np.complex64)


def f16(v):
    """Binary16 rounding of complex64 values (round to nearest even)."""
    return v.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)


def test_hip_f16_storage_f32_compute_matches_cpu(hip_ctx):
    # hip/runtime.rs:3345-3396: N=64, expected = reference on binary16-quantized
    # input, quantized again; max error <= 1e-3 * N
    n = 64
    x = ref_input(n)
    ir = ir_for([n], 1, F16S)
    y = hip_ctx.execute_transform_f32(ir, x)
    assert y.dtype == np.complex64
    expected = f16(o.fft(f16(x).astype(np.complex128)).astype(np.complex64))
    assert np.max(np.abs(y - expected)) <= 1e-3 * n


def test_hip_f64_compute_f32_storage_matches_cpu(hip_ctx):
    # hip/runtime.rs:3398-3448: N=64, error < 2e-5 * N against the f64 reference
    n = 64
    x = ref_input(n)
    ir = ir_for([n], 1, F64C)
    y = hip_ctx.execute_transform_f32(ir, x)
    assert y.dtype == np.complex64
    expected = o.fft(x.astype(np.complex128))
    assert np.max(np.abs(y.astype(np.complex128) - expected)) < 2e-5 * n


@pytest.mark.parametrize("dims,batch,fused", [([1024], 16, True), ([4099], 4, False), ([64, 48], 2, False),
                                              ([1 << 20], 1, True), ([3 << 16], 1, False), ([97], 5, False)])
def test_f64_compute_f32_storage(hip_ctx, dims, batch, fused):
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 991, np.complex64)
    ir = ir_for(dims, batch, F64C)
    y = hip_ctx.execute_transform_f32(ir, x)
    ref = o.fft_nd(x, dims, batch, threads=8) if len(dims) > 1 else \
        o.fft_batch(x.astype(np.complex128), dims[0], "forward", False, threads=8)
    # f64 passes: the only error left is rounding the result to f32
    assert o.rel_l2(y, ref) <= 1e-7
    desc = hip_ctx.plan(ir).describe()
    # a 1-D one-upload Stockham pass, and the two passes of a two-upload
    # length with fixed edge shapes (2^20 = 1024 x 1024), convert in their
    # own loads and stores; N-D, other four-step (3 * 2^16 = 512 x 384) and
    # Rader plans keep boundary passes, and so do Bluestein plans whose
    # convolution length has no fixed shape in f64 (4099: M = 8232)
    assert desc["boundary"]["fused_edges"] == fused
    boundary = desc["passes"][0]["kernel"] == "boundary_in" and desc["passes"][-1]["kernel"] == "boundary_out"
    assert boundary != fused
    assert desc["precision"] == "f64_compute_f32_storage"


@pytest.mark.parametrize("dims,batch", [([1024], 16), ([4099], 2), ([256, 64], 2)])
def test_f16_storage_f32_compute(hip_ctx, dims, batch):
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 977, np.complex64)
    ir = ir_for(dims, batch, F16S)
    y = hip_ctx.execute_transform_f32(ir, x)
    xq = f16(x)
    ref = o.fft_nd(xq, dims, batch, threads=8) if len(dims) > 1 else \
        o.fft_batch(xq.astype(np.complex128), dims[0], "forward", False, threads=8)
    # binary16 output rounding (unit roundoff 2^-11) dominates
    assert o.rel_l2(y, ref) <= 1e-3
    assert np.array_equal(y, f16(y))


def test_mixed_real_round_trip(hip_ctx):
    n, batch = 1 << 14, 3
    x = o.normal(n * batch, 12, np.float32)
    for prec, tol in ((F64C, 1e-7), (F16S, 2e-3)):
        r2c = ir_for([n], batch, prec, FWD, vk.TransformKind.RealToComplex)
        c2r = ir_for([n], batch, prec, INV, vk.TransformKind.ComplexToReal, True)
        X = hip_ctx.execute_transform(r2c, x)
        xin = x if prec == F64C else x.astype(np.float16).astype(np.float32)
        ref = o.r2c_batch(xin.astype(np.float64), n)
        h = n // 2 + 1
        assert o.rel_l2(X, ref) <= tol, prec
        z = hip_ctx.execute_transform(c2r, X)
        assert o.rel_l2(z, xin) <= 2 * tol, prec
        assert X[:h].dtype == np.complex64


def test_f16_device_resident_matches_host(hip_ctx):
    import torch
    n, batch = 1024, 8
    x = o.complex_uniform(n * batch, 13, np.complex64)
    ir = ir_for([n], batch, F16S)
    plan = hip_ctx.plan(ir)
    assert plan.in_bytes == n * batch * 4 and plan.out_bytes == n * batch * 4
    xs = torch.from_numpy(x.view(np.float32).astype(np.float16)).cuda()
    ys = torch.empty_like(xs)
    plan.execute_tensors(xs, ys)
    torch.cuda.synchronize()
    y_dev = ys.cpu().numpy().astype(np.float32).view(np.complex64)
    assert np.array_equal(y_dev, hip_ctx.execute_transform_f32(ir, x))


def test_mixed_ticket_and_chain(hip_ctx):
    n, batch = 2048, 4
    x = o.complex_uniform(n * batch, 14, np.complex64)
    fwd = ir_for([n], batch, F64C)
    inv = ir_for([n], batch, F64C, INV, normalize=True)
    t = hip_ctx.submit_transform_async(fwd, x)
    assert np.array_equal(t.wait(), hip_ctx.execute_transform_f32(fwd, x))
    z = hip_ctx.execute_chain([fwd, inv], x)
    assert o.rel_l2(z, x) <= 1e-7


# ------------------------------------ the reference's mixed-storage FFTW corpora

MIXED_CORPORA = {
    # tests/fftw_medium_f16_storage_golden.rs:230-252: within 2 binary16 ulps or 2e-3
    "f16": ("fftw_precision_medium_f16_storage_v1.txt", F16S, 2, 2e-3),
    # tests/fftw_medium_f64_f32_storage_golden.rs:217-240: within 4 f32 ulps or 1e-6
    "f64_f32": ("fftw_precision_medium_f64_f32_storage_v1.txt", F64C, 4, 1e-6),
}


@pytest.mark.parametrize("corpus", sorted(MIXED_CORPORA))
@pytest.mark.parametrize("case", ["c2c-bluestein-n103", "c2c-rader-n257", "c2c-smooth-n1536",
                                  "c2c-large-smooth-n4096", "r2c-nd-17x34", "r2c-nd-64x64", "dct2-nd-17x34"])
def test_fftw_medium_mixed_storage_on_gpu(hip_ctx, corpus, case):
    """run_native_medium_*_storage_fftw of the reference: the f32 input
    formulas (rounded to binary16 by the F16 plan's storage), a forward plan
    of the case's kind, every output scalar against FFTW's committed bits at
    the reference's tolerances, and the planner families of the C2C cases
    (Bluestein under max_rader_fft_prime = 100, Rader, Stockham)."""
    import os

    import golden_bits as gb
    from conftest import GOLDEN
    name, prec, max_ulps, max_abs = MIXED_CORPORA[corpus]
    width, cases = gb.parse(os.path.join(GOLDEN, name))
    c = cases[case]
    kind = {"c2c": vk.TransformKind.ComplexToComplex, "r2c": vk.TransformKind.RealToComplex,
            "dct2": vk.TransformKind.dct(2)}[c["kind"]]
    cfg = vk.FftConfig.new(c["shape"]).with_precision(prec).with_transform(kind)
    if case == "c2c-bluestein-n103":
        t = vk.PlannerTuning.portable()
        t.max_rader_fft_prime = 100
        cfg = cfg.with_tuning(t)
    ir = vk.TransformIr.build(cfg, FWD)
    family = {"c2c-bluestein-n103": vk.AlgorithmKind.Bluestein, "c2c-rader-n257": vk.AlgorithmKind.Rader,
              "c2c-smooth-n1536": vk.AlgorithmKind.Stockham, "c2c-large-smooth-n4096": vk.AlgorithmKind.Stockham}
    if case in family:
        assert ir.axis_algorithms == [family[case]]
    n = int(np.prod(c["shape"]))
    x = o.fixture_input("complex-f32-v1" if c["kind"] == "c2c" else "real-f32-v1", n)
    y = hip_ctx.execute_transform_f32(ir, x)
    got = gb.scalars(y, c["kind"]).astype(np.float32)
    assert got.size == c["bits"].size and np.all(np.isfinite(got))
    if width == 16:   # caller-visible binary16 storage
        assert np.array_equal(got.astype(np.float16).astype(np.float32), got)
    expected = gb.from_bits(c["bits"], width)
    d = gb.ulps(gb.to_bits(got, width), c["bits"], width)
    ok = (d <= max_ulps) | (np.abs(got - expected) <= max_abs)
    bad = np.flatnonzero(~ok)
    assert bad.size == 0, [(int(i), float(got[i]), float(expected[i]), int(d[i])) for i in bad[:8]]
