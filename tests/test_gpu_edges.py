"""Boundary work inside the FFT passes (KF_EDGE): the storage conversion of
mixed precisions (src/config.rs:108-145) and the zero intervals of 1-D zero
padding (src/zero_pad_ir.rs:320-345, 607-647) in the first pass's loads and
the last pass's stores of C2C plans made of one-upload Stockham passes. Each
case runs with the fused passes and with the boundary passes
(VKFX_FUSED_EDGES=0) and both are checked against the oracle; the fused plan
must have no boundary pass. Every test takes the session context first so
that torch's HIP runtime is the one the library binds to."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
SPATIAL, FREQ = vk.ZeroPaddingDomain.Spatial, vk.ZeroPaddingDomain.Frequency


def f16(v):
    """Binary16 rounding of complex64 values (round to nearest even)."""
    return v.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)


def ref_c2c(x, dims, batch, direction, normalize=False):
    v = x.reshape((batch,) + tuple(dims)).astype(np.complex128)
    if len(dims) == 1:
        y = o.fft_batch(v.reshape(-1), dims[0], "forward" if direction == FWD else "inverse", normalize, threads=8)
        return np.asarray(y).reshape(-1)
    axes = tuple(range(1, len(dims) + 1))
    if direction == FWD:
        return np.fft.fftn(v, axes=axes).reshape(-1)
    return (np.fft.ifftn(v, axes=axes) * (1 if normalize else int(np.prod(dims)))).reshape(-1)


def run_both(monkeypatch, c, direction, x):
    """(fused output, fused describe, boundary-pass output); the fused plan
    also runs with staged ends only (VKFX_EDGE_DIRECT=0) and must give the
    same values as with HBM-direct ends up to rounding."""
    out = []
    for fused, direct in (("1", "1"), ("1", "0"), ("0", "1")):
        monkeypatch.setenv("VKFX_FUSED_EDGES", fused)
        monkeypatch.setenv("VKFX_EDGE_DIRECT", direct)
        ctx = vk.HipExecutionContext(0)  # own plan cache: plans read the switches when built
        try:
            ir = vk.TransformIr.build(c, direction)
            y = ctx.execute_transform(ir, x)
            desc = ctx.plan(ir).describe()
        finally:
            ctx.close()
        assert (desc["boundary"]["fused_edges"] or desc["boundary"]["fused_layout"]) == (fused == "1")
        kernels = [p["kernel"] for p in desc["passes"]]
        assert ("boundary_in" in kernels or "boundary_out" in kernels) == (fused == "0"), kernels
        out.append((y, desc))
    (y, desc), (ys, _), (yb, _) = out
    scale = max(float(np.max(np.abs(y))), 1e-30)
    tol = {F16S: 2e-3, F32: 1e-5, F64C: 1e-6, F64: 1e-12}[c.precision]
    assert float(np.max(np.abs(y - ys))) <= tol * scale
    return y, desc, yb


@pytest.mark.parametrize("dims,batch", [([1024], 7), ([4096], 3), ([720], 5), ([1000], 2)])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_mixed_storage_fused(hip_ctx, monkeypatch, dims, batch, direction):
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 983, np.complex64)
    for prec, tol in ((F64C, 1e-7), (F16S, 1e-3)):
        c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
        y, desc, yb = run_both(monkeypatch, c, direction, x)
        xin = f16(x) if prec == F16S else x
        ref = ref_c2c(xin, dims, batch, direction, normalize=True)
        assert o.rel_l2(y, ref) <= tol, prec
        assert o.rel_l2(yb, ref) <= tol, prec
        if prec == F16S:
            assert np.array_equal(y, f16(y))
        assert [p["kernel"] for p in desc["passes"]] == ["stockham"]


@pytest.mark.parametrize("dims,batch", [([16, 24, 40], 2), ([64, 48], 3), ([6, 10, 12, 14], 1), ([4096, 16], 2),
                                        ([8, 2048, 24], 1), ([8, 97, 40], 1)])
def test_mixed_storage_nd_flat_boundary(hip_ctx, dims, batch):
    """N-D mixed storage: the first and last passes of each chunk convert in
    their own loads and stores when both have fixed shapes with edge
    variants, else the fixed-shape passes run between two boundary passes
    (flat vectorized conversions for dense layouts)."""
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 983, np.complex64)
    for prec, tol in ((F64C, 1e-7), (F16S, 1e-3)):
        c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec)
        ir = vk.TransformIr.build(c, FWD)
        y = hip_ctx.execute_transform(ir, x)
        desc = hip_ctx.plan(ir).describe()
        kernels = [p["kernel"] for p in desc["passes"]]
        boundary = kernels[0] == "boundary_in" and kernels[-1] == "boundary_out"
        assert boundary != desc["boundary"]["fused_edges"], kernels
        xin = f16(x) if prec == F16S else x
        assert o.rel_l2(y, ref_c2c(xin, dims, batch, FWD)) <= tol, prec


@pytest.mark.parametrize("direction,domain", [(FWD, SPATIAL), (INV, SPATIAL), (FWD, FREQ), (INV, FREQ)])
@pytest.mark.parametrize("n,left,right", [(1024, 100, 300), (720, 0, 1), (4096, 4000, 4096), (1000, 0, 1000)])
def test_zero_padding_fused(hip_ctx, monkeypatch, direction, domain, n, left, right):
    batch = 3
    x = o.complex_uniform(n * batch, n + left, np.complex64)
    for prec, dt, tol in ((F32, np.complex64, 1e-5), (F64, np.complex128, 1e-13), (F16S, np.complex64, 1e-3)):
        xs = x.astype(dt)
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
            .with_zero_padding(0, left, right).with_zero_padding_domain(domain)
        y, desc, yb = run_both(monkeypatch, c, direction, xs)
        mask = np.zeros((batch, n), dtype=bool)
        mask[:, left:right] = True
        mask = mask.reshape(-1)
        input_side = (direction == FWD) == (domain == SPATIAL)
        xin = f16(xs) if prec == F16S else xs
        xin = np.where(mask, 0, xin) if input_side else xin
        expect = ref_c2c(xin, [n], batch, direction)
        if not input_side:
            expect = np.where(mask, 0, expect)
            assert (y[mask] == 0).all() and (yb[mask] == 0).all()
        if left == 0 and right == n:
            # the whole axis is zero on one side: the result is exactly zero
            assert (y == 0).all() and (yb == 0).all()
            continue
        assert o.rel_l2(y, expect) <= tol, prec
        assert o.rel_l2(yb, expect) <= tol, prec


def test_fused_edges_device_resident_and_chunks(hip_ctx, monkeypatch):
    """Device-resident f16 buffers through the fused plan, a batch large
    enough for several chunks, and a plan that does not qualify (a
    two-upload length without fixed edge shapes) keeping its boundary
    passes."""
    import torch
    n, batch = 1024, 4096
    x = o.complex_uniform(n * batch, 31, np.complex64)
    ctx = vk.HipExecutionContext(0)
    try:
        ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F16S), FWD)
        plan = ctx.plan(ir)
        assert plan.describe()["boundary"]["fused_edges"]
        xs = torch.from_numpy(x.view(np.float32).astype(np.float16)).cuda()
        ys = torch.empty_like(xs)
        plan.execute_tensors(xs, ys)
        torch.cuda.synchronize()
        y = ys.cpu().numpy().astype(np.float32).view(np.complex64)
        for b in (0, 1, 2047, 4095):
            ref = o.fft(f16(x[b * n:(b + 1) * n]).astype(np.complex128))
            assert o.rel_l2(y[b * n:(b + 1) * n], ref) <= 1e-3, b
        # 3 * 2^16 = 512 x 384: no fixed edge shape for the 384-point rows
        big = vk.TransformIr.build(vk.FftConfig.new([3 << 16]).with_batch_count(2).with_precision(F16S), FWD)
        assert not ctx.plan(big).describe()["boundary"]["fused_edges"]
    finally:
        ctx.close()


FOUR_STEP = ["four_step_columns", "four_step_rows"]


@pytest.mark.parametrize("n,batch", [(1 << 16, 3), (1 << 18, 2), (1 << 20, 1)])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_mixed_storage_four_step(hip_ctx, monkeypatch, n, batch, direction):
    """Two-upload C2C lengths whose factors have fixed edge shapes: the
    column pass reads the storage type and the row pass writes it (no
    boundary pass, no compute-type copy), against the oracle and against the
    boundary-pass plan."""
    x = o.complex_uniform(n * batch, n % 997 + batch, np.complex64)
    for prec, tol in ((F64C, 1e-7), (F16S, 1e-3)):
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
        y, desc, yb = run_both(monkeypatch, c, direction, x)
        assert desc["boundary"]["four_step_edges"]
        assert [p["kernel"] for p in desc["passes"]] == FOUR_STEP, desc["passes"]
        xin = f16(x) if prec == F16S else x
        ref = ref_c2c(xin, [n], batch, direction, normalize=True)
        assert o.rel_l2(y, ref) <= tol, prec
        assert o.rel_l2(yb, ref) <= tol, prec
        if prec == F16S:
            assert np.array_equal(y, f16(y))


@pytest.mark.parametrize("direction,domain", [(FWD, SPATIAL), (INV, SPATIAL), (FWD, FREQ)])
@pytest.mark.parametrize("left,right", [(1000, 40000), (0, 1), (65000, 65536)])
def test_mixed_storage_four_step_zero_padding(hip_ctx, monkeypatch, direction, domain, left, right):
    """The zero interval of a 1-D zero padding in the mixed-storage
    four-step passes: element n2 + n1 * N2 of the column pass reads as zero,
    element k1 + k2 * N1 of the row pass is written as zero."""
    n, batch = 1 << 16, 2
    x = o.complex_uniform(n * batch, left + 3, np.complex64)
    mask = np.zeros((batch, n), dtype=bool)
    mask[:, left:right] = True
    mask = mask.reshape(-1)
    input_side = (direction == FWD) == (domain == SPATIAL)
    for prec, tol in ((F64C, 1e-7), (F16S, 1e-3)):
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
            .with_zero_padding(0, left, right).with_zero_padding_domain(domain)
        y, desc, yb = run_both(monkeypatch, c, direction, x)
        assert desc["boundary"]["four_step_edges"]
        xin = f16(x) if prec == F16S else x
        xin = np.where(mask, 0, xin) if input_side else xin
        expect = ref_c2c(xin, [n], batch, direction)
        if not input_side:
            expect = np.where(mask, 0, expect)
            assert (y[mask] == 0).all() and (yb[mask] == 0).all()
        assert o.rel_l2(y, expect) <= tol, prec
        assert o.rel_l2(yb, expect) <= tol, prec


def test_mixed_storage_four_step_chunks(hip_ctx, monkeypatch):
    """Batch chunks of the mixed-storage four-step plan on two stream lanes
    (a 1 MB work budget: five chunks of two lines in f32 compute, nine of
    one line in f64 compute), every line against the oracle."""
    monkeypatch.setenv("VKFX_WORK_BUDGET_MB", "1")
    n, batch = 1 << 16, 9
    x = o.complex_uniform(n * batch, 57, np.complex64)
    for prec, tol, chunks in ((F16S, 1e-3, 5), (F64C, 1e-7, 9)):
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
        y, desc, yb = run_both(monkeypatch, c, FWD, x)
        assert desc["boundary"]["four_step_edges"] and desc["lanes"] == 2
        assert [p["kernel"] for p in desc["passes"]] == FOUR_STEP * chunks
        xin = f16(x) if prec == F16S else x
        ref = ref_c2c(xin, [n], batch, FWD)
        assert o.rel_l2(y, ref) <= tol and o.rel_l2(yb, ref) <= tol, prec


def layout_cfg(dims, batch, prec, fmt_in, fmt_out):
    """Formatted strides on the chosen sides: every axis but the fastest
    padded by a few elements, and the batch stride padded too."""
    c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec)
    for side, on in (("input", fmt_in), ("output", fmt_out)):
        if not on:
            continue
        st = 1
        for ax in range(len(dims) - 1, -1, -1):
            if ax < len(dims) - 1:
                st = st + 3 + ax
                c = getattr(c, f"with_{side}_buffer_axis_stride")(ax, st)
            st *= dims[ax]
        c = getattr(c, f"with_{side}_buffer_batch_stride")(st + 5)
    return c


@pytest.mark.parametrize("dims,batch", [([1024], 3), ([32, 48], 3), ([8, 12, 40], 2), ([64, 64], 2), ([4, 300], 2),
                                        ([3, 5, 512], 2)])
@pytest.mark.parametrize("sides", [(True, False), (False, True), (True, True)])
def test_formatted_layout_fused(hip_ctx, monkeypatch, dims, batch, sides):
    """Formatted strides read and written by the first and last passes
    (rank <= 3): alone, and together with storage conversion."""
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 887, np.complex64)
    for prec, tol in ((F32, 1e-5), (F64, 1e-12), (F16S, 1e-3), (F64C, 1e-7)):
        if len(dims) == 1 and prec in (F32, F64):
            continue  # the 1-D batch stride alone is the passes' own stride (test_gpu_layout)
        xs = x.astype(np.complex128) if prec == F64 else x
        c = layout_cfg(dims, batch, prec, *sides)
        if len(dims) > 1 and prec in (F16S, F64C):
            # N-D mixed storage: boundary passes carry both the layout and the conversion
            ir = vk.TransformIr.build(c, FWD)
            y = hip_ctx.execute_transform(ir, xs)
            assert not hip_ctx.plan(ir).describe()["boundary"]["fused_layout"]
            assert o.rel_l2(y, ref_c2c(f16(xs) if prec == F16S else xs, dims, batch, FWD)) <= tol, prec
            continue
        y, desc, yb = run_both(monkeypatch, c, FWD, xs)
        assert desc["boundary"]["fused_layout"], desc["boundary"]
        xin = f16(xs) if prec == F16S else xs
        ref = ref_c2c(xin, dims, batch, FWD)
        assert o.rel_l2(y, ref) <= tol, prec
        assert o.rel_l2(yb, ref) <= tol, prec


@pytest.mark.parametrize("dims,prec", [([8, 12, 40], F32), ([1000], F16S)])
def test_formatted_layout_fused_gaps_untouched(hip_ctx, dims, prec):
    """The fused last pass writes only the logical positions of a formatted
    output (gaps keep their NaN), from a formatted input."""
    import torch
    batch = 2
    c = layout_cfg(dims, batch, prec, True, True)
    ir = vk.TransformIr.build(c, FWD)
    plan = hip_ctx.plan(ir)
    assert plan.describe()["boundary"]["fused_layout"]
    x = o.complex_uniform(int(np.prod(dims)) * batch, 41, np.complex64)
    xs = ir.to_storage(ir.pack_input(x))
    tdt = torch.float16 if prec == F16S else torch.float32
    dx = torch.from_numpy(np.ascontiguousarray(xs).view(np.float16 if prec == F16S else np.float32)).cuda()
    dy = torch.full((plan.out_bytes // (2 if prec == F16S else 4),), float("nan"), device="cuda", dtype=tdt)
    plan.execute_tensors(dx, dy)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().astype(np.float32).view(np.complex64)
    idx, _ = ir._physical_index(True)
    gaps = np.ones(y.size, dtype=bool)
    gaps[idx] = False
    assert gaps.any() and np.isnan(y[gaps].real).all() and np.isnan(y[gaps].imag).all()
    xin = f16(x) if prec == F16S else x
    assert o.rel_l2(y[idx], ref_c2c(xin, dims, batch, FWD)) <= (1e-3 if prec == F16S else 1e-5)


# prime lengths whose one-upload Bluestein convolution length M has a fixed
# shape with an edge variant (f32 compute: M = 8232, 4096, 1024, 16384, 256;
# f64 compute: M = 3430, 2048, 8192, 512), batches spanning several blocks
def ref_np(x, n, batch, direction, normalize=False):
    """pocketfft's float64 1-D transform (the f64 gate of the Bluestein
    tests: the oracle's own f64 Bluestein sits near 1e-12)."""
    v = x.astype(np.complex128).reshape(batch, n)
    y = np.fft.fft(v, axis=1) if direction == FWD else np.fft.ifft(v, axis=1) * (1 if normalize else n)
    return y.reshape(-1)


BLUE_EDGE = [(4099, F16S, 5), (1583, F16S, 3), (409, F16S, 9), (6133, F16S, 2), (103, F16S, 35),
             (1583, F64C, 3), (1019, F64C, 4), (3461, F64C, 2), (137, F64C, 17)]


@pytest.mark.parametrize("n,prec,batch", BLUE_EDGE)
@pytest.mark.parametrize("direction", [FWD, INV])
def test_mixed_storage_bluestein(hip_ctx, monkeypatch, n, prec, batch, direction):
    """Mixed-storage 1-D Bluestein transforms in one kernel: the edge variant
    of the fixed shape reads the storage type before the chirp weighting and
    writes it after the chirp and scale (no boundary pass), against the
    oracle and against the boundary-pass plan."""
    x = o.complex_uniform(n * batch, n % 997 + batch, np.complex64)
    tol = {F16S: 1e-3, F64C: 1e-7}[prec]
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
    y, desc, yb = run_both(monkeypatch, c, direction, x)
    assert desc["boundary"]["bluestein_edges"]
    assert [p["kernel"] for p in desc["passes"]] == ["bluestein_single"], desc["passes"]
    xin = f16(x) if prec == F16S else x
    ref = ref_np(xin, n, batch, direction, normalize=True)
    assert o.rel_l2(y, ref) <= tol
    assert o.rel_l2(yb, ref) <= tol
    if prec == F16S:
        assert np.array_equal(y, f16(y))


def test_mixed_storage_bluestein_without_edge_shape(hip_ctx):
    """A Bluestein length whose convolution length has no fixed shape in the
    compute precision (4099 in f64: M = 8232) keeps its boundary passes."""
    n, batch = 4099, 2
    x = o.complex_uniform(n * batch, 11, np.complex64)
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F64C)
    ir = vk.TransformIr.build(c, FWD)
    y = hip_ctx.execute_transform(ir, x)
    desc = hip_ctx.plan(ir).describe()
    assert not desc["boundary"]["bluestein_edges"]
    kernels = [p["kernel"] for p in desc["passes"]]
    assert "boundary_in" in kernels and "boundary_out" in kernels, kernels
    assert o.rel_l2(y, ref_np(x, n, batch, FWD)) <= 1e-7


@pytest.mark.parametrize("direction,domain", [(FWD, SPATIAL), (INV, SPATIAL), (FWD, FREQ), (INV, FREQ)])
@pytest.mark.parametrize("prec", [F32, F64, F16S, F64C])
def test_bluestein_zero_padding_fused(hip_ctx, monkeypatch, direction, domain, prec):
    """The 1-D zero interval inside the one-upload Bluestein kernel, on the
    plain and the mixed precisions: input elements [l, r) read as zero before
    the chirp weighting, output elements [l, r) written as zero."""
    n, batch, left, right = 1583, 3, 100, 1200
    cdt = np.complex128 if prec == F64 else np.complex64
    x = o.complex_uniform(n * batch, 29, cdt)
    mask = np.zeros((batch, n), dtype=bool)
    mask[:, left:right] = True
    mask = mask.reshape(-1)
    input_side = (direction == FWD) == (domain == SPATIAL)
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_zero_padding(0, left, right).with_zero_padding_domain(domain)
    y, desc, yb = run_both(monkeypatch, c, direction, x)
    assert desc["boundary"]["bluestein_edges"]
    assert [p["kernel"] for p in desc["passes"]] == ["bluestein_single"], desc["passes"]
    xin = f16(x) if prec == F16S else x
    xin = np.where(mask, 0, xin) if input_side else xin
    expect = ref_np(xin, n, batch, direction)
    if not input_side:
        expect = np.where(mask, 0, expect)
        assert (y[mask] == 0).all() and (yb[mask] == 0).all()
    tol = {F32: 2e-5, F64: 2e-13, F16S: 1e-3, F64C: 1e-7}[prec]
    assert o.rel_l2(y, expect) <= tol
    assert o.rel_l2(yb, expect) <= tol


R2C, C2R = vk.TransformKind.RealToComplex, vk.TransformKind.ComplexToReal
# even lengths whose half length has a fixed real row shape with an edge
# variant (f32 compute: 8192, 512, 1536, 640; f64 compute: 4096, 512, 384, 160)
REAL_EDGE = [(16384, F16S, 3), (1024, F16S, 9), (3072, F16S, 5), (1280, F16S, 4),
             (8192, F64C, 2), (1024, F64C, 7), (768, F64C, 3), (320, F64C, 10)]


def f16_real(v):
    return v.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("n,prec,batch", REAL_EDGE)
def test_mixed_storage_real(hip_ctx, monkeypatch, n, prec, batch):
    """Mixed-storage 1-D even-length R2C and C2R in one kernel each: the edge
    variant of the fixed real row shape reads and writes the storage type (no
    boundary pass), against pocketfft and against the boundary-pass plan."""
    x = o.normal(n * batch, n % 991 + batch, np.float32)
    tol = {F16S: 2e-3, F64C: 1e-7}[prec]
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_transform(R2C)
    X, desc, Xb = run_both(monkeypatch, c, FWD, x)
    assert desc["boundary"]["real_edges"]
    assert [p["kernel"] for p in desc["passes"]] == ["r2c_even_half"], desc["passes"]
    xin = f16_real(x) if prec == F16S else x
    ref = np.fft.rfft(xin.astype(np.float64).reshape(batch, n), axis=1).reshape(-1)
    assert o.rel_l2(X, ref) <= tol and o.rel_l2(Xb, ref) <= tol
    if prec == F16S:
        assert np.array_equal(X, f16(X))
    ci = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_transform(C2R) \
        .with_inverse_normalization(True)
    z, desc, zb = run_both(monkeypatch, ci, INV, ref.astype(np.complex64))
    assert desc["boundary"]["real_edges"]
    assert [p["kernel"] for p in desc["passes"]] == ["c2r_even_half"], desc["passes"]
    assert o.rel_l2(z, xin.astype(np.float64)) <= tol and o.rel_l2(zb, xin.astype(np.float64)) <= tol
    if prec == F16S:
        assert np.array_equal(z, f16_real(z))


@pytest.mark.parametrize("prec", [F32, F64, F16S, F64C])
def test_real_zero_padding_fused(hip_ctx, monkeypatch, prec):
    """The zero interval of a 1-D zero padding inside the even-length real
    kernels, over real elements (an odd left end splits a packed pair): R2C
    reads reals [l, r) as zero, C2R writes them as zero."""
    n, batch, left, right = 2048, 3, 101, 1500
    rdt = np.float64 if prec == F64 else np.float32
    x = o.normal(n * batch, 71, rdt)
    mask = np.zeros((batch, n), dtype=bool)
    mask[:, left:right] = True
    tol = {F32: 2e-5, F64: 2e-13, F16S: 2e-3, F64C: 1e-7}[prec]
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_transform(R2C) \
        .with_zero_padding(0, left, right)
    X, desc, Xb = run_both(monkeypatch, c, FWD, x)
    assert desc["boundary"]["real_edges"]
    xin = (f16_real(x) if prec == F16S else x).astype(np.float64).reshape(batch, n)
    ref = np.fft.rfft(np.where(mask, 0, xin), axis=1).reshape(-1)
    assert o.rel_l2(X, ref) <= tol and o.rel_l2(Xb, ref) <= tol
    # C2R of a spectrum: the output reals [l, r) written as zero
    S = np.fft.rfft(xin, axis=1).astype(np.complex128 if prec == F64 else np.complex64)
    ci = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_transform(C2R) \
        .with_zero_padding(0, left, right)
    z, desc, zb = run_both(monkeypatch, ci, INV, S.reshape(-1))
    assert desc["boundary"]["real_edges"]
    Sin = f16(S.astype(np.complex64)) if prec == F16S else S
    expect = np.where(mask, 0, np.fft.irfft(Sin.astype(np.complex128), n, axis=1) * n).reshape(-1)
    m = mask.reshape(-1)
    assert (z[m] == 0).all() and (zb[m] == 0).all()
    assert o.rel_l2(z, expect) <= tol and o.rel_l2(zb, expect) <= tol


@pytest.mark.parametrize("n,batch", [(1024, 33), (4096, 5), (512, 17), (1000, 7), (8, 100), (96, 40), (2048, 9),
                                     (720, 6)])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_mixed_storage_fixed_rows(hip_ctx, monkeypatch, n, batch, direction):
    """Mixed-storage one-upload 1-D C2C keeps the fixed row shape of its
    length where that shape has an edge variant (3/5-family rows; in f64
    compute also the power-of-two rows), else runs the runtime-shape edge
    kernel (f32 power-of-two rows, short rows, round lengths such as 720),
    against pocketfft and the boundary-pass plan."""
    x = o.complex_uniform(n * batch, n % 977 + batch, np.complex64)
    fixed_edge = {F16S: {1000}, F64C: {1024, 4096, 512, 1000, 2048}}
    for prec, tol in ((F16S, 1e-3), (F64C, 1e-7)):
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
        y, desc, yb = run_both(monkeypatch, c, direction, x)
        assert [p["kernel"] for p in desc["passes"]] == ["stockham"]
        assert desc["passes"][0]["fixed_shape"] == (n in fixed_edge[prec]), (prec, desc["passes"][0])
        xin = f16(x) if prec == F16S else x
        ref = ref_np(xin, n, batch, direction, normalize=True)
        assert o.rel_l2(y, ref) <= tol and o.rel_l2(yb, ref) <= tol, prec
        # VKFX_FIXED_EDGES=0: the same plan on the runtime-shape edge kernel
        monkeypatch.setenv("VKFX_FUSED_EDGES", "1")
        monkeypatch.setenv("VKFX_FIXED_EDGES", "0")
        ctx = vk.HipExecutionContext(0)
        try:
            ir = vk.TransformIr.build(c, direction)
            yr = ctx.execute_transform(ir, x)
            assert not ctx.plan(ir).describe()["passes"][0]["fixed_shape"]
        finally:
            ctx.close()
            monkeypatch.delenv("VKFX_FIXED_EDGES")
        assert o.rel_l2(yr, ref) <= tol, prec
        if prec == F16S:
            assert np.array_equal(y, f16(y))


@pytest.mark.parametrize("dims,batch,precs", [([256, 256], 2, (F16S, F64C)), ([64, 512], 3, (F16S, F64C)),
                                              ([4096, 4096], 1, (F16S,)), ([96, 360], 2, (F16S, F64C)),
                                              ([32, 256, 256], 2, (F16S, F64C))])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_mixed_storage_nd_fused(hip_ctx, monkeypatch, dims, batch, precs, direction):
    """Mixed-storage N-D plans whose chunks start and end on fixed shapes with
    edge variants: the row pass reads the storage type, the column (or split
    second) pass writes it, the passes between run on a compute-type stage;
    against pocketfft and the boundary-pass plan."""
    count = int(np.prod(dims)) * batch
    x = o.complex_uniform(count, count % 971, np.complex64)
    for prec in precs:
        tol = {F16S: 1e-3, F64C: 1e-7}[prec]
        c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
        y, desc, yb = run_both(monkeypatch, c, direction, x)
        kernels = [p["kernel"] for p in desc["passes"]]
        assert "boundary_in" not in kernels and "boundary_out" not in kernels, kernels
        assert desc["passes"][0]["fixed_shape"] and desc["passes"][-1]["fixed_shape"]
        xin = (f16(x) if prec == F16S else x).astype(np.complex128).reshape((batch,) + tuple(dims))
        axes = tuple(range(1, len(dims) + 1))
        ref = (np.fft.fftn(xin, axes=axes) if direction == FWD else np.fft.ifftn(xin, axes=axes)).reshape(-1)
        assert o.rel_l2(y, ref) <= tol and o.rel_l2(yb, ref) <= tol, prec
        if prec == F16S:
            assert np.array_equal(y, f16(y))
