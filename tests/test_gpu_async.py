"""Async tickets and device-resident chains through the C ABI (the HIP side
of NativeAsyncRuntime, src/backend/native_runtime.rs:406-451, and of the
resident program chains, src/backend/cuda/runtime.rs:1744-1809).

Results of a ticket or a chain must equal the synchronous execute of the same
plans bit for bit (same kernels, own buffers), and the oracle within the
parity tolerances (f32 relative L2 1e-5, f64 1e-13)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse


def c2c_ir(dims, batch, prec=F32, direction=FWD, normalize=False):
    cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec) \
        .with_inverse_normalization(normalize)
    return vk.TransformIr.build(cfg, direction)


def real_irs(n, batch):
    r2c = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch)
                               .with_transform(vk.TransformKind.RealToComplex), FWD)
    c2r = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch)
                               .with_transform(vk.TransformKind.ComplexToReal)
                               .with_inverse_normalization(True), INV)
    return r2c, c2r


def test_tickets_in_flight(hip_ctx):
    # hip/runtime.rs:3038-3095: several submissions in flight from one thread
    cases = [(c2c_ir([1024], 64), o.complex_uniform(1024 * 64, 1, np.complex64)),
             (c2c_ir([1024], 64), o.complex_uniform(1024 * 64, 2, np.complex64)),
             (c2c_ir([4099], 8), o.complex_uniform(4099 * 8, 3, np.complex64)),
             (c2c_ir([96, 80], 3, F64), o.complex_uniform(96 * 80 * 3, 4, np.complex128))]
    tickets = [hip_ctx.submit_transform_async(ir, x) for ir, x in cases]
    outs = [t.wait() for t in tickets]
    for (ir, x), y in zip(cases, outs):
        sync = hip_ctx.execute_transform(ir, x)
        assert np.array_equal(y, sync)
        dims = ir.config.dimensions
        ref = o.fft_nd(x, dims, ir.config.batch_count, threads=8) if len(dims) > 1 else \
            o.fft_batch(x.astype(np.complex128), dims[0], "forward", False, threads=8)
        tol = 1e-5 if ir.config.precision == F32 else 1e-13
        assert o.rel_l2(y, ref) <= tol


def test_ticket_ready_and_drop(hip_ctx):
    ir = c2c_ir([2048], 32)
    x = o.complex_uniform(2048 * 32, 5, np.complex64)
    t = hip_ctx.submit_transform_async(ir, x)
    y = t.wait()
    assert np.array_equal(y, hip_ctx.execute_transform(ir, x))
    # a ticket dropped without wait synchronises and returns its buffers
    t2 = hip_ctx.submit_transform_async(ir, x)
    t2.close()
    t3 = hip_ctx.submit_transform_async(ir, x)
    while not t3.ready():
        pass
    assert np.array_equal(t3.wait(), y)


def test_tickets_two_lane_plan_isolated(hip_ctx):
    """A chunked plan (four-step, two stream lanes) in two concurrent tickets:
    each ticket has its own workspace."""
    ir = c2c_ir([1 << 20], 64)
    plan = hip_ctx.plan(ir)
    assert plan.describe()["lanes"] == 2
    xa = o.complex_uniform((1 << 20) * 64, 6, np.complex64)
    xb = o.complex_uniform((1 << 20) * 64, 7, np.complex64)
    ta = hip_ctx.submit_transform_async(ir, xa)
    tb = hip_ctx.submit_transform_async(ir, xb)
    ya, yb = ta.wait(), tb.wait()
    assert np.array_equal(ya, hip_ctx.execute_transform(ir, xa))
    assert np.array_equal(yb, hip_ctx.execute_transform(ir, xb))
    n = 1 << 20
    for b in (0, 63):
        ref = o.fft(xb[b * n:(b + 1) * n].astype(np.complex128))
        assert o.rel_l2(yb[b * n:(b + 1) * n], ref) <= 1e-5


def test_real_ticket(hip_ctx):
    r2c, c2r = real_irs(1 << 14, 6)
    x = o.normal((1 << 14) * 6, 8, np.float32)
    t = hip_ctx.submit_transform_async(r2c, x)
    X = t.wait()
    assert np.array_equal(X, hip_ctx.execute_transform(r2c, x))
    h = (1 << 14) // 2 + 1
    ref = o.r2c_batch(x[: 1 << 14].astype(np.float64), 1 << 14)
    assert o.rel_l2(X[:h], ref) <= 1e-5


def test_chain_host_round_trips(hip_ctx):
    fwd = c2c_ir([1024], 16)
    inv = c2c_ir([1024], 16, direction=INV, normalize=True)
    x = o.complex_uniform(1024 * 16, 9, np.complex64)
    z = hip_ctx.execute_chain([fwd, inv], x)
    seq = hip_ctx.execute_transform(inv, hip_ctx.execute_transform(fwd, x))
    assert np.array_equal(z, seq)
    assert o.rel_l2(z, x) <= 2e-5
    r2c, c2r = real_irs(1 << 20, 2)
    xr = o.normal((1 << 20) * 2, 10, np.float32)
    zr = hip_ctx.execute_chain([r2c, c2r], xr)
    assert zr.dtype == np.float32
    assert o.rel_l2(zr, xr) <= 2e-5
    # three transforms: fwd, inv, fwd == fwd
    y3 = hip_ctx.execute_chain([fwd, inv, fwd], x)
    assert o.rel_l2(y3, hip_ctx.execute_transform(fwd, x)) <= 2e-5


def test_chain_device_resident(hip_ctx):
    import torch
    fwd = c2c_ir([64, 64], 4, F64)
    inv = c2c_ir([64, 64], 4, F64, INV, True)
    x = o.complex_uniform(64 * 64 * 4, 11, np.complex128)
    dx = torch.from_numpy(x.view(np.float64).copy()).cuda()
    dy = torch.empty_like(dx)
    s = torch.cuda.current_stream()
    vk.execute_chain([hip_ctx.plan(fwd), hip_ctx.plan(inv)], dx.data_ptr(), dy.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().view(np.complex128)
    assert o.rel_l2(y, x) <= 1e-13


def test_chain_transition_mismatch(hip_ctx):
    a = c2c_ir([1024], 2)
    b = c2c_ir([2048], 2)
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.execute_chain([a, b], o.complex_uniform(2048, 1, np.complex64))
    assert ei.value.status == -5
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.execute_chain([a], o.complex_uniform(100, 1, np.complex64))
    assert ei.value.status == -5


def test_runtime_caches_and_clear(hip_ctx):
    """hip/runtime.rs:3038-3095, 3225-3343: with two tickets in flight the
    caches cannot be cleared; afterwards the pooled streams and transient
    buffers are counted, clearing empties them and later submissions work."""
    a = (c2c_ir([64], 1), o.complex_uniform(64, 6, np.complex64))
    b = (c2c_ir([96], 1), o.complex_uniform(96, 7, np.complex64))
    ta = hip_ctx.submit_transform_async(*a)
    tb = hip_ctx.submit_transform_async(*b)
    assert hip_ctx.in_flight_submission_count() == 2
    with pytest.raises(vk.VkFftError):
        hip_ctx.clear_runtime_caches()
    yb, ya = tb.wait(), ta.wait()
    tb.close()
    ta.close()
    assert hip_ctx.in_flight_submission_count() == 0
    assert hip_ctx.pooled_stream_count() >= 2
    assert hip_ctx.cached_transient_buffer_count() > 0
    for (ir, x), y in ((a, ya), (b, yb)):
        ref = o.fft_batch(x.astype(np.complex128), ir.config.dimensions[0], "forward", False)
        assert np.max(np.abs(y - ref)) <= 2e-3 * x.size  # the reference test's bound
    hip_ctx.clear_runtime_caches()
    assert hip_ctx.pooled_stream_count() == 0 and hip_ctx.cached_transient_buffer_count() == 0
    t = hip_ctx.submit_transform_async(*a)
    assert np.array_equal(t.wait(), ya)
    t.close()


def test_pass_resource_reports(hip_ctx):
    """compiled_pass_resource_reports / theoretical_occupancy_reports
    (native_runtime.rs:96-131): one report per distinct pass, with the
    compiled kernel's registers and the blocks of the launch that fit a CU."""
    c1 = hip_ctx.plan(c2c_ir([1024], 8192)).resources()
    assert len(c1) == 1 and c1[0]["pass"] == "stockham"
    r = c1[0]
    assert 0 < r["registers_per_thread"] <= 512 and r["local_bytes_per_thread"] == 0
    assert r["block_threads"] == 128 and r["dynamic_shared_bytes"] >= 1024 * 8
    assert 1 <= r["resident_blocks_per_cu"] and r["waves_per_cu"] <= 64
    real = hip_ctx.plan(real_irs(1 << 20, 4)[0]).resources()
    assert [p["pass"] for p in real] == ["r2c_four_step_columns", "r2c_four_step_rows"] or len(real) == 2
    assert all(p["resident_blocks_per_cu"] >= 1 for p in real)
    # mixed storage: converted inside the one-upload pass or the two four-step
    # passes with fixed edge shapes, else boundary passes around the plan
    mixed = vk.TransformIr.build(vk.FftConfig.new([1024]).with_batch_count(4)
                                 .with_precision(vk.Precision.F64ComputeF32Storage), FWD)
    fused = hip_ctx.plan(mixed).resources()
    assert [p["pass"] for p in fused] == ["stockham"] and fused[0]["resident_blocks_per_cu"] >= 1
    mixed = vk.TransformIr.build(vk.FftConfig.new([1 << 20]).with_batch_count(1)
                                 .with_precision(vk.Precision.F64ComputeF32Storage), FWD)
    names = [p["pass"] for p in hip_ctx.plan(mixed).resources()]
    assert names == ["four_step_columns", "four_step_rows"], names
    mixed = vk.TransformIr.build(vk.FftConfig.new([3 << 16]).with_batch_count(1)
                                 .with_precision(vk.Precision.F64ComputeF32Storage), FWD)
    names = [p["pass"] for p in hip_ctx.plan(mixed).resources()]
    assert names[0] == "boundary_in" and names[-1] == "boundary_out"


def _shim_ticket_wait(ctx, ir, x):
    """What the reference-side Rust shim's Mi355xTicket32/64 does: submit the
    plan's input bytes, size the wait buffer from vkfx_plan_output_info's
    widened bytes as Complex32/64 elements, wait with exactly that byte count
    and hand the complex vector on (finish_transform_output32/64 then takes
    `.re` for real outputs, native_runtime.rs:2045-2087)."""
    import ctypes
    L = ctx._L
    plan = ctx.plan(ir)
    xs = np.ascontiguousarray(x)
    assert xs.nbytes == plan.in_bytes
    real = ctypes.c_int32()
    widened = ctypes.c_uint64()
    vk._check(L.vkfx_plan_output_info(plan.handle, ctypes.byref(real), ctypes.byref(widened)), L)
    cdt = np.complex64 if ir.config.precision == F32 else np.complex128
    out_len = int(widened.value) // np.dtype(cdt).itemsize  # Vec<Complex32>::len
    t = ctypes.c_void_p()
    vk._check(L.vkfx_submit_host(plan.handle, xs.ctypes.data, xs.nbytes, ctypes.byref(t)), L)
    try:
        # the size the round-1 shim passed (out_len * 8 of a real output) is refused
        if real.value:
            bad = np.empty(plan.out_bytes // np.dtype(cdt).itemsize // 2 + 1, dtype=cdt)
            rc = L.vkfx_ticket_wait_complex(t, bad.ctypes.data, bad.nbytes)
            assert rc == -5
        out = np.empty(out_len, dtype=cdt)
        vk._check(L.vkfx_ticket_wait_complex(t, out.ctypes.data, out_len * np.dtype(cdt).itemsize), L)
    finally:
        vk._check(L.vkfx_ticket_destroy(t), L)
    return bool(real.value), out


@pytest.mark.parametrize("prec", [F32, F64])
def test_shim_real_output_tickets(hip_ctx, prec):
    rd = np.float32 if prec == F32 else np.float64
    tol = 1e-5 if prec == F32 else 1e-12
    # C2R: widened to {v, 0}; .re is the oracle's C2R
    n, batch = 4096, 3
    x = o.normal(n * batch, 31, rd)
    r2c = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
                               .with_transform(vk.TransformKind.RealToComplex), FWD)
    c2r = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
                               .with_transform(vk.TransformKind.ComplexToReal), INV)
    real, X = _shim_ticket_wait(hip_ctx, r2c, x)
    assert not real and X.size == batch * (n // 2 + 1)
    assert o.rel_l2(X, o.r2c_batch(x.astype(np.float64), n, threads=8)) <= tol
    real, y = _shim_ticket_wait(hip_ctx, c2r, X)
    assert real and y.size == n * batch
    assert np.all(y.imag == 0)
    ref = o.c2r_batch(X.astype(np.complex128), n, threads=8)
    assert o.rel_l2(y.real, ref) <= tol
    assert np.array_equal(y.real, hip_ctx.execute_transform(c2r, X))
    # DCT-II: real in, real out, widened the same way
    m, mb = 256, 8
    xr = o.uniform(m * mb, 32, rd)
    dct = vk.TransformIr.build(vk.FftConfig.new([m]).with_batch_count(mb).with_precision(prec)
                               .with_transform(vk.TransformKind.dct(2)), FWD)
    real, z = _shim_ticket_wait(hip_ctx, dct, xr)
    assert real and z.size == m * mb and np.all(z.imag == 0)
    assert o.rel_l2(z.real, o.r2r_batch(xr.astype(np.float64), m, "dct2", threads=8)) <= tol


def test_shim_f16_storage_tickets(hip_ctx):
    """The shim's F16StorageF32Compute ticket path: binary16 input
    (Binary16::from_f32), out_len = widened bytes / 4 (binary16 pairs), the
    wait decoded to Complex32 (native_runtime.rs:1111-1120 decodes F16
    storage on readback). Equal to the synchronous execute of the same plan;
    C2C and C2R (a real output widened to {v, 0})."""
    import ctypes
    L = hip_ctx._L
    F16 = vk.Precision.F16StorageF32Compute
    n, batch = 4096, 3
    cases = [
        (vk.TransformIr.build(vk.FftConfig.new([1024]).with_batch_count(4).with_precision(F16), FWD),
         o.complex_uniform(1024 * 4, 41, np.complex64)),
        (vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F16)
                              .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True), INV),
         # a Hermitian spectrum (C2R of anything else has no unique real inverse)
         (o.r2c_batch(o.normal(n * batch, 42), n) / n).astype(np.complex64)),
    ]
    for ir, x in cases:
        plan = hip_ctx.plan(ir)
        x16 = np.ascontiguousarray(x.view(np.float32).astype(np.float16))
        assert x16.nbytes == plan.in_bytes
        real, widened = ctypes.c_int32(), ctypes.c_uint64()
        vk._check(L.vkfx_plan_output_info(plan.handle, ctypes.byref(real), ctypes.byref(widened)), L)
        out_len = int(widened.value) // 4
        t = ctypes.c_void_p()
        vk._check(L.vkfx_submit_host(plan.handle, x16.ctypes.data, x16.nbytes, ctypes.byref(t)), L)
        try:
            raw = np.empty(2 * out_len, dtype=np.float16)
            vk._check(L.vkfx_ticket_wait_complex(t, raw.ctypes.data, raw.nbytes), L)
        finally:
            L.vkfx_ticket_destroy(t)
        y = raw.astype(np.float32).view(np.complex64)
        sync = hip_ctx.execute_transform(ir, x)
        if real.value:
            assert np.all(y.imag == 0) and np.array_equal(y.real, sync)
            xin = x16.astype(np.float32).view(np.complex64).astype(np.complex128)
            assert o.rel_l2(y.real, o.c2r_batch(xin, n, normalize=True, threads=8)) <= 2e-3
        else:
            assert np.array_equal(y, sync)
            xin = x16.astype(np.float32).view(np.complex64).astype(np.complex128)
            assert o.rel_l2(y, o.fft_batch(xin, 1024)) <= 2e-3


def test_context_close_releases_tickets_and_plans():
    """Closing a context with a live ticket destroys the ticket and its plan
    first; the ticket then refuses to wait instead of reading freed memory.
    The C ABI refuses to destroy a plan with live tickets or a context with
    live plans."""
    import ctypes
    import os
    if not os.path.exists("/dev/kfd"):
        pytest.skip("no GPU in this container")
    ctx = vk.HipExecutionContext(0)
    ir = c2c_ir([1024], 8)
    x = o.complex_uniform(1024 * 8, 33, np.complex64)
    t = ctx.submit_transform_async(ir, x)
    L = ctx._L
    plan = ctx.plan(ir)
    assert L.vkfx_plan_destroy(plan.handle) == -2       # its ticket is alive
    assert L.vkfx_context_destroy(ctx.handle) == -2     # plans and tickets are alive
    ctx.close()
    assert not ctx.handle and not plan.handle
    with pytest.raises(vk.VkFftError):
        t.wait()
    with pytest.raises(vk.VkFftError):
        t.ready()
