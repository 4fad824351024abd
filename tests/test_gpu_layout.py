"""Formatted device layouts, zero padding and grouped batch through the C ABI
(FftConfig::with_*_buffer_axis_stride / _batch_stride, with_zero_padding,
with_zero_padding_domain, with_grouped_batch: src/config.rs:869-1025;
boundary semantics src/zero_pad_ir.rs:38-46, 320-345, 607-647; formatted copies
src/nd_ir.rs:1105-1260)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
C2C, R2C, C2R = vk.TransformKind.ComplexToComplex, vk.TransformKind.RealToComplex, vk.TransformKind.ComplexToReal
FREQ = vk.ZeroPaddingDomain.Frequency


def cfg(dims, batch, prec=F32, kind=C2C, normalize=False):
    return vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind) \
        .with_inverse_normalization(normalize)


def build(c, direction=FWD):
    return vk.TransformIr.build(c, direction)


def ref_c2c(x, dims, batch, direction=FWD, normalize=False):
    v = x.reshape((batch,) + tuple(dims)).astype(np.complex128)
    axes = tuple(range(1, len(dims) + 1))
    if direction == FWD:
        return np.fft.fftn(v, axes=axes).reshape(-1)
    y = np.fft.ifftn(v, axes=axes) * (1 if normalize else int(np.prod(dims)))
    return y.reshape(-1)


def zero_mask(dims, batch, ranges):
    """zero_pad_ir.rs:607-617: zero where any coordinate lies in its interval."""
    m = np.zeros((batch,) + tuple(dims), dtype=bool)
    for ax, r in enumerate(ranges):
        if r is None:
            continue
        idx = [slice(None)] * (len(dims) + 1)
        idx[ax + 1] = slice(r[0], r[1])
        m[tuple(idx)] = True
    return m.reshape(-1)


@pytest.mark.parametrize("prec", [F32, F64])
def test_formatted_1d_batch_strides(hip_ctx, prec):
    n, batch = 1024, 5
    dt = np.complex64 if prec == F32 else np.complex128
    x = o.complex_uniform(n * batch, 21, dt)
    ir = build(cfg([n], batch, prec).with_input_buffer_batch_stride(1100).with_output_buffer_batch_stride(1030))
    y = hip_ctx.execute_transform(ir, x)
    tol = 1e-5 if prec == F32 else 1e-13
    assert o.rel_l2(y, ref_c2c(x, [n], batch)) <= tol
    desc = hip_ctx.plan(ir).describe()
    # a 1-D batch stride is the passes' own per-transform stride: no boundary pass
    assert not desc["boundary"]["input"] and not desc["boundary"]["output"]
    assert desc["boundary"]["fused_batch_stride"] == [True, True]
    assert hip_ctx.plan(ir).in_bytes == 1100 * batch * np.dtype(dt).itemsize


@pytest.mark.parametrize("n,batch,prec,env", [
    (1024, 7, F32, {}), (1024, 9, F32, {"VKFX_REGISTER_EXCHANGE": "1"}), (1000, 5, F32, {}), (1000, 5, F64, {}),
    (1 << 18, 5, F32, {"VKFX_WORK_BUDGET_MB": "2"}), (4096, 4, F32, {"VKFX_MAX_UPLOAD": "16"}),
    (4099, 3, F32, {}), (65537, 2, F32, {}), (97, 6, F32, {}), (47, 6, F64, {})])
def test_formatted_1d_batch_strides_fused(hip_ctx, n, batch, prec, env):
    """1-D C2C with formatted batch strides on both sides, read and written
    by the FFT passes themselves (one-upload, runtime-shape, register-exchange,
    four-step over several chunks and lanes, three-upload, Bluestein one- and
    three-pass, Rader FFT and direct): results against numpy, and the gaps of
    the output layout keep their contents."""
    import os

    import torch
    dt = np.complex64 if prec == F32 else np.complex128
    sin, sout = n + 13, n + 5
    c = cfg([n], batch, prec).with_input_buffer_batch_stride(sin).with_output_buffer_batch_stride(sout)
    ir = build(c)
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        plan = vk.Plan(hip_ctx, ir)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    try:
        desc = plan.describe()
        assert desc["boundary"]["fused_batch_stride"] == [True, True], desc["boundary"]
        assert not any(p.get("kernel", "").startswith("boundary") for p in desc["passes"])
        x = o.complex_uniform(n * batch, 60 + n % 89, dt)
        xin = np.zeros(sin * batch, dtype=dt)
        xin.reshape(batch, sin)[:, :n] = x.reshape(batch, n)
        rdt = torch.float32 if prec == F32 else torch.float64
        dx = torch.from_numpy(xin.view(np.float32 if prec == F32 else np.float64).copy()).cuda()
        dy = torch.full((sout * batch * 2,), float("nan"), device="cuda", dtype=rdt)
        plan.execute_tensors(dx, dy)
        torch.cuda.synchronize()
        y = dy.cpu().numpy().view(dt).reshape(batch, sout)
        assert np.isnan(y[:, n:].real).all() and np.isnan(y[:, n:].imag).all()
        tol = 1e-5 if prec == F32 else 1e-12
        assert o.rel_l2(y[:, :n].reshape(-1), ref_c2c(x, [n], batch)) <= tol
    finally:
        plan.close()


def test_formatted_2d_axis_and_batch_strides(hip_ctx):
    dims, batch = [32, 48], 3
    x = o.complex_uniform(32 * 48 * batch, 22, np.complex64)
    c = cfg(dims, batch).with_input_buffer_axis_stride(0, 64).with_input_buffer_batch_stride(2100) \
        .with_output_buffer_axis_stride(0, 50).with_output_buffer_batch_stride(1700)
    y = hip_ctx.execute_transform(build(c), x)
    assert o.rel_l2(y, ref_c2c(x, dims, batch)) <= 1e-5


def test_formatted_device_gaps_untouched(hip_ctx):
    """The output scatter writes only logical positions of the formatted layout."""
    import torch
    dims, batch = [16, 40], 2
    c = cfg(dims, batch).with_output_buffer_axis_stride(0, 44).with_output_buffer_batch_stride(16 * 44 + 8)
    ir = build(c)
    plan = hip_ctx.plan(ir)
    x = o.complex_uniform(16 * 40 * batch, 23, np.complex64)
    dx = torch.from_numpy(x.view(np.float32).copy()).cuda()
    phys = plan.out_bytes // 8
    dy = torch.full((phys * 2,), float("nan"), device="cuda")
    plan.execute_tensors(dx, dy)
    torch.cuda.synchronize()
    y = dy.cpu().numpy().view(np.complex64)
    idx, _ = ir._physical_index(True)
    gaps = np.ones(phys, dtype=bool)
    gaps[idx] = False
    assert np.isnan(y[gaps].real).all() and np.isnan(y[gaps].imag).all()
    assert o.rel_l2(y[idx], ref_c2c(x, dims, batch)) <= 1e-5


def test_formatted_real_round_trip(hip_ctx):
    n, batch = 4096, 3
    h = n // 2 + 1
    x = o.normal(n * batch, 24, np.float32)
    r2c = build(cfg([n], batch, kind=R2C).with_input_buffer_batch_stride(4100).with_output_buffer_batch_stride(2100))
    c2r = build(cfg([n], batch, kind=C2R, normalize=True).with_input_buffer_batch_stride(2100)
                .with_output_buffer_batch_stride(4100), INV)
    X = hip_ctx.execute_transform(r2c, x)
    ref = np.fft.rfft(x.reshape(batch, n).astype(np.float64), axis=1).reshape(-1)
    assert X.size == h * batch
    assert o.rel_l2(X, ref) <= 1e-5
    z = hip_ctx.execute_transform(c2r, X)
    assert o.rel_l2(z, x) <= 2e-5


@pytest.mark.parametrize("direction,domain", [(FWD, vk.ZeroPaddingDomain.Spatial), (INV, vk.ZeroPaddingDomain.Spatial),
                                              (FWD, FREQ), (INV, FREQ)])
def test_zero_padding_1d(hip_ctx, direction, domain):
    n, batch, left, right = 1024, 4, 100, 300
    x = o.complex_uniform(n * batch, 25, np.complex64)
    c = cfg([n], batch).with_zero_padding(0, left, right).with_zero_padding_domain(domain)
    y = hip_ctx.execute_transform(build(c, direction), x)
    mask = zero_mask([n], batch, [(left, right)])
    input_side = (direction == FWD) == (domain == vk.ZeroPaddingDomain.Spatial)
    xin = np.where(mask, 0, x) if input_side else x
    expect = ref_c2c(xin, [n], batch, direction)
    if not input_side:
        expect = np.where(mask, 0, expect)
        assert (y[mask] == 0).all()
    assert o.rel_l2(y, expect) <= 1e-5


def test_zero_padding_nd_any_axis(hip_ctx):
    dims, batch = [64, 48], 2
    ranges = [(8, 16), (40, 48)]
    x = o.complex_uniform(64 * 48 * batch, 26, np.complex64)
    c = cfg(dims, batch).with_zero_padding(0, *ranges[0]).with_zero_padding(1, *ranges[1])
    y = hip_ctx.execute_transform(build(c), x)
    mask = zero_mask(dims, batch, ranges)
    assert o.rel_l2(y, ref_c2c(np.where(mask, 0, x), dims, batch)) <= 1e-5
    # 3-D, inverse spatial: the output interval is zero (application.rs:1330-1345 shape)
    dims3 = [16, 16, 16]
    x3 = o.complex_uniform(16 ** 3, 27, np.complex128)
    c3 = cfg(dims3, 1, F64, normalize=True)
    for ax in range(3):
        c3 = c3.with_zero_padding(ax, 8, 16)
    y3 = hip_ctx.execute_transform(build(c3, INV), x3)
    m3 = zero_mask(dims3, 1, [(8, 16)] * 3)
    assert (y3[m3] == 0).all()
    assert o.rel_l2(y3, np.where(m3, 0, ref_c2c(x3, dims3, 1, INV, True))) <= 1e-13


@pytest.mark.parametrize("length", [206, 578])
def test_zero_padding_real_round_trip(hip_ctx, length):
    # application.rs:1045-1110: R2C with [3N/4, N) zero-padded ignores the
    # garbage there; C2R with the same padding restores exact zeros
    left = length * 3 // 4
    x = np.sin(0.37 * np.arange(length)) + 0.25 * np.cos(1.3 * np.arange(length))
    x[left:] = 10_000.0 + np.arange(length - left)
    manual = x.copy()
    manual[left:] = 0.0
    fwd = build(vk.FftConfig.new([length]).with_transform(R2C).with_precision(F64).with_zero_padding(0, left, length))
    X = hip_ctx.execute_transform(fwd, x)
    assert np.max(np.abs(X - np.fft.rfft(manual))) <= 2e-8 * length
    inv = build(vk.FftConfig.new([length]).with_transform(C2R).with_precision(F64).with_inverse_normalization(True)
                .with_zero_padding(0, left, length), INV)
    z = hip_ctx.execute_transform(inv, X)
    assert (z[left:] == 0.0).all()
    assert np.max(np.abs(z - manual)) <= 2e-8 * length


def test_frequency_zero_padding_real_fails_closed(hip_ctx):
    c = vk.FftConfig.new([256]).with_transform(R2C).with_zero_padding(0, 10, 20) \
        .with_zero_padding_domain(FREQ)
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.plan(build(c))
    assert ei.value.status == -3


def test_grouped_batch_hint_and_mixed_layout(hip_ctx):
    n, batch = 512, 6
    x = o.complex_uniform(n * batch, 28, np.complex64)
    c = cfg([n], batch, vk.Precision.F16StorageF32Compute).with_grouped_batch(0, 3) \
        .with_input_buffer_batch_stride(520).with_zero_padding(0, 500, 512)
    ir = build(c)
    y = hip_ctx.execute_transform(ir, x)
    xq = x.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)
    mask = zero_mask([n], batch, [(500, 512)])
    assert o.rel_l2(y, ref_c2c(np.where(mask, 0, xq), [n], batch)) <= 1e-3
    assert hip_ctx.plan(ir).describe()["boundary"]["grouped_batch"] == [3]
    with pytest.raises(vk.VkFftError):
        hip_ctx.plan(build(cfg([n], 2).with_grouped_batch(0, 3)))


def test_invalid_formatted_strides(hip_ctx):
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.plan(build(cfg([8, 16], 1).with_input_buffer_axis_stride(0, 12)))
    assert ei.value.status == -7
    with pytest.raises(vk.VkFftError):
        hip_ctx.plan(build(cfg([8, 16], 1).with_input_buffer_axis_stride(1, 2)))
    with pytest.raises(vk.VkFftError):
        hip_ctx.plan(build(cfg([8, 16], 2).with_output_buffer_batch_stride(100)))
