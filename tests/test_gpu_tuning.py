"""FftConfig::with_tuning (config.rs:367-420, 820-832) and kernel-spectrum
preparation with kernelConvolution (config.rs:746-749, 806-818, 1101-1136)
through the C ABI."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD = vk.Direction.Forward


def test_tuning_moves_rader_prime_to_bluestein(hip_ctx):
    n, batch = 1009, 3
    assert vk.planner_axis(n)[0] == vk.AlgorithmKind.Rader
    tuned = vk.PlannerTuning(max_rader_fft_prime=1000)
    assert vk.planner_axis(n, tuning=tuned)[0] == vk.AlgorithmKind.Bluestein
    x = o.complex_uniform(n * batch, 61, np.complex128)
    ref = np.fft.fft(x.reshape(batch, n), axis=1).reshape(-1)
    outs = []
    for t in (None, tuned):
        c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F64)
        if t is not None:
            c = c.with_tuning(t)
        ir = vk.TransformIr.build(c, FWD)
        desc = hip_ctx.plan(ir).describe()
        assert desc["axes"][0]["algorithm"] == ("bluestein" if t else "rader")
        y = hip_ctx.execute_transform(ir, x)
        assert o.rel_l2(y, ref) <= 1e-13
        outs.append(y)
    # the library planner honours the same tuning for a real transform's full-complex C2C
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F64) \
        .with_transform(vk.TransformKind.RealToComplex).with_tuning(tuned)
    xr = o.normal(n * batch, 62, np.float64)
    yr = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), xr)
    assert o.rel_l2(yr, np.fft.rfft(xr.reshape(batch, n), axis=1).reshape(-1)) <= 1e-13
    # back to the device tuning
    assert vk.TransformIr.build(c.with_device_tuning(), FWD).config.tuning is None


def test_kernel_preparation_feeds_convolution(hip_ctx):
    # 1-D C2C: prepare FFT(h) over coordinate_features * batch systems
    n = 512
    h = o.complex_uniform(n * 2, 63, np.complex64)
    prep = vk.FftConfig.new([n]).with_batch_count(2).with_coordinate_features(1).with_kernel_convolution(True)
    spec = hip_ctx.execute_transform(vk.TransformIr.build(prep, FWD), h)
    assert o.rel_l2(spec, np.fft.fft(h.reshape(2, n).astype(np.complex128), axis=1).reshape(-1)) <= 1e-5
    x = o.complex_uniform(n, 64, np.complex64)
    conv = vk.ConvolutionIr.build(vk.FftConfig.new([n]).with_convolution(True).with_convolution_kernel_count(2), spec)
    y = hip_ctx.execute_convolution(conv, x).reshape(2, n)
    for k in range(2):
        ref = np.fft.ifft(np.fft.fft(x.astype(np.complex128)) * np.fft.fft(h[k * n:(k + 1) * n].astype(np.complex128)))
        assert o.rel_l2(y[k], ref) <= 1e-5
    # sample_52-style 2-D R2C preparation (batch 2, coordinates 2) for a
    # real-application convolution with 2 kernels over 2 coordinates
    dims = [32, 48]
    hr = o.normal(4 * 32 * 48, 65, np.float32)
    prep2 = vk.FftConfig.new(dims).with_batch_count(2).with_coordinate_features(2) \
        .with_transform(vk.TransformKind.RealToComplex).with_kernel_convolution(True)
    ir2 = vk.TransformIr.build(prep2, FWD)
    assert ir2.input_count() == 4 * 32 * 48
    spec2 = hip_ctx.execute_transform(ir2, hr)
    ref2 = np.fft.rfftn(hr.reshape(4, 32, 48).astype(np.float64), axes=(1, 2)).reshape(-1)
    assert o.rel_l2(spec2, ref2) <= 1e-5
    xr = o.normal(2 * 32 * 48, 66, np.float32)
    cc = vk.FftConfig.new(dims).with_transform(vk.TransformKind.RealToComplex).with_convolution(True) \
        .with_coordinate_features(2).with_convolution_kernel_count(2)
    yr = hip_ctx.execute_convolution(vk.ConvolutionIr.build(cc, spec2), xr)
    assert o.rel_l2(yr, o.convolution_real(xr, spec2, dims, coords=2, kernel_count=2)) <= 1e-5
