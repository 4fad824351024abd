"""FftConfig::omit_dimension through the C ABI (config.rs:844-853, 1053-1067;
nd_ir.rs:1692-1725): omitted axes stay untransformed, the others transform
with their own normalization; the real axis of R2C/C2R cannot be omitted."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse


@pytest.mark.parametrize("dims,omit,prec", [([3, 4], [0], F64), ([3, 4], [1], F64), ([16, 12, 10], [1], F64),
                                            ([64, 48, 8], [0, 2], F32), ([4096, 64], [1], F32),
                                            ([8, 1, 4], [0], F64)])
def test_omit_c2c(hip_ctx, dims, omit, prec):
    batch = 2
    cd = np.complex64 if prec == F32 else np.complex128
    x = o.complex_uniform(int(np.prod(dims)) * batch, 41, cd)
    active = tuple(ax + 1 for ax in range(len(dims)) if ax not in omit)
    v = x.reshape((batch,) + tuple(dims)).astype(np.complex128)
    for direction, normalize in ((FWD, False), (INV, True), (INV, False)):
        c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_inverse_normalization(normalize)
        for ax in omit:
            c = c.with_omit_dimension(ax, True)
        y = hip_ctx.execute_transform(vk.TransformIr.build(c, direction), x)
        if direction == FWD:
            ref = np.fft.fftn(v, axes=active)
        else:
            ref = np.fft.ifftn(v, axes=active) * (1 if normalize else int(np.prod([dims[a - 1] for a in active])))
        assert o.rel_l2(y, ref.reshape(-1)) <= (1e-5 if prec == F32 else 1e-13), (dims, omit, direction)


def test_omit_real(hip_ctx):
    dims, batch = [8, 16], 3
    x = o.normal(8 * 16 * batch, 42, np.float64)
    c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(F64) \
        .with_transform(vk.TransformKind.RealToComplex).with_omit_dimension(0, True)
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    ref = np.fft.rfft(x.reshape(batch, 8, 16), axis=2)
    assert o.rel_l2(y, ref.reshape(-1)) <= 1e-13
    ci = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(F64) \
        .with_transform(vk.TransformKind.ComplexToReal).with_omit_dimension(0, True).with_inverse_normalization(True)
    z = hip_ctx.execute_transform(vk.TransformIr.build(ci, INV), y)
    assert o.rel_l2(z, x) <= 1e-13


def test_omit_rejections(hip_ctx):
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.plan(vk.TransformIr.build(vk.FftConfig.new([16]).with_omit_dimension(0, True), FWD))
    assert ei.value.status == -3
    c = vk.FftConfig.new([8, 4]).with_transform(vk.TransformKind.RealToComplex).with_omit_dimension(1, True)
    with pytest.raises(vk.VkFftError) as ei:
        hip_ctx.plan(vk.TransformIr.build(c, FWD))
    assert ei.value.status == -3
