"""N-D R2C / C2R through the C ABI (NdRealFftIr, src/nd_real_ir.rs:754-870):
the fastest axis as a 1-D real transform, the other axes as C2C over the
compact [.., N/2+1] spectrum, against the oracle's N-D C2C of the promoted
input (f32) and pocketfft's rfftn / irfftn (f64)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
R2C, C2R = vk.TransformKind.RealToComplex, vk.TransformKind.ComplexToReal


def cfg(dims, batch, prec, kind, normalize=False):
    return vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind) \
        .with_inverse_normalization(normalize)


def compact_ref(x, dims, batch, threads=8):
    """Forward N-D DFT of the real input (oracle, f64), compact last axis."""
    full = o.fft_nd(x.astype(np.complex128), dims, batch, threads=threads).reshape((batch,) + tuple(dims))
    return full[..., :dims[-1] // 2 + 1].reshape(-1)


ND = [([64, 48], 3, F32), ([16, 12, 10], 2, F64), ([32, 45], 2, F32), ([8, 4, 6, 10], 2, F64),
      ([4, 1 << 16], 2, F32), ([1009, 6], 2, F32), ([512, 1024], 2, F32), ([1, 256], 3, F32), ([6, 1], 2, F64)]


@pytest.mark.parametrize("dims,batch,prec", ND)
def test_nd_r2c(hip_ctx, dims, batch, prec):
    rd = np.float32 if prec == F32 else np.float64
    count = int(np.prod(dims)) * batch
    x = o.uniform(count, count % 997, rd)
    ir = vk.TransformIr.build(cfg(dims, batch, prec, R2C), FWD)
    y = hip_ctx.execute_transform(ir, x)
    assert y.size == ir.output_count() == batch * int(np.prod(dims[:-1])) * (dims[-1] // 2 + 1)
    if prec == F32:
        assert o.rel_l2(y, compact_ref(x, dims, batch)) <= 1e-5, dims
    else:
        ref = np.fft.rfftn(x.reshape((batch,) + tuple(dims)), axes=tuple(range(1, len(dims) + 1)))
        assert o.rel_l2(y, ref.reshape(-1)) <= 1e-13, dims
    if len(dims) > 1 and int(np.prod(dims[:-1])) > 1:
        assert "real_nd" in hip_ctx.plan(ir).describe()


@pytest.mark.parametrize("dims,batch,prec", ND)
def test_nd_c2r(hip_ctx, dims, batch, prec):
    """Unnormalized C2R of a Hermitian spectrum (pocketfft's rfftn of a real
    tensor) returns prod(dims) times the tensor. (A spectrum that is not
    Hermitian has no unique real inverse: the half-size real-axis algebra of
    real_ir.rs:1086-1099 and irfftn disagree on it.)"""
    cd = np.complex64 if prec == F32 else np.complex128
    h = dims[-1] // 2 + 1
    x = o.uniform(batch * int(np.prod(dims)), 17, np.float64).reshape((batch,) + tuple(dims))
    axes = tuple(range(1, len(dims) + 1))
    X = np.fft.rfftn(x, axes=axes).astype(cd).reshape(-1)
    ir = vk.TransformIr.build(cfg(dims, batch, prec, C2R), INV)
    z = hip_ctx.execute_transform(ir, X)
    assert z.size == batch * int(np.prod(dims)) and X.size == ir.input_count()
    ref = x.reshape(-1) * int(np.prod(dims))
    assert o.rel_l2(z, ref) <= (1e-5 if prec == F32 else 1e-13), dims
    # the input stays untouched on the device path
    if prec == F64:
        import torch
        plan = hip_ctx.plan(ir)
        dx = torch.from_numpy(X.view(np.float64).copy()).cuda()
        dz = torch.empty(z.size, dtype=torch.float64, device="cuda")
        plan.execute_tensors(dx, dz)
        torch.cuda.synchronize()
        assert np.array_equal(dx.cpu().numpy(), X.view(np.float64))
        assert np.array_equal(dz.cpu().numpy(), z)


@pytest.mark.parametrize("dims,batch,prec", [([64, 48], 2, F32), ([16, 12, 10], 2, F64), ([256, 254], 1, F32)])
def test_nd_round_trip(hip_ctx, dims, batch, prec):
    rd = np.float32 if prec == F32 else np.float64
    x = o.normal(int(np.prod(dims)) * batch, 31, rd)
    X = hip_ctx.execute_transform(vk.TransformIr.build(cfg(dims, batch, prec, R2C), FWD), x)
    z = hip_ctx.execute_transform(vk.TransformIr.build(cfg(dims, batch, prec, C2R, True), INV), X)
    assert o.rel_l2(z, x) <= (2e-5 if prec == F32 else 1e-13)


def test_nd_real_c3_shape(hip_ctx):
    """4096 x 4096 real images (the C3 geometry as R2C + C2R), round trip."""
    dims, batch = [4096, 4096], 2
    x = o.normal(4096 * 4096 * batch, 32, np.float32)
    X = hip_ctx.execute_transform(vk.TransformIr.build(cfg(dims, batch, F32, R2C), FWD), x)
    # spot rows against pocketfft
    ref0 = np.fft.rfft2(x[:4096 * 4096].reshape(dims).astype(np.float64))
    assert o.rel_l2(X[:4096 * 2049], ref0.reshape(-1)) <= 1e-5
    z = hip_ctx.execute_transform(vk.TransformIr.build(cfg(dims, batch, F32, C2R, True), INV), X)
    assert o.rel_l2(z, x) <= 2e-5


def test_nd_real_layouts_and_mixed(hip_ctx):
    dims, batch = [32, 40], 2
    x = o.normal(32 * 40 * batch, 33, np.float32)
    ref = np.fft.rfftn(x.reshape(batch, 32, 40).astype(np.float64), axes=(1, 2)).reshape(-1)
    # formatted output batch stride
    c = cfg(dims, batch, F32, R2C).with_output_buffer_batch_stride(32 * 21 + 5)
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    assert o.rel_l2(y, ref) <= 1e-5
    # spatial zero padding of the real input
    cz = cfg(dims, batch, F32, R2C).with_zero_padding(1, 30, 40)
    yz = hip_ctx.execute_transform(vk.TransformIr.build(cz, FWD), x)
    xm = x.reshape(batch, 32, 40).copy()
    xm[:, :, 30:] = 0
    assert o.rel_l2(yz, np.fft.rfftn(xm.astype(np.float64), axes=(1, 2)).reshape(-1)) <= 1e-5
    # f64 compute with f32 storage, both directions
    for kind, direction in ((R2C, FWD), (C2R, INV)):
        ir = vk.TransformIr.build(cfg(dims, batch, vk.Precision.F64ComputeF32Storage, kind, True), direction)
        if kind == R2C:
            ym = hip_ctx.execute_transform(ir, x)
            assert o.rel_l2(ym, ref) <= 1e-7
        else:
            zm = hip_ctx.execute_transform(ir, ym)
            assert o.rel_l2(zm, x) <= 1e-7
