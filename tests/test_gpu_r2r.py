"""DCT / DST types I-IV through the C ABI (TransformKind::Dct/Dst, the
definitions of src/r2r_ir.rs:2351-2434) against the oracle's direct sums and
scipy.fft (pocketfft) for f64."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
KINDS = ["dct1", "dct2", "dct3", "dct4", "dst1", "dst2", "dst3", "dst4"]


def kind_of(name):
    t = int(name[-1])
    return vk.TransformKind.dct(t) if name.startswith("dct") else vk.TransformKind.dst(t)


def r2r_ir(name, n, batch, prec, direction=FWD, normalize=False):
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_transform(kind_of(name)) \
        .with_inverse_normalization(normalize)
    return vk.TransformIr.build(c, direction)


def scipy_ref(name, x):
    import scipy.fft as sf
    return (sf.dct if name.startswith("dct") else sf.dst)(x, type=int(name[-1]), axis=-1)


@pytest.mark.parametrize("name", KINDS)
@pytest.mark.parametrize("prec", [F32, F64])
def test_r2r_forward(hip_ctx, name, prec):
    rd = np.float32 if prec == F32 else np.float64
    for n in (2, 9, 64, 257, 1000, 4096):
        batch = 3
        x = o.uniform(n * batch, n + len(name), rd)
        y = hip_ctx.execute_transform(r2r_ir(name, n, batch, prec), x)
        assert y.dtype == rd and y.size == n * batch
        if prec == F32:
            ref = o.r2r_batch(x.astype(np.float64), n, name, threads=8)
            assert o.rel_l2(y, ref) <= 1e-5, (name, n)
        else:
            ref = scipy_ref(name, x.reshape(batch, n)).reshape(-1)
            assert o.rel_l2(y, ref) <= 1e-13, (name, n)


@pytest.mark.parametrize("name", KINDS)
def test_r2r_inverse_round_trip(hip_ctx, name):
    n, batch = 300, 4
    x = o.uniform(n * batch, 7, np.float64)
    y = hip_ctx.execute_transform(r2r_ir(name, n, batch, F64), x)
    z = hip_ctx.execute_transform(r2r_ir(name, n, batch, F64, INV, True), y)
    assert o.rel_l2(z, x) <= 1e-13
    # unnormalized inverse: the partner transform itself
    partner = {"dct2": "dct3", "dct3": "dct2", "dst2": "dst3", "dst3": "dst2"}.get(name, name)
    u = hip_ctx.execute_transform(r2r_ir(name, n, batch, F64, INV), y)
    assert o.rel_l2(u, scipy_ref(partner, y.reshape(batch, n)).reshape(-1)) <= 1e-13


def test_reference_medium_dct_goldens(hip_ctx):
    """application.rs:1112-1155: DCT-II / DCT-III of N=257 against the direct
    sums within 2e-8 * N, and the normalized inverse DCT-II restores x."""
    n = 257
    x = np.sin(0.37 * np.arange(n)) + 0.25 * np.cos(1.3 * np.arange(n))
    d2 = hip_ctx.execute_transform(r2r_ir("dct2", n, 1, F64), x)
    assert np.max(np.abs(d2 - o.r2r_batch(x, n, "dct2"))) <= 2e-8 * n
    d3 = hip_ctx.execute_transform(r2r_ir("dct3", n, 1, F64), x)
    assert np.max(np.abs(d3 - o.r2r_batch(x, n, "dct3"))) <= 2e-8 * n
    back = hip_ctx.execute_transform(r2r_ir("dct2", n, 1, F64, INV, True), d2)
    assert np.max(np.abs(back - x)) <= 2e-8 * n


def test_r2r_zero_padding(hip_ctx):
    """Forward masks the input interval, inverse the output interval
    (execute_r2r_ir, r2r_ir.rs:1227-1279)."""
    n, batch, left, right = 128, 2, 96, 128
    x = o.uniform(n * batch, 11, np.float64)
    c = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F64).with_transform(vk.TransformKind.DctII) \
        .with_zero_padding(0, left, right)
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    xm = x.reshape(batch, n).copy()
    xm[:, left:right] = 0
    assert o.rel_l2(y, scipy_ref("dct2", xm).reshape(-1)) <= 1e-13
    ci = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(F64).with_transform(vk.TransformKind.DctII) \
        .with_inverse_normalization(True).with_zero_padding(0, left, right)
    z = hip_ctx.execute_transform(vk.TransformIr.build(ci, INV), y).reshape(batch, n)
    assert (z[:, left:right] == 0).all()
    assert o.rel_l2(z[:, :left], xm[:, :left]) <= 1e-13


def test_r2r_mixed_precision_and_device_in_place(hip_ctx):
    import torch
    n, batch = 1000, 5
    x = o.uniform(n * batch, 12, np.float32)
    ir = r2r_ir("dct2", n, batch, vk.Precision.F64ComputeF32Storage)
    y = hip_ctx.execute_transform_f32(ir, x)
    assert o.rel_l2(y, o.r2r_batch(x.astype(np.float64), n, "dct2", threads=8)) <= 1e-7
    irh = r2r_ir("dst4", n, batch, vk.Precision.F16StorageF32Compute)
    yh = hip_ctx.execute_transform_f32(irh, x)
    xq = x.astype(np.float16).astype(np.float64)
    assert o.rel_l2(yh, o.r2r_batch(xq, n, "dst4", threads=8)) <= 2e-3
    # in place on device buffers
    ir32 = r2r_ir("dct4", n, batch, F32)
    plan = hip_ctx.plan(ir32)
    d = torch.from_numpy(x.copy()).cuda()
    plan.execute(d.data_ptr(), d.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), hip_ctx.execute_transform(ir32, x))


def test_dct1_length_one_rejected(hip_ctx):
    with pytest.raises(vk.VkFftError):
        hip_ctx.plan(r2r_ir("dct1", 1, 1, F32))


# ---- N-D (NdR2rIr, src/r2r_ir.rs:1769-1990, execute_nd_r2r_ir :2216-2300) ----

def oracle_nd(x, dims, batch, name, axes):
    """The oracle's 1-D direct sums along each axis in `axes`."""
    v = x.reshape((batch,) + tuple(dims)).astype(np.float64)
    for ax in axes:
        moved = np.moveaxis(v, ax + 1, -1)
        shp = moved.shape
        out = o.r2r_batch(np.ascontiguousarray(moved).reshape(-1), shp[-1], name, threads=8).reshape(shp)
        v = np.moveaxis(out, -1, ax + 1)
    return v.reshape(-1)


def r2r_nd_cfg(name, dims, batch, prec, normalize=False):
    return vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_transform(kind_of(name)) \
        .with_inverse_normalization(normalize)


@pytest.mark.parametrize("name", KINDS)
def test_r2r_nd_forward(hip_ctx, name):
    import scipy.fft as sf
    dims, batch = [12, 10, 6], 2
    x = o.uniform(int(np.prod(dims)) * batch, 51, np.float64)
    y = hip_ctx.execute_transform(vk.TransformIr.build(r2r_nd_cfg(name, dims, batch, F64), FWD), x)
    f = sf.dctn if name.startswith("dct") else sf.dstn
    ref = f(x.reshape((batch,) + tuple(dims)), type=int(name[-1]), axes=(1, 2, 3)).reshape(-1)
    assert o.rel_l2(y, ref) <= 1e-13
    dims32 = [64, 48]
    x32 = o.uniform(64 * 48 * 3, 52, np.float32)
    y32 = hip_ctx.execute_transform(vk.TransformIr.build(r2r_nd_cfg(name, dims32, 3, F32), FWD), x32)
    assert o.rel_l2(y32, oracle_nd(x32, dims32, 3, name, (0, 1))) <= 1e-5


@pytest.mark.parametrize("name", ["dct1", "dct2", "dst3", "dst4"])
def test_r2r_nd_round_trip_and_omit(hip_ctx, name):
    import scipy.fft as sf
    dims, batch = [20, 1, 36], 2
    x = o.uniform(20 * 36 * batch, 53, np.float64)
    y = hip_ctx.execute_transform(vk.TransformIr.build(r2r_nd_cfg(name, dims, batch, F64), FWD), x)
    z = hip_ctx.execute_transform(vk.TransformIr.build(r2r_nd_cfg(name, dims, batch, F64, True), INV), y)
    assert o.rel_l2(z, x) <= 1e-13
    # omitting axis 0 transforms axis 2 only
    c = r2r_nd_cfg(name, dims, batch, F64).with_omit_dimension(0, True)
    yo = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    f = sf.dct if name.startswith("dct") else sf.dst
    ref = f(x.reshape(batch, 20, 1, 36), type=int(name[-1]), axis=3).reshape(-1)
    assert o.rel_l2(yo, ref) <= 1e-13


def test_r2r_nd_layouts(hip_ctx):
    import scipy.fft as sf
    dims, batch = [24, 30], 2
    x = o.uniform(24 * 30 * batch, 54, np.float64)
    c = r2r_nd_cfg("dct2", dims, batch, F64).with_zero_padding(1, 25, 30).with_output_buffer_batch_stride(24 * 30 + 7)
    y = hip_ctx.execute_transform(vk.TransformIr.build(c, FWD), x)
    xm = x.reshape(batch, 24, 30).copy()
    xm[:, :, 25:] = 0
    assert o.rel_l2(y, sf.dctn(xm, type=2, axes=(1, 2)).reshape(-1)) <= 1e-13
    irm = vk.TransformIr.build(r2r_nd_cfg("dst2", dims, batch, vk.Precision.F64ComputeF32Storage), FWD)
    ym = hip_ctx.execute_transform(irm, x.astype(np.float32))
    assert o.rel_l2(ym, sf.dstn(x.astype(np.float32).astype(np.float64).reshape(batch, 24, 30), type=2,
                                axes=(1, 2)).reshape(-1)) <= 1e-7


@pytest.mark.parametrize("name", KINDS)
def test_r2r_fft_lengths_follow_reference_reductions(hip_ctx, name):
    """The complex FFT inside each type has the length of the reference's
    reduction (r2r_ir.rs:76-110): 2(N-1) for DCT-I, 2(N+1) for DST-I, N for
    types II and III, N/2 for even type IV and 2N for odd type IV; both
    directions (the inverse runs the partner type)."""
    for n in (64, 63):
        for direction in (FWD, INV):
            d = hip_ctx.plan(r2r_ir(name, n, 2, F32, direction)).describe()["r2r"]
            t = int(name[-1])
            expect = {1: 2 * (n - 1) if name.startswith("dct") else 2 * (n + 1), 2: n, 3: n,
                      4: n // 2 if n % 2 == 0 else 2 * n}[t]
            assert d["fft_len"] == expect, (name, n, direction, d)
