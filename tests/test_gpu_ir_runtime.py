"""The IR-driven boundary on the GPU: NativeRuntime plans each IR on first
use from desc_from_ir, with the IR built from its own fields (no FftConfig),
as vkfft-rs's execute_transform_f32/f64 and submit_transform_*_async receive
only the TransformIr (native_runtime.rs:339-359, 458-529). Every family is
checked against the oracle (f32 relative L2 <= 1e-5, f64 <= 1e-13)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
S = vk.ScalarType
K = vk.TransformKind


@pytest.fixture(scope="module")
def rt(hip_ctx):
    r = vk.NativeRuntime(hip_ctx)
    yield r
    r.close()


def test_c2c_stockham_from_ir_fields(rt):
    ir = vk.RecursiveFftIr(logical_len=1024, batch_count=16, direction=FWD, scalar=S.F32, external_scalar=S.F32)
    x = o.complex_uniform(1024 * 16, 1, np.complex64)
    y = rt.execute_transform_f32(ir, x)
    assert o.rel_l2(y, o.fft_batch(x.astype(np.complex128), 1024)) <= 1e-5
    # the plan is created once and found again by an equal IR
    p = rt.plan_for(ir)
    assert rt.plan_for(vk.RecursiveFftIr(1024, 16, FWD, S.F32, S.F32)) is p
    inv = vk.RecursiveFftIr(1024, 16, INV, S.F64, S.F64, normalize=True)
    z = rt.execute_transform_f64(inv, x.astype(np.complex128))
    assert o.rel_l2(z, o.fft_batch(x.astype(np.complex128), 1024, "inverse", True)) <= 1e-13


def test_c2c_rader_and_bluestein_from_ir_fields(rt):
    rader = vk.RecursiveFftIr(17, 9, FWD, S.F32, S.F32, rader_primes=(17,))
    x = o.complex_uniform(17 * 9, 2, np.complex64)
    assert o.rel_l2(rt.execute_transform_f32(rader, x), o.fft_batch(x.astype(np.complex128), 17)) <= 1e-5
    assert "rader" in rt.plan_for(rader).describe()
    blue = vk.BluesteinPipelineIr(logical_len=4099, convolution_len=8232, batch_count=8, direction=FWD,
                                  scalar=S.F32, external_scalar=S.F32)
    x = o.complex_uniform(4099 * 8, 3, np.complex64)
    assert o.rel_l2(rt.execute_transform_f32(blue, x), o.fft_batch(x.astype(np.complex128), 4099)) <= 1e-5
    desc = rt.plan_for(blue).describe()
    assert desc["axes"][0]["convolution_len"] == 8232
    # recursive Rader tree from the IR's own tuning
    tree = vk.RecursiveFftIr(4099, 2, FWD, S.F32, S.F32, rader_primes=(4099,),
                             scheduler_tuning=(17, 89, 17, 16384, True))
    x = o.complex_uniform(4099 * 2, 4, np.complex64)
    assert o.rel_l2(rt.execute_transform_f32(tree, x), o.fft_batch(x.astype(np.complex128), 4099)) <= 1e-5
    assert rt.plan_for(tree).describe()["rader"]["convolution_len"] == 4098


def test_c2c_nd_from_ir_fields(rt):
    axes = (vk.NdAxisIr(0, vk.RecursiveFftIr(64, 1, FWD, S.F32, S.F32)),
            vk.NdAxisIr(1, vk.RecursiveFftIr(96, 1, FWD, S.F32, S.F32)))
    ir = vk.NdFftIr(dimensions=(64, 96), batch_count=3, direction=FWD, scalar=S.F32, external_scalar=S.F32,
                    axes=axes)
    x = o.complex_uniform(64 * 96 * 3, 5, np.complex64)
    assert o.rel_l2(rt.execute_transform_f32(ir, x), o.fft_nd(x, [64, 96], 3, threads=8)) <= 1e-5
    # a Bluestein axis inside an N-D IR, f64, normalized inverse
    axes = (vk.NdAxisIr(0, vk.RecursiveFftIr(32, 1, INV, S.F64, S.F64, normalize=True)),
            vk.NdAxisIr(1, vk.BluesteinPipelineIr(263, vk.bluestein_padding(263, 32, vk.Precision.F64), 1, INV,
                                                  S.F64, S.F64, normalize=True)))
    ir = vk.NdFftIr((32, 263), 2, INV, S.F64, S.F64, axes)
    x = o.complex_uniform(32 * 263 * 2, 6, np.complex128)
    ref = np.fft.ifftn(x.reshape(2, 32, 263), axes=(1, 2)).reshape(-1)
    assert o.rel_l2(rt.execute_transform_f64(ir, x), ref) <= 1e-13


def test_real_from_ir_fields(rt):
    n, batch = 4096, 6
    r2c = vk.RealFftIr(K.RealToComplex, n, batch, S.F32, S.F32, S.F32)
    c2r = vk.RealFftIr(K.ComplexToReal, n, batch, S.F32, S.F32, S.F32, normalize=True)
    x = o.normal(n * batch, 7).astype(np.float32)
    X = rt.execute_transform_f32(r2c, x)
    assert o.rel_l2(X, o.r2c_batch(x.astype(np.float64), n)) <= 1e-5
    back = rt.execute_transform_f32(c2r, X)
    assert o.rel_l2(back, o.c2r_batch(X.astype(np.complex128), n, normalize=True)) <= 1e-5
    # async: the same lazy plan; real outputs arrive widened to {v, 0}
    t = rt.submit_transform_async(c2r, X)
    w = t.wait()
    assert np.array_equal(w.real, back) and not np.any(w.imag)
    nd = vk.NdRealFftIr(K.RealToComplex, (32, 64), 2, S.F64, S.F64, S.F64)
    x = o.normal(32 * 64 * 2, 8)
    ref = np.fft.rfftn(x.reshape(2, 32, 64), axes=(1, 2)).reshape(-1)
    assert o.rel_l2(rt.execute_transform_f64(nd, x), ref) <= 1e-13


def test_mixed_storage_and_r2r_from_ir_fields(rt):
    ir = vk.RecursiveFftIr(512, 4, FWD, S.F32, S.F16)
    x = o.complex_uniform(512 * 4, 9, np.complex64)
    x16 = x.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)
    y = rt.execute_transform_f32(ir, x)
    assert o.rel_l2(y, o.fft_batch(x16.astype(np.complex128), 512)) <= 2e-3
    dct = vk.R2rIr(K.dct(2), 100, 4, FWD, S.F64, S.F64)
    x = o.uniform(400, 10)
    assert o.rel_l2(rt.execute_transform_f64(dct, x), o.r2r_batch(x, 100, "dct2")) <= 1e-13


def test_input_length_mismatch_from_ir(rt):
    ir = vk.RecursiveFftIr(256, 2, FWD, S.F32, S.F32)
    with pytest.raises(vk.VkFftError) as e:
        rt.execute_transform_f32(ir, np.zeros(256, np.complex64))
    assert "InputLengthMismatch" in str(e.value)
