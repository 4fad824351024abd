"""desc_from_ir (vkfft_amd.py): the plan descriptor derived from the IR's own
fields (the reference's NativeRuntime entry points receive only the
TransformIr, native_runtime.rs:339-359, 458-529) equals the descriptor the
FftConfig route builds, for every IR family the HIP boundary serves: 1-D C2C
(Stockham, Rader, recursive Rader, Bluestein; tuning; zero padding; mixed
storage), N-D C2C (formatted strides, omitted axes, zero padding, Bluestein
and Rader axes), 1-D and N-D R2C / C2R, and DCT / DST. The `normalize` field
of a forward descriptor is ignored by the library (only inverse plans scale)
and is compared for inverse plans only."""
import ctypes

import pytest

import vkfft_amd as vk

FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
P = vk.Precision
K = vk.TransformKind


def _bytes(d, forward):
    if forward:
        d.normalize = 0
    return bytes(d)


def _check(cfg, direction):
    ir = vk.TransformIr.build(cfg, direction)
    low = ir.lower()
    a = _bytes(vk.desc_from_ir(low), direction == FWD)
    b = _bytes(ir.desc(), direction == FWD)
    assert a == b, (cfg, low)
    hash(low)  # IRs key the runtime's plan cache
    return low


def cfgs():
    yield vk.FftConfig.new([1024]).with_batch_count(8), FWD
    yield vk.FftConfig.new([1024]).with_batch_count(8).with_inverse_normalization(True), INV
    yield vk.FftConfig.new([17]).with_batch_count(3).with_precision(P.F64), FWD
    yield vk.FftConfig.new([89 * 2]).with_batch_count(3), INV
    yield vk.FftConfig.new([4099]).with_batch_count(4), FWD
    yield vk.FftConfig.new([65537]).with_batch_count(2).with_inverse_normalization(True), INV
    c = vk.FftConfig.new([4099]).with_batch_count(2)
    c.allow_recursive_fft_rader = True
    yield c, FWD
    yield vk.FftConfig.new([4099]).with_batch_count(2).with_tuning(vk.PlannerTuning().with_recursive_fft_rader()), FWD
    yield vk.FftConfig.new([1000]).with_batch_count(5).with_zero_padding(0, 100, 300), FWD
    yield vk.FftConfig.new([512]).with_batch_count(4).with_precision(P.F16StorageF32Compute), FWD
    yield vk.FftConfig.new([512]).with_batch_count(4).with_precision(P.F64ComputeF32Storage) \
        .with_inverse_normalization(True), INV
    yield vk.FftConfig.new([64, 96]).with_batch_count(3), FWD
    yield vk.FftConfig.new([64, 4099]).with_batch_count(1).with_inverse_normalization(True), INV
    yield vk.FftConfig.new([17, 32, 8]).with_batch_count(2).with_precision(P.F64), FWD
    yield vk.FftConfig.new([32, 64]).with_batch_count(2).with_input_buffer_axis_stride(0, 80) \
        .with_output_buffer_batch_stride(4096), FWD
    yield vk.FftConfig.new([32, 64, 16]).with_batch_count(2).with_omit_dimension(0), FWD
    yield vk.FftConfig.new([32, 64]).with_batch_count(2).with_zero_padding(1, 8, 16) \
        .with_zero_padding_domain(vk.ZeroPaddingDomain.Frequency), FWD
    yield vk.FftConfig.new([4096]).with_batch_count(3).with_transform(K.RealToComplex), FWD
    yield vk.FftConfig.new([4096]).with_batch_count(3).with_transform(K.ComplexToReal) \
        .with_inverse_normalization(True), INV
    yield vk.FftConfig.new([1 << 20]).with_batch_count(2).with_transform(K.RealToComplex), FWD
    yield vk.FftConfig.new([45]).with_batch_count(3).with_transform(K.ComplexToReal).with_precision(P.F64), INV
    yield vk.FftConfig.new([64, 64]).with_batch_count(2).with_transform(K.RealToComplex), FWD
    yield vk.FftConfig.new([16, 32, 34]).with_batch_count(1).with_transform(K.ComplexToReal) \
        .with_inverse_normalization(True).with_output_buffer_axis_stride(1, 40), INV
    yield vk.FftConfig.new([100]).with_batch_count(4).with_transform(K.dct(2)), FWD
    yield vk.FftConfig.new([100]).with_batch_count(4).with_transform(K.dst(4)).with_precision(P.F64) \
        .with_inverse_normalization(True), INV


@pytest.mark.parametrize("case", list(range(len(list(cfgs())))))
def test_desc_from_ir_matches_config_route(case):
    cfg, direction = list(cfgs())[case]
    _check(cfg, direction)


def test_ir_families():
    irs = [vk.TransformIr.build(c, d).lower() for c, d in cfgs()]
    kinds = {type(x).__name__ for x in irs}
    assert kinds == {"RecursiveFftIr", "BluesteinPipelineIr", "NdFftIr", "RealFftIr", "NdRealFftIr", "R2rIr"}
    rec = [x for x in irs if isinstance(x, vk.RecursiveFftIr) and x.logical_len == 4099]
    assert rec and all(x.rader_primes == (4099,) for x in rec)


def test_desc_from_ir_rejects_unsupported():
    with pytest.raises(vk.VkFftError):
        vk.desc_from_ir(vk.RecursiveFftIr(64, 1, FWD, vk.ScalarType.F16, vk.ScalarType.F16))
    with pytest.raises(vk.VkFftError):
        vk.desc_from_ir(object())
    with pytest.raises(vk.VkFftError):
        vk.desc_from_ir(vk.RealFftIr(K.ComplexToComplex, 64, 1, vk.ScalarType.F32, vk.ScalarType.F32,
                                     vk.ScalarType.F32))
