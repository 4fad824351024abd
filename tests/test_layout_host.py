"""Host side of formatted layouts and zero padding in the Python mirror:
resolution rules of resolve_formatted_axis_strides / _batch_stride
(src/config.rs:1463-1522) and the pack / unpack of the reference's runtime
boundary (src/nd_ir.rs:1115-1150, 1191-1260). No GPU needed."""
import numpy as np
import pytest

import vkfft_amd as vk


def ir(c, direction=vk.Direction.Forward):
    return vk.TransformIr.build(c, direction)


def test_dense_layout_is_not_formatted():
    t = ir(vk.FftConfig.new([8, 16]).with_batch_count(2))
    assert not t.is_formatted(False) and not t.is_formatted(True)
    x = np.arange(256).astype(np.complex64)
    assert t.pack_input(x) is x


def test_pack_unpack_round_trip():
    c = vk.FftConfig.new([3, 4]).with_batch_count(2).with_input_buffer_axis_stride(0, 6) \
        .with_input_buffer_batch_stride(20).with_output_buffer_axis_stride(0, 5).with_output_buffer_batch_stride(16)
    t = ir(c)
    x = (np.arange(24) + 1).astype(np.complex64)
    p = t.pack_input(x)
    assert p.size == 40
    # element (b, i, j) sits at b*20 + i*6 + j; the gaps stay zero
    for b in range(2):
        for i in range(3):
            for j in range(4):
                assert p[b * 20 + i * 6 + j] == x[b * 12 + i * 4 + j]
    assert np.count_nonzero(p) == 24
    idx, n = t._physical_index(True)
    assert n == 32
    y = np.zeros(32, dtype=np.complex64)
    y[idx] = x
    assert np.array_equal(t.unpack_output(y), x)


def test_real_sides_use_half_spectrum_extent():
    c = vk.FftConfig.new([10]).with_batch_count(3).with_transform(vk.TransformKind.RealToComplex) \
        .with_output_buffer_batch_stride(8)
    t = ir(c)
    assert t._side_dims(False) == [10] and t._side_dims(True) == [6]
    assert t.physical_output_count() == 24
    with pytest.raises(vk.VkFftError):
        ir(vk.FftConfig.new([10]).with_transform(vk.TransformKind.RealToComplex)
           .with_output_buffer_batch_stride(5))._side_strides(True)


@pytest.mark.parametrize("setup", [lambda c: c.with_input_buffer_axis_stride(1, 2),
                                   lambda c: c.with_input_buffer_axis_stride(0, 15),
                                   lambda c: c.with_input_buffer_batch_stride(100)])
def test_invalid_layouts_rejected(setup):
    c = setup(vk.FftConfig.new([8, 16]).with_batch_count(2))
    with pytest.raises(vk.VkFftError):
        ir(c)._side_strides(False)


def test_zero_padding_validation():
    c = vk.FftConfig.new([64])
    with pytest.raises(vk.VkFftError):
        c.with_zero_padding(0, 10, 65)
    with pytest.raises(vk.VkFftError):
        c.with_zero_padding(0, 20, 10)
    with pytest.raises(vk.VkFftError):
        c.with_zero_padding(1, 0, 1)
    assert c.with_zero_padding(0, 5, 5).zero_padding[0] is None
    d = ir(c.with_zero_padding(0, 8, 16).with_zero_padding_domain(vk.ZeroPaddingDomain.Frequency)).desc()
    assert (d.zero_left[0], d.zero_right[0], d.zero_frequency) == (8, 16, 1)
