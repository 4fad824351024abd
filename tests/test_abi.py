"""The C ABI library loads and exports every symbol include/vkfx.h declares
(no compute without a GPU), and its host-side validation behaves like the
reference's error contract."""
import ctypes
import os

import pytest

import vkfft_amd as vk


def test_library_exports_every_declared_symbol():
    lib = vk.lib()
    names = vk.header_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name


def test_version_string():
    assert b"gfx950" in vk.lib().vkfx_version()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="only meaningful without a GPU")
def test_context_without_gpu_is_native_unavailable():
    with pytest.raises(vk.VkFftError) as e:
        vk.HipExecutionContext(0)
    assert e.value.kind == "NativeUnavailable"


def test_transform_ir_direction_contract():
    # application.rs:49-61: R2C must be forward, C2R inverse
    cfg = vk.FftConfig.new([64]).with_transform(vk.TransformKind.RealToComplex)
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(cfg, vk.Direction.Inverse)
    cfg = vk.FftConfig.new([64]).with_transform(vk.TransformKind.ComplexToReal)
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(cfg, vk.Direction.Forward)
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(vk.FftConfig.new([0]), vk.Direction.Forward)


def test_ir_counts():
    ir = vk.TransformIr.build(vk.FftConfig.new([1 << 20]).with_batch_count(256)
                              .with_transform(vk.TransformKind.RealToComplex), vk.Direction.Forward)
    assert ir.input_count() == 256 << 20 and ir.output_count() == 256 * ((1 << 19) + 1)
    ir = vk.TransformIr.build(vk.FftConfig.new([4096, 4096]).with_batch_count(16), vk.Direction.Forward)
    assert ir.axis_algorithms == [vk.AlgorithmKind.Stockham] * 2


def test_null_arguments_are_rejected():
    lib = vk.lib()
    assert lib.vkfx_plan_create(None, None, None) == -7
    assert lib.vkfx_execute(None, None, None, None, None) == -7
    assert b"null" in lib.vkfx_last_error()
    out = ctypes.c_uint64()
    assert lib.vkfx_planner_bluestein_padding(1, 1, 0, 0, ctypes.byref(out)) == -7


def test_integration_rust_extern_block_declares_every_symbol():
    """The Rust `extern "C"` block of the integration guide at the repository
    root declares every function of include/vkfx.h, so a maintainer copying
    it has the whole ABI."""
    import re
    text = open(os.path.join(os.path.dirname(vk.HEADER_PATH), "..", "INTEGRATION.md")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    declared = set(re.findall(r"pub fn (vkfx_[a-z_0-9]+)\(", block))
    assert declared == set(vk.header_symbols())


def test_lifetime_guards_without_gpu():
    lib = vk.lib()
    assert lib.vkfx_plan_destroy(None) == 0
    assert lib.vkfx_context_destroy(None) == 0
    assert lib.vkfx_plan_output_info(None, None, None) == -7
    assert lib.vkfx_ticket_wait_complex(None, None, 0) == -7
