"""Planner restatement (vkfft-rs_amd/csrc/planner.cpp) pinned against values
the reference asserts or that follow from its tables, called through the C ABI."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

A = vk.AlgorithmKind


def test_readme_axis_classes():
    # README.md:39-43 / planner.rs:1095-1101: [1024, 17, 65537] -> Stockham / Rader / Bluestein
    assert vk.planner_axis(1024)[0] == A.Stockham
    assert vk.planner_axis(17)[0] == A.Rader
    assert vk.planner_axis(65537)[0] == A.Bluestein


def test_config_c5_bluestein_lengths():
    # 4098 = 2*3*683 fails the safe-prime gate (planner.rs:498-503): Bluestein,
    # first "good" 2357-smooth M >= 8197 (scheduler.rs:283-357)
    assert vk.planner_axis(4099, 4096) == (A.Bluestein, 8232)
    # 65537 pads past 2^17 = 131072 < 2N-1: first good smooth length is 131220
    assert vk.planner_axis(65537, 4096) == (A.Bluestein, 131220)
    assert vk.planner_axis(4099, 4096, vk.Precision.F64) == (A.Bluestein, 8232)


def test_recursive_rader_opt_in_changes_4099():
    # PlannerTuning::with_recursive_fft_rader (config.rs:376-379, planner.rs:414-422)
    assert vk.planner_axis(4099, 4096, recursive_rader=True)[0] == A.Rader


def test_bluestein_table_rows():
    # tests/f32_bluestein_higher_axis_grouped_padding.rs:114-118: AMD p263 -> 625
    assert vk.bluestein_padding(263, 1, vk.Precision.F32, 32 * 1024) == 625
    # table edges (scheduler.rs:178-208): 103 in [89,129) -> 256; 3281 in [2593,3282) -> 6561
    assert vk.bluestein_padding(103) == 256
    assert vk.bluestein_padding(3281) == 6561
    assert vk.bluestein_padding(3300) == 8192
    # wide table (scheduler.rs:121-176) for F64
    assert vk.bluestein_padding(103, 1, vk.Precision.F64) == 243
    assert vk.bluestein_padding(1000, 1, vk.Precision.F64) == 2016
    assert vk.bluestein_padding(1009, 1, vk.Precision.F64) == 2048


@pytest.mark.parametrize("n", [4099, 5003, 65537, 100003, 12289])
def test_generic_padding_is_smooth_and_long_enough(n):
    m = vk.bluestein_padding(n, 64)
    assert m >= 2 * n - 1
    assert all(p in (2, 3, 5, 7) for p in o.prime_factorization(m))
    # it is never below the plain smooth search of reference::fft
    assert m >= o.next_smooth_at_least(2 * n - 1)


@pytest.mark.parametrize("n,alg", [(2, A.Stockham), (13, A.Stockham), (26, A.Stockham), (34, A.Rader),
                                   (89, A.Rader), (257, A.Rader), (263, A.Bluestein), (97, A.Rader)])
def test_small_axis_classes(n, alg):
    # direct Rader for 17 <= p < 89; FFT-Rader for primes whose p-1 has only
    # factors below 17 (the safe-prime gate, planner.rs:498-503: 89-1 = 2^3*11,
    # 97-1 = 2^5*3, 257-1 = 2^8); Bluestein otherwise (263-1 = 2*131)
    assert vk.planner_axis(n)[0] == alg


def test_f64_rader_limit_follows_lds_capacity():
    # planner.rs:442-463: the FFT-Rader scan stops at LDS/complex_bytes; 160 KiB
    # holds 10240 f64 complex values, so 12289 is Rader in F32, Bluestein in F64
    assert vk.planner_axis(12289, 1, vk.Precision.F32)[0] == A.Rader
    assert vk.planner_axis(12289, 1, vk.Precision.F64)[0] == A.Bluestein


def test_next_smooth_matches_oracle():
    for t in [1, 2, 7, 11, 2061, 8197, 131073, 99991]:
        assert vk.next_smooth_at_least(t) == o.next_smooth_at_least(t)


def test_mixed_precisions_plan_like_their_compute_type():
    """PlannerTuning::for_device (config.rs:411-417) and the LUT rule
    (scheduler.rs:231-239) treat F64ComputeF32Storage as F64 and
    F16StorageF32Compute as F32."""
    F32, F64 = vk.Precision.F32, vk.Precision.F64
    F16S, F64C = vk.Precision.F16StorageF32Compute, vk.Precision.F64ComputeF32Storage
    for n in (4099, 65537, 1000, 1009, 12289, 23, 31):
        assert vk.planner_axis(n, 4, F64C) == vk.planner_axis(n, 4, F64)
        assert vk.planner_axis(n, 4, F16S) == vk.planner_axis(n, 4, F32)
    for n in (1000, 4099, 65537):
        assert vk.bluestein_padding(n, 1, F64C) == vk.bluestein_padding(n, 1, F64)
        assert vk.bluestein_padding(n, 1, F16S) == vk.bluestein_padding(n, 1, F32)


def test_mixed_precision_host_storage_conversion():
    ir = vk.TransformIr.build(vk.FftConfig.new([8]).with_precision(vk.Precision.F16StorageF32Compute),
                              vk.Direction.Forward)
    assert ir.complex_dtype == np.complex64 and ir.storage_scalar_dtype == np.float16
    x = (np.arange(8) / 3 + 1j * np.arange(8) / 7).astype(np.complex64)
    s = ir.to_storage(x)
    assert s.dtype == np.float16 and s.size == 16
    back = ir.from_storage(s, True)
    assert back.dtype == np.complex64
    np.testing.assert_array_equal(back.view(np.float32), x.view(np.float32).astype(np.float16).astype(np.float32))
    ir64 = vk.TransformIr.build(vk.FftConfig.new([8]).with_precision(vk.Precision.F64ComputeF32Storage),
                                vk.Direction.Forward)
    assert ir64.complex_dtype == np.complex64 and ir64.storage_scalar_dtype == np.float32
    assert ir64.to_storage(x) is x


def test_tuned_planner_and_kernel_preparation_rules():
    """PlannerTuning moves a Rader prime to Bluestein above max_rader_fft_prime
    (config.rs:367-420); kernelConvolution is a forward-only preparation of
    coordinate_features * batch systems with the pinned ownerships
    (config.rs:806-818, 1101-1136)."""
    assert vk.planner_axis(1009)[0] == vk.AlgorithmKind.Rader
    assert vk.planner_axis(1009, tuning=vk.PlannerTuning(max_rader_fft_prime=1000))[0] == vk.AlgorithmKind.Bluestein
    assert vk.planner_axis(4099, tuning=vk.PlannerTuning().with_recursive_fft_rader())[0] == vk.AlgorithmKind.Rader
    ir = vk.TransformIr.build(vk.FftConfig.new([64]).with_batch_count(3).with_coordinate_features(2)
                              .with_kernel_convolution(True), vk.Direction.Forward)
    assert ir.input_count() == ir.output_count() == 64 * 6 and ir.desc().batch == 6
def test_kernel_preparation_rejections():
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(vk.FftConfig.new([64]).with_kernel_convolution(True), vk.Direction.Inverse)
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(vk.FftConfig.new([64, 32]).with_kernel_convolution(True), vk.Direction.Forward)  # 2-D C2C
    with pytest.raises(vk.VkFftError):
        vk.TransformIr.build(vk.FftConfig.new([64]).with_kernel_convolution(True).with_convolution(True), vk.Direction.Forward)
