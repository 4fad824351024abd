"""Host-side mirror of vkfft-rs's transform API over the MI355X C ABI.

The names follow the Rust crate so callers and tests read like its own code:
`FftConfig` (src/config.rs:609-1034), `Direction`/`TransformKind`/`Precision`,
`TransformIr.build` (src/application.rs:48-167) and a `HipExecutionContext`
with `execute_transform_f32/f64` (src/backend/native_runtime.rs:339-359,
src/backend/hip/runtime.rs:1982-1988). Everything below calls
libvkfft_mi355x.so through ctypes; there is no CPU fallback: if the library
or the GPU is missing, the calls raise.
"""
from __future__ import annotations

import ctypes
import enum
import json
import os
import weakref
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvkfft_mi355x.so")
# index-map test build (identity arithmetic): tests only
INDEX_LIB_PATH = os.path.join(_HERE, "libvkfft_mi355x_index.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "vkfx.h")
MAX_RANK = 4

_libs = {}


class VkFftError(RuntimeError):
    """Mirrors vkfft-rs `VkFftError` (src/error.rs:6-57)."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, "Unknown")
        super().__init__(f"{self.kind}: {message}")


STATUS_NAMES = {
    -1: "NativeUnavailable",
    -2: "NativeRuntime",
    -3: "UnsupportedKernelPath",
    -4: "UnsupportedPrecision",
    -5: "InputLengthMismatch",
    -6: "ResourceLimitExceeded",
    -7: "InvalidArgument",
    -8: "ArithmeticOverflow",
}


class Direction(enum.IntEnum):
    Forward = -1
    Inverse = 1


class TransformKind(enum.IntEnum):
    """TransformKind (config.rs:35-41); Dct(DctType::I..IV) and Dst(DstType::I..IV)
    are flattened to one value each."""
    ComplexToComplex = 0
    RealToComplex = 1
    ComplexToReal = 2
    DctI = 3
    DctII = 4
    DctIII = 5
    DctIV = 6
    DstI = 7
    DstII = 8
    DstIII = 9
    DstIV = 10

    @staticmethod
    def dct(t: int) -> "TransformKind":
        return TransformKind(2 + t)

    @staticmethod
    def dst(t: int) -> "TransformKind":
        return TransformKind(6 + t)

    @property
    def is_r2r(self) -> bool:
        return self >= TransformKind.DctI


class Precision(enum.IntEnum):
    """Precision (config.rs:108-145): storage / compute."""
    F32 = 0
    F64 = 1
    F16StorageF32Compute = 2
    F64ComputeF32Storage = 3


def _f32_family(p: Precision) -> bool:
    return p != Precision.F64


class ZeroPaddingDomain(enum.IntEnum):
    """ZeroPaddingDomain (config.rs): which boundary owns the zero interval."""
    Spatial = 0
    Frequency = 1


class ConvolutionConjugation(enum.IntEnum):
    """configuration.conjugateConvolution (config.rs:595-612)."""
    Off = 0
    Sequence = 1
    Kernel = 2


class AlgorithmKind(enum.IntEnum):
    Stockham = 0
    Rader = 1
    Bluestein = 2


class _PassResources(ctypes.Structure):
    _fields_ = [
        ("pass_", ctypes.c_char * 48),
        ("registers_per_thread", ctypes.c_uint32),
        ("static_shared_bytes", ctypes.c_uint32),
        ("dynamic_shared_bytes", ctypes.c_uint32),
        ("local_bytes_per_thread", ctypes.c_uint32),
        ("max_threads_per_block", ctypes.c_uint32),
        ("block_threads", ctypes.c_uint32),
        ("resident_blocks_per_cu", ctypes.c_uint32),
        ("waves_per_cu", ctypes.c_uint32),
    ]


class _PassTiming(ctypes.Structure):
    _fields_ = [
        ("pass_", ctypes.c_char * 48),
        ("fft_len", ctypes.c_uint32),
        ("launches", ctypes.c_uint32),
        ("lines", ctypes.c_uint64),
        ("total_ms", ctypes.c_double),
        ("min_ms", ctypes.c_double),
        ("max_ms", ctypes.c_double),
    ]


class _PlannerTuning(ctypes.Structure):
    _fields_ = [
        ("min_rader_direct_prime", ctypes.c_uint64),
        ("max_rader_direct_prime", ctypes.c_uint64),
        ("min_rader_fft_prime", ctypes.c_uint64),
        ("max_rader_fft_prime", ctypes.c_uint64),
        ("allow_recursive_fft_rader", ctypes.c_int32),
    ]


class _PlanDesc(ctypes.Structure):
    _fields_ = [
        ("rank", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * MAX_RANK),
        ("batch", ctypes.c_uint64),
        ("transform", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("direction", ctypes.c_int32),
        ("normalize", ctypes.c_int32),
        ("use_library_planner", ctypes.c_int32),
        ("axis_algorithm", ctypes.c_int32 * MAX_RANK),
        ("convolution_len", ctypes.c_uint64 * MAX_RANK),
        ("in_axis_stride", ctypes.c_uint64 * MAX_RANK),
        ("out_axis_stride", ctypes.c_uint64 * MAX_RANK),
        ("in_batch_stride", ctypes.c_uint64),
        ("out_batch_stride", ctypes.c_uint64),
        ("zero_left", ctypes.c_uint64 * MAX_RANK),
        ("zero_right", ctypes.c_uint64 * MAX_RANK),
        ("zero_frequency", ctypes.c_int32),
        ("grouped_batch", ctypes.c_uint32 * MAX_RANK),
        ("perform_convolution", ctypes.c_int32),
        ("conjugate_sequence", ctypes.c_int32),
        ("cross_power_normalize", ctypes.c_int32),
        ("coordinate_features", ctypes.c_uint32),
        ("matrix_convolution", ctypes.c_uint32),
        ("symmetric_kernel", ctypes.c_int32),
        ("independent_coordinates", ctypes.c_int32),
        ("kernel_count", ctypes.c_uint32),
        ("kernel_spectrum", ctypes.c_void_p),
        ("kernel_spectrum_bytes", ctypes.c_uint64),
        ("omit_dimension", ctypes.c_uint32),
        ("custom_tuning", ctypes.c_int32),
        ("tuning", _PlannerTuning),
    ]


class _Profile(ctypes.Structure):
    _fields_ = [
        ("shared_memory_bytes", ctypes.c_uint64),
        ("shared_memory_pow2_bytes", ctypes.c_uint64),
        ("max_threads_per_block", ctypes.c_uint64),
        ("warp_size", ctypes.c_uint64),
        ("compute_units", ctypes.c_uint64),
        ("global_memory_bytes", ctypes.c_uint64),
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
    ]


def lib(path: Optional[str] = None):
    """Loads libvkfft_mi355x.so (or the library at `path`, e.g. the index-map
    test build INDEX_LIB_PATH); raises if it has not been built."""
    path = path or LIB_PATH
    if path not in _libs:
        if not os.path.exists(path):
            raise VkFftError(-1, f"{path} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(path)
        vp, u64, i32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32
        L.vkfx_last_error.restype = ctypes.c_char_p
        L.vkfx_version.restype = ctypes.c_char_p
        L.vkfx_context_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.vkfx_context_destroy.argtypes = [vp]
        L.vkfx_context_profile.argtypes = [vp, ctypes.POINTER(_Profile)]
        L.vkfx_context_synchronize.argtypes = [vp]
        L.vkfx_plan_create.argtypes = [vp, ctypes.POINTER(_PlanDesc), ctypes.POINTER(vp)]
        L.vkfx_plan_destroy.argtypes = [vp]
        L.vkfx_plan_io_bytes.argtypes = [vp, ctypes.POINTER(u64), ctypes.POINTER(u64)]
        L.vkfx_plan_workspace_bytes.argtypes = [vp, ctypes.POINTER(u64)]
        L.vkfx_plan_describe.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.vkfx_execute.argtypes = [vp, vp, vp, vp, vp]
        L.vkfx_execute_noalloc.argtypes = [vp, vp, vp, vp]
        L.vkfx_execute_host.argtypes = [vp, vp, u64, vp, u64]
        L.vkfx_planner_axis.argtypes = [u64, u64, i32, i32, i32, u64, ctypes.POINTER(i32), ctypes.POINTER(u64)]
        L.vkfx_planner_axis_tuned.argtypes = [u64, u64, i32, i32, ctypes.POINTER(_PlannerTuning), u64,
                                              ctypes.POINTER(i32), ctypes.POINTER(u64)]
        L.vkfx_planner_bluestein_padding.argtypes = [u64, u64, i32, u64, ctypes.POINTER(u64)]
        L.vkfx_planner_next_smooth.argtypes = [u64]
        L.vkfx_planner_next_smooth.restype = u64
        L.vkfx_submit_host.argtypes = [vp, vp, u64, ctypes.POINTER(vp)]
        L.vkfx_ticket_ready.argtypes = [vp, ctypes.POINTER(i32)]
        L.vkfx_ticket_wait.argtypes = [vp, vp, u64]
        L.vkfx_ticket_wait_complex.argtypes = [vp, vp, u64]
        L.vkfx_plan_output_info.argtypes = [vp, ctypes.POINTER(i32), ctypes.POINTER(u64)]
        L.vkfx_ticket_destroy.argtypes = [vp]
        L.vkfx_context_cache_stats.argtypes = [vp, ctypes.POINTER(u64), ctypes.POINTER(u64), ctypes.POINTER(u64)]
        L.vkfx_context_clear_caches.argtypes = [vp]
        L.vkfx_plan_resources.argtypes = [vp, ctypes.POINTER(_PassResources), ctypes.c_uint32,
                                          ctypes.POINTER(ctypes.c_uint32)]
        L.vkfx_plan_timing_start.argtypes = [vp, ctypes.c_uint32]
        L.vkfx_plan_timing_stop.argtypes = [vp, ctypes.POINTER(_PassTiming), ctypes.c_uint32,
                                            ctypes.POINTER(ctypes.c_uint32)]
        L.vkfx_execute_chain.argtypes = [ctypes.POINTER(vp), ctypes.c_uint32, vp, vp, vp]
        L.vkfx_execute_chain_host.argtypes = [ctypes.POINTER(vp), ctypes.c_uint32, vp, u64, vp, u64]
        _libs[path] = L
    return _libs[path]


def _check(rc: int, L=None):
    if rc != 0:
        raise VkFftError(rc, (L or lib()).vkfx_last_error().decode(errors="replace"))


def header_symbols() -> List[str]:
    """Function names declared in include/vkfx.h."""
    import re
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(vkfx_[a-z_0-9]+)\s*\(", text)))


# ------------------------------------------------------------------ planner

@dataclass
class PlannerTuning:
    """PlannerTuning (src/config.rs:367-420): Rader ranges (max bounds exclusive)
    and the recursive-Rader opt-in."""
    min_rader_direct_prime: int = 17
    max_rader_direct_prime: int = 89
    min_rader_fft_prime: int = 17
    max_rader_fft_prime: int = 16_384
    allow_recursive_fft_rader: bool = False

    @staticmethod
    def portable() -> "PlannerTuning":
        return PlannerTuning()

    def with_recursive_fft_rader(self, enabled: bool = True) -> "PlannerTuning":
        self.allow_recursive_fft_rader = bool(enabled)
        return self

    def _c(self) -> _PlannerTuning:
        return _PlannerTuning(self.min_rader_direct_prime, self.max_rader_direct_prime, self.min_rader_fft_prime,
                              self.max_rader_fft_prime, int(self.allow_recursive_fft_rader))


def planner_axis(length: int, batch: int = 1, precision: Precision = Precision.F32, strided: bool = False,
                 recursive_rader: bool = False, shared_memory_bytes: int = 160 * 1024,
                 tuning: Optional[PlannerTuning] = None):
    """plan_c2c_axis_algorithm_for_device on the HIP/AMD profile (planner.rs:349-440),
    with the device tuning or an explicit PlannerTuning."""
    alg, m = ctypes.c_int32(), ctypes.c_uint64()
    if tuning is None:
        _check(lib().vkfx_planner_axis(length, batch, int(precision), int(strided), int(recursive_rader),
                                       shared_memory_bytes, ctypes.byref(alg), ctypes.byref(m)))
    else:
        t = tuning._c()
        t.allow_recursive_fft_rader = int(tuning.allow_recursive_fft_rader or recursive_rader)
        _check(lib().vkfx_planner_axis_tuned(length, batch, int(precision), int(strided), ctypes.byref(t),
                                             shared_memory_bytes, ctypes.byref(alg), ctypes.byref(m)))
    return AlgorithmKind(alg.value), int(m.value)


def bluestein_padding(length: int, batch: int = 1, precision: Precision = Precision.F32,
                      shared_memory_bytes: int = 160 * 1024) -> int:
    """upstream_bluestein_auto_padding for HIP/AMD (scheduler.rs:361-373)."""
    out = ctypes.c_uint64()
    _check(lib().vkfx_planner_bluestein_padding(length, batch, int(precision), shared_memory_bytes,
                                                ctypes.byref(out)))
    return int(out.value)


def next_smooth_at_least(target: int) -> int:
    return int(lib().vkfx_planner_next_smooth(target))


# ------------------------------------------------------------------- config

@dataclass
class FftConfig:
    """Builder mirroring vkfft-rs `FftConfig` (dims slowest -> fastest)."""
    dimensions: List[int]
    batch_count: int = 1
    precision: Precision = Precision.F32
    transform: TransformKind = TransformKind.ComplexToComplex
    normalize_inverse: bool = False
    allow_recursive_fft_rader: bool = False
    input_buffer_axis_strides: List[int] = field(default_factory=lambda: [0] * MAX_RANK)
    output_buffer_axis_strides: List[int] = field(default_factory=lambda: [0] * MAX_RANK)
    input_buffer_batch_stride: int = 0
    output_buffer_batch_stride: int = 0
    zero_padding: List[Optional[tuple]] = field(default_factory=lambda: [None] * MAX_RANK)
    zero_padding_domain: ZeroPaddingDomain = ZeroPaddingDomain.Spatial
    grouped_batch: List[int] = field(default_factory=lambda: [0] * MAX_RANK)
    perform_convolution: bool = False
    convolution_conjugation: ConvolutionConjugation = ConvolutionConjugation.Off
    cross_power_spectrum_normalization: bool = False
    coordinate_features: int = 1
    matrix_convolution: int = 1
    symmetric_convolution_kernel: bool = False
    convolution_kernel_count: int = 1
    omit_dimension: List[bool] = field(default_factory=lambda: [False] * MAX_RANK)
    kernel_convolution: bool = False
    tuning: Optional["PlannerTuning"] = None  # None: the device tuning

    @staticmethod
    def new(dimensions: Sequence[int]) -> "FftConfig":
        return FftConfig(list(int(d) for d in dimensions))

    def with_batch_count(self, batch: int) -> "FftConfig":
        self.batch_count = int(batch)
        return self

    def with_precision(self, precision: Precision) -> "FftConfig":
        self.precision = Precision(precision)
        return self

    def with_transform(self, transform: TransformKind) -> "FftConfig":
        self.transform = TransformKind(transform)
        return self

    def with_inverse_normalization(self, normalize: bool = True) -> "FftConfig":
        self.normalize_inverse = bool(normalize)
        return self

    def _axis(self, axis: int, field_name: str) -> int:
        if not 0 <= axis < len(self.dimensions):
            raise VkFftError(-7, f"ValueOutOfRange {{ field: {field_name!r} }}")
        return axis

    def with_input_buffer_axis_stride(self, axis: int, stride: int) -> "FftConfig":
        """Formatted input stride in stored elements (config.rs:892-905); 0 clears."""
        self.input_buffer_axis_strides[self._axis(axis, "formatted input axis stride")] = int(stride)
        return self

    def with_output_buffer_axis_stride(self, axis: int, stride: int) -> "FftConfig":
        self.output_buffer_axis_strides[self._axis(axis, "formatted output axis stride")] = int(stride)
        return self

    def with_input_buffer_batch_stride(self, stride: int) -> "FftConfig":
        self.input_buffer_batch_stride = int(stride)
        return self

    def with_output_buffer_batch_stride(self, stride: int) -> "FftConfig":
        self.output_buffer_batch_stride = int(stride)
        return self

    def with_zero_padding(self, axis: int, left: int, right: int) -> "FftConfig":
        """Logical zero interval [left, right) on one axis (config.rs:1004-1025)."""
        if not 0 <= axis < len(self.dimensions):
            raise VkFftError(-7, f"InvalidZeroPaddingRange {{ axis: {axis}, left: {left}, right: {right}, length: 0 }}")
        n = self.dimensions[axis]
        if left > right or right > n:
            raise VkFftError(-7, f"InvalidZeroPaddingRange {{ axis: {axis}, left: {left}, right: {right}, length: {n} }}")
        self.zero_padding[axis] = (int(left), int(right)) if left != right else None
        return self

    def with_zero_padding_domain(self, domain: ZeroPaddingDomain) -> "FftConfig":
        self.zero_padding_domain = ZeroPaddingDomain(domain)
        return self

    def with_tuning(self, tuning: "PlannerTuning") -> "FftConfig":
        """config.rs:820-824: explicit planner tuning."""
        self.tuning = tuning
        return self

    def with_device_tuning(self) -> "FftConfig":
        """config.rs:828-832: back to the device/precision defaults."""
        self.tuning = None
        return self

    def with_kernel_convolution(self, enabled: bool = True) -> "FftConfig":
        """config.rs:746-749: a forward transform that prepares a convolution
        kernel spectrum over coordinate_features * batch_count systems."""
        self.kernel_convolution = bool(enabled)
        return self

    def with_omit_dimension(self, axis: int, omit: bool = True) -> "FftConfig":
        """config.rs:844-853: leave `axis` untransformed."""
        if not 0 <= axis < len(self.dimensions):
            raise VkFftError(-7, "ValueOutOfRange { field: omitDimension axis }")
        self.omit_dimension[axis] = bool(omit)
        return self

    # convolution knobs (config.rs:734-800)
    def with_convolution(self, enabled: bool = True) -> "FftConfig":
        self.perform_convolution = bool(enabled)
        return self

    def with_convolution_conjugation(self, conjugation: ConvolutionConjugation) -> "FftConfig":
        self.convolution_conjugation = ConvolutionConjugation(conjugation)
        return self

    def with_cross_power_spectrum_normalization(self, enabled: bool = True) -> "FftConfig":
        self.cross_power_spectrum_normalization = bool(enabled)
        return self

    def with_coordinate_features(self, n: int) -> "FftConfig":
        self.coordinate_features = int(n)
        return self

    def with_matrix_convolution(self, matrix_size: int) -> "FftConfig":
        self.matrix_convolution = int(matrix_size)
        if matrix_size > 1:
            self.coordinate_features = int(matrix_size)
        return self

    def with_symmetric_convolution_kernel(self, symmetric: bool = True) -> "FftConfig":
        self.symmetric_convolution_kernel = bool(symmetric)
        return self

    def with_convolution_kernel_count(self, kernel_count: int) -> "FftConfig":
        self.convolution_kernel_count = int(kernel_count)
        return self

    def with_grouped_batch(self, axis: int, grouped_batch: int) -> "FftConfig":
        """configuration.groupedBatch[axis] override (config.rs:869-880); 0 clears."""
        self.grouped_batch[self._axis(axis, "groupedBatch axis")] = int(grouped_batch)
        return self

    def validate(self):
        # FftConfig::validate (src/config.rs:1036): non-empty, non-zero dims
        if not self.dimensions or len(self.dimensions) > MAX_RANK:
            raise VkFftError(-7, "dimensions must hold 1..4 axes")
        for axis, d in enumerate(self.dimensions):
            if d <= 0:
                raise VkFftError(-7, f"ZeroLength {{ axis: {axis} }}")
        if self.batch_count <= 0:
            raise VkFftError(-7, "batch_count must be >= 1")
        if self.coordinate_features <= 0:
            raise VkFftError(-7, "ValueOutOfRange { field: coordinateFeatures }")
        if self.kernel_convolution:
            # config.rs:1101-1136: the pinned kernel-preparation ownerships
            rank = len(self.dimensions)
            padded = [z is not None for z in self.zero_padding[:rank]]
            real = self.transform == TransformKind.RealToComplex
            dense_1d = rank == 1 and not any(padded)
            s52 = real and rank == 2 and self.batch_count == 2 and self.coordinate_features == 2 and not any(padded)
            s51 = real and rank == 3 and self.batch_count == 1 and self.coordinate_features == 9 and all(padded) \
                and self.zero_padding_domain == ZeroPaddingDomain.Spatial
            formatted = any(self.input_buffer_axis_strides[:rank]) or any(self.output_buffer_axis_strides[:rank]) \
                or bool(self.input_buffer_batch_stride) or bool(self.output_buffer_batch_stride)
            if self.perform_convolution:
                raise VkFftError(-3, "kernelConvolution prepares a kernel spectrum and must not be combined with "
                                     "performConvolution")
            if self.transform not in (TransformKind.ComplexToComplex, TransformKind.RealToComplex) \
                    or not (dense_1d or s52 or s51) or self.matrix_convolution != 1 \
                    or self.symmetric_convolution_kernel or self.convolution_kernel_count != 1 \
                    or self.precision not in (Precision.F32, Precision.F64) or formatted \
                    or self.convolution_conjugation != ConvolutionConjugation.Off \
                    or self.cross_power_spectrum_normalization:
                raise VkFftError(-3, "kernelConvolution currently requires dense 1D C2C/R2C independent "
                                     "batch/coordinate K1 preparation, sample_52-style 2D R2C B2/C2 preparation, "
                                     "or sample_51-style batch1 3D R2C C9 Spatial-padding preparation in F32/F64")

    def system_count(self) -> int:
        """Independent transforms of a plan: coordinate_features * batch_count
        for kernel preparation (config.rs:806-818), else batch_count."""
        return self.batch_count * (self.coordinate_features if self.kernel_convolution else 1)


@dataclass
class TransformIr:
    """The plan-time object of application.rs:48-167 for this path."""
    config: FftConfig
    direction: Direction
    axis_algorithms: List[AlgorithmKind] = field(default_factory=list)
    convolution_lens: List[int] = field(default_factory=list)

    @staticmethod
    def build(config: FftConfig, direction: Direction) -> "TransformIr":
        config.validate()
        direction = Direction(direction)
        if config.transform == TransformKind.RealToComplex and direction != Direction.Forward:
            raise VkFftError(-7, "RealToComplex requires Direction::Forward")
        if config.transform == TransformKind.ComplexToReal and direction != Direction.Inverse:
            raise VkFftError(-7, "ComplexToReal requires Direction::Inverse")
        if config.kernel_convolution and direction != Direction.Forward:
            raise VkFftError(-3, "kernelConvolution prepares a kernel spectrum with a forward transform")
        ir = TransformIr(config, direction)
        rank = len(config.dimensions)
        for axis, n in enumerate(config.dimensions):
            if config.transform == TransformKind.ComplexToComplex:
                alg, m = planner_axis(n, config.system_count(), config.precision, strided=axis + 1 != rank,
                                      recursive_rader=config.allow_recursive_fft_rader, tuning=config.tuning)
            else:
                alg, m = AlgorithmKind.Stockham, 0
            ir.axis_algorithms.append(alg)
            ir.convolution_lens.append(m)
        return ir

    def lower(self):
        """The IR variant TransformIr::build makes for this config
        (application.rs:48-167), with the fields the HIP boundary reads."""
        c = self.config
        prec = c.precision
        scalar = ScalarType.F64 if prec in (Precision.F64, Precision.F64ComputeF32Storage) else ScalarType.F32
        storage = {Precision.F32: ScalarType.F32, Precision.F64: ScalarType.F64,
                   Precision.F16StorageF32Compute: ScalarType.F16,
                   Precision.F64ComputeF32Storage: ScalarType.F32}[prec]
        if c.perform_convolution or c.kernel_convolution:
            raise VkFftError(-3, "convolutions lower to ConvolutionIr, not TransformIr")
        rank = len(c.dimensions)
        zeros = tuple(ZeroPadPassIr(z[0], z[1], c.zero_padding_domain == ZeroPaddingDomain.Frequency)
                      if z is not None else None for z in c.zero_padding[:rank])
        norm = bool(c.normalize_inverse) and self.direction == Direction.Inverse
        tun = None
        if c.tuning is not None:
            t = c.tuning
            tun = (t.min_rader_direct_prime, t.max_rader_direct_prime, t.min_rader_fft_prime,
                   t.max_rader_fft_prime, bool(t.allow_recursive_fft_rader or c.allow_recursive_fft_rader))

        def one_dim(axis, n, batch):
            alg, m = self.axis_algorithms[axis], self.convolution_lens[axis]
            if alg == AlgorithmKind.Bluestein:
                return BluesteinPipelineIr(n, m, batch, self.direction, scalar, storage, norm,
                                           zeros[axis] if rank == 1 else None)
            primes = tuple(p for p in _prime_factors(n) if p > 13) if alg == AlgorithmKind.Rader else ()
            return RecursiveFftIr(n, batch, self.direction, scalar, storage, norm, primes, tun,
                                  zeros[axis] if rank == 1 else None)

        dense = all(v == 0 for v in c.input_buffer_axis_strides[:rank] + c.output_buffer_axis_strides[:rank]) and \
            not c.input_buffer_batch_stride and not c.output_buffer_batch_stride
        if c.transform == TransformKind.ComplexToComplex:
            if rank == 1 and dense and not any(c.omit_dimension[:1]):
                return one_dim(0, c.dimensions[0], c.batch_count)
            return NdFftIr(tuple(c.dimensions), c.batch_count, self.direction, scalar, storage,
                           tuple(NdAxisIr(i, one_dim(i, n, 1)) for i, n in enumerate(c.dimensions)),
                           tuple(c.input_buffer_axis_strides[:rank]), tuple(c.output_buffer_axis_strides[:rank]),
                           c.input_buffer_batch_stride, c.output_buffer_batch_stride,
                           tuple(bool(o) for o in c.omit_dimension[:rank]), zeros)
        if c.transform in (TransformKind.RealToComplex, TransformKind.ComplexToReal):
            r2c = c.transform == TransformKind.RealToComplex
            real_norm = bool(c.normalize_inverse) and not r2c
            if rank == 1 and dense:
                return RealFftIr(c.transform, c.dimensions[0], c.batch_count, scalar, storage, storage, real_norm,
                                 zeros[0])
            return NdRealFftIr(c.transform, tuple(c.dimensions), c.batch_count, scalar, storage, storage, real_norm,
                               tuple(c.input_buffer_axis_strides[:rank]), tuple(c.output_buffer_axis_strides[:rank]),
                               c.input_buffer_batch_stride, c.output_buffer_batch_stride,
                               tuple(bool(o) for o in c.omit_dimension[:rank]), zeros)
        if rank == 1 and dense:
            return R2rIr(c.transform, c.dimensions[0], c.batch_count, self.direction, scalar, storage,
                         bool(c.normalize_inverse) and self.direction == Direction.Inverse, zeros[0])
        raise VkFftError(-3, "N-D or formatted DCT/DST IRs are planned from FftConfig here")

    def desc(self) -> _PlanDesc:
        c = self.config
        d = _PlanDesc()
        d.rank = len(c.dimensions)
        for i, n in enumerate(c.dimensions):
            d.dims[i] = n
        d.batch = c.batch_count
        d.transform = int(c.transform)
        d.precision = int(c.precision)
        d.direction = int(self.direction)
        d.normalize = int(c.normalize_inverse)
        d.use_library_planner = 0 if self.config.transform == TransformKind.ComplexToComplex else 1
        for i, (a, m) in enumerate(zip(self.axis_algorithms, self.convolution_lens)):
            d.axis_algorithm[i] = int(a)
            d.convolution_len[i] = m
        for i in range(len(c.dimensions)):
            d.in_axis_stride[i] = c.input_buffer_axis_strides[i]
            d.out_axis_stride[i] = c.output_buffer_axis_strides[i]
            d.grouped_batch[i] = c.grouped_batch[i]
            if c.zero_padding[i] is not None:
                d.zero_left[i], d.zero_right[i] = c.zero_padding[i]
        d.in_batch_stride = c.input_buffer_batch_stride
        d.out_batch_stride = c.output_buffer_batch_stride
        d.zero_frequency = int(c.zero_padding_domain == ZeroPaddingDomain.Frequency)
        # a convolution config without its kernel spectrum fails at plan time
        d.perform_convolution = int(c.perform_convolution)
        d.omit_dimension = sum(1 << i for i in range(len(c.dimensions)) if c.omit_dimension[i])
        if c.tuning is not None:
            d.custom_tuning = 1
            d.tuning = c.tuning._c()
            d.tuning.allow_recursive_fft_rader = int(c.tuning.allow_recursive_fft_rader or c.allow_recursive_fft_rader)
        if c.kernel_convolution:
            d.batch = c.system_count()
        return d

    # ---- formatted layouts (the host-side pack/unpack of the reference's
    # runtime boundary, nd_ir.rs:1115-1150, 1191-1260)
    def _side_dims(self, output: bool) -> List[int]:
        c = self.config
        dims = list(c.dimensions)
        if (c.transform == TransformKind.RealToComplex and output) or \
                (c.transform == TransformKind.ComplexToReal and not output):
            dims[-1] = dims[-1] // 2 + 1
        return dims

    def _side_strides(self, output: bool):
        """resolve_formatted_axis_strides / _batch_stride (config.rs:1463-1522)."""
        c = self.config
        dims = self._side_dims(output)
        over = c.output_buffer_axis_strides if output else c.input_buffer_axis_strides
        rank = len(dims)
        if over[rank - 1] not in (0, 1):
            raise VkFftError(-7, "formatted fastest-axis stride must remain one stored element")
        st = [1] * rank
        for ax in range(rank - 2, -1, -1):
            minimum = st[ax + 1] * dims[ax + 1]
            st[ax] = over[ax] or minimum
            if st[ax] < minimum:
                raise VkFftError(-7, "formatted axis stride overlaps the next faster logical axis")
        b = (c.output_buffer_batch_stride if output else c.input_buffer_batch_stride) or st[0] * dims[0]
        if b < st[0] * dims[0]:
            raise VkFftError(-7, "formatted batch stride overlaps the logical tensor")
        return dims, st, b

    def _physical_index(self, output: bool) -> np.ndarray:
        dims, st, b = self._side_strides(output)
        idx = np.zeros((self.config.batch_count,) + tuple(dims), dtype=np.int64)
        idx += (np.arange(self.config.batch_count) * b).reshape((-1,) + (1,) * len(dims))
        for ax, (n, s) in enumerate(zip(dims, st)):
            shape = [1] * (len(dims) + 1)
            shape[ax + 1] = n
            idx += (np.arange(n) * s).reshape(shape)
        return idx.reshape(-1), self.config.batch_count * b

    def is_formatted(self, output: bool) -> bool:
        dims, st, b = self._side_strides(output)
        dense = [int(np.prod(dims[ax + 1:])) for ax in range(len(dims))]
        return st != dense or b != int(np.prod(dims))

    def pack_input(self, x: np.ndarray) -> np.ndarray:
        """Logical input -> the formatted physical buffer (gaps zero)."""
        if not self.is_formatted(False):
            return x
        idx, n = self._physical_index(False)
        out = np.zeros(n, dtype=x.dtype)
        out[idx] = x
        return out

    def unpack_output(self, y: np.ndarray) -> np.ndarray:
        if not self.is_formatted(True):
            return y
        idx, _ = self._physical_index(True)
        return y[idx]

    def physical_output_count(self) -> int:
        return self._physical_index(True)[1] if self.is_formatted(True) else self.output_count()

    @property
    def real_dtype(self):
        """Host-side element type (Complex32 / f32 for every F32-family precision)."""
        return np.float32 if _f32_family(self.config.precision) else np.float64

    @property
    def complex_dtype(self):
        return np.complex64 if _f32_family(self.config.precision) else np.complex128

    @property
    def storage_scalar_dtype(self):
        """Scalar type of the device buffers (binary16 for F16StorageF32Compute)."""
        p = self.config.precision
        return np.float16 if p == Precision.F16StorageF32Compute else (np.float64 if p == Precision.F64
                                                                         else np.float32)

    def to_storage(self, x: np.ndarray) -> np.ndarray:
        """Host values -> the scalars the device buffers hold (binary16 rounds to
        nearest even, like Binary16::from_f32)."""
        if self.config.precision != Precision.F16StorageF32Compute:
            return x
        scal = x.view(np.float32) if np.iscomplexobj(x) else x
        return scal.astype(np.float16)

    def from_storage(self, s: np.ndarray, complex_out: bool) -> np.ndarray:
        if self.config.precision != Precision.F16StorageF32Compute:
            return s
        v = s.astype(np.float32)
        return v.view(np.complex64) if complex_out else v

    def input_count(self) -> int:
        """Logical input elements: the compact [.., N/2+1] spectrum for C2R."""
        return int(np.prod(self._side_dims(False))) * self.config.system_count()

    def output_count(self) -> int:
        """Logical output elements: the compact [.., N/2+1] spectrum for R2C."""
        return int(np.prod(self._side_dims(True))) * self.config.system_count()


class Plan:
    """A built plan: launch list, tables and workspace on one device."""

    def __init__(self, ctx: "HipExecutionContext", ir: TransformIr, desc: Optional[_PlanDesc] = None):
        self.ctx = ctx
        self._L = ctx._L
        self.ir = ir
        self.handle = ctypes.c_void_p()
        d = desc if desc is not None else ir.desc()
        _check(self._L.vkfx_plan_create(ctx.handle, ctypes.byref(d), ctypes.byref(self.handle)), self._L)
        ctx._live_plans.add(self)
        i, o, w = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(self._L.vkfx_plan_io_bytes(self.handle, ctypes.byref(i), ctypes.byref(o)), self._L)
        _check(self._L.vkfx_plan_workspace_bytes(self.handle, ctypes.byref(w)), self._L)
        self.in_bytes, self.out_bytes, self.workspace_bytes = int(i.value), int(o.value), int(w.value)

    def resources(self) -> List[dict]:
        """compiled_pass_resource_reports + theoretical_occupancy_reports
        (native_runtime.rs:96-131): one entry per distinct pass."""
        count = ctypes.c_uint32()
        _check(self._L.vkfx_plan_resources(self.handle, None, 0, ctypes.byref(count)), self._L)
        arr = (_PassResources * max(1, count.value))()
        _check(self._L.vkfx_plan_resources(self.handle, arr, count.value, ctypes.byref(count)), self._L)
        out = []
        for r in arr[:count.value]:
            d = {name: getattr(r, name) for name, _ in _PassResources._fields_ if name != "pass_"}
            d["pass"] = r.pass_.decode()
            out.append(d)
        return out

    def timing_start(self, max_launches: int):
        """Arms kernel timing: the next `max_launches` FFT kernel dispatches
        of this plan carry HIP events bound to the dispatch itself."""
        _check(self._L.vkfx_plan_timing_start(self.handle, int(max_launches)), self._L)

    def timing_stop(self) -> List[dict]:
        """Waits for the timed dispatches and returns one record per (pass
        label, line length, lines per launch), in launch order: launches and
        total/min/max/avg kernel ms."""
        count = ctypes.c_uint32()
        arr = (_PassTiming * 256)()
        _check(self._L.vkfx_plan_timing_stop(self.handle, arr, 256, ctypes.byref(count)), self._L)
        out = []
        for r in arr[:min(256, count.value)]:
            out.append({"pass": r.pass_.decode(), "fft_len": int(r.fft_len), "lines": int(r.lines),
                        "launches": int(r.launches), "total_ms": r.total_ms,
                        "min_ms": r.min_ms, "max_ms": r.max_ms,
                        "avg_ms": r.total_ms / r.launches if r.launches else None})
        return out

    def describe(self) -> dict:
        n = self._L.vkfx_plan_describe(self.handle, None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        self._L.vkfx_plan_describe(self.handle, buf, n + 1)
        return json.loads(buf.value.decode())

    def execute(self, d_in: int, d_out: int, d_work: int = 0, stream: int = 0):
        """Device-resident asynchronous execute (raw device pointers)."""
        _check(self._L.vkfx_execute(self.handle, ctypes.c_void_p(d_in), ctypes.c_void_p(d_out),
                                  ctypes.c_void_p(d_work or None), ctypes.c_void_p(stream or None)), self._L)

    def execute_noalloc(self, d_in: int, d_out: int, stream: int = 0):
        """vkfx_execute_noalloc: the same passes with the library's static
        device scratch as the workspace; allocates nothing."""
        _check(self._L.vkfx_execute_noalloc(self.handle, ctypes.c_void_p(d_in), ctypes.c_void_p(d_out),
                                          ctypes.c_void_p(stream or None)), self._L)

    def execute_tensors(self, x, y, stream=None):
        """Execute on torch tensors already resident on the GPU."""
        if x.numel() * x.element_size() != self.in_bytes or y.numel() * y.element_size() != self.out_bytes:
            raise VkFftError(-5, f"InputLengthMismatch: expected {self.in_bytes}/{self.out_bytes} bytes")
        if not (x.is_cuda and y.is_cuda and x.is_contiguous() and y.is_contiguous()):
            raise VkFftError(-7, "tensors must be contiguous device tensors")
        s = stream.cuda_stream if stream is not None else 0
        self.execute(x.data_ptr(), y.data_ptr(), 0, s)

    def close(self):
        # a plan outliving its context only drops its handle: the context's
        # close already destroyed it (vkfx_plan_destroy needs a live context)
        if self.handle and self.ctx.handle:
            for t in list(self.ctx._live_tickets):  # a plan's tickets go first
                if t.plan is self:
                    t.close()
            _check(self._L.vkfx_plan_destroy(self.handle), self._L)
        self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ConvolutionIr:
    """ConvolutionIr / NdConvolutionIr / NdRealConvolutionIr (convolution_ir.rs):
    forward transform of every [batch][coordinate] tensor, multiply by
    `kernel_spectrum` (frequency domain, [kernel][plane][tensor]), normalized
    inverse. C2C configs convolve complex tensors; an N-D RealToComplex config
    (batch 1) is the real application: R2C, multiply over the compact
    [.., N/2+1] spectra, C2R, real tensors on both sides."""

    def __init__(self, config: FftConfig, kernel_spectrum: np.ndarray):
        if config.convolution_conjugation == ConvolutionConjugation.Kernel:
            raise VkFftError(-3, "kernel-conjugated convolution is not executable in the pinned VkFFT codegen")
        cfg = FftConfig(**{k: (list(v) if isinstance(v, list) else v) for k, v in config.__dict__.items()})
        cfg.perform_convolution = True
        self.ir = TransformIr.build(cfg, Direction.Forward)
        self.config = cfg
        dt = self.ir.complex_dtype if cfg.precision != Precision.F64ComputeF32Storage else np.complex128
        self.kernel = np.ascontiguousarray(kernel_spectrum, dtype=dt).reshape(-1)
        m = cfg.matrix_convolution if cfg.matrix_convolution > 1 else 0
        self.coordinates = m if m else max(1, cfg.coordinate_features)
        self.kernel_count = max(1, cfg.convolution_kernel_count)
        self.independent = (not m) and self.coordinates > 1
        self.real = cfg.transform == TransformKind.RealToComplex
        # caller-side layouts: `coordinates` input tensors, K * coordinates
        # output tensors, full (real or complex) dims on both sides
        systems_out = self.kernel_count if self.kernel_count > 1 else cfg.batch_count
        self._sides = []
        for systems in (cfg.batch_count * self.coordinates, systems_out * self.coordinates):
            side = FftConfig(**{k: (list(v) if isinstance(v, list) else v) for k, v in cfg.__dict__.items()})
            side.transform = TransformKind.ComplexToComplex
            side.batch_count = systems
            self._sides.append(TransformIr(side, Direction.Forward))

    @staticmethod
    def build(config: FftConfig, kernel_spectrum: np.ndarray) -> "ConvolutionIr":
        return ConvolutionIr(config, kernel_spectrum)

    def tensor_len(self) -> int:
        """Elements of one input / output tensor (real for the real application)."""
        return int(np.prod(self.config.dimensions))

    def spectrum_len(self) -> int:
        """Elements of one kernel-spectrum plane (compact for the real application)."""
        dims = list(self.config.dimensions)
        if self.real:
            dims[-1] = dims[-1] // 2 + 1
        return int(np.prod(dims))

    def input_count(self) -> int:
        return self.config.batch_count * self.coordinates * self.tensor_len()

    def output_count(self) -> int:
        systems = self.kernel_count if self.kernel_count > 1 else self.config.batch_count
        return systems * self.coordinates * self.tensor_len()

    def desc(self) -> _PlanDesc:
        d = self.ir.desc()
        c = self.config
        d.perform_convolution = 1
        d.conjugate_sequence = int(c.convolution_conjugation == ConvolutionConjugation.Sequence)
        d.cross_power_normalize = int(c.cross_power_spectrum_normalization)
        d.coordinate_features = self.coordinates
        d.matrix_convolution = c.matrix_convolution if c.matrix_convolution > 1 else 0
        d.symmetric_kernel = int(c.symmetric_convolution_kernel)
        d.independent_coordinates = int(self.independent)
        d.kernel_count = self.kernel_count
        d.kernel_spectrum = self.kernel.ctypes.data
        d.kernel_spectrum_bytes = self.kernel.nbytes
        return d


class TransformTicket:
    """NativeAsyncTransformTicket32/64 (native_runtime.rs:372-401): a submitted
    transform; `wait()` returns the output and releases the ticket."""

    def __init__(self, plan: "Plan", x: np.ndarray, out_dtype, out_count: int):
        self.plan = plan
        self._L = plan._L
        ir = plan.ir
        self._complex_out = np.dtype(out_dtype).kind == "c"
        x = np.ascontiguousarray(ir.to_storage(ir.pack_input(x)))
        self._x = x  # kept alive until the submit has copied it
        out_count = ir.physical_output_count()
        self._out = np.empty(out_count * (2 if self._complex_out else 1), dtype=ir.storage_scalar_dtype) \
            if ir.config.precision == Precision.F16StorageF32Compute else np.empty(out_count, dtype=out_dtype)
        self.handle = ctypes.c_void_p()
        _check(self._L.vkfx_submit_host(plan.handle, x.ctypes.data, x.nbytes, ctypes.byref(self.handle)), self._L)
        plan.ctx._live_tickets.add(self)

    def _live(self):
        if not self.handle:
            raise VkFftError(-2, "ticket was released (waited, closed, or its context was closed)")

    def ready(self) -> bool:
        self._live()
        r = ctypes.c_int32()
        _check(self._L.vkfx_ticket_ready(self.handle, ctypes.byref(r)), self._L)
        return bool(r.value)

    def wait(self) -> np.ndarray:
        self._live()
        _check(self._L.vkfx_ticket_wait(self.handle, self._out.ctypes.data, self._out.nbytes), self._L)
        self.close()
        ir = self.plan.ir
        return ir.unpack_output(ir.from_storage(self._out, self._complex_out))

    def close(self):
        # the context's close destroys its live tickets first, so a ticket
        # never outlives the plan and context it references
        if self.handle:
            self._L.vkfx_ticket_destroy(self.handle)
        self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _plan_array(plans):
    arr = (ctypes.c_void_p * len(plans))()
    for i, p in enumerate(plans):
        arr[i] = p.handle
    return arr


def execute_chain(plans, d_in: int, d_out: int, stream: int = 0):
    """Device-resident chain (cuda/runtime.rs:1744-1809): plans[i]'s output feeds
    plans[i+1] on the device; raw device pointers, asynchronous on `stream`."""
    L = plans[0]._L
    _check(L.vkfx_execute_chain(_plan_array(plans), len(plans), ctypes.c_void_p(d_in), ctypes.c_void_p(d_out),
                                ctypes.c_void_p(stream or None)), L)


# ------------------------------------------------- IR-driven runtime boundary
#
# vkfft-rs's NativeRuntime entry points receive only the built IR:
# execute_transform_f32/f64(&TransformIr, input) (src/backend/native_runtime.rs:
# 339-359) and submit_transform_f32/f64_async (:458-529), and callers build that
# IR with TransformIr::build (e.g. native_runtime.rs:2206-2220). The classes
# below mirror the fields of the IR variants the HIP boundary reads; desc_from_ir
# derives the library's plan descriptor from those fields alone, and
# NativeRuntime plans each IR on first use, keyed by the IR itself.

class ScalarType(enum.IntEnum):
    """ScalarType of the IRs (src/precision.rs): compute `scalar` and the
    caller-visible storage scalar."""
    F16 = 0
    F32 = 1
    F64 = 2


@dataclass(frozen=True)
class ZeroPadPassIr:
    """ZeroPadPassIr (src/zero_pad_ir.rs:50-64): the zero interval [left, right)
    of the logical axis and its domain (spatial: forward input / inverse
    output; frequency: forward output / inverse input, zero_pad_ir.rs:38-46)."""
    left: int
    right: int
    frequency: bool = False


@dataclass(frozen=True)
class RecursiveFftIr:
    """RecursiveFftIr (src/recursive_ir.rs:1662-1696). `rader_primes`: the
    primes of the DirectRader / FftRader nodes of `root` at any depth
    (RecursiveFftNodeIr, recursive_ir.rs:917-922); `normalize`: the
    StoreSharedToGlobal normalize flag of the root's final store
    (kernel_ir.rs:1442-1445, set at :1582-1585)."""
    logical_len: int
    batch_count: int
    direction: Direction
    scalar: ScalarType
    external_scalar: ScalarType
    normalize: bool = False
    rader_primes: Tuple[int, ...] = ()
    # the effective PlannerTuning (config.rs:367-380) as (min/max direct prime,
    # min/max FFT prime, allow_recursive_fft_rader); None = the device default
    scheduler_tuning: Optional[Tuple[int, int, int, int, bool]] = None
    zero_pad_pass: Optional[ZeroPadPassIr] = None


@dataclass(frozen=True)
class BluesteinPipelineIr:
    """BluesteinPipelineIr (src/bluestein_ir.rs:436-451); `normalize` is the
    postprocess pass's Postprocess { normalize } (bluestein_ir.rs:29, 658)."""
    logical_len: int
    convolution_len: int
    batch_count: int
    direction: Direction
    scalar: ScalarType
    external_scalar: ScalarType
    normalize: bool = False
    zero_pad_pass: Optional[ZeroPadPassIr] = None


@dataclass(frozen=True)
class NdAxisIr:
    """NdAxisIr (src/nd_ir.rs:528-537): the axis and its one-dimensional
    transform (OneDimFftIr::Recursive or ::Bluestein)."""
    axis: int
    transform: object


@dataclass(frozen=True)
class NdFftIr:
    """NdFftIr (src/nd_ir.rs:541-557). Strides are in stored elements, 0 =
    dense; `zero_padding` holds one ZeroPadPassIr (or None) per axis, the
    ranges of the NdZeroPadPassIr."""
    dimensions: Tuple[int, ...]
    batch_count: int
    direction: Direction
    scalar: ScalarType
    external_scalar: ScalarType
    axes: Tuple[NdAxisIr, ...]
    input_buffer_axis_strides: Tuple[int, ...] = ()
    output_buffer_axis_strides: Tuple[int, ...] = ()
    input_buffer_batch_stride: int = 0
    output_buffer_batch_stride: int = 0
    omitted_axes: Tuple[bool, ...] = ()
    zero_padding: Tuple[Optional[ZeroPadPassIr], ...] = ()


@dataclass(frozen=True)
class RealFftIr:
    """RealFftIr (src/real_ir.rs:264-279): R2C (forward) or C2R (inverse) of
    `length` reals; `normalize` is the C2R PreprocessEvenHalf { normalize }
    (real_ir.rs:55, 412) or the odd-length inner transform's store flag."""
    kind: TransformKind
    length: int
    batch_count: int
    scalar: ScalarType
    input_storage_scalar: ScalarType
    output_storage_scalar: ScalarType
    normalize: bool = False
    zero_pad_pass: Optional[ZeroPadPassIr] = None


@dataclass(frozen=True)
class NdRealFftIr:
    """NdRealFftIr (src/nd_real_ir.rs:754-870): R2C / C2R over `dimensions`
    (the last axis real), with the formatted layouts and zero padding of the
    compact-spectrum application."""
    kind: TransformKind
    dimensions: Tuple[int, ...]
    batch_count: int
    scalar: ScalarType
    input_storage_scalar: ScalarType
    output_storage_scalar: ScalarType
    normalize: bool = False
    input_buffer_axis_strides: Tuple[int, ...] = ()
    output_buffer_axis_strides: Tuple[int, ...] = ()
    input_buffer_batch_stride: int = 0
    output_buffer_batch_stride: int = 0
    omitted_axes: Tuple[bool, ...] = ()
    zero_padding: Tuple[Optional[ZeroPadPassIr], ...] = ()


@dataclass(frozen=True)
class R2rIr:
    """R2rIr (src/r2r_ir.rs:600-620): one DCT/DST type over `length` reals,
    normalize / normalization_scale of the inverse partner."""
    kind: TransformKind
    length: int
    batch_count: int
    direction: Direction
    scalar: ScalarType
    external_scalar: ScalarType
    normalize: bool = False
    zero_pad_pass: Optional[ZeroPadPassIr] = None


def _prime_factors(n: int) -> List[int]:
    out, p = [], 2
    while p * p <= n:
        while n % p == 0:
            out.append(p)
            n //= p
        p += 1
    if n > 1:
        out.append(n)
    return out


def _precision_of(scalar: ScalarType, storage: ScalarType) -> Precision:
    """(compute scalar, storage scalar) -> Precision (config.rs:108-145)."""
    table = {(ScalarType.F32, ScalarType.F32): Precision.F32, (ScalarType.F64, ScalarType.F64): Precision.F64,
             (ScalarType.F32, ScalarType.F16): Precision.F16StorageF32Compute,
             (ScalarType.F64, ScalarType.F32): Precision.F64ComputeF32Storage}
    if (scalar, storage) not in table:
        raise VkFftError(-4, f"UnsupportedPrecision: no MI355X kernels for {scalar.name} compute with "
                             f"{storage.name} storage")
    return table[(scalar, storage)]


def _one_dim_algorithm(t) -> Tuple[AlgorithmKind, int, bool]:
    """(axis algorithm, Bluestein M, normalize) of a OneDimFftIr."""
    if isinstance(t, BluesteinPipelineIr):
        return AlgorithmKind.Bluestein, t.convolution_len, t.normalize
    if isinstance(t, RecursiveFftIr):
        return (AlgorithmKind.Rader if t.rader_primes else AlgorithmKind.Stockham), 0, t.normalize
    raise VkFftError(-7, f"InvalidKernelIr: {type(t).__name__} is not a one-dimensional FFT IR")


def _set_zero(d: _PlanDesc, axis: int, z: Optional[ZeroPadPassIr]):
    if z is not None and z.right > z.left:
        d.zero_left[axis], d.zero_right[axis] = z.left, z.right
        d.zero_frequency = int(z.frequency)


def _set_layout(d: _PlanDesc, ir):
    for i, v in enumerate(ir.input_buffer_axis_strides):
        d.in_axis_stride[i] = v
    for i, v in enumerate(ir.output_buffer_axis_strides):
        d.out_axis_stride[i] = v
    d.in_batch_stride = ir.input_buffer_batch_stride
    d.out_batch_stride = ir.output_buffer_batch_stride
    d.omit_dimension = sum(1 << i for i, o in enumerate(ir.omitted_axes) if o)
    for i, z in enumerate(ir.zero_padding):
        _set_zero(d, i, z)


def desc_from_ir(ir) -> _PlanDesc:
    """The library's plan descriptor from the IR's own fields (the planner's
    per-axis decisions included): no FftConfig is consulted."""
    d = _PlanDesc()
    if isinstance(ir, (RecursiveFftIr, BluesteinPipelineIr)):      # TransformIr::Complex1d
        d.rank, d.dims[0], d.batch = 1, ir.logical_len, ir.batch_count
        d.transform = int(TransformKind.ComplexToComplex)
        d.precision = int(_precision_of(ir.scalar, ir.external_scalar))
        d.direction = int(ir.direction)
        alg, m, norm = _one_dim_algorithm(ir)
        d.axis_algorithm[0], d.convolution_len[0], d.normalize = int(alg), m, int(norm)
        _set_zero(d, 0, ir.zero_pad_pass)
        t = getattr(ir, "scheduler_tuning", None)
        if t is not None:
            d.custom_tuning, d.tuning = 1, _PlannerTuning(t[0], t[1], t[2], t[3], int(t[4]))
        return d
    if isinstance(ir, NdFftIr):                                      # TransformIr::ComplexNd
        d.rank = len(ir.dimensions)
        for i, n in enumerate(ir.dimensions):
            d.dims[i] = n
        d.batch = ir.batch_count
        d.transform = int(TransformKind.ComplexToComplex)
        d.precision = int(_precision_of(ir.scalar, ir.external_scalar))
        d.direction = int(ir.direction)
        norm = False
        for ax in ir.axes:
            alg, m, n_ = _one_dim_algorithm(ax.transform)
            d.axis_algorithm[ax.axis], d.convolution_len[ax.axis] = int(alg), m
            norm = norm or n_
        d.normalize = int(norm)
        _set_layout(d, ir)
        return d
    if isinstance(ir, (RealFftIr, NdRealFftIr)):                     # TransformIr::Real / RealNd
        dims = (ir.length,) if isinstance(ir, RealFftIr) else ir.dimensions
        d.rank = len(dims)
        for i, n in enumerate(dims):
            d.dims[i] = n
        d.batch = ir.batch_count
        if ir.kind not in (TransformKind.RealToComplex, TransformKind.ComplexToReal):
            raise VkFftError(-7, "InvalidKernelIr: a real FFT IR is R2C or C2R")
        d.transform = int(ir.kind)
        storage = ir.input_storage_scalar if ir.kind == TransformKind.RealToComplex else ir.output_storage_scalar
        d.precision = int(_precision_of(ir.scalar, storage))
        d.direction = int(Direction.Forward if ir.kind == TransformKind.RealToComplex else Direction.Inverse)
        d.normalize = int(ir.normalize)
        d.use_library_planner = 1          # half-length / full-complex axes are planned inside
        if isinstance(ir, RealFftIr):
            _set_zero(d, 0, ir.zero_pad_pass)
        else:
            _set_layout(d, ir)
        return d
    if isinstance(ir, R2rIr):                                        # TransformIr::RealToReal
        d.rank, d.dims[0], d.batch = 1, ir.length, ir.batch_count
        if not ir.kind.is_r2r:
            raise VkFftError(-7, "InvalidKernelIr: an R2rIr is a DCT or DST")
        d.transform = int(ir.kind)
        d.precision = int(_precision_of(ir.scalar, ir.external_scalar))
        d.direction = int(ir.direction)
        d.normalize = int(ir.normalize)
        d.use_library_planner = 1
        _set_zero(d, 0, ir.zero_pad_pass)
        return d
    raise VkFftError(-3, f"UnsupportedKernelPath: no MI355X plan for {type(ir).__name__}")


class NativeRuntime:
    """The IR-driven boundary, the Python side of a Rust HipNativeRuntime
    over the C ABI (NativeRuntime::execute_transform_f32/f64 and the async
    submit, src/backend/native_runtime.rs:339-359, 406-451): they take only
    the IR, plan it on first use from desc_from_ir and keep the plan keyed by
    the IR."""

    def __init__(self, ctx: "HipExecutionContext"):
        self.ctx = ctx
        self._plans = {}

    def plan_for(self, ir) -> "Plan":
        p = self._plans.get(ir)
        if p is None or not p.handle:
            p = Plan(self.ctx, ir, desc=desc_from_ir(ir))
            self._plans[ir] = p
        return p

    @staticmethod
    def _storage(ir):
        if isinstance(ir, (RealFftIr, NdRealFftIr)):
            return ir.input_storage_scalar if ir.kind == TransformKind.RealToComplex else ir.output_storage_scalar
        return ir.external_scalar

    def _run(self, ir, x: np.ndarray, host_scalar):
        plan = self.plan_for(ir)
        storage = self._storage(ir)
        xs = np.ascontiguousarray(x).reshape(-1)
        scal = xs.view(host_scalar) if np.iscomplexobj(xs) else xs.astype(host_scalar, copy=False)
        if storage == ScalarType.F16:
            scal = scal.astype(np.float16)      # Binary16::from_f32, round to nearest even
        scal = np.ascontiguousarray(scal)
        if scal.nbytes != plan.in_bytes:
            raise VkFftError(-5, f"InputLengthMismatch {{ expected: {plan.in_bytes}, actual: {scal.nbytes} }}")
        real = ctypes.c_int32()
        _check(self.ctx._L.vkfx_plan_output_info(plan.handle, ctypes.byref(real), None), self.ctx._L)
        sdt = {ScalarType.F16: np.float16, ScalarType.F32: np.float32, ScalarType.F64: np.float64}[storage]
        out = np.empty(plan.out_bytes // np.dtype(sdt).itemsize, dtype=sdt)
        _check(self.ctx._L.vkfx_execute_host(plan.handle, scal.ctypes.data, scal.nbytes, out.ctypes.data,
                                             out.nbytes), self.ctx._L)
        y = out.astype(host_scalar, copy=False)
        return y if real.value else y.view(np.complex64 if host_scalar == np.float32 else np.complex128)

    def execute_transform_f32(self, ir, x: np.ndarray) -> np.ndarray:
        """native_runtime.rs:339-349: Complex32 / f32 in, Complex32 / f32 out."""
        if ir.scalar == ScalarType.F64 and self._storage(ir) == ScalarType.F64:
            raise VkFftError(-4, "execute_transform_f32 needs an F32-family TransformIr")
        return self._run(ir, x, np.float32)

    def execute_transform_f64(self, ir, x: np.ndarray) -> np.ndarray:
        """native_runtime.rs:351-359: Complex64 / f64 in and out."""
        if ir.scalar != ScalarType.F64 or self._storage(ir) != ScalarType.F64:
            raise VkFftError(-4, "execute_transform_f64 needs an F64 TransformIr")
        return self._run(ir, x, np.float64)

    def submit_transform_async(self, ir, x: np.ndarray) -> "IrTicket":
        """NativeAsyncRuntime::submit_transform_f32/f64_async (native_runtime.rs:
        458-529): the same lazy plan; the ticket's wait returns complex values
        for every IR kind ({v, 0} for real outputs, whose .re
        finish_transform_output32/64 takes, native_runtime.rs:2045-2087)."""
        plan = self.plan_for(ir)
        host = np.float64 if ir.scalar == ScalarType.F64 and self._storage(ir) == ScalarType.F64 else np.float32
        return IrTicket(self, plan, ir, x, host)

    def close(self):
        for p in self._plans.values():
            p.close()
        self._plans.clear()


class IrTicket:
    """A submitted IR transform (vkfx_submit_host / vkfx_ticket_wait_complex)."""

    def __init__(self, rt: NativeRuntime, plan: "Plan", ir, x: np.ndarray, host_scalar):
        L = rt.ctx._L
        self._L, self.plan, self._host = L, plan, host_scalar
        storage = rt._storage(ir)
        xs = np.ascontiguousarray(x).reshape(-1)
        scal = xs.view(host_scalar) if np.iscomplexobj(xs) else xs.astype(host_scalar, copy=False)
        if storage == ScalarType.F16:
            scal = scal.astype(np.float16)
        self._x = np.ascontiguousarray(scal)
        self._sdt = {ScalarType.F16: np.float16, ScalarType.F32: np.float32, ScalarType.F64: np.float64}[storage]
        widened = ctypes.c_uint64()
        _check(L.vkfx_plan_output_info(plan.handle, None, ctypes.byref(widened)), L)
        self._out = np.empty(int(widened.value) // np.dtype(self._sdt).itemsize, dtype=self._sdt)
        self.handle = ctypes.c_void_p()
        _check(L.vkfx_submit_host(plan.handle, self._x.ctypes.data, self._x.nbytes, ctypes.byref(self.handle)), L)
        plan.ctx._live_tickets.add(self)

    def wait(self) -> np.ndarray:
        if not self.handle:
            raise VkFftError(-2, "ticket was released")
        _check(self._L.vkfx_ticket_wait_complex(self.handle, self._out.ctypes.data, self._out.nbytes), self._L)
        self.close()
        y = self._out.astype(self._host, copy=False)
        return y.view(np.complex64 if self._host == np.float32 else np.complex128)

    def close(self):
        if self.handle:
            self._L.vkfx_ticket_destroy(self.handle)
        self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipExecutionContext:
    """`HipExecutionContext::new(device_index)` over the C ABI. `library`
    selects another build of the library (INDEX_LIB_PATH for the index-map
    tests); the default is the product library."""

    def __init__(self, device_index: int = 0, library: Optional[str] = None):
        self._L = lib(library)
        self.handle = ctypes.c_void_p()
        _check(self._L.vkfx_context_create(device_index, ctypes.byref(self.handle)), self._L)
        self._plans = {}
        self._live_plans = weakref.WeakSet()  # every Plan built on this context
        self._live_tickets = weakref.WeakSet()  # every TransformTicket submitted on it

    def device_profile(self) -> dict:
        p = _Profile()
        _check(self._L.vkfx_context_profile(self.handle, ctypes.byref(p)), self._L)
        return {k: (getattr(p, k).decode() if isinstance(getattr(p, k), bytes) else int(getattr(p, k)))
                for k, _ in _Profile._fields_}

    def device_name(self) -> str:
        return self.device_profile()["name"]

    def plan(self, ir: TransformIr) -> Plan:
        # keyed on every field the library sees
        key = bytes(ir.desc())
        if key not in self._plans:
            self._plans[key] = Plan(self, ir)
        return self._plans[key]

    def _execute_host(self, ir: TransformIr, x: np.ndarray, in_dtype, out_dtype, out_count):
        x = np.ascontiguousarray(x, dtype=in_dtype).reshape(-1)
        if x.size != ir.input_count():
            raise VkFftError(-5, f"InputLengthMismatch {{ expected: {ir.input_count()}, actual: {x.size} }}")
        plan = self.plan(ir)
        xs = np.ascontiguousarray(ir.to_storage(ir.pack_input(x)))
        logical_count = out_count
        out_count = ir.physical_output_count()
        complex_out = np.dtype(out_dtype).kind == "c"
        out = np.empty(out_count * (2 if complex_out else 1), dtype=ir.storage_scalar_dtype) \
            if ir.config.precision == Precision.F16StorageF32Compute else np.empty(out_count, dtype=out_dtype)
        _check(self._L.vkfx_execute_host(plan.handle, xs.ctypes.data, xs.nbytes, out.ctypes.data, out.nbytes),
               self._L)
        y = ir.unpack_output(ir.from_storage(out, complex_out))
        assert y.size == logical_count
        return y

    def execute_transform(self, ir: TransformIr, x: np.ndarray) -> np.ndarray:
        kind = ir.config.transform
        if kind.is_r2r:
            return self._execute_host(ir, x, ir.real_dtype, ir.real_dtype, ir.output_count())
        if kind == TransformKind.RealToComplex:
            return self._execute_host(ir, x, ir.real_dtype, ir.complex_dtype, ir.output_count())
        if kind == TransformKind.ComplexToReal:
            return self._execute_host(ir, x, ir.complex_dtype, ir.real_dtype, ir.output_count())
        return self._execute_host(ir, x, ir.complex_dtype, ir.complex_dtype, ir.output_count())

    def execute_convolution(self, conv: ConvolutionIr, x: np.ndarray) -> np.ndarray:
        """Host round trip of a convolution (the plan is built once per ConvolutionIr)."""
        ir = conv.ir
        vdt = ir.real_dtype if conv.real else ir.complex_dtype
        x = np.ascontiguousarray(x, dtype=vdt).reshape(-1)
        if x.size != conv.input_count():
            raise VkFftError(-5, f"InputLengthMismatch {{ expected: {conv.input_count()}, actual: {x.size} }}")
        plan = getattr(conv, "_plan", None)
        if plan is None or plan.ctx is not self:
            plan = Plan(self, ir, desc=conv.desc())
            conv._plan = plan
        side_in, side_out = conv._sides
        xs = np.ascontiguousarray(ir.to_storage(side_in.pack_input(x)))
        n_out = side_out.physical_output_count()
        f16 = ir.config.precision == Precision.F16StorageF32Compute
        scal = 1 if conv.real else 2
        out = np.empty(scal * n_out, dtype=np.float16) if f16 else np.empty(n_out, dtype=vdt)
        _check(self._L.vkfx_execute_host(plan.handle, xs.ctypes.data, xs.nbytes, out.ctypes.data, out.nbytes),
               self._L)
        return side_out.unpack_output(ir.from_storage(out, not conv.real))

    def _io_dtypes(self, ir: TransformIr):
        kind = ir.config.transform
        if kind.is_r2r:
            return ir.real_dtype, ir.real_dtype
        if kind == TransformKind.RealToComplex:
            return ir.real_dtype, ir.complex_dtype
        if kind == TransformKind.ComplexToReal:
            return ir.complex_dtype, ir.real_dtype
        return ir.complex_dtype, ir.complex_dtype

    def submit_transform_async(self, ir: TransformIr, x: np.ndarray) -> TransformTicket:
        """NativeAsyncRuntime::submit_transform_f32/f64_async (native_runtime.rs:406-451)."""
        in_dt, out_dt = self._io_dtypes(ir)
        x = np.ascontiguousarray(x, dtype=in_dt).reshape(-1)
        if x.size != ir.input_count():
            raise VkFftError(-5, f"InputLengthMismatch {{ expected: {ir.input_count()}, actual: {x.size} }}")
        return TransformTicket(self.plan(ir), x, out_dt, ir.output_count())

    def execute_chain(self, irs, x: np.ndarray) -> np.ndarray:
        """execute_program_chain_complex32_into (cuda/runtime.rs:1765-1809): host input,
        the transforms run back to back on the device, one download."""
        plans = [self.plan(ir) for ir in irs]
        in_dt, _ = self._io_dtypes(irs[0])
        _, out_dt = self._io_dtypes(irs[-1])
        x = np.ascontiguousarray(irs[0].to_storage(irs[0].pack_input(np.ascontiguousarray(x, dtype=in_dt)
                                                                                 .reshape(-1))))
        last = irs[-1]
        complex_out = np.dtype(out_dt).kind == "c"
        n_out = last.physical_output_count()
        out = np.empty(n_out * (2 if complex_out else 1), dtype=last.storage_scalar_dtype) \
            if last.config.precision == Precision.F16StorageF32Compute else np.empty(n_out, dtype=out_dt)
        _check(self._L.vkfx_execute_chain_host(_plan_array(plans), len(plans), x.ctypes.data, x.nbytes,
                                             out.ctypes.data, out.nbytes), self._L)
        return last.unpack_output(last.from_storage(out, complex_out))

    def execute_transform_f32(self, ir: TransformIr, x: np.ndarray) -> np.ndarray:
        if not _f32_family(ir.config.precision):
            raise VkFftError(-4, "execute_transform_f32 needs an F32-family TransformIr")
        return self.execute_transform(ir, x)

    def execute_transform_f64(self, ir: TransformIr, x: np.ndarray) -> np.ndarray:
        if ir.config.precision != Precision.F64:
            raise VkFftError(-4, "execute_transform_f64 needs an F64 TransformIr")
        return self.execute_transform(ir, x)

    def synchronize(self):
        _check(self._L.vkfx_context_synchronize(self.handle), self._L)

    def _cache_stats(self):
        b, s, a = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(self._L.vkfx_context_cache_stats(self.handle, ctypes.byref(b), ctypes.byref(s), ctypes.byref(a)),
               self._L)
        return int(b.value), int(s.value), int(a.value)

    def cached_transient_buffer_count(self) -> int:
        """hip/runtime.rs:1828-1833: pooled device and pinned buffers."""
        return self._cache_stats()[0]

    def pooled_stream_count(self) -> int:
        """hip/runtime.rs:1835-1840."""
        return self._cache_stats()[1]

    def in_flight_submission_count(self) -> int:
        return self._cache_stats()[2]

    def clear_runtime_caches(self):
        """hip/runtime.rs:2275-2330: fails while tickets are in flight."""
        _check(self._L.vkfx_context_clear_caches(self.handle), self._L)

    def close(self):
        # tickets, then plans, then the context (the C ABI refuses any other order)
        for t in list(self._live_tickets):
            t.close()
        for p in list(self._live_plans):
            p.close()
        self._plans.clear()
        if self.handle:
            _check(self._L.vkfx_context_destroy(self.handle), self._L)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
