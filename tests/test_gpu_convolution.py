"""performConvolution through the C ABI (ConvolutionIr / NdConvolutionIr,
src/convolution_ir.rs:2583-3110, 3642-3760; multiply rules :4252-4440;
ownership rules of FftConfig::validate, src/config.rs:1156-1300): forward C2C,
kernel-spectrum multiply, normalized inverse C2C, against the oracle's
restatement (itself pinned to brute-force circular convolution)."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
# two chained transforms (forward, normalized inverse), each within the
# transform bar of 1e-5 (f32) or 1e-13 (f64)
TOL = {F32: 1e-5, F64: 2e-13}


def conv_cfg(dims, batch, prec, matrix=1, symmetric=False, kernels=1, conj=False, cross=False):
    c = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec).with_convolution(True) \
        .with_convolution_kernel_count(kernels)
    if matrix > 1:
        c = c.with_matrix_convolution(matrix).with_symmetric_convolution_kernel(symmetric)
    if conj:
        c = c.with_convolution_conjugation(vk.ConvolutionConjugation.Sequence)
    if cross:
        c = c.with_cross_power_spectrum_normalization(True)
    return c


def planes(matrix, symmetric):
    if matrix <= 1:
        return 1
    return matrix * (matrix + 1) // 2 if symmetric else matrix * matrix


def run_case(ctx, dims, batch, prec, matrix=1, symmetric=False, kernels=1, conj=False, cross=False, seed=0):
    t = int(np.prod(dims))
    coords = matrix if matrix > 1 else 1
    dt = np.complex64 if prec == F32 else np.complex128
    x = o.complex_uniform(batch * coords * t, 100 + seed, dt)
    k = o.complex_uniform(kernels * planes(matrix, symmetric) * t, 200 + seed, dt)
    conv = vk.ConvolutionIr.build(conv_cfg(dims, batch, prec, matrix, symmetric, kernels, conj, cross), k)
    y = ctx.execute_convolution(conv, x)
    # f64 against pocketfft transforms: the oracle's own f64 error is near 1e-13
    ref = o.convolution(x, k, dims, batch, matrix if matrix > 1 else 0, symmetric, kernels, conj, cross, threads=8,
                        backend="numpy" if prec == F64 else "oracle")
    assert y.size == conv.output_count() == ref.size
    err = o.rel_l2(y, ref)
    assert err <= TOL[prec], (dims, batch, prec, matrix, kernels, err)
    return conv, x, y


@pytest.mark.parametrize("dims,batch,prec", [([1024], 8, F32), ([2048], 4, F64), ([4099], 3, F32),
                                             ([1009], 2, F64), ([1 << 20], 1, F32), ([360], 5, F32),
                                             ([64, 48], 2, F32), ([16, 12, 10], 2, F64), ([256, 256], 1, F32),
                                             ([97, 16], 2, F32), ([48, 97], 3, F64), ([8, 6, 5, 4], 3, F32),
                                             ([1024, 48], 2, F32), ([768, 16, 4], 1, F32),
                                             ([1024, 8], 2, F64), ([3 << 16], 2, F64)])
def test_scalar_kernel(hip_ctx, dims, batch, prec):
    conv, _, _ = run_case(hip_ctx, dims, batch, prec)
    desc = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    labels = [p["kernel"] for p in desc["passes"]]
    if dims in ([1024], [2048], [360]):
        # one upload: forward FFT, multiply and normalized inverse in one pass
        assert desc["convolution"]["fused"] and labels == ["convolution_fused"], labels
    elif dims == [1 << 20]:
        # two uploads: forward column pass, row pass with the multiply between
        # its forward and inverse FFTs, inverse column pass
        assert desc["convolution"]["fused"] and labels == FOUR_STEP_LABELS, labels
    elif len(dims) > 1 and ((dims[0] > 640 and prec == F32) or dims[0] in FIXED_CONV_COLUMNS):
        # N-D over Stockham axes whose axis 0 has a fixed-shape convolution
        # column kernel (64, 128, 256, 512), or which the plain plan splits
        # (and whose runtime geometry holds 8 or more columns per block: 1024,
        # 768): the forward FFT of axes 1.., one kernel per axis-0 line
        # (forward FFT, multiply, inverse FFT), the inverse of axes 1..: 2D - 1
        # passes
        assert desc["convolution"]["fused"] and desc["convolution"]["fused_axis"] == 0, desc["convolution"]
        assert labels.count("convolution_fused_axis0") == 1 and "convolution_multiply" not in labels, labels
        assert len(labels) == 2 * len(dims) - 1, labels
    else:
        # a Rader axis, an axis 0 of one pass without a fixed-shape column
        # kernel, (f64) too few columns per block for the fused kernel, or a
        # two-upload length whose rows (384 for 3 * 2^16 = 512 x 384) have no
        # fixed-shape row pass keep the separate multiply
        assert not desc["convolution"]["fused"] and "convolution_multiply" in labels
    assert desc["convolution"]["kernels"] == 1 and desc["convolution"]["matrix"] == 0


FOUR_STEP_LABELS = ["convolution_columns", "convolution_rows", "convolution_columns_out"]
# axis-0 lengths with a fixed-shape one-upload convolution column kernel
FIXED_CONV_COLUMNS = (64, 128, 256, 512)


@pytest.mark.parametrize("dims,batch,prec", [([1 << 17], 3, F64), ([100000], 2, F32), ([1000000], 1, F64),
                                             ([1 << 16], 5, F32)])
def test_fused_four_step(hip_ctx, dims, batch, prec):
    """A 1-D scalar convolution over a two-upload length whose row length has
    a fixed-shape row pass runs as three passes (forward columns with the W_N
    twiddle; rows: forward FFT, natural-order spectrum multiply, inverse FFT,
    inverse twiddle; inverse columns) and matches the oracle."""
    conv, _, _ = run_case(hip_ctx, dims, batch, prec, seed=21)
    desc = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    labels = [p["kernel"] for p in desc["passes"]]
    assert desc["convolution"]["fused"] and labels == FOUR_STEP_LABELS, labels
    assert desc["convolution"]["n1"] * desc["convolution"]["n2"] == dims[0]


@pytest.mark.parametrize("matrix,symmetric,batch,kernels", [(0, False, 1, 3), (2, False, 2, 1), (2, True, 1, 2),
                                                             (3, False, 1, 1)])
def test_two_upload_fan_out_and_matrix(hip_ctx, matrix, symmetric, batch, kernels):
    """Multi-kernel and matrix convolutions over a two-upload length keep
    the separate multiply (the three-pass plan is scalar only), against the
    oracle."""
    conv, _, _ = run_case(hip_ctx, [1 << 16], batch, F32, matrix, symmetric, kernels, seed=24)
    d = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    assert not d["convolution"]["fused"] and "convolution_multiply" in [p["kernel"] for p in d["passes"]]


@pytest.mark.parametrize("conj,cross", [(True, False), (False, True), (True, True)])
def test_fused_four_step_policies(hip_ctx, conj, cross):
    """Sequence conjugation and cross-power normalization in the four-step
    row pass, batch 3, against the oracle."""
    conv, _, _ = run_case(hip_ctx, [1 << 16], 3, F32, conj=conj, cross=cross, seed=22)
    assert vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()["convolution"]["fused"]


def test_fused_four_step_chunks(monkeypatch, hip_ctx):
    """Batch chunks of the fused four-step convolution on two stream lanes
    (a 1 MB work budget: two lines of 2^16 per chunk, five chunks, the last
    partial), every line against the oracle."""
    monkeypatch.setenv("VKFX_WORK_BUDGET_MB", "1")
    ctx = vk.HipExecutionContext(0)
    try:
        conv, _, _ = run_case(ctx, [1 << 16], 9, F32, seed=23)
        desc = vk.Plan(ctx, conv.ir, desc=conv.desc()).describe()
        labels = [p["kernel"] for p in desc["passes"]]
        assert desc["convolution"]["chunk"] == 2 and labels == FOUR_STEP_LABELS * 5, labels
        assert desc["lanes"] == 2
    finally:
        ctx.close()


@pytest.mark.parametrize("dims,prec", [([1024, 24], F32), ([768, 10, 3], F32)])
@pytest.mark.parametrize("conj,cross", [(True, False), (False, True), (True, True)])
def test_fused_nd_policies(hip_ctx, dims, prec, conj, cross):
    """Sequence conjugation and cross-power normalization in the fused axis-0
    kernel of an N-D convolution (the spectrum of each axis-0 column indexed
    by its position in the tensor), batch 3, against the oracle."""
    conv, _, _ = run_case(hip_ctx, dims, 3, prec, conj=conj, cross=cross, seed=12)
    assert vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()["convolution"]["fused_axis"] == 0


@pytest.mark.parametrize("conj,cross,batch", [(True, False, 3), (False, True, 2), (True, True, 5)])
@pytest.mark.parametrize("n,prec", [(1536, F32), (1024, F32), (8192, F32), (4096, F64)])
def test_fused_convolution_policies(hip_ctx, conj, cross, batch, n, prec):
    """Sequence conjugation and cross-power normalization inside the fused
    one-pass kernel (runtime shape for 1536, fixed shapes with the product in
    the forward FFT's last stage otherwise), against the oracle's three-step
    definition."""
    conv, _, _ = run_case(hip_ctx, [n], batch, prec, conj=conj, cross=cross, seed=5)
    d = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    assert d["convolution"]["fused"] and d["passes"][0]["fixed_shape"] == (n != 1536), d["passes"]


@pytest.mark.parametrize("dims,prec", [([256, 20], F32), ([64, 33], F32), ([128, 12, 3], F64), ([512, 9], F64)])
@pytest.mark.parametrize("conj,cross", [(False, False), (True, True)])
def test_fused_nd_fixed_columns(hip_ctx, dims, prec, conj, cross):
    """N-D convolutions whose axis 0 fits one pass with a fixed-shape column
    kernel: 2D - 1 passes with the fused axis-0 kernel, batch 3, against the
    oracle."""
    conv, _, _ = run_case(hip_ctx, dims, 3, prec, conj=conj, cross=cross, seed=13)
    d = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    labels = [p["kernel"] for p in d["passes"]]
    assert d["convolution"]["fused_axis"] == 0 and len(labels) == 2 * len(dims) - 1, labels
    fused = [p for p in d["passes"] if p["kernel"] == "convolution_fused_axis0"]
    assert len(fused) == 1 and fused[0]["fixed_shape"], fused


@pytest.mark.parametrize("dims,prec", [([1024], F32), ([256], F64), ([1536], F32), ([4099], F32), ([32, 40], F64)])
def test_multi_kernel_fan_out(hip_ctx, dims, prec):
    """K kernels over one input: a one-upload 1-D Stockham length runs one
    fused kernel line per kernel (the input read by every line, spectrum
    plane k); other lengths keep the separate multiply."""
    conv, _, _ = run_case(hip_ctx, dims, 1, prec, kernels=3, seed=1)
    d = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    fused = len(dims) == 1 and dims[0] != 4099
    assert d["convolution"]["fused"] == fused, d["convolution"]
    if fused:
        assert [p["kernel"] for p in d["passes"]] == ["convolution_fused"]


@pytest.mark.parametrize("matrix,symmetric,batch,kernels,prec",
                         [(2, False, 3, 1, F32), (3, False, 2, 1, F64), (2, True, 4, 1, F64), (3, False, 1, 2, F32),
                          (2, True, 1, 3, F32)])
@pytest.mark.parametrize("n", [512, 2048])
def test_matrix_1d(hip_ctx, matrix, symmetric, batch, kernels, prec, n):
    """Matrix convolutions of one-upload 1-D lengths: one fused kernel whose
    blocks hold whole systems of coordinate lines and mix them between the
    forward and inverse FFTs."""
    conv, _, _ = run_case(hip_ctx, [n], batch, prec, matrix, symmetric, kernels, seed=2)
    d = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    assert d["convolution"]["fused"] and [p["kernel"] for p in d["passes"]] == ["convolution_fused"], d["passes"]
    assert d["passes"][0]["lines_per_block"] % matrix == 0, d["passes"][0]


@pytest.mark.parametrize("matrix,symmetric,kernels", [(2, False, 1), (3, False, 2), (2, True, 1)])
@pytest.mark.parametrize("conj,cross", [(True, False), (False, True)])
def test_matrix_1d_policies(hip_ctx, matrix, symmetric, kernels, conj, cross):
    """Sequence conjugation and cross-power normalization of the mixed
    product (the normalization applies to the row sum), against the oracle."""
    batch = 2 if kernels == 1 else 1
    conv, _, _ = run_case(hip_ctx, [1024], batch, F32, matrix, symmetric, kernels, conj, cross, seed=4)
    assert vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()["convolution"]["fused"]


def test_matrix_nd_batch1(hip_ctx):
    run_case(hip_ctx, [16, 32], 1, F32, matrix=2, seed=3)
    run_case(hip_ctx, [8, 8, 8], 1, F64, matrix=3, seed=4)


@pytest.mark.parametrize("conj,cross", [(True, False), (False, True), (True, True)])
def test_conjugation_and_cross_power(hip_ctx, conj, cross):
    run_case(hip_ctx, [1000], 3, F64, conj=conj, cross=cross, seed=5)
    run_case(hip_ctx, [1024], 2, F32, conj=conj, cross=cross, seed=6)


def test_phase_correlation_finds_shift(hip_ctx):
    """Cross-power spectrum of x and a shifted copy: a delta at the shift."""
    dims, shift = [128, 96], (37, 11)
    x = o.complex_uniform(128 * 96, 7, np.complex64)
    k = np.fft.fft2(np.roll(x.reshape(dims), shift, axis=(0, 1))).astype(np.complex64)
    cfg = conv_cfg(dims, 1, F32, conj=True, cross=True)
    y = hip_ctx.execute_convolution(vk.ConvolutionIr.build(cfg, k), x).reshape(dims)
    assert np.unravel_index(np.argmax(np.abs(y)), dims) == shift
    e = np.zeros(dims)
    e[shift] = 1
    assert np.max(np.abs(y - e)) <= 1e-5


@pytest.mark.parametrize("n", [4096, 1 << 16])
def test_mixed_storage_scalar(hip_ctx, n):
    """Mixed storage around the one-upload fused kernel (4096) and the
    three-pass two-upload convolution (2^16)."""
    x = o.complex_uniform(n, 8, np.complex64)
    k = o.complex_uniform(n, 9, np.complex128)
    for prec, tol in ((vk.Precision.F64ComputeF32Storage, 1e-7), (vk.Precision.F16StorageF32Compute, 2e-3)):
        conv = vk.ConvolutionIr.build(conv_cfg([n], 1, prec), k)
        y = hip_ctx.execute_convolution(conv, x)
        assert vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()["convolution"]["fused"], (n, prec)
        xin = x if prec == vk.Precision.F64ComputeF32Storage else \
            x.view(np.float32).astype(np.float16).astype(np.float32).view(np.complex64)
        kin = k if prec == vk.Precision.F64ComputeF32Storage else k.astype(np.complex64)
        assert o.rel_l2(y, o.convolution(xin, kin, [n], 1)) <= tol, prec


def test_device_resident_in_place(hip_ctx):
    import torch
    n, batch = 1024, 6
    x = o.complex_uniform(n * batch, 10, np.complex64)
    k = o.complex_uniform(n, 11, np.complex64)
    conv = vk.ConvolutionIr.build(conv_cfg([n], batch, F32), k)
    plan = vk.Plan(hip_ctx, conv.ir, desc=conv.desc())
    assert plan.in_bytes == plan.out_bytes == n * batch * 8
    d = torch.from_numpy(x.view(np.float32).copy()).cuda()
    plan.execute(d.data_ptr(), d.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y = d.cpu().numpy().view(np.complex64)
    assert np.array_equal(y, hip_ctx.execute_convolution(conv, x))


def _rejects(ctx, cfg, k, status=None):
    with pytest.raises(vk.VkFftError) as ei:
        conv = vk.ConvolutionIr.build(cfg, k)  # keeps the kernel spectrum alive through plan creation
        vk.Plan(ctx, conv.ir, desc=conv.desc())
    if status is not None:
        assert ei.value.status == status
    return ei.value


def test_fail_closed_layouts(hip_ctx):
    k1 = o.complex_uniform(256, 12, np.complex64)
    unsupported = -3
    # kernel spectrum length must match the plane layout
    _rejects(hip_ctx, conv_cfg([256], 1, F32, kernels=2), k1)
    # numberKernels is a one-input fan-out
    _rejects(hip_ctx, conv_cfg([256], 2, F32, kernels=2), np.tile(k1, 2), unsupported)
    # coordinates without a matrix belong to real application convolution
    _rejects(hip_ctx, conv_cfg([256], 1, F32).with_coordinate_features(2), np.tile(k1, 2), unsupported)
    # 3x3 symmetric aliases two planes upstream
    _rejects(hip_ctx, conv_cfg([256], 1, F32, matrix=3, symmetric=True), np.tile(k1, 6), unsupported)
    # N-D matrix needs batch 1
    _rejects(hip_ctx, conv_cfg([16, 16], 2, F32, matrix=2), np.tile(k1, 4), unsupported)
    # non-finite kernel values
    bad = k1.copy()
    bad[7] = np.nan
    _rejects(hip_ctx, conv_cfg([256], 1, F32), bad)
    # zero padding and formatted strides are real-application features
    _rejects(hip_ctx, conv_cfg([256], 1, F32).with_zero_padding(0, 10, 20), k1, unsupported)
    _rejects(hip_ctx, conv_cfg([256], 1, F32).with_input_buffer_batch_stride(300), k1, unsupported)
    # mixed storage only for the batch-1 scalar K=1 default policy
    _rejects(hip_ctx, conv_cfg([256], 2, vk.Precision.F64ComputeF32Storage), k1.astype(np.complex128), unsupported)
    # kernel conjugation has no executable codegen upstream
    with pytest.raises(vk.VkFftError):
        vk.ConvolutionIr.build(conv_cfg([256], 1, F32).with_convolution_conjugation(vk.ConvolutionConjugation.Kernel),
                               k1)
    # a convolution config run as a plain transform has no kernel spectrum
    with pytest.raises(vk.VkFftError):
        hip_ctx.plan(vk.TransformIr.build(conv_cfg([256], 1, F32), vk.Direction.Forward))


# ---- real application (NdRealConvolutionIr, convolution_ir.rs:3884-4251) ----

def real_conv_cfg(dims, prec, coords=1, matrix=1, symmetric=False, kernels=1, conj=False, cross=False):
    c = conv_cfg(dims, 1, prec, matrix, symmetric, kernels, conj, cross).with_transform(vk.TransformKind.RealToComplex)
    if matrix <= 1:
        c = c.with_coordinate_features(coords)
    return c


def run_real_case(ctx, dims, prec, coords=1, matrix=1, symmetric=False, kernels=1, conj=False, cross=False, seed=0):
    rd = np.float32 if prec == F32 else np.float64
    cd = np.complex64 if prec == F32 else np.complex128
    coords = matrix if matrix > 1 else coords
    n = int(np.prod(dims))
    x = o.normal(coords * n, 300 + seed, rd)
    pl = planes(matrix, symmetric) if matrix > 1 else coords
    hk = o.normal(kernels * pl * n, 400 + seed, np.float64).reshape((kernels * pl,) + tuple(dims))
    k = np.fft.rfftn(hk, axes=tuple(range(1, len(dims) + 1))).astype(cd).reshape(-1)  # Hermitian spectra
    conv = vk.ConvolutionIr.build(real_conv_cfg(dims, prec, coords, matrix, symmetric, kernels, conj, cross), k)
    assert conv.real and conv.input_count() == coords * n and conv.output_count() == kernels * coords * n
    y = ctx.execute_convolution(conv, x)
    assert y.dtype == rd
    ref = o.convolution_real(x, k, dims, coords, matrix if matrix > 1 else 0, symmetric, kernels, conj, cross)
    err = o.rel_l2(y, ref)
    assert err <= TOL[prec], (dims, prec, coords, matrix, kernels, err)
    return conv


@pytest.mark.parametrize("dims,prec,coords,kernels", [([64, 48], F32, 1, 1), ([32, 40], F64, 3, 1),
                                                      ([16, 12, 10], F32, 2, 3), ([128, 130], F32, 1, 2),
                                                      ([1, 64], F64, 1, 1), ([4096, 4096], F32, 1, 1)])
def test_real_convolution_independent(hip_ctx, dims, prec, coords, kernels):
    conv = run_real_case(hip_ctx, dims, prec, coords=coords, kernels=kernels)
    desc = vk.Plan(hip_ctx, conv.ir, desc=conv.desc()).describe()
    assert desc["convolution"]["real"] and "convolution_multiply" in [p["kernel"] for p in desc["passes"]]


@pytest.mark.parametrize("matrix,symmetric,kernels,prec", [(2, False, 1, F32), (3, False, 2, F64), (2, True, 1, F64)])
def test_real_convolution_matrix(hip_ctx, matrix, symmetric, kernels, prec):
    run_real_case(hip_ctx, [24, 32], prec, matrix=matrix, symmetric=symmetric, kernels=kernels, seed=1)


def test_real_convolution_policies_and_mixed(hip_ctx):
    run_real_case(hip_ctx, [48, 40], F64, conj=True, seed=2)
    run_real_case(hip_ctx, [48, 40], F64, conj=True, cross=True, seed=3)
    # mixed storage: scalar ownership and independent-coordinate K>1 fan-out
    dims, n = [32, 36], 32 * 36
    x = o.normal(n, 5, np.float32)
    hk = o.normal(n, 6, np.float64).reshape(dims)
    k = np.fft.rfftn(hk).reshape(-1)
    for prec, tol in ((vk.Precision.F64ComputeF32Storage, 1e-7), (vk.Precision.F16StorageF32Compute, 3e-3)):
        kk = k if prec == vk.Precision.F64ComputeF32Storage else k.astype(np.complex64)
        y = hip_ctx.execute_convolution(vk.ConvolutionIr.build(real_conv_cfg(dims, prec), kk), x)
        xin = x if prec == vk.Precision.F64ComputeF32Storage else x.astype(np.float16).astype(np.float32)
        assert o.rel_l2(y, o.convolution_real(xin, kk, dims)) <= tol, prec


def test_real_convolution_zero_padding_and_layout(hip_ctx):
    """Spatial zero padding masks the input of the forward R2C and the output
    of the inverse C2R; formatted strides for scalar K=1 ownership."""
    dims, n = [40, 36], 40 * 36
    x = o.normal(2 * n, 7, np.float64)
    hk = o.normal(4 * n, 8, np.float64).reshape(4, 40, 36)
    k = np.fft.rfftn(hk, axes=(1, 2)).reshape(-1)
    c = real_conv_cfg(dims, F64, matrix=2).with_zero_padding(0, 30, 40).with_zero_padding(1, 20, 36)
    y = hip_ctx.execute_convolution(vk.ConvolutionIr.build(c, k), x).reshape(2, 40, 36)
    mask = np.zeros((40, 36), dtype=bool)
    mask[30:, :] = True
    mask[:, 20:] = True
    xm = x.reshape(2, 40, 36).copy()
    xm[:, mask] = 0
    ref = o.convolution_real(xm, k, dims, 2, 2).reshape(2, 40, 36)
    ref[:, mask] = 0
    assert (y[:, mask] == 0).all()
    assert o.rel_l2(y, ref) <= TOL[F64]
    # formatted input / output row strides (scalar, K = 1)
    k1 = k[:40 * 19]
    cf = real_conv_cfg(dims, F64).with_input_buffer_axis_stride(0, 40).with_output_buffer_axis_stride(0, 38)
    conv = vk.ConvolutionIr.build(cf, k1)
    yf = hip_ctx.execute_convolution(conv, x[:n])
    assert o.rel_l2(yf, o.convolution_real(x[:n], k1, dims)) <= TOL[F64]


def test_real_convolution_fail_closed(hip_ctx):
    dims = [16, 16]
    k1 = np.fft.rfftn(np.ones(dims)).astype(np.complex64).reshape(-1)
    unsupported = -3
    _rejects(hip_ctx, real_conv_cfg(dims, F32).with_batch_count(2), k1, unsupported)
    _rejects(hip_ctx, real_conv_cfg(dims, F32, matrix=2, symmetric=True).with_zero_padding(0, 8, 16),
             np.tile(k1, 3), unsupported)
    _rejects(hip_ctx, real_conv_cfg(dims, F32, coords=2).with_output_buffer_batch_stride(300), np.tile(k1, 2),
             unsupported)
    # mixed storage: a 2x2 matrix is not among the pinned real ownerships
    _rejects(hip_ctx, real_conv_cfg(dims, vk.Precision.F64ComputeF32Storage, matrix=2), np.tile(k1, 4).astype(np.complex128),
             unsupported)
    # 1-D real convolution is not a real application
    with pytest.raises(vk.VkFftError):
        hip_ctx.execute_convolution(vk.ConvolutionIr.build(real_conv_cfg([64], F32), k1[:33]), np.ones(64, np.float32))
