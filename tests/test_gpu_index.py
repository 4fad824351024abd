"""Bit-exact addressing: the index-map test build of the library
(libvkfft_mi355x_index.so, identity butterflies / twiddles / chirps /
spectra / scale) against the CPU index maps of oracle/index_maps.py.

Inputs are integer-tagged (exact in f32 and f64), so every output element
must equal the input element the maps name, bit for bit: this checks the
direct HBM stages, LDS slot arithmetic, line mappings (rows, columns, split
axes, chunks, stream lanes, formatted layouts), four-step transposes and
Bluestein padding / truncation of every C2C kernel family. The even R2C / C2R
kernels (one upload and four-step) combine each element with its mirror:
with random integer tags their identity-arithmetic results (sums and
differences of the paired elements) are exact, so the pairing and placement
are checked bit for bit too, and likewise the FFT-mode Rader kernel's
gather, slot-0 sum and scatter. The direct-multiplication Rader kernel and
the Rader stages of mixed-radix lengths convolve with the unit impulse under
identity arithmetic (the FFT-mode stages run their convolution's identity
Stockham maps), so their gathers and scatters are checked bit for bit too."""
import os

import numpy as np
import pytest

import vkfft_amd as vk
from oracle import index_maps as im

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse


@pytest.fixture(scope="module")
def idx_ctx():
    if not os.path.exists("/dev/kfd"):
        pytest.skip("no GPU in this container")
    import torch
    torch.cuda.init()
    ctx = vk.HipExecutionContext(0, library=vk.INDEX_LIB_PATH)
    assert b"index-map test build" in ctx._L.vkfx_version()
    yield ctx
    ctx.close()


def tagged(count, prec):
    k = np.arange(count, dtype=np.float64)
    x = (k + 1) - 1j * ((k % 65521) + 0.5)
    return x.astype(np.complex64 if prec == F32 else np.complex128)


def run(ctx, dims, batch, prec, direction, x, env=None):
    """Fresh plan (plans read the chunk budgets when built), host round trip."""
    old = {}
    for k, v in (env or {}).items():
        old[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec)
        ir = vk.TransformIr.build(cfg, direction)
        plan = vk.Plan(ctx, ir)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    out = np.empty(ir.output_count(), dtype=x.dtype)
    vk._check(ctx._L.vkfx_execute_host(plan.handle, x.ctypes.data, x.nbytes, out.ctypes.data, out.nbytes), ctx._L)
    desc = plan.describe()
    plan.close()
    return out, desc


def first_passes(desc):
    """Passes of the first chunk, in launch order (labels repeat per chunk)."""
    seen, out = set(), []
    for p in desc["passes"]:
        if p["kernel"] in seen and p["kernel"] not in ("stockham_rows", "stockham_columns", "split_axis_pass1",
                                                        "split_axis_pass2", "bluestein_axis"):
            break
        seen.add(p["kernel"])
        out.append(p)
    return out


def line_map_1d(n, desc):
    ps = first_passes(desc)
    names = [p["kernel"] for p in ps]
    if names[0] == "stockham":
        return im.stockham_perm(n, ps[0]["radices"])
    if names[:2] == ["four_step_columns", "four_step_rows"]:
        a, b = ps[0], ps[1]
        return im.four_step_perm(a["fft_len"], a["radices"], b["fft_len"], b["radices"])
    if names[:3] == ["three_upload_pass1", "three_upload_pass2", "three_upload_pass3"]:
        a, b, c = ps[:3]
        return im.three_pass_perm(a["fft_len"], a["radices"], b["fft_len"], b["radices"], c["fft_len"],
                                  c["radices"])
    if names[0] == "bluestein_single":
        return im.bluestein_single_perm(n, ps[0]["fft_len"], ps[0]["radices"])
    if names[:3] == ["bluestein_columns", "bluestein_rows", "bluestein_columns_out"]:
        a, b, c = ps[:3]
        return im.bluestein_three_pass_perm(n, a["fft_len"], a["radices"], b["fft_len"], b["radices"],
                                            c["radices"])
    raise AssertionError(f"unmodelled pass list {names}")


def check_1d(ctx, n, batch, prec, direction=FWD, env=None):
    x = tagged(n * batch, prec)
    out, desc = run(ctx, [n], batch, prec, direction, x, env)
    src = line_map_1d(n, desc)
    expect = im.gather(x, src, n, batch, n)
    assert np.array_equal(out, expect), (n, batch, [p["kernel"] for p in desc["passes"][:4]])
    return desc


SINGLE = [2, 3, 5, 7, 8, 11, 13, 16, 18, 25, 27, 32, 36, 49, 60, 64, 96, 100, 121, 125, 128, 169, 243,
          343, 360, 512, 625, 1000, 1024, 1536, 2048, 2187, 2401, 3125, 4096, 6561, 8192, 10000, 15625, 16384,
          # the 3*2^k / 5*2^k fixed families
          12, 20, 24, 40, 48, 80, 160, 192, 320, 384, 640, 768, 1280, 2560, 3072, 5120, 6144, 10240, 12288]


ROUND = [200, 240, 300, 400, 480, 500, 600, 720, 750, 800, 900, 960, 1200, 1500, 1600, 1800, 1920, 2000, 2400,
         2500, 3000, 3200, 3600, 4000, 4800, 5000, 6000, 6400, 7200, 8000, 9000, 9600, 12000, 16000]


@pytest.mark.parametrize("prec", [F32, F64])
def test_round_length_rows(idx_ctx, prec):
    """The generated round-length row shapes (kf_round_*), both directions."""
    for n in ROUND:
        if prec == F64 and n > 8192:
            continue
        d = check_1d(idx_ctx, n, 3, prec)
        assert d["passes"][0]["fixed_shape"], n
        check_1d(idx_ctx, n, 2, prec, INV)


@pytest.mark.parametrize("prec", [F32, F64])
def test_single_upload_lengths(idx_ctx, prec):
    for n in SINGLE:
        check_1d(idx_ctx, n, 3, prec)
        check_1d(idx_ctx, n, 2, prec, INV)


def test_config_shapes_1d(idx_ctx):
    d = check_1d(idx_ctx, 1024, 64, F32)          # C1 kernel (fixed, two waves per line)
    assert d["passes"][0]["fixed_shape"]
    check_1d(idx_ctx, 1024, 33, F32, INV)
    check_1d(idx_ctx, 4096, 5, F32)
    check_1d(idx_ctx, 512, 9, F64)


def test_register_exchange_kernel(idx_ctx):
    """The one-wave 1024-point kernel whose exchanges are DPP moves and
    permlane swaps: with identity arithmetic it must apply exactly the
    Stockham (16, 4, 16) digit-reversal permutation, for full and partial
    blocks of 4 lines, both directions."""
    env = {"VKFX_REGISTER_EXCHANGE": "1"}
    for batch, direction in ((64, FWD), (33, FWD), (5, INV), (1, INV)):
        d = check_1d(idx_ctx, 1024, batch, F32, direction, env=env)
        (p,) = d["passes"]
        assert p["lds_bytes"] == 0 and p["lines_per_block"] == 4 and p["radices"] == [16, 4, 16], p


@pytest.mark.parametrize("n,cap,prec", [(4096, 16, F32), (2187, 27, F64), (3072, 16, F32), (1 << 20, 128, F32)])
def test_three_upload(idx_ctx, n, cap, prec):
    """Lengths with no two-upload split (forced by capping the one-upload
    length): three passes, every chunk and lane."""
    env = {"VKFX_MAX_UPLOAD": str(cap)}
    for batch, direction in ((3, FWD), (2, INV)):
        d = check_1d(idx_ctx, n, batch, prec, direction, env=env)
        assert d["four_step"]["uploads"] == 3, d["four_step"]
    d = check_1d(idx_ctx, n, 9, prec, env=dict(env, VKFX_WORK_BUDGET_MB="0"))


@pytest.mark.parametrize("n,kind,pick", [(1024, 0, 0), (1024, 0, 1), (4099, 12, 0), (4099, 12, 1), (4099, 12, 2),
                                         (4115, 12, 0)])
def test_fixed_shape_variants(idx_ctx, n, kind, pick):
    """Per-stage twiddle tables and pads, ping-pong LDS buffers and the
    product-tree forms of the C1 and M = 8232 shapes move the same elements."""
    env = {f"VKFX_FIXED_PICK_K{kind}": str(pick)}
    for batch, direction in ((5, FWD), (3, INV)):
        d = check_1d(idx_ctx, n, batch, F32, direction, env=env)
        assert d["passes"][0]["fixed_shape"]


@pytest.mark.parametrize("n,batch,prec", [(1 << 20, 2, F32), (1 << 17, 3, F32), (3 ** 12, 1, F32),
                                          (1 << 18, 2, F64), (5 ** 8, 1, F64),
                                          # kf_round_fs_* factors
                                          (1 << 16, 2, F32), (60000, 2, F64), (100000, 2, F32),
                                          (250000, 1, F64), (1000000, 1, F32), (4000000, 1, F32)])
def test_four_step(idx_ctx, n, batch, prec):
    d = check_1d(idx_ctx, n, batch, prec)
    assert [p["kernel"] for p in d["passes"][:2]] == ["four_step_columns", "four_step_rows"]
    check_1d(idx_ctx, n, batch, prec, INV)


def test_four_step_chunks_and_lanes(idx_ctx):
    """Many small chunks on two stream lanes: offsets of every chunk."""
    d = check_1d(idx_ctx, 1 << 18, 12, F32, env={"VKFX_WORK_BUDGET_MB": "4"})
    assert d["lanes"] == 2
    assert len(d["passes"]) == 2 * 6


@pytest.mark.parametrize("n,prec", [(4099, F32), (65537, F32), (12289, F64), (20011, F32),
                                    # one-kernel fixed rows: M = 256 (four lines per block), 5184, 16384, 1323, 8192
                                    (103, F32), (2309, F32), (6131, F32), (659, F64), (4093, F64)])
def test_bluestein(idx_ctx, n, prec):
    alg, _ = vk.planner_axis(n, 4, prec)
    if alg != vk.AlgorithmKind.Bluestein:
        pytest.skip(f"N={n} plans as {alg.name}")
    check_1d(idx_ctx, n, 4, prec)
    check_1d(idx_ctx, n, 3, prec, INV)


ND = [([64, 48], 2, F32), ([256, 256], 2, F32), ([8, 4096], 2, F32), ([4096, 8], 1, F32), ([1024, 6], 2, F32),
      ([512, 8], 2, F64), ([8, 512], 2, F64), ([16, 12, 10], 2, F64), ([6, 20, 64, 40], 1, F32),
      ([64, 64, 64], 1, F64), ([3, 768, 5], 2, F32), ([4099, 4], 1, F32),
      # power-of-two column shapes and split strided axes (32 x 32, 64 x 32, 128 x 64)
      ([32, 16, 8], 3, F32), ([128, 64], 2, F64), ([16, 128], 5, F32), ([256, 3], 2, F64),
      ([1024, 4], 1, F64), ([2048, 3], 1, F32), ([8192, 2], 1, F32), ([8192, 2], 1, F64),
      # 3*2^k / 5*2^k / 10^k / 360 column shapes
      ([96, 20], 2, F32), ([360, 12], 1, F64), ([100, 40, 6], 1, F32), ([640, 3], 2, F32), ([640, 3], 1, F64),
      ([80, 160, 2], 1, F64), ([384, 24], 1, F32), ([12, 48, 5], 2, F64),
      # round-length rows, columns and split passes (kf_round_*)
      ([120, 120, 12], 1, F32), ([720, 30], 1, F32), ([1000, 40], 1, F64), ([2000, 6], 1, F32),
      ([75, 45, 27], 1, F64), ([6, 10, 9, 15], 2, F32), ([625, 18], 1, F32), ([4800, 3], 1, F64)]


def nd_axis_maps(dims, desc):
    """Per-axis line maps from the pass list: axes run last to first, one pass
    each, two for a split strided axis."""
    passes = desc["passes"]
    maps = [None] * len(dims)
    i = 0
    for ax in range(len(dims) - 1, -1, -1):
        n = dims[ax]
        if n == 1:
            continue
        p = passes[i]
        if p["kernel"] in ("stockham_rows", "stockham_columns"):
            maps[ax] = im.stockham_perm(n, p["radices"])
            i += 1
        elif p["kernel"] == "split_axis_pass1":
            q = passes[i + 1]
            maps[ax] = im.four_step_perm(p["fft_len"], p["radices"], q["fft_len"], q["radices"])
            i += 2
        elif p["kernel"] == "bluestein_axis":
            src = im.bluestein_single_perm(n, p["fft_len"], p["radices"])
            maps[ax] = src
            i += 1
        else:
            raise AssertionError(f"unmodelled pass {p['kernel']}")
    return maps


@pytest.mark.parametrize("dims,batch,prec", ND)
def test_nd(idx_ctx, dims, batch, prec):
    count = int(np.prod(dims)) * batch
    x = tagged(count, prec)
    out, desc = run(idx_ctx, dims, batch, prec, FWD, x)
    maps = nd_axis_maps(dims, desc)
    v = x.reshape((batch,) + tuple(dims))
    for ax, src in enumerate(maps):
        if src is None:
            continue
        safe = np.where(src >= 0, src, 0)
        v = np.take(v, safe, axis=ax + 1)
        if (src < 0).any():
            idx = [slice(None)] * v.ndim
            idx[ax + 1] = np.nonzero(src < 0)[0]
            v[tuple(idx)] = 0
    assert np.array_equal(out, v.reshape(-1)), (dims, batch, [p["kernel"] for p in desc["passes"]])


def test_nd_slab_chunks(idx_ctx):
    """Slab-chunked volume (axes 1.. per slab chunk, axis 0 last)."""
    dims, batch = [32, 64, 48], 2
    x = tagged(int(np.prod(dims)) * batch, F64)
    out, desc = run(idx_ctx, dims, batch, F64, FWD, x, env={"VKFX_ND_CHUNK_MB": "1"})
    assert desc["nd"]["slabs_per_chunk"] > 0
    rad = {}
    for p in desc["passes"]:
        rad.setdefault(p["fft_len"], p["radices"])
    v = x.reshape((batch,) + tuple(dims))
    for ax, n in enumerate(dims):
        v = np.take(v, im.stockham_perm(n, rad[n]), axis=ax + 1)
    assert np.array_equal(out, v.reshape(-1))


def _padded_layout(c, dims):
    """Formatted strides on both sides: every axis but the fastest padded by a
    few elements, and the batch stride padded too."""
    for side in ("input", "output"):
        st = 1
        for ax in range(len(dims) - 1, -1, -1):
            if ax < len(dims) - 1:
                st = st + 3 + ax
                c = getattr(c, f"with_{side}_buffer_axis_stride")(ax, st)
            st *= dims[ax]
        c = getattr(c, f"with_{side}_buffer_batch_stride")(st + 5)
    return c


@pytest.mark.parametrize("dims,batch", [([32, 48], 2), ([8, 12, 40], 2), ([4, 300], 3)])
def test_formatted_layout_in_passes(idx_ctx, dims, batch):
    """Formatted input and output read and written by the first and last
    passes (three line levels): every logical element lands where the
    per-axis Stockham maps send it, through the caller's strides."""
    cfg = _padded_layout(vk.FftConfig.new(dims).with_batch_count(batch).with_precision(F64), dims)
    ir = vk.TransformIr.build(cfg, FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        assert desc["boundary"]["fused_layout"] and not desc["boundary"]["input"]
        x = tagged(int(np.prod(dims)) * batch, F64)
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    rad = {}
    for p in desc["passes"]:
        rad.setdefault(p["fft_len"], p["radices"])
    v = x.reshape((batch,) + tuple(dims))
    for ax, n in enumerate(dims):
        v = np.take(v, im.stockham_perm(n, rad[n]), axis=ax + 1)
    assert np.array_equal(out, v.reshape(-1))


@pytest.mark.parametrize("n,left,right,domain", [(1024, 100, 300, "spatial"), (1000, 0, 7, "frequency"),
                                                 (720, 700, 720, "spatial")])
def test_storage_and_zero_interval_in_pass(idx_ctx, n, left, right, domain):
    """1-D F64ComputeF32Storage with a zero interval, converted and masked
    inside the one pass (HBM-direct ends): f32 tags survive the f64 pass
    exactly; the input interval reads as zero (spatial, forward) or the
    output interval is written as zero (frequency, forward)."""
    batch = 3
    zd = vk.ZeroPaddingDomain.Spatial if domain == "spatial" else vk.ZeroPaddingDomain.Frequency
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(vk.Precision.F64ComputeF32Storage) \
        .with_zero_padding(0, left, right).with_zero_padding_domain(zd)
    ir = vk.TransformIr.build(cfg, FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        assert desc["boundary"]["fused_edges"] and [p["kernel"] for p in desc["passes"]] == ["stockham"]
        x = tagged(n * batch, F32)
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    perm = im.stockham_perm(n, desc["passes"][0]["radices"])
    v = x.reshape(batch, n).copy()
    if domain == "spatial":
        v[:, left:right] = 0
    v = v[:, perm]
    if domain == "frequency":
        v[:, left:right] = 0
    assert np.array_equal(out, v.reshape(-1))


def _muli(v, s):
    """(s i) * v, s = +-1 (fft_device.hpp muli)."""
    return (-v.imag + 1j * v.real) if s > 0 else (v.imag - 1j * v.real)


@pytest.mark.parametrize("n", [64, 210, 1000, 1024, 4096, 6000, 8192, 2400, 16000, 20000, 32000])
@pytest.mark.parametrize("prec", [F32, F64])
def test_r2c_half_addressing(idx_ctx, n, prec):
    """Even one-upload R2C (real pairs -> half-length FFT -> postprocess):
    with identity butterflies and twiddles the postprocess computes
    (A + conj Z[M-k]) - i (A - conj Z[M-k]) from A = Z[k] (k = 0 and M both
    take Z[0]). Random integer tags make a wrong pairing or placement show:
    the result must match bit for bit."""
    if prec == F64 and n > 16384:
        pytest.skip("an f64 half length above 8192 runs as two uploads (the four-step addressing tests)")
    batch, M = 3, n // 2
    rng = np.random.default_rng(n)
    x = rng.integers(0, 1 << 18, n * batch).astype(np.float32 if prec == F32 else np.float64)
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.RealToComplex)
    ir = vk.TransformIr.build(cfg, FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    assert len(desc["passes"]) == 1, desc["passes"]
    z = (x[0::2] + 1j * x[1::2]).reshape(batch, M)
    z = z[:, im.stockham_perm(M, desc["passes"][0]["radices"])]
    k = np.arange(M + 1)
    a = z[:, np.where(k == M, 0, k)]
    b = np.conj(z[:, np.where(k == 0, 0, M - k)])
    expect = (a + b) + _muli(a - b, -1)
    assert np.array_equal(out.reshape(batch, M + 1), expect.astype(out.dtype))


@pytest.mark.parametrize("n", [64, 210, 1000, 1024, 4096, 6000, 8192, 2400, 16000, 20000, 32000])
@pytest.mark.parametrize("prec", [F32, F64])
def test_c2r_half_addressing(idx_ctx, n, prec):
    """Even one-upload C2R (preprocess -> half-length inverse FFT -> real
    pairs): with identity arithmetic Z[k] = (X[k] + conj X[M-k]) +
    i (X[k] - conj X[M-k]) for k < M, then the Stockham map, then the
    complex results as real pairs; random integer tags, bit for bit."""
    if prec == F64 and n > 16384:
        pytest.skip("an f64 half length above 8192 runs as two uploads (the four-step addressing tests)")
    batch, M = 3, n // 2
    rng = np.random.default_rng(n + 1)
    re = rng.integers(0, 1 << 18, (M + 1) * batch)
    im_ = rng.integers(0, 1 << 18, (M + 1) * batch)
    X = (re + 1j * im_).astype(np.complex64 if prec == F32 else np.complex128)
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.ComplexToReal)
    ir = vk.TransformIr.build(cfg, INV)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, X)
    finally:
        plan.close()
    assert len(desc["passes"]) == 1, desc["passes"]
    Xb = X.reshape(batch, M + 1).astype(np.complex128)
    k = np.arange(M)
    xk = Xb[:, k]
    xm = np.conj(Xb[:, M - k])
    z = (xk + xm) + _muli(xk - xm, 1)
    z = z[:, im.stockham_perm(M, desc["passes"][0]["radices"])]
    expect = np.empty((batch, n))
    expect[:, 0::2] = z.real
    expect[:, 1::2] = z.imag
    assert np.array_equal(out.reshape(batch, n), expect.astype(out.dtype))


def _real_four_step(desc, first, second):
    names = [p["kernel"] for p in desc["passes"]]
    assert names[:2] == [first, second], names
    a, b = desc["passes"][0], desc["passes"][1]
    return im.four_step_perm(a["fft_len"], a["radices"], b["fft_len"], b["radices"])


@pytest.mark.parametrize("n,batch", [(1 << 17, 3), (1 << 20, 2), (3 << 16, 2)])
@pytest.mark.parametrize("prec", [F32, F64])
def test_r2c_four_step_addressing(idx_ctx, n, batch, prec):
    """Two-upload R2C (column pass, then the row pass with the postprocess
    of each row beside its mirror row): X[k] from Z[k] and Z[(M-k) mod M] of
    the four-step map, X[M] = Re Z[0] - Im Z[0]; integer tags, bit for bit."""
    M = n // 2
    rng = np.random.default_rng(n + batch)
    x = rng.integers(0, 1 << 18, n * batch).astype(np.float32 if prec == F32 else np.float64)
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.RealToComplex)
    ir = vk.TransformIr.build(cfg, FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    src = _real_four_step(desc, "r2c_columns", "r2c_rows_post")
    z = (x[0::2] + 1j * x[1::2]).reshape(batch, M)[:, src]
    k = np.arange(M)
    a = z
    b = np.conj(z[:, (M - k) % M])
    expect = np.empty((batch, M + 1), dtype=np.complex128)
    expect[:, :M] = (a + b) + _muli(a - b, -1)
    expect[:, M] = z[:, 0].real - z[:, 0].imag
    assert np.array_equal(out.reshape(batch, M + 1), expect.astype(out.dtype))


@pytest.mark.parametrize("n,batch", [(1 << 17, 3), (1 << 20, 2), (3 << 16, 2)])
@pytest.mark.parametrize("prec", [F32, F64])
def test_c2r_four_step_addressing(idx_ctx, n, batch, prec):
    """Two-upload C2R (column pass forming the preprocess from X[k] and
    X[M-k], then the row pass): the four-step map of Z, as real pairs;
    integer tags, bit for bit."""
    M = n // 2
    rng = np.random.default_rng(n + batch + 7)
    X = (rng.integers(0, 1 << 18, (M + 1) * batch) + 1j * rng.integers(0, 1 << 18, (M + 1) * batch))
    X = X.astype(np.complex64 if prec == F32 else np.complex128)
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.ComplexToReal)
    ir = vk.TransformIr.build(cfg, INV)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, X)
    finally:
        plan.close()
    src = _real_four_step(desc, "c2r_columns_pre", "c2r_rows")
    Xb = X.reshape(batch, M + 1).astype(np.complex128)
    k = np.arange(M)
    xk, xm = Xb[:, k], np.conj(Xb[:, M - k])
    z = ((xk + xm) + _muli(xk - xm, 1))[:, src]
    expect = np.empty((batch, n))
    expect[:, 0::2] = z.real
    expect[:, 1::2] = z.imag
    assert np.array_equal(out.reshape(batch, n), expect.astype(out.dtype))


@pytest.mark.parametrize("p", [97, 193, 257, 769, 3457])
@pytest.mark.parametrize("prec", [F32, F64])
def test_rader_fft_addressing(idx_ctx, p, prec):
    """FFT-mode Rader of a prime p (rader_ir.rs, lut.rs:374-435): gather
    a[s] = x[g^-s], length p-1 FFT, kernel multiply, inverse FFT, scatter to
    g^m plus x[0], and X[0] = x[0] + (the FFT's slot 0). With identity
    arithmetic both FFTs are the Stockham map of the plan's radices, so
    X[0] = x0 + a[P[0]] and X[g^m] = x0 + a[P[P[m]]]; random integer tags,
    bit for bit."""
    from oracle import oracle as orc
    batch, L = 3, p - 1
    rng = np.random.default_rng(p)
    x = (rng.integers(0, 1 << 18, p * batch) + 1j * rng.integers(0, 1 << 18, p * batch))
    x = x.astype(np.complex64 if prec == F32 else np.complex128)
    cfg = vk.FftConfig.new([p]).with_batch_count(batch).with_precision(prec)
    ir = vk.TransformIr.build(cfg, FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    assert [q["kernel"] for q in desc["passes"]] == ["rader_fft"], desc["passes"]
    g = orc.primitive_root(p)
    pw = np.array([pow(g, e, p) for e in range(L)])
    pin = pw[(L - np.arange(L)) % L]
    perm = im.stockham_perm(L, desc["passes"][0]["radices"])
    xb = x.reshape(batch, p).astype(np.complex128)
    a = xb[:, pin]
    f = a[:, perm]
    h = f[:, perm]
    expect = np.empty((batch, p), dtype=np.complex128)
    expect[:, 0] = xb[:, 0] + f[:, 0]
    expect[:, pw] = xb[:, :1] + h
    assert np.array_equal(out.reshape(batch, p), expect.astype(out.dtype))


@pytest.mark.parametrize("p", [47, 59, 83])
@pytest.mark.parametrize("prec", [F32, F64])
def test_rader_direct_addressing(idx_ctx, p, prec):
    """Direct-multiplication Rader of a prime p (rader_ir.rs:1957-2101): with
    identity arithmetic the kernel build convolves with the unit impulse and
    takes a[0] for the DC sum, so X[g^m] = x0 + x[g^-m] and X[0] = x0 + x[1]
    (the gather of a[s] = x[g^-s] and the scatter to g^m), bit for bit on
    random integer tags."""
    from oracle import oracle as orc
    batch = 4
    rng = np.random.default_rng(1000 + p)
    x = (rng.integers(0, 1 << 18, p * batch) + 1j * rng.integers(0, 1 << 18, p * batch))
    x = x.astype(np.complex64 if prec == F32 else np.complex128)
    ir = vk.TransformIr.build(vk.FftConfig.new([p]).with_batch_count(batch).with_precision(prec), FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    assert [q["kernel"] for q in desc["passes"]] == ["rader_direct"], desc["passes"]
    expect = im.rader_butterfly(x.reshape(batch, p).astype(np.complex128), p, orc.primitive_root(p), "impulse")
    assert np.array_equal(out.reshape(batch, p), expect.astype(out.dtype))


RADER_STAGE_LENGTHS = [17 * 4, 19 * 12, 2 * 29 * 31, 17 * 17 * 3, 47 * 4, 89 * 4, 97 * 8, 113 * 2, 257 * 4]


@pytest.mark.parametrize("n", RADER_STAGE_LENGTHS)
@pytest.mark.parametrize("prec", [F32, F64])
def test_rader_stage_addressing(idx_ctx, n, prec):
    """Rader stages inside a mixed-radix runtime radix list: the Stockham
    stage maps with identity butterflies, and at each prime radix the
    identity Rader butterfly (direct stages below 89: unit impulse; FFT-mode
    stages: the convolution's two identity Stockham maps of the plan's
    sub-radices), against oracle/index_maps.py bit for bit."""
    from oracle import oracle as orc
    batch = 3
    rng = np.random.default_rng(2000 + n)
    x = (rng.integers(0, 1 << 16, n * batch) + 1j * rng.integers(0, 1 << 16, n * batch))
    x = x.astype(np.complex64 if prec == F32 else np.complex128)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec), FWD)
    plan = vk.Plan(idx_ctx, ir)
    try:
        desc = plan.describe()
        out = idx_ctx.execute_transform(ir, x)
    finally:
        plan.close()
    assert len(desc["passes"]) == 1, desc["passes"]
    radices = desc["passes"][0]["radices"]
    fft_stages = {int(k): v for k, v in desc["rader_mixed"]["fft_convolution"].items()}
    rader = {r: (orc.primitive_root(r), im.stockham_perm(r - 1, fft_stages[r]) if r in fft_stages else None)
             for r in radices if r > 16}
    assert rader, radices
    expect = im.stockham_identity(x.reshape(batch, n).astype(np.complex128), radices, rader)
    assert np.array_equal(out.reshape(batch, n), expect.astype(out.dtype)), (n, radices)
