"""GPU parity: the HIP path (through the C ABI) against the CPU oracle
(restated src/reference.rs) on identical seeded inputs.

Tolerances: f32 relative L2 <= 1e-5 against the f64 oracle of the
same f32-rounded input; f64 <= 1e-13. Where the oracle's own algorithm is
less accurate than 1e-13 (reference::fft's Bluestein at large N), f64 is
checked against pocketfft at 1e-13 and against the oracle within its own
measured error. Config-scale shapes run on sampled batches against the
oracle plus size-independent properties (round trips, separability).
"""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse
TOL = {F32: 1e-5, F64: 1e-13}


def _cdtype(prec):
    return np.complex64 if prec == F32 else np.complex128


def c2c(ctx, dims, batch, x, prec=F32, direction=FWD, normalize=False):
    cfg = vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec) \
        .with_inverse_normalization(normalize)
    ir = vk.TransformIr.build(cfg, direction)
    return ctx.execute_transform(ir, x), ir


def oracle_c2c(x, n, direction=FWD, normalize=False):
    return o.fft_batch(x.astype(np.complex128), n, "forward" if direction == FWD else "inverse",
                       normalize, threads=8)


def rand(count, seed, prec=F32):
    return o.complex_uniform(count, seed, _cdtype(prec))


# ------------------------------------------------ reference HIP unit tests

def test_hip_stockham_matches_cpu_n64(hip_ctx):
    # hip/runtime.rs:3451-3490: N=64 vs reference::dft, max error < 2e-3 * N
    x = rand(64, 1)
    y, _ = c2c(hip_ctx, [64], 1, x)
    assert np.max(np.abs(y - o.dft(x))) < 2e-3 * 64


def test_hip_round_trip_n4096_batch8(hip_ctx):
    # hip/runtime.rs:3172-3218: N4096 x 8 round trip <= 2e-4
    x = rand(4096 * 8, 2)
    y, _ = c2c(hip_ctx, [4096], 8, x)
    z, _ = c2c(hip_ctx, [4096], 8, y, direction=INV, normalize=True)
    assert np.max(np.abs(z - x)) <= 2e-4


# ------------------------------------------------------- 1-D C2C sweep

SMALL = list(range(1, 65)) + [96, 100, 121, 125, 128, 169, 192, 243, 343, 360, 512, 625, 1000, 1024, 1536,
                             2048, 2187, 2401, 3125, 4096, 6561, 8192, 10000, 15625, 16384,
                             # fixed 3*2^k / 5*2^k family lengths
                             80, 160, 320, 384, 640, 768, 1280, 2560, 3072, 5120, 6144, 10240, 12288]


@pytest.mark.parametrize("prec", [F32, F64])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_c2c_length_sweep(hip_ctx, prec, direction):
    worst = {}
    for n in SMALL:
        batch = 3
        x = rand(n * batch, n, prec)
        y, _ = c2c(hip_ctx, [n], batch, x, prec, direction, normalize=direction == INV)
        ref = oracle_c2c(x, n, direction, direction == INV)
        err = o.rel_l2(y, ref)
        if prec == F64 and err > TOL[F64]:
            # reference::fft's own Bluestein error can exceed 1e-13: pin to pocketfft
            npref = (np.fft.fft if direction == FWD else np.fft.ifft)(x.reshape(batch, n), axis=1).reshape(-1)
            err = o.rel_l2(y, npref)
        worst[n] = err
    bad = {n: e for n, e in worst.items() if e > TOL[prec]}
    assert not bad, bad


@pytest.mark.parametrize("prec", [F32, F64])
def test_runtime_kernels_on_registered_lengths(hip_ctx, monkeypatch, prec):
    """VKFX_DISABLE_FIXED=1: lengths that normally run fixed shapes go through
    the runtime-shape kernels (rows, columns, split axes), against the oracle,
    so the runtime path stays covered as the fixed families grow."""
    monkeypatch.setenv("VKFX_DISABLE_FIXED", "1")
    ctx = vk.HipExecutionContext(0)
    try:
        for n in (8, 12, 30, 100, 720, 1000, 1024, 2000, 4096):
            x = rand(n * 5, n, prec)
            y, ir = c2c(ctx, [n], 5, x, prec)
            assert not any(p.get("fixed_shape") for p in ctx.plan(ir).describe()["passes"]), n
            assert o.rel_l2(y, oracle_c2c(x, n)) <= TOL[prec], (n, prec)
        for dims in ([120, 30], [1000, 6], [25, 12, 8]):
            count = int(np.prod(dims))
            x = rand(count * 2, count, prec)
            y, ir = c2c(ctx, dims, 2, x, prec)
            assert not any(p.get("fixed_shape") for p in ctx.plan(ir).describe()["passes"]), dims
            assert o.rel_l2(y, o.fft_nd(x, dims, 2, threads=8)) <= TOL[prec], (dims, prec)
    finally:
        ctx.close()


@pytest.mark.parametrize("prec", [F32, F64])
def test_many_lines_per_block(hip_ctx, prec):
    """Short lengths at batch 70 and 133: blocks of up to 64 lines, partial
    last blocks, every line checked (the line placement of the cooperative
    copies and of each thread's butterflies), against pocketfft."""
    bad = {}
    for n in list(range(2, 70)) + [96, 100, 120, 125, 128, 130]:
        for batch in (70, 133):
            x = rand(n * batch, 7 * n + batch, prec)
            y, _ = c2c(hip_ctx, [n], batch, x, prec)
            ref = np.fft.fft(x.reshape(batch, n).astype(np.complex128), axis=1)
            lines = np.linalg.norm(y.reshape(batch, n) - ref, axis=1) / np.linalg.norm(ref, axis=1)
            if lines.max() > 4 * TOL[prec]:
                bad[(n, batch)] = np.nonzero(lines > 4 * TOL[prec])[0][:8].tolist()
    assert not bad, bad


@pytest.mark.parametrize("prec", [F32, F64])
def test_c1_shape_sampled_full_size(hip_ctx, prec):
    """C1: N=1024, batch 8192; every 97th transform against the oracle, all
    of them through a forward/inverse round trip."""
    n, batch = 1024, 8192
    x = rand(n * batch, 101, prec)
    y, ir = c2c(hip_ctx, [n], batch, x, prec)
    assert hip_ctx.plan(ir).describe()["axes"][0]["algorithm"] == "stockham"
    idx = np.arange(0, batch, 97)
    xs = x.reshape(batch, n)[idx].reshape(-1)
    assert o.rel_l2(y.reshape(batch, n)[idx].reshape(-1), oracle_c2c(xs, n)) <= TOL[prec]
    z, _ = c2c(hip_ctx, [n], batch, y, prec, INV, normalize=True)
    assert o.rel_l2(z, x) <= 4 * TOL[prec]


@pytest.mark.parametrize("n", [1 << 15, 3 * (1 << 14), 1 << 17, 1 << 20])
def test_c2c_four_step(hip_ctx, n):
    x = rand(n * 2, n)
    y, ir = c2c(hip_ctx, [n], 2, x)
    assert "four_step" in hip_ctx.plan(ir).describe()
    assert o.rel_l2(y, oracle_c2c(x, n)) <= TOL[F32]
    z, _ = c2c(hip_ctx, [n], 2, y, direction=INV, normalize=True)
    assert o.rel_l2(z, x) <= 2 * TOL[F32]


@pytest.mark.parametrize("n", [1 << 16, 60000, 100000, 250000, 1000000, 1 << 22, 4000000])
@pytest.mark.parametrize("prec", [F32, F64])
def test_c2c_four_step_round_factors(hip_ctx, n, prec):
    """Two-upload four-step over the factors of kf_round_fs_* (fixed column
    and row passes, both directions), against pocketfft in f64."""
    batch = 2
    x = rand(n * batch, n % 1009, prec)
    y, ir = c2c(hip_ctx, [n], batch, x, prec)
    passes = hip_ctx.plan(ir).describe()["passes"]
    assert [p["kernel"] for p in passes[:2]] == ["four_step_columns", "four_step_rows"], passes[:2]
    assert all(p["fixed_shape"] for p in passes), [(p["kernel"], p["fft_len"]) for p in passes]
    ref = np.fft.fft(x.reshape(batch, n).astype(np.complex128), axis=1).reshape(-1)
    assert o.rel_l2(y, ref) <= TOL[prec]
    z, ir2 = c2c(hip_ctx, [n], batch, y, prec, INV, normalize=True)
    assert all(p["fixed_shape"] for p in hip_ctx.plan(ir2).describe()["passes"])
    assert o.rel_l2(z, x) <= 4 * TOL[prec]


def test_c2c_four_step_f64(hip_ctx):
    n = 1 << 14
    x = rand(n * 2, 7, F64)
    y, _ = c2c(hip_ctx, [n], 2, x, F64)
    assert o.rel_l2(y, oracle_c2c(x, n)) <= TOL[F64]


# ----------------------------------------------------------- Bluestein

@pytest.mark.parametrize("n,batch", [(4099, 8), (65537, 2), (103, 5), (17, 4), (257, 3), (1031, 2)])
def test_bluestein_and_rader_classified_f32(hip_ctx, n, batch):
    x = rand(n * batch, n)
    y, ir = c2c(hip_ctx, [n], batch, x)
    assert ir.axis_algorithms[0] in (vk.AlgorithmKind.Bluestein, vk.AlgorithmKind.Rader)
    assert o.rel_l2(y, oracle_c2c(x, n)) <= TOL[F32]
    z, _ = c2c(hip_ctx, [n], batch, x, direction=INV, normalize=True)
    assert o.rel_l2(z, oracle_c2c(x, n, INV, True)) <= TOL[F32]


def _assert_f64_gate(prec, x, n, batch, y, z):
    """The f64 gate itself (relative L2 <= 1e-13) against pocketfft, forward
    and normalized inverse: the oracle's own f64 Rader/Bluestein error can
    approach 1e-12 for these lengths, so the comparison with the oracle above
    alone would let a GPU error of that size through."""
    if prec != F64:
        return
    xs = x.reshape(batch, n).astype(np.complex128)
    assert o.rel_l2(y, np.fft.fft(xs, axis=1).reshape(-1)) <= TOL[F64]
    assert o.rel_l2(z, np.fft.ifft(xs, axis=1).reshape(-1)) <= TOL[F64]


@pytest.mark.parametrize("n,mode", [(17, "fft"), (97, "fft"), (257, "fft"), (89, "fft"), (12289, "fft"),
                                    (47, "direct"), (59, "direct"), (83, "direct")])
@pytest.mark.parametrize("prec", [F32, F64])
def test_rader(hip_ctx, n, mode, prec):
    """Rader-classified primes execute as Rader (FFT convolution when p-1 is
    Stockham-smooth, direct multiplication below 89), rader_ir.rs:1957-2101."""
    if prec == F64 and n == 12289:
        pytest.skip("F64 LDS capacity (10240 elements) makes the planner pick Bluestein for 12289")
    batch = 3
    x = rand(n * batch, n + 7, prec)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec), FWD)
    assert ir.axis_algorithms == [vk.AlgorithmKind.Rader]
    desc = hip_ctx.plan(ir).describe()
    assert desc["rader"]["mode"] == mode and desc["rader"]["prime"] == n
    y = hip_ctx.execute_transform(ir, x)
    ref = oracle_c2c(x, n)
    tol = TOL[prec] if prec == F32 else max(TOL[F64], 2 * o.rel_l2(ref, np.fft.fft(x.reshape(batch, n), axis=1).reshape(-1)))
    assert o.rel_l2(y, ref) <= tol
    z, _ = c2c(hip_ctx, [n], batch, x, prec, INV, normalize=True)
    assert o.rel_l2(z, oracle_c2c(x, n, INV, True)) <= tol
    _assert_f64_gate(prec, x, n, batch, y, z)


@pytest.mark.parametrize("prec", [F32, F64])
def test_rader_recursive_opt_in_runs_the_rader_tree(hip_ctx, prec):
    """PlannerTuning::with_recursive_fft_rader (planner.rs:414-422): 4099 is a
    Rader prime whose convolution length 4098 = 2 * 3 * 683 has the Rader
    prime 683 (rader_ir.rs:706-745, 1957-2101). The FFT-mode Rader kernel
    runs its length-4098 FFTs with 683 as a Rader stage."""
    n, batch = 4099, 3
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
    cfg.allow_recursive_fft_rader = True
    ir = vk.TransformIr.build(cfg, FWD)
    assert ir.axis_algorithms == [vk.AlgorithmKind.Rader]
    desc = hip_ctx.plan(ir).describe()
    assert "rader_fallback" not in desc
    assert desc["rader"]["mode"] == "fft" and desc["rader"]["convolution_len"] == 4098
    assert desc["rader"]["nested_rader_primes"] == [683]
    # 683 -> 682 = 2 * 11 * 31 convolves by FFT, 31 by direct multiplication
    assert desc["rader"]["nested"]["fft_convolution"] == {"683": RADER_FFT_STAGES[683]}
    x = rand(n * batch, 3, prec)
    ref = oracle_c2c(x, n)
    tol = TOL[F32] if prec == F32 else max(TOL[F64], 2 * o.rel_l2(ref, np.fft.fft(x.reshape(batch, n), axis=1)
                                                                  .reshape(-1)))
    y = hip_ctx.execute_transform(ir, x)
    assert o.rel_l2(y, ref) <= tol
    cfg_i = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(True)
    cfg_i.allow_recursive_fft_rader = True
    ir_i = vk.TransformIr.build(cfg_i, INV)
    z = hip_ctx.execute_transform(ir_i, x)
    assert o.rel_l2(z, oracle_c2c(x, n, INV, True)) <= tol
    _assert_f64_gate(prec, x, n, batch, y, z)


# composite lengths whose prime factors above 13 are Rader primes: the
# reference folds Rader into the mixed-radix tree (mixed_ir.rs); here each
# such factor is a Rader stage of the Stockham sequence
RADER_MIXED = [(17 * 64, [17]), (19 * 12, [19]), (23 * 5, [23]), (17 * 19, [17, 19]), (2 * 29 * 31, [29, 31]),
               (47 * 4, [47]), (97 * 8, [97]), (17 * 17 * 3, [17, 17]), (89 * 4, [89]), (113 * 2, [113]),
               (193 * 2, [193]), (257 * 4, [257])]
# Rader stages from 89 on convolve by FFT (the reference's FFT-Rader node):
# the plan reports the sub-radices of each such stage's length p - 1 FFTs
RADER_FFT_STAGES = {89: [8, 11], 97: [8, 4, 3], 113: [16, 7], 193: [8, 8, 3], 257: [16, 16], 683: [2, 11, 31]}


@pytest.mark.parametrize("n,primes", RADER_MIXED)
@pytest.mark.parametrize("prec", [F32, F64])
def test_rader_inside_mixed_radix(hip_ctx, n, primes, prec):
    batch = 5
    x = rand(n * batch, n + 11, prec)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec), FWD)
    assert ir.axis_algorithms == [vk.AlgorithmKind.Rader]
    desc = hip_ctx.plan(ir).describe()
    assert "rader_fallback" not in desc, desc
    assert desc["rader_mixed"]["rader_primes"] == primes
    fft_stages = {int(k): v for k, v in desc["rader_mixed"]["fft_convolution"].items()}
    assert fft_stages == {p: RADER_FFT_STAGES[p] for p in primes if p >= 89}, fft_stages
    ref = oracle_c2c(x, n)
    npref = np.fft.fft(x.reshape(batch, n).astype(np.complex128), axis=1).reshape(-1)
    tol = TOL[prec] if prec == F32 else max(TOL[F64], 2 * o.rel_l2(ref, npref))
    y = hip_ctx.execute_transform(ir, x)
    assert o.rel_l2(y, ref) <= tol
    z, _ = c2c(hip_ctx, [n], batch, x, prec, INV, normalize=True)
    assert o.rel_l2(z, oracle_c2c(x, n, INV, True)) <= tol
    _assert_f64_gate(prec, x, n, batch, y, z)


@pytest.mark.parametrize("dims", [[8, 17 * 16], [17 * 4, 32], [3, 19 * 4, 5]])
def test_rader_inside_mixed_radix_nd(hip_ctx, dims):
    """Composite Rader axes of N-D transforms, contiguous and strided."""
    batch = 2
    total = int(np.prod(dims)) * batch
    x = rand(total, 77)
    ir = vk.TransformIr.build(vk.FftConfig.new(dims).with_batch_count(batch), FWD)
    assert vk.AlgorithmKind.Rader in ir.axis_algorithms
    desc = hip_ctx.plan(ir).describe()
    assert "rader_mixed" in desc and "rader_fallback" not in desc, desc
    y = hip_ctx.execute_transform(ir, x)
    assert o.rel_l2(y, o.fft_nd(x, dims, batch, threads=8)) <= TOL[F32]


def test_bluestein_plan_uses_planner_length(hip_ctx):
    for n, m in [(4099, 8232), (65537, 131220)]:
        ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(4096), FWD)
        assert ir.convolution_lens == [m]
        plan_small = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(2), FWD)
        desc = hip_ctx.plan(plan_small).describe()
        assert desc["axes"][0]["algorithm"] == "bluestein"


@pytest.mark.parametrize("n", [4099, 65537])
def test_bluestein_f64(hip_ctx, n):
    x = rand(n * 2, n + 1, F64)
    y, _ = c2c(hip_ctx, [n], 2, x, F64)
    npref = np.fft.fft(x.reshape(2, n), axis=1).reshape(-1)
    assert o.rel_l2(y, npref) <= 1e-13
    ref = oracle_c2c(x, n)
    assert o.rel_l2(y, ref) <= max(1e-13, 2 * o.rel_l2(ref, npref))


# A prime per convolution length M of the one-kernel Bluestein rows
# (kf_blue_rows_*): the planner's padding tables give that M for the prime.
BLUE_PRIMES = {F32: {103: 256, 137: 512, 263: 625, 317: 768, 389: 1024, 523: 1296, 653: 2048, 1031: 2187,
                     1097: 2304, 1163: 2500, 1259: 2592, 1303: 3072, 1543: 3125, 1567: 3136, 1571: 4096,
                     2053: 4375, 2203: 4608, 2309: 5184, 2609: 6561, 3299: 8192, 6131: 16384},
               F64: {239: 512, 311: 625, 317: 640, 373: 750, 383: 768, 431: 875, 509: 1024, 647: 1296, 659: 1323,
                     743: 1512, 887: 1792, 997: 2016, 1021: 2048, 1091: 2187, 1567: 3136, 1709: 3430, 1789: 3584,
                     2039: 4096, 2153: 4375, 2239: 4480, 2351: 4704, 2551: 5103, 2687: 5376, 3023: 6048,
                     3067: 6144, 4093: 8192}}


@pytest.mark.parametrize("prec", [F32, F64])
def test_bluestein_fixed_rows(hip_ctx, prec):
    """Primes whose Bluestein convolution length has a fixed one-kernel row
    shape run on it (bluestein_ir.rs's single-upload path), forward and
    inverse. f32 against the oracle; f64 against pocketfft at 1e-13 and against
    the oracle within twice the oracle's own distance from pocketfft."""
    for n, m in BLUE_PRIMES[prec].items():
        batch = 3
        x = rand(n * batch, n + 11, prec)
        y, ir = c2c(hip_ctx, [n], batch, x, prec)
        desc = hip_ctx.plan(ir).describe()
        assert desc["bluestein"]["m"] == m, (n, desc["bluestein"])
        assert desc["passes"][0]["kernel"] == "bluestein_single" and desc["passes"][0]["fixed_shape"], n
        ref = oracle_c2c(x, n)
        if prec == F32:
            assert o.rel_l2(y, ref) <= TOL[F32], n
        else:
            npref = np.fft.fft(x.reshape(batch, n), axis=1).reshape(-1)
            assert o.rel_l2(y, npref) <= 1e-13, n
            assert o.rel_l2(y, ref) <= max(1e-13, 2 * o.rel_l2(ref, npref)), n
        z, iir = c2c(hip_ctx, [n], batch, y, prec, INV, normalize=True)
        idesc = hip_ctx.plan(iir).describe()
        assert idesc["passes"][0]["kernel"] == "bluestein_single" and idesc["passes"][0]["fixed_shape"], n
        assert o.rel_l2(z, x) <= 4 * TOL[prec], n


# -------------------------------------------------------------- R2C / C2R

def r2c(ctx, n, batch, x, prec=F32):
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.RealToComplex)
    ir = vk.TransformIr.build(cfg, FWD)
    return ctx.execute_transform(ir, x), ir


def c2r(ctx, n, batch, X, prec=F32, normalize=True):
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(normalize)
    ir = vk.TransformIr.build(cfg, INV)
    return ctx.execute_transform(ir, X), ir


@pytest.mark.parametrize("n", [2, 4, 8, 10, 45, 64, 105, 1000, 4096, 32768, 1 << 16, 1 << 20])
@pytest.mark.parametrize("prec", [F32, F64])
def test_r2c_c2r(hip_ctx, n, prec):
    if prec == F64 and n > 1 << 16:
        pytest.skip("f64 four-step real path is covered at 2^16")
    batch = 2
    rdt = np.float32 if prec == F32 else np.float64
    x = o.normal(n * batch, n, rdt)
    X, _ = r2c(hip_ctx, n, batch, x, prec)
    ref = o.r2c_batch(x.astype(np.float64), n, threads=8)
    assert o.rel_l2(X, ref) <= TOL[prec] * (1 if prec == F32 else 10)
    # C2R of the exact spectrum against the oracle's C2R
    xr, _ = c2r(hip_ctx, n, batch, ref.astype(_cdtype(prec)), prec)
    back = o.c2r_batch(ref, n, normalize=True, threads=8)
    assert o.rel_l2(xr, back) <= TOL[prec] * (1 if prec == F32 else 10)


@pytest.mark.parametrize("n", [6, 18, 22, 26, 196, 210, 686, 1078, 2002, 5880, 9000, 18018])
@pytest.mark.parametrize("prec", [F32, F64])
def test_r2c_c2r_runtime_lengths(hip_ctx, n, prec):
    """Even lengths without a registered shape (runtime-radix kernels whose
    first R2C stage loads, and last C2R stage stores, HBM directly), over a
    batch that leaves the last block of lines partly empty."""
    batch = 37
    rdt = np.float32 if prec == F32 else np.float64
    x = o.normal(n * batch, 4000 + n, rdt)
    X, _ = r2c(hip_ctx, n, batch, x, prec)
    ref = o.r2c_batch(x.astype(np.float64), n, threads=8)
    assert o.rel_l2(X, ref) <= TOL[prec] * (1 if prec == F32 else 10)
    xr, _ = c2r(hip_ctx, n, batch, ref.astype(_cdtype(prec)), prec)
    back = o.c2r_batch(ref, n, normalize=True, threads=8)
    assert o.rel_l2(xr, back) <= TOL[prec] * (1 if prec == F32 else 10)
    # unnormalized C2R of the R2C output returns n * x
    xu, _ = c2r(hip_ctx, n, batch, X, prec, normalize=False)
    assert o.rel_l2(xu, n * x.astype(np.float64)) <= TOL[prec] * (1 if prec == F32 else 10)


def test_c2r_runtime_variants_covered(hip_ctx):
    """The host rule for the runtime-shape C2R half-length kernels: HBM-direct
    last stage always; the first stage forms the preprocess from HBM whenever
    its loads span 128 bytes or more (any first radix but 2, both precisions;
    n=210 has radix 3 first), else the staged preprocess (f64 n=6, 18: one
    stage or a short span). n=18018 (M=9009) needs the wide geometry. Each case
    named here also runs in test_r2c_c2r_runtime_lengths."""
    def c2r_launch(n, prec):
        cfg = vk.FftConfig.new([n]).with_batch_count(37).with_precision(prec) \
            .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True)
        plan = hip_ctx.plan(vk.TransformIr.build(cfg, INV))
        ls = [L for L in plan.describe()["passes"] if "runtime_variant" in L and not L["fixed_shape"]]
        assert len(ls) == 1, plan.describe()
        return ls[0]
    for prec in (F32, F64):
        L = c2r_launch(210, prec)
        assert L["radices"][0] == 3 and L["runtime_variant"]["hbm_direct"]
        assert L["runtime_variant"]["direct_preprocess"]
    L = c2r_launch(18018, F32)
    assert L["runtime_variant"]["wide"] and L["runtime_variant"]["hbm_direct"]
    assert L["runtime_variant"]["direct_preprocess"]
    L = c2r_launch(2800, F32)
    assert L["radices"][0] == 8 and L["runtime_variant"]["direct_preprocess"]
    for n in (6, 18):
        L = c2r_launch(n, F64)
        assert L["runtime_variant"]["hbm_direct"] and not L["runtime_variant"]["direct_preprocess"]


HALF_FIXED = {F32: [256, 384, 512, 640, 768, 1024, 1280, 1536, 2048, 2560, 3072, 4096, 5120, 6144, 8192, 320,
                   # round half lengths and 10^k / 360 (kf_round_real_*)
                   200, 360, 500, 750, 1000, 1200, 1500, 2400, 3000, 5000, 8000, 10000, 16000],
              F64: [64, 128, 160, 192, 256, 320, 384, 512, 640, 768, 1024, 1280, 1536, 2048, 2560, 3072, 4096,
                    240, 360, 600, 1000, 1800, 3000, 4800, 8000]}


ROUND = [200, 240, 300, 400, 480, 500, 600, 720, 750, 800, 900, 960, 1200, 1500, 1600, 1800, 1920, 2000, 2400,
         2500, 3000, 3200, 3600, 4000, 4800, 5000, 6000, 6400, 7200, 8000, 9000, 9600, 12000, 16000]


@pytest.mark.parametrize("prec", [F32, F64])
def test_round_length_fixed_rows(hip_ctx, prec):
    """The round lengths with factors 2, 3 and 5 (kf_round_*) run on their
    fixed row shapes, forward and inverse, against the oracle."""
    for n in ROUND:
        if prec == F64 and n > 8192:
            continue  # longer f64 lines are two uploads
        batch = 3
        x = rand(n * batch, n, prec)
        y, ir = c2c(hip_ctx, [n], batch, x, prec)
        assert hip_ctx.plan(ir).describe()["passes"][0]["fixed_shape"], n
        assert o.rel_l2(y, oracle_c2c(x, n)) <= TOL[prec], (n, prec)
        z, _ = c2c(hip_ctx, [n], batch, y, prec, INV, normalize=True)
        assert o.rel_l2(z, x) <= 4 * TOL[prec], (n, prec)


def _lines_against_pocketfft(y, x, n, batch, direction, tol):
    """Indices of the lines of y whose relative L2 error against numpy's FFT of
    the same line exceeds tol (normalized inverse for direction INV)."""
    xs = x.reshape(batch, n).astype(np.complex128)
    ref = np.fft.fft(xs, axis=1) if direction == FWD else np.fft.ifft(xs, axis=1)
    err = np.linalg.norm(y.reshape(batch, n) - ref, axis=1) / np.linalg.norm(ref, axis=1)
    return np.nonzero(err > tol)[0][:8].tolist()


@pytest.mark.parametrize("prec", [F32, F64])
def test_fixed_rows_several_blocks(hip_ctx, prec):
    """Round-length and Bluestein fixed row shapes at a batch of 3*G + 1 lines
    (G = the shape's lines per block): three full blocks and a partial one, so
    the line placement of the second and later blocks and of the partial block
    runs on each shape's own length. Every line, forward and normalized inverse,
    against pocketfft."""
    round_sample = [200, 240, 480, 600, 720, 1200, 2000, 3000, 5000, 8000, 16000]
    blue = BLUE_PRIMES[prec]
    blue_sample = [p for i, p in enumerate(sorted(blue)) if i % 3 == 0]
    tol = 4 * TOL[prec]
    bad, seen_g = {}, set()
    for n in round_sample + blue_sample:
        if prec == F64 and n in ROUND and n > 8192:
            continue  # longer f64 lines are two uploads
        probe = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(1).with_precision(prec), FWD)
        first = hip_ctx.plan(probe).describe()["passes"][0]
        assert first["fixed_shape"], n
        g = int(first["lines_per_block"])
        seen_g.add(g)
        batch = 3 * g + 1
        x = rand(n * batch, 3 * n + g, prec)
        for direction in (FWD, INV):
            y, ir = c2c(hip_ctx, [n], batch, x, prec, direction, normalize=True)
            p0 = hip_ctx.plan(ir).describe()["passes"][0]
            assert p0["fixed_shape"] and p0["lines_per_block"] == g, (n, direction, p0)
            assert p0["grid"] >= 4, (n, p0["grid"])
            lines = _lines_against_pocketfft(y, x, n, batch, direction, tol)
            if lines:
                bad[(n, direction)] = lines
    assert not bad, bad
    assert max(seen_g) >= 4, seen_g  # the sample holds multi-line blocks


@pytest.mark.parametrize("prec", [F32, F64])
def test_r2c_c2r_fixed_half_lengths(hip_ctx, prec):
    """Even lengths whose half-size FFT has a fixed shape, at batch 37 (several
    lines per block, a partial last block), every line against pocketfft."""
    rdt = np.float32 if prec == F32 else np.float64
    cdt = _cdtype(prec)
    bad = {}
    for m in HALF_FIXED[prec]:
        n, batch = 2 * m, 37
        x = o.normal(n * batch, m, rdt).reshape(batch, n)
        X, ir = r2c(hip_ctx, n, batch, x.reshape(-1), prec)
        assert hip_ctx.plan(ir).describe()["passes"][0]["fixed_shape"], n
        ref = np.fft.rfft(x.astype(np.float64), axis=1)
        e1 = o.rel_l2(X, ref.reshape(-1))
        xr, _ = c2r(hip_ctx, n, batch, ref.astype(cdt).reshape(-1), prec)
        e2 = o.rel_l2(xr, x.astype(np.float64).reshape(-1))
        if max(e1, e2) > TOL[prec] * (1 if prec == F32 else 10):
            bad[n] = (e1, e2)
    assert not bad, bad


def test_c2_shape_round_trip_full_size(hip_ctx):
    """C2: R2C N=2^20 batch 256 then C2R with normalization; two sampled
    transforms against the oracle, the whole batch through the round trip."""
    n, batch = 1 << 20, 256
    x = o.normal(n * batch, 2024, np.float32)
    X, ir = r2c(hip_ctx, n, batch, x)
    desc = hip_ctx.plan(ir).describe()
    assert desc["real"]["uploads"] == 2
    h = n // 2 + 1
    for b in (0, 255):
        ref = o.r2c_batch(x[b * n:(b + 1) * n].astype(np.float64), n)
        assert o.rel_l2(X[b * h:(b + 1) * h], ref) <= TOL[F32]
    xr, _ = c2r(hip_ctx, n, batch, X)
    assert o.rel_l2(xr, x) <= 2 * TOL[F32]
    # the full-size C2R itself on sampled lines: the oracle's C2R of the same
    # (f32) spectrum the GPU consumed
    for b in (0, 131, 255):
        back = o.c2r_batch(X[b * h:(b + 1) * h].astype(np.complex128), n, normalize=True)
        assert o.rel_l2(xr[b * n:(b + 1) * n], back) <= TOL[F32]


# ------------------------------------------------------------------ N-D

@pytest.mark.parametrize("dims,batch,prec", [([64, 48], 2, F32), ([256, 256], 2, F32), ([17, 34], 1, F32),
                                             ([16, 12, 10], 2, F64), ([64, 64, 64], 1, F64),
                                             ([8, 6, 5, 4], 1, F32), ([4099, 4], 1, F32),
                                             # strided axes long enough to run as two split passes
                                             ([1024, 8], 2, F32), ([2048, 3], 1, F32), ([1000, 6], 1, F64),
                                             ([3, 768, 5], 2, F32),
                                             # Rader axes inside N-D transforms (contiguous and strided)
                                             ([8, 17], 2, F32), ([47, 8], 1, F32), ([97, 6], 1, F64),
                                             # round-length rows, columns and split passes (kf_round_*)
                                             ([120, 120, 12], 1, F32), ([720, 30], 1, F32), ([1000, 40], 1, F64),
                                             ([2000, 6], 1, F32), ([75, 45, 27], 1, F64), ([6, 10, 9, 15], 2, F32),
                                             ([625, 18], 1, F32), ([4800, 3], 1, F64)])
def test_nd_c2c(hip_ctx, dims, batch, prec):
    count = int(np.prod(dims)) * batch
    x = rand(count, count % 1000, prec)
    y, _ = c2c(hip_ctx, dims, batch, x, prec)
    ref = o.fft_nd(x, dims, batch, threads=8)
    assert o.rel_l2(y, ref) <= TOL[prec]
    z, _ = c2c(hip_ctx, dims, batch, y, prec, INV, normalize=True)
    assert o.rel_l2(z, x) <= 4 * TOL[prec]


@pytest.mark.parametrize("dims,batch,prec", [([64, 64, 64], 1, F64), ([8, 4096, 8], 1, F32),
                                             ([32, 64, 48], 2, F64), ([6, 20, 64, 40], 2, F32)])
def test_nd_slab_chunks(hip_ctx, monkeypatch, dims, batch, prec):
    """Volumes above the chunk budget run axes 1.. slab chunk by slab chunk
    (ragged last chunk, split strided middle axis, several batches), then
    axis 0 over the whole volume."""
    monkeypatch.setenv("VKFX_ND_CHUNK_MB", "1")
    ctx = vk.HipExecutionContext(0)  # own plan cache: plans read the budget when built
    try:
        count = int(np.prod(dims)) * batch
        x = rand(count, count % 997, prec)
        y, ir = c2c(ctx, dims, batch, x, prec)
        desc = ctx.plan(ir).describe()
        assert desc["nd"]["slabs_per_chunk"] > 0
        assert desc["lanes"] == 1
        ref = o.fft_nd(x, dims, batch, threads=8)
        assert o.rel_l2(y, ref) <= TOL[prec]
    finally:
        ctx.close()


def test_c3_shape_full_size(hip_ctx):
    """C3: 4096 x 4096, batch 16, f32. Image 0 against the f64 oracle on a
    sample of rows of the row pass is too slow, so image 0 is checked against
    pocketfft (f64) and every image through a round trip."""
    dims, batch = [4096, 4096], 16
    x = rand(4096 * 4096 * batch, 33)
    y, _ = c2c(hip_ctx, dims, batch, x)
    ref0 = np.fft.fft2(x[: 4096 * 4096].reshape(4096, 4096).astype(np.complex128))
    assert o.rel_l2(y[: 4096 * 4096], ref0.reshape(-1)) <= TOL[F32]
    z, _ = c2c(hip_ctx, dims, batch, y, direction=INV, normalize=True)
    assert o.rel_l2(z, x) <= 4 * TOL[F32]


def test_c4_shape_full_size_f64(hip_ctx):
    """C4: 512^3 f64 (2 GiB). Checked against pocketfft at 1e-13."""
    dims = [512, 512, 512]
    x = rand(512 ** 3, 44, F64)
    y, _ = c2c(hip_ctx, dims, 1, x, F64)
    ref = np.fft.fftn(x.reshape(dims))
    assert o.rel_l2(y, ref.reshape(-1)) <= TOL[F64]


def test_c5_shape_sampled_full_size(hip_ctx):
    """C5: N=4099 and N=65537 at batch 4096; sampled transforms against the oracle."""
    for n, seed in [(4099, 5), (65537, 6)]:
        batch = 4096
        x = rand(n * batch, seed)
        y, _ = c2c(hip_ctx, [n], batch, x)
        for b in (0, 1, 2047, 4095):
            ref = o.fft(x[b * n:(b + 1) * n].astype(np.complex128))
            assert o.rel_l2(y[b * n:(b + 1) * n], ref) <= TOL[F32], (n, b)


# ----------------------------------------------------- FFTW golden (GPU)

@pytest.mark.parametrize("case", ["c2c-bluestein-n103", "c2c-rader-n257", "c2c-smooth-n1536",
                                  "c2c-large-smooth-n4096"])
def test_fftw_medium_f32_on_gpu(hip_ctx, case):
    # tests/fftw_medium_f32_golden.rs:162-172: F32 GPU tolerance 1e-4 * N max-abs
    import os
    from conftest import GOLDEN
    c = o.parse_fixture(os.path.join(GOLDEN, "fftw_precision_medium_f32_v1.txt"))["cases"][case]
    n = int(c["meta"]["shape"])
    x = o.fixture_input("complex-f32-v1", n)
    rows = np.array(c["rows"])
    expected = rows[:, 0] + 1j * rows[:, 1]
    y, _ = c2c(hip_ctx, [n], 1, x)
    assert np.max(np.abs(y - expected)) <= 1e-4 * n
    assert o.rel_l2(y, expected) <= TOL[F32]


# ------------------------------------------------------------ contracts

def test_input_length_mismatch(hip_ctx):
    ir = vk.TransformIr.build(vk.FftConfig.new([64]).with_batch_count(2), FWD)
    with pytest.raises(vk.VkFftError) as e:
        hip_ctx.execute_transform(ir, np.zeros(100, np.complex64))
    assert e.value.kind == "InputLengthMismatch"


def test_device_profile(hip_ctx):
    p = hip_ctx.device_profile()
    assert p["arch"].startswith("gfx950") and p["warp_size"] == 64
    assert p["shared_memory_bytes"] >= 64 * 1024


def test_device_resident_execute_matches_host(hip_ctx):
    import torch
    n, batch = 1024, 64
    x = rand(n * batch, 77)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch), FWD)
    plan = hip_ctx.plan(ir)
    xt = torch.from_numpy(x.view(np.float32).copy()).cuda()
    yt = torch.empty_like(xt)
    plan.execute_tensors(xt, yt)
    hip_ctx.synchronize()
    y_dev = yt.cpu().numpy().view(np.complex64)
    assert np.array_equal(y_dev, hip_ctx.execute_transform(ir, x))
    # in place (d_in == d_out) gives the same result
    plan.execute_tensors(xt, xt)
    hip_ctx.synchronize()
    assert np.array_equal(xt.cpu().numpy().view(np.complex64), y_dev)


@pytest.mark.parametrize("n,prec", [(206, F64), (578, F32), (323, F32), (1009, F64), (131074, F32), (17, F32)])
def test_real_full_complex_lengths(hip_ctx, n, prec):
    """Real lengths whose half-size (even) or own (odd) FFT has no Stockham
    geometry run as a full-length C2C (real_ir.rs:935-946, 1038-1053)."""
    batch = 3
    rd = np.float32 if prec == F32 else np.float64
    x = o.normal(n * batch, n, rd)
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec)
    r2c = vk.TransformIr.build(cfg.with_transform(vk.TransformKind.RealToComplex), FWD)
    X = hip_ctx.execute_transform(r2c, x)
    h = n // 2 + 1
    ref = np.concatenate([o.r2c_batch(x[b * n:(b + 1) * n].astype(np.float64), n) for b in range(batch)])
    assert X.size == h * batch
    err = o.rel_l2(X, ref)
    if prec == F64 and err > TOL[F64]:
        # reference::fft's Bluestein for large primes is itself less accurate
        # than 1e-13: pin to pocketfft
        err = o.rel_l2(X, np.fft.rfft(x.reshape(batch, n), axis=1).reshape(-1))
    assert err <= TOL[prec]
    cfg2 = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec) \
        .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True)
    c2r = vk.TransformIr.build(cfg2, INV)
    z = hip_ctx.execute_transform(c2r, X)
    assert o.rel_l2(z, x) <= 4 * TOL[prec]


@pytest.mark.parametrize("prec", [F32, F64])
def test_length_sweep_sampled_against_numpy(hip_ctx, prec):
    """Every 7th length through the planner's kernel choice (registered
    shapes, runtime-radix kernels with HBM-direct stages, Rader, Bluestein,
    four-step): even R2C/C2R lengths 2..4096 and C2C lengths 1..2048, batch 3,
    against numpy's float64 FFT (a full sweep of every length passes the same
    bounds)."""
    rdt, cdt = (np.float32, np.complex64) if prec == F32 else (np.float64, np.complex128)
    tol = 2e-5 if prec == F32 else 2e-13
    rng = np.random.default_rng(11)
    batch = 3
    for n in range(2, 4097, 14):
        x = rng.standard_normal(n * batch).astype(rdt)
        X, _ = r2c(hip_ctx, n, batch, x, prec)
        ref = np.fft.rfft(x.astype(np.float64).reshape(batch, n), axis=1).reshape(-1)
        assert o.rel_l2(X, ref) <= tol, ("r2c", n)
        xr, _ = c2r(hip_ctx, n, batch, ref.astype(cdt), prec)
        assert o.rel_l2(xr, x.astype(np.float64)) <= tol, ("c2r", n)
    for n in range(1, 2049, 7):
        z = (rng.standard_normal(n * batch) + 1j * rng.standard_normal(n * batch)).astype(cdt)
        y = c2c(hip_ctx, [n], batch, z, prec)[0]
        ref = np.fft.fft(z.astype(np.complex128).reshape(batch, n), axis=1).reshape(-1)
        assert o.rel_l2(y, ref) <= tol, ("c2c", n)


def _plan_with_env(ctx, ir, env):
    """A fresh plan built under the given environment knobs (read at plan time)."""
    import os
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return vk.Plan(ctx, ir)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _run_plan(ctx, plan, x, out_count):
    out = np.empty(out_count, dtype=x.dtype)
    vk._check(ctx._L.vkfx_execute_host(plan.handle, x.ctypes.data, x.nbytes, out.ctypes.data, out.nbytes), ctx._L)
    return out


@pytest.mark.parametrize("batch", [1, 3, 5, 37, 8192])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_register_exchange_kernel_1024(hip_ctx, batch, direction):
    """The one-wave register-exchange kernel (DPP and permlane exchanges, no
    LDS) for 1024-point f32 rows, against the oracle: partial blocks of 4
    lines, both directions, normalized inverse; bit-identical to itself on
    repeat and within 1e-5 of the LDS-staged default."""
    n = 1024
    normalize = direction == INV
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_inverse_normalization(normalize)
    ir = vk.TransformIr.build(cfg, direction)
    plan = _plan_with_env(hip_ctx, ir, {"VKFX_REGISTER_EXCHANGE": "1"})
    try:
        (p,) = plan.describe()["passes"]
        assert p["block"] == 256 and p["lines_per_block"] == 4 and p["lds_bytes"] == 0, p
        assert p["radices"] == [16, 4, 16]
        x = rand(n * batch, 700 + batch)
        y = _run_plan(hip_ctx, plan, x, n * batch)
        idx = np.arange(0, batch, max(1, batch // 64))
        xs = x.reshape(batch, n)[idx].reshape(-1)
        ref = o.fft_batch(xs.astype(np.complex128), n, "forward" if direction == FWD else "inverse", normalize,
                          threads=8)
        assert o.rel_l2(y.reshape(batch, n)[idx].reshape(-1), ref) <= TOL[F32]
        assert np.array_equal(_run_plan(hip_ctx, plan, x, n * batch), y)
        y_default = hip_ctx.execute_transform(ir, x)
        assert o.rel_l2(y, y_default) <= TOL[F32]
    finally:
        plan.close()


@pytest.mark.parametrize("n,batch,kind,pick,lds", [
    (1024, 37, 0, 0, 1088 * 8), (1024, 37, 0, 1, 1088 * 8), (1024, 37, 0, 3, 1056 * 8),
    (4099, 6, 12, 0, 9261 * 8), (4099, 6, 12, 1, 2 * 9261 * 8), (4099, 6, 12, 2, 8489 * 8),
    (4115, 5, 12, 0, 9261 * 8)])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_fixed_shape_variants(hip_ctx, n, batch, kind, pick, lds, direction):
    """Each registered variant of the C1 and M = 8232 Bluestein shapes
    (per-stage twiddle tables and pads, ping-pong LDS buffers, product-tree
    twiddles with one uniform pad) against the oracle, both directions."""
    if n == 1024 and pick == 3 and direction == INV:
        pytest.skip("the one-slot-per-32 padding is registered for the forward direction only")
    normalize = direction == INV
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_inverse_normalization(normalize)
    ir = vk.TransformIr.build(cfg, direction)
    plan = _plan_with_env(hip_ctx, ir, {f"VKFX_FIXED_PICK_K{kind}": str(pick)})
    try:
        (p,) = plan.describe()["passes"]
        assert p["fixed_shape"] and p["lds_bytes"] == lds, p
        x = rand(n * batch, 300 + pick)
        y = _run_plan(hip_ctx, plan, x, n * batch)
        assert o.rel_l2(y, oracle_c2c(x, n, direction, normalize)) <= TOL[F32]
    finally:
        plan.close()


@pytest.mark.parametrize("n,cap,prec", [(4096, 16, F32), (2187, 27, F64), (3072, 16, F32), (1 << 20, 128, F64)])
@pytest.mark.parametrize("direction", [FWD, INV])
def test_three_upload_four_step(hip_ctx, n, cap, prec, direction):
    """Three-upload four-step (FourStepThreeUpload, kernel_ir.rs:1206-1236,
    recursive_ir.rs:756-893) forced at small sizes by capping the one-upload
    length, against the oracle; normalized inverse."""
    batch = 3
    normalize = direction == INV
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(normalize)
    ir = vk.TransformIr.build(cfg, direction)
    plan = _plan_with_env(hip_ctx, ir, {"VKFX_MAX_UPLOAD": str(cap)})
    try:
        fs = plan.describe()["four_step"]
        assert fs["uploads"] == 3 and fs["n1"] * fs["m1"] * fs["m2"] == n and max(fs["n1"], fs["m1"], fs["m2"]) <= cap
        x = rand(n * batch, 40 + n % 97, prec)
        y = _run_plan(hip_ctx, plan, x, n * batch)
        ref = oracle_c2c(x, n, direction, normalize)
        tol = TOL[prec] if prec == F32 else max(TOL[F64], 4 * o.rel_l2(ref, (np.fft.fft if direction == FWD else
                                                                              np.fft.ifft)(x.reshape(batch, n).astype(np.complex128), axis=1).reshape(-1)))
        assert o.rel_l2(y, ref) <= tol
    finally:
        plan.close()


@pytest.mark.parametrize("log2n,prec,tol", [(29, F32, 1e-5), (27, F64, 1e-12)])
def test_three_upload_full_length(hip_ctx, log2n, prec, tol):
    """Lengths past the two-upload limit (f32 2^29, f64 2^27: one line of
    4 and 2 GiB): three uploads without a cap. Input = three tones, whose
    spectrum is N a_t at bin f_t and zero elsewhere (closed form); then the
    normalized inverse returns the input."""
    import torch
    n = 1 << log2n
    cdt = torch.complex64 if prec == F32 else torch.complex128
    freqs, amps = [3, 12345, n - 77], [1.0, 0.5 - 0.25j, -0.75j]
    k = torch.arange(n, device="cuda", dtype=torch.int64)
    x = torch.zeros(n, device="cuda", dtype=torch.complex128)
    one = torch.ones(n, device="cuda", dtype=torch.float64)
    for f, a in zip(freqs, amps):
        # exact integer reduction of the phase f k / n before the float conversion
        x += a * torch.polar(one, (2 * np.pi / n) * ((k * f) % n).to(torch.float64))
    del k, one
    x = x.to(cdt)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_precision(prec), FWD)
    plan = hip_ctx.plan(ir)
    assert plan.describe()["four_step"]["uploads"] == 3
    y = torch.empty_like(x)
    plan.execute_tensors(x, y)
    torch.cuda.synchronize()
    ref_norm = n * float(np.sqrt(sum(abs(a) ** 2 for a in amps)))
    err = y.clone()
    for f, a in zip(freqs, amps):
        err[f] -= n * a
    assert float(torch.linalg.vector_norm(err.to(torch.complex128))) / ref_norm <= tol
    del err
    plan.close()
    iir = vk.TransformIr.build(vk.FftConfig.new([n]).with_precision(prec).with_inverse_normalization(True), INV)
    iplan = hip_ctx.plan(iir)
    z = torch.empty_like(x)
    iplan.execute_tensors(y, z)
    torch.cuda.synchronize()
    rel = float(torch.linalg.vector_norm((z - x).to(torch.complex128)) / torch.linalg.vector_norm(x.to(torch.complex128)))
    assert rel <= tol
    iplan.close()


@pytest.mark.parametrize("prec", [F32, F64])
@pytest.mark.parametrize("batch", [1, 3, 4096, 100003])
def test_length_one_is_a_copy(hip_ctx, prec, batch):
    """A transform whose only axis has length 1 is X[0] = x[0] in both
    directions (normalized or not): one copy pass, 16-byte body and 8-byte
    tail, bit-exact."""
    x = rand(batch, 5 + batch % 7, prec)
    for direction, normalize in ((FWD, False), (INV, True), (INV, False)):
        cfg = vk.FftConfig.new([1]).with_batch_count(batch).with_precision(prec).with_inverse_normalization(normalize)
        ir = vk.TransformIr.build(cfg, direction)
        plan = hip_ctx.plan(ir)
        assert [p["kernel"] for p in plan.describe()["passes"]] == ["copy"]
        y = hip_ctx.execute_transform(ir, x)
        assert np.array_equal(y, x)


def test_register_exchange_kernel_nd_rows(hip_ctx):
    """The register-exchange kernel as the contiguous-axis pass of N-D plans."""
    for dims, batch in (([8, 1024], 2), ([3, 5, 1024], 1)):
        cfg = vk.FftConfig.new(dims).with_batch_count(batch)
        ir = vk.TransformIr.build(cfg, FWD)
        plan = _plan_with_env(hip_ctx, ir, {"VKFX_REGISTER_EXCHANGE": "1"})
        try:
            assert any(p.get("lds_bytes") == 0 and p.get("fft_len") == 1024 and p.get("lines_per_block") == 4
                       for p in plan.describe()["passes"])
            total = int(np.prod(dims)) * batch
            x = rand(total, 900)
            y = _run_plan(hip_ctx, plan, x, total)
            assert o.rel_l2(y, o.fft_nd(x, dims, batch, threads=8)) <= TOL[F32]
        finally:
            plan.close()
