"""The library's tuning switches (VKFX_* environment variables, read when a
plan is built): each one, set, still gives the transform's results, and its
effect shows in the plan description. These switches select between
measured alternatives (comparison runs); the defaults are the product."""
import os

import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32, F64 = vk.Precision.F32, vk.Precision.F64
FWD, INV = vk.Direction.Forward, vk.Direction.Inverse


@pytest.fixture
def fresh_ctx(hip_ctx):
    """A context of its own, so no plan built under another setting is reused."""
    ctx = vk.HipExecutionContext(0)
    yield ctx
    ctx.close()


def c2c_ir(dims, batch, prec=F32, direction=FWD):
    return vk.TransformIr.build(vk.FftConfig.new(dims).with_batch_count(batch).with_precision(prec), direction)


def run_c2c(ctx, dims, batch, seed, prec=F32):
    ir = c2c_ir(dims, batch, prec)
    dt = np.complex64 if prec == F32 else np.complex128
    x = o.complex_uniform(batch * int(np.prod(dims)), seed, dt)
    y = ctx.execute_transform(ir, x)
    axes = tuple(range(1, len(dims) + 1))
    ref = np.fft.fftn(x.reshape([batch] + list(dims)).astype(np.complex128), axes=axes).reshape(-1)
    assert o.rel_l2(y, ref) <= (1e-5 if prec == F32 else 1e-13), dims
    return ctx.plan(ir).describe()


def test_c2r_pair_loads(monkeypatch, hip_ctx):
    """VKFX_C2R_PAIR_LOADS=0: the C2R column pass of N = 2^20 reads X[k] and
    X[M-k] per element instead of once per pair."""
    n, batch = 1 << 20, 2
    h = n // 2 + 1
    x = o.normal(n * batch, 31, np.float32).reshape(batch, n)
    X = np.fft.rfft(x.astype(np.float64), axis=1).astype(np.complex64).reshape(-1)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch)
                              .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True), INV)
    for value, expect in (("0", False), (None, True)):
        if value is None:
            monkeypatch.delenv("VKFX_C2R_PAIR_LOADS", raising=False)
        else:
            monkeypatch.setenv("VKFX_C2R_PAIR_LOADS", value)
        ctx = vk.HipExecutionContext(0)
        try:
            y = ctx.execute_transform(ir, X)
            assert o.rel_l2(y, x.reshape(-1)) <= 2e-5
            cols = [p for p in ctx.plan(ir).describe()["passes"] if p["kernel"] == "c2r_columns_pre"]
            assert cols and all(p["pair_loads"] == expect for p in cols), cols
        finally:
            ctx.close()
    assert X.size == batch * h


def test_c2r_staged_preprocess(monkeypatch, fresh_ctx):
    """VKFX_C2R_PRE=0: the runtime-shape even C2R keeps its preprocess staged."""
    monkeypatch.setenv("VKFX_C2R_PRE", "0")
    n, batch = 6000, 3
    x = o.normal(n * batch, 32, np.float32).reshape(batch, n)
    X = np.fft.rfft(x.astype(np.float64), axis=1).astype(np.complex64).reshape(-1)
    ir = vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch)
                              .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True), INV)
    y = fresh_ctx.execute_transform(ir, X)
    assert o.rel_l2(y, x.reshape(-1)) <= 2e-5
    passes = fresh_ctx.plan(ir).describe()["passes"]
    assert not any(p["runtime_variant"]["direct_preprocess"] for p in passes), passes


@pytest.mark.parametrize("pick", ["1", "2"])
def test_fixed_variant_pick(monkeypatch, fresh_ctx, pick):
    """VKFX_FIXED_PICK=k: the k-th registered variant of every fixed shape
    (or its last), here the C1 and C5a shapes."""
    monkeypatch.setenv("VKFX_FIXED_PICK", pick)
    d = run_c2c(fresh_ctx, [1024], 64, 33)
    assert d["passes"][0]["fixed_shape"]
    if pick == "1":
        assert d["passes"][0]["twiddles"] == "per_stage_tables"
    d = run_c2c(fresh_ctx, [4099], 8, 34)
    assert d["passes"][0]["kernel"] == "bluestein_single" and d["passes"][0]["fixed_shape"]


def test_one_lane(monkeypatch, fresh_ctx):
    """VKFX_LANES=1: a chunked plan runs every chunk on the caller's stream."""
    monkeypatch.setenv("VKFX_WORK_BUDGET_MB", "8")
    monkeypatch.setenv("VKFX_LANES", "1")
    d = run_c2c(fresh_ctx, [1 << 18], 16, 35)
    assert d["lanes"] == 1 and d["four_step"]["chunk"] < 16, d["four_step"]


def test_lds_budget(monkeypatch, fresh_ctx):
    """VKFX_LDS_BUDGET_KB=40: a 512-point strided axis no longer fits 16
    columns per block in the budget and runs as two split passes."""
    monkeypatch.setenv("VKFX_LDS_BUDGET_KB", "40")
    d = run_c2c(fresh_ctx, [512, 64], 2, 36)
    labels = [p["kernel"] for p in d["passes"]]
    assert "split_axis_pass1" in labels and "split_axis_pass2" in labels, labels


def test_nontemporal_roles_off(monkeypatch, fresh_ctx):
    """VKFX_NT_ROLES=0: each fixed shape keeps its first registered variant
    (no nontemporal choice by role)."""
    monkeypatch.setenv("VKFX_NT_ROLES", "0")
    d = run_c2c(fresh_ctx, [4096, 256], 1, 37)
    assert all(p["fixed_shape"] for p in d["passes"])


def test_split_launches(monkeypatch, fresh_ctx):
    """VKFX_SPLIT=3: a one-upload batch runs as three launches."""
    monkeypatch.setenv("VKFX_SPLIT", "3")
    d = run_c2c(fresh_ctx, [1024], 10, 38)
    assert [p["kernel"] for p in d["passes"]].count("stockham") == 3, d["passes"]


@pytest.mark.parametrize("value", ["0", "1"])
def test_xcd_groups_forced(monkeypatch, fresh_ctx, value):
    """VKFX_XCD_GROUPS=0/1 forces the contiguous dealing of line groups to
    XCDs off / on for every launch (the three-pass Bluestein of 65537 uses it
    by default)."""
    monkeypatch.setenv("VKFX_XCD_GROUPS", value)
    d = run_c2c(fresh_ctx, [65537], 3, 39)
    assert d["passes"] and all(p["xcd_groups"] == (value == "1") for p in d["passes"] if "xcd_groups" in p)


def test_xcd_groups_default(fresh_ctx):
    if "VKFX_XCD_GROUPS" in os.environ:
        pytest.skip("VKFX_XCD_GROUPS is set in this environment")
    d = run_c2c(fresh_ctx, [65537], 3, 40)
    blue = [p for p in d["passes"] if p["kernel"].startswith("bluestein")]
    assert blue and all(p["xcd_groups"] for p in blue), blue
    d = run_c2c(fresh_ctx, [1024], 8, 41)
    assert not d["passes"][0]["xcd_groups"]
