"""Kernel timing of a plan (vkfx_plan_timing_start / _stop): HIP events bound
to each FFT kernel dispatch, the measurement bench.py's roofline uses. The
durations are positive, count every dispatch up to the armed capacity, are
grouped per (pass, length, lines) in launch order, and never exceed the host
clock around the same launches."""
import time

import numpy as np
import pytest

import vkfft_amd as vk

pytestmark = pytest.mark.gpu


def _buffers(plan):
    import torch
    x = torch.rand(plan.in_bytes // 4, device="cuda", dtype=torch.float32)
    y = torch.empty(plan.out_bytes // 4, device="cuda", dtype=torch.float32)
    return x, y


def test_one_pass_plan_times_each_dispatch(hip_ctx):
    import torch
    plan = hip_ctx.plan(vk.TransformIr.build(vk.FftConfig.new([1024]).with_batch_count(512), vk.Direction.Forward))
    x, y = _buffers(plan)
    plan.execute_tensors(x, y)
    torch.cuda.synchronize()
    plan.timing_start(16)
    t0 = time.perf_counter()
    for _ in range(5):
        plan.execute_tensors(x, y)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    recs = plan.timing_stop()
    assert [r["pass"] for r in recs] == ["stockham"], recs
    r = recs[0]
    assert r["launches"] == 5 and r["fft_len"] == 1024 and r["lines"] == 512
    assert 0 < r["min_ms"] <= r["avg_ms"] <= r["max_ms"]
    assert r["total_ms"] <= wall_ms
    # disarmed: further executes are untimed, and a second stop is an error
    plan.execute_tensors(x, y)
    with pytest.raises(vk.VkFftError):
        plan.timing_stop()


def test_capacity_bounds_the_timed_dispatches(hip_ctx):
    import torch
    plan = hip_ctx.plan(vk.TransformIr.build(vk.FftConfig.new([256]).with_batch_count(64), vk.Direction.Forward))
    x, y = _buffers(plan)
    plan.timing_start(2)
    for _ in range(4):
        plan.execute_tensors(x, y)
    torch.cuda.synchronize()
    recs = plan.timing_stop()
    assert sum(r["launches"] for r in recs) == 2
    with pytest.raises(vk.VkFftError):
        plan.timing_start(0)


def test_multi_pass_plan_groups_passes_in_launch_order(hip_ctx):
    """A two-upload four-step over several batch chunks on two stream lanes:
    one record per (pass, length, lines), in launch order, every dispatch
    counted; the output still matches numpy."""
    import torch
    n, batch = 1 << 20, 64
    plan = hip_ctx.plan(vk.TransformIr.build(vk.FftConfig.new([n]).with_batch_count(batch), vk.Direction.Forward))
    desc = plan.describe()
    passes = desc["passes"]
    x, y = _buffers(plan)
    plan.timing_start(4 * len(passes))
    plan.execute_tensors(x, y)
    plan.execute_tensors(x, y)
    torch.cuda.synchronize()
    recs = plan.timing_stop()
    fft_passes = [p for p in passes if "fft_len" in p and "lines" in p]
    assert sum(r["launches"] for r in recs) == 2 * len(fft_passes)
    seen = []
    for p in fft_passes:
        key = (p["kernel"], p["fft_len"], p["lines"])
        if key not in seen:
            seen.append(key)
    assert [(r["pass"], r["fft_len"], r["lines"]) for r in recs] == seen
    assert all(r["min_ms"] > 0 for r in recs)
    xs = x.cpu().numpy().view(np.complex64)[: 2 * n].astype(np.complex128).reshape(2, n)
    ys = y.cpu().numpy().view(np.complex64)[: 2 * n].reshape(2, n)
    ref = np.fft.fft(xs, axis=1)
    assert np.linalg.norm(ys - ref) / np.linalg.norm(ref) <= 1e-5
