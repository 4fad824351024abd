"""Benchmark of the MI355X batched-FFT path (one JSON line on stdout).

Default workload (metric "batched f32 C2C effective HBM GB/s"):
C1 = 1-D C2C forward, f32, N=1024, batch 8192, inputs resident in HBM.
A step is one execute of the plan over one batch. Buffers rotate over 8
input/output pairs (1 GiB) so the 256 MB Infinity Cache cannot hold the
working set between steps.

Every configuration is timed the same way, after max(3, --warmup) untimed
steps, over three runs of the same K = max(20, --steps) steps:

  value      = algorithmic bytes (2 * N * batch * 8) / mean step time, GB/s;
               the step time is the host clock between the synchronizes that
               bracket the K steps (no timing event in that region)
  ms_per_step_median = median of 20 host-clocked blocks of B steps each
               (B: about 2 ms of work per block), a per-step figure robust to
               outliers (a HIP event pair around each step slows the launches
               it brackets, so none is used)
  roofline   = the dominant kernel's algorithmic bytes per launch / its mean
               duration, from HIP events bound to each kernel dispatch
               (vkfx_plan_timing_start: hipExtLaunchKernel begin/end, the
               durations a rocprofv3 kernel trace reports, without the gaps
               between launches), against 8 TB/s; `traffic` is that kernel's
               HBM bytes per launch from the committed rocprofv3 counters
  cpu_baseline = the oracle (a port of vkfft-rs src/reference.rs) timed on
               this host's cores over a bounded sample of the same workload

The default line also carries `configs`: every other BASELINE configuration
(C2-C5b) timed in the same process by the same protocol (K at least 50, and
the warmup continued until at least 50 ms of work has run; the row reports
`warmup_steps_run`), each with its own
roofline, HBM sweeps per step, CPU baseline and the relative L2 error of a
sampled slice of its timed output against the oracle. `accuracy` is the same
check for the headline's timed output (plus the sample-11 metrics of
vkfft-rs src/precision.rs:31-101).

--config selects another benchmark configuration (c2, c3, c4, c5a, c5b,
c5a_rader) for measurement runs; --all prints one line per config;
--headline-only skips the `configs` field. Every line but the default C1
line warms up for at least 50 ms as the rows do (`warmup_steps_run`).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "vkfft-rs_amd"))

PEAK_HBM_GBS = 8000.0

CONFIGS = {
    "c1": dict(workload="1d_c2c_fwd_f32_n1024_b8192", dims=[1024], batch=8192, kind="c2c", prec="f32"),
    "c2": dict(workload="1d_r2c_fwd_c2r_inv_f32_n1048576_b256", dims=[1 << 20], batch=256, kind="r2c_c2r",
               prec="f32"),
    "c3": dict(workload="2d_c2c_fwd_f32_4096x4096_b16", dims=[4096, 4096], batch=16, kind="c2c", prec="f32"),
    "c4": dict(workload="3d_c2c_fwd_f64_512x512x512_b1", dims=[512, 512, 512], batch=1, kind="c2c", prec="f64"),
    "c5a": dict(workload="1d_c2c_fwd_f32_n4099_b4096_bluestein", dims=[4099], batch=4096, kind="c2c",
                prec="f32"),
    "c5b": dict(workload="1d_c2c_fwd_f32_n65537_b4096_bluestein", dims=[65537], batch=4096, kind="c2c",
                prec="f32"),
    # C5a's length under PlannerTuning::with_recursive_fft_rader (planner.rs:414-422):
    # the FFT-Rader tree 4099 -> 4098 = 2 * 3 * 683 instead of Bluestein
    "c5a_rader": dict(workload="1d_c2c_fwd_f32_n4099_b4096_rader", dims=[4099], batch=4096, kind="c2c",
                      prec="f32", recursive_rader=True),
}
# BASELINE.json's configurations (the others are extra measurement runs)
BASELINE_CONFIGS = ["c1", "c2", "c3", "c4", "c5a", "c5b"]


# The metric of the default workload; the other configs report the
# same quantities for their own transform.
METRICS = {
    "c1": "batched f32 C2C effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c2": "batched f32 R2C + C2R effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c3": "batched f32 2-D C2C effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c4": "f64 3-D C2C effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c5a": "batched f32 C2C (Bluestein axis) effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c5b": "batched f32 C2C (Bluestein axis) effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
    "c5a_rader": "batched f32 C2C (Rader axis) effective HBM GB/s and % of peak; GFLOP/s (5NlogN); 1 GPU",
}


def algorithmic(cfg):
    """(bytes, flops) of one step: one read + one write of the logical data
    (for R2C/C2R: N*4 + (N/2+1)*8 bytes per direction and transform); flops
    5 N log2 N per transform (logical N)."""
    n = 1
    for d in cfg["dims"]:
        n *= d
    b = cfg["batch"]
    if cfg["kind"] == "r2c_c2r":
        per_dir = n * 4 + (n // 2 + 1) * 8
        return 2 * per_dir * b, 2 * 5 * n * math.log2(n) * b
    es = 8 if cfg["prec"] == "f32" else 16
    return 2 * n * b * es, 5 * n * math.log2(n) * b


def build_plans(vk, ctx, cfg):
    prec = vk.Precision.F32 if cfg["prec"] == "f32" else vk.Precision.F64
    if cfg["kind"] == "r2c_c2r":
        f = vk.TransformIr.build(vk.FftConfig.new(cfg["dims"]).with_batch_count(cfg["batch"]).with_precision(prec)
                                 .with_transform(vk.TransformKind.RealToComplex), vk.Direction.Forward)
        i = vk.TransformIr.build(vk.FftConfig.new(cfg["dims"]).with_batch_count(cfg["batch"]).with_precision(prec)
                                 .with_transform(vk.TransformKind.ComplexToReal).with_inverse_normalization(True),
                                 vk.Direction.Inverse)
        return [ctx.plan(f), ctx.plan(i)]
    c = vk.FftConfig.new(cfg["dims"]).with_batch_count(cfg["batch"]).with_precision(prec)
    if cfg.get("recursive_rader"):
        c.allow_recursive_fft_rader = True
    ir = vk.TransformIr.build(c, vk.Direction.Forward)
    return [ctx.plan(ir)]


def run_gpu(cfg, steps, warmup, rotate, check=None, warm_ms=0.0):
    """Times one configuration: `warmup` untimed steps, then three runs of
    the same `steps` steps. Returns a dict with
      ms_mean    host clock between the synchronizes around run 1 / steps
                 (no timing event in that region: HIP timing events in the
                 stream slow the launches around them);
      block_ms   run 2: mean step time of each of 20 host-clocked blocks of
                 block_steps steps (a HIP event pair around every step slows
                 the launches of every step it brackets, 10-15% for the
                 multi-pass configs and 2x for C1, so none is used);
      kernels    run 3: per-pass kernel durations from HIP events bound to
                 each FFT kernel dispatch (vkfx_plan_timing_start), one list
                 per plan; with --profile-region, run 3 is the region a
                 `rocprofv3 --selected-regions` trace collects;
      info       device, plan descriptions, buffer pairs, accuracy.
    `check(bufs, pairs, steps)` runs on the timed output before the buffers
    are released. With `warm_ms` > 0 the warmup continues past `warmup` steps
    until that much host-clocked work has run (info["warmup_steps_run"])."""
    import torch

    torch.cuda.init()  # torch's HIP runtime first: the library then binds to the same one
    import vkfft_amd as vk

    ctx = vk.HipExecutionContext(0, library=vk.INDEX_LIB_PATH if _INDEX_BUILD["on"] else None)
    plans = build_plans(vk, ctx, cfg)
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device="cuda").manual_seed(1234)
    # buffers: rotate pairs unless the working set is already >= 1 GiB
    in_bytes, out_bytes = plans[0].in_bytes, plans[0].out_bytes
    pairs = max(1, min(rotate, (1 << 30) // max(in_bytes + out_bytes, 1) + 1)) if in_bytes + out_bytes < (1 << 30) else 1
    bufs = []
    fdt = torch.float32 if cfg["prec"] == "f32" else torch.float64
    fsz = 4 if cfg["prec"] == "f32" else 8
    for _ in range(pairs):
        if cfg["kind"] == "r2c_c2r":  # BASELINE C2: i.i.d. normal(0,1) real samples
            x = torch.randn(in_bytes // fsz, device="cuda", generator=gen, dtype=fdt)
        else:                         # uniform[-1,1) re and im
            x = torch.rand(in_bytes // fsz, device="cuda", generator=gen, dtype=fdt) * 2 - 1
        y = torch.zeros(out_bytes // fsz, device="cuda", dtype=fdt)  # touched before timing
        z = torch.zeros(in_bytes // fsz, device="cuda", dtype=fdt) if len(plans) == 2 else None
        bufs.append((x, y, z))
    s = stream.cuda_stream

    def step(i):
        x, y, z = bufs[i % pairs]
        plans[0].execute(x.data_ptr(), y.data_ptr(), 0, s)
        if len(plans) == 2:
            plans[1].execute(y.data_ptr(), z.data_ptr(), 0, s)

    for i in range(warmup):
        step(i)
    # a floor on the warmup's duration: a kernel bound by VALU issue runs its
    # first milliseconds slower while the GPU's clocks leave their idle state
    # (C5a: 20 steps averaged 226 us after 5 warmup steps, 193 us after 200)
    warm_done = warmup
    if warm_ms > 0:
        torch.cuda.synchronize()
        t_w = time.perf_counter()
        while (time.perf_counter() - t_w) * 1e3 < warm_ms:
            for _ in range(4):
                step(warm_done)
                warm_done += 1
            torch.cuda.synchronize()
    # run 1: host clock, no event in the region
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t0) * 1e3
    # run 2: 20 host-clocked blocks of B steps (B chosen so a block holds
    # about 2 ms of work), for the median per-step time; a synchronize ends
    # each block, so its cost is spread over the block
    per_step = total_ms / steps
    B = max(1, int(math.ceil(2.0 / max(per_step, 1e-3))))
    block_ms = []
    for blk in range(MEDIAN_BLOCKS):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(B):
            step(blk * B + i)
        torch.cuda.synchronize()
        block_ms.append((time.perf_counter() - t0) * 1e3 / B)
    # run 3: kernel durations from events bound to each dispatch
    launches = [p.describe() for p in plans]
    for p, d in zip(plans, launches):
        p.timing_start(steps * max(1, len(d.get("passes", []))))
    _profile_region(True)
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    _profile_region(False)
    kernels = [p.timing_stop() for p in plans]
    info = {"device": ctx.device_name(), "profile": ctx.device_profile(), "plans": launches, "pairs": pairs,
            "warmup_steps_run": warm_done}
    if check is not None:
        # the last timed step's pair holds its output (runs 2 and 3 rewrote
        # the same inputs' outputs with the same plans)
        info["accuracy"] = check(bufs, pairs, steps)
    del bufs
    ctx.close()
    torch.cuda.empty_cache()
    return {"ms_mean": total_ms / steps, "block_ms": block_ms, "block_steps": B, "kernels": kernels, "info": info}


MEDIAN_BLOCKS = 20
_ROCTX = {"on": False, "lib": None}
# --index-build: time the identity-arithmetic build of the same kernels (the
# index-map test library: every butterfly, twiddle, chirp and spectrum
# product replaced by the identity), i.e. the plan's data movement alone:
# the same loads, stores, LDS exchanges and barriers
_INDEX_BUILD = {"on": False}


def _profile_region(begin):
    """roctxProfilerResume / roctxProfilerPause around the kernel-timing run
    (only with --profile-region), so that `rocprofv3 --selected-regions`
    traces exactly the dispatches whose durations the roofline uses."""
    if not _ROCTX["on"]:
        return
    import ctypes
    if _ROCTX["lib"] is None:
        _ROCTX["lib"] = ctypes.CDLL("librocprofiler-sdk-roctx.so.1")
    (_ROCTX["lib"].roctxProfilerResume if begin else _ROCTX["lib"].roctxProfilerPause)(ctypes.c_uint64(0))


# Pass label -> the IO policy its kernels are instantiated with (the
# rocprofv3 kernel names carry it, with the line length of fixed shapes).
PASS_IO = {
    "stockham": ["IoPlain", "IoPlainStaged"], "stockham_columns": ["IoPlain", "IoPlainStaged"],
    "stockham_rows": ["IoPlain", "IoPlainStaged"],
    "split_axis_pass1": ["IoFsA"], "split_axis_pass2": ["IoPlain", "IoPlainStaged"],
    "four_step_columns": ["IoFsA"], "four_step_rows": ["IoFsB"],
    "r2c_columns": ["IoFsA"], "r2c_rows_post": ["IoFsBR2C"],
    "c2r_columns_pre": ["IoFsAC2R", "IoFsAC2RDirect"], "c2r_rows": ["IoFsB"],
    "bluestein_single": ["IoBlue1"], "bluestein_columns": ["IoFsABlue"], "bluestein_rows": ["IoBlueB"],
    "bluestein_columns_out": ["IoFsCBlue"], "rader_fft": ["IoRader"], "rader_mixed": ["IoPlain"],
}


def pass_bytes(rec, cfg, plan_desc):
    """Algorithmic HBM bytes of one launch of a pass: each line's elements
    read once and written once. A Bluestein column pass faces the caller on
    one side, where a line holds the logical N of its M points."""
    es = 8 if cfg["prec"] == "f32" else 16
    elems = rec["lines"] * rec["fft_len"]
    if rec["pass"] == "bluestein_single":
        n = cfg["dims"][0]
        return 2 * rec["lines"] * n * es
    if rec["pass"] in ("bluestein_columns", "bluestein_columns_out"):
        m = _plan_m(plan_desc)
        return int(elems * es * (1 + cfg["dims"][-1] / m))
    return 2 * elems * es


def dominant_kernel(kernels, plans, cfg):
    """The pass (label, line length, lines per launch) with the largest total
    kernel time over the timed steps, its mean launch duration and its
    algorithmic bytes per launch."""
    best = None
    for recs, desc in zip(kernels, plans):
        for r in recs:
            if best is None or r["total_ms"] > best[0]["total_ms"]:
                best = (r, desc)
    if best is None:
        return None
    r, desc = best
    total = sum(x["total_ms"] for recs in kernels for x in recs)
    grid = None
    for p in desc.get("passes", []):
        if p.get("kernel") == r["pass"] and p.get("fft_len") == r["fft_len"] and p.get("lines") == r["lines"]:
            grid = p["grid"] * p["block"]
            break
    return {"pass": r["pass"], "fft_len": r["fft_len"], "lines_per_launch": r["lines"], "launches": r["launches"],
            "avg_ms": r["avg_ms"], "min_ms": r["min_ms"], "max_ms": r["max_ms"],
            "share_of_kernel_time": round(r["total_ms"] / total, 4) if total else None,
            "bytes_per_launch": pass_bytes(r, cfg, desc), "grid_threads": grid}


def roofline_of(dom, workload):
    if not dom or not dom["avg_ms"]:
        return None
    ach = dom["bytes_per_launch"] / (dom["avg_ms"] * 1e-3) / 1e9
    traffic, kname = profiled_traffic(workload, dom["pass"], dom["fft_len"], dom.get("grid_threads"))
    return {"bound": "hbm", "achieved": round(ach, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic,
            "traffic_ratio": round(traffic / dom["bytes_per_launch"], 3) if traffic else None,
            "kernel": dom["pass"], "fft_len": dom["fft_len"], "lines_per_launch": dom["lines_per_launch"],
            "profile_kernel": kname, "grid_threads": dom["grid_threads"], "launch_ms": round(dom["avg_ms"], 5),
            "launches": dom["launches"],
            "bytes_per_launch": dom["bytes_per_launch"], "share_of_kernel_time": dom["share_of_kernel_time"],
            "timing": "HIP events bound to each dispatch of the kernel (hipExtLaunchKernel begin/end), mean over "
                      "the timed steps"}


def plain_copy_bandwidth(nbytes=1 << 30, reps=10):
    """The library's own copy (a transform whose only axis has length 1:
    dims [1], f64, 1 GiB) on device buffers. Its kernel (k_copy16, 16-byte
    nontemporal loads and stores) streams HBM like the FFT kernels' direct
    stages, so its FETCH_SIZE / WRITE_SIZE counters calibrate theirs."""
    import torch

    torch.cuda.init()
    import vkfft_amd as vk

    ctx = vk.HipExecutionContext(0)
    ir = vk.TransformIr.build(vk.FftConfig.new([1]).with_batch_count(nbytes // 16).with_precision(vk.Precision.F64),
                              vk.Direction.Forward)
    plan = ctx.plan(ir)
    x = torch.zeros(nbytes // 4, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    s = torch.cuda.current_stream()
    plan.execute(x.data_ptr(), y.data_ptr(), 0, s.cuda_stream)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(reps):
        plan.execute(x.data_ptr(), y.data_ptr(), 0, s.cuda_stream)
    b.record(s)
    torch.cuda.synchronize()
    ctx.close()
    return 2 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9


def copy_bandwidth(nbytes=1 << 30, reps=20):
    """Measured device-to-device copy rate (read + write bytes / time), the
    practical HBM ceiling on this box next to the nominal 8 TB/s."""
    import torch
    x = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    return 2 * nbytes * reps / (a.elapsed_time(b) * 1e-3) / 1e9


def _host(t, complex_=True):
    import numpy as np
    a = t.detach().cpu().numpy()
    if not complex_:
        return a
    return a.view(np.complex64 if a.dtype == np.float32 else np.complex128)


def _partial_dft_weights(n, k):
    """exp(-2 pi i (j k mod n) / n) for j < n, with the index product reduced
    exactly in integers before the float conversion."""
    import numpy as np
    j = (np.arange(n, dtype=np.int64) * k) % n
    return np.exp(-2j * np.pi * j.astype(np.float64) / n)


def make_check(cfg, threads):
    """Checker of a sampled slice of the timed output against the oracle (the
    C port of vkfft-rs src/reference.rs, f64): relative L2 over the slice."""
    import numpy as np

    from oracle import oracle as o

    dims, kind = cfg["dims"], cfg["kind"]
    tol = 1e-5 if cfg["prec"] == "f32" else 1e-13

    def check(bufs, pairs, steps):
        x, y, z = bufs[(steps - 1) % pairs]
        if kind == "r2c_c2r":
            n = dims[0]
            h = n // 2 + 1
            xr = _host(x[:n], False).astype(np.float64)
            X = _host(y[: 2 * h])
            ref = o.r2c_batch(xr, n, threads=threads)
            back = o.c2r_batch(X.astype(np.complex128), n, normalize=True, threads=threads)
            zr = _host(z[:n], False)
            e1, e2 = o.rel_l2(X, ref), o.rel_l2(zr, back)
            return {"rel_l2": max(e1, e2), "rel_l2_r2c": e1, "rel_l2_c2r": e2, "tolerance": tol,
                    "sample": "batch 0: R2C vs oracle r2c, C2R (of the GPU spectrum) vs oracle c2r"}
        if len(dims) == 1:
            n = dims[0]
            lines = 16 if n <= 8192 else 2
            xs = _host(x[: 2 * n * lines]).astype(np.complex128)
            ys = _host(y[: 2 * n * lines])
            ref = o.fft_batch(xs, n, threads=threads)
            out = {"rel_l2": o.rel_l2(ys, ref), "tolerance": tol,
                   "sample": f"first {lines} of {cfg['batch']} lines vs oracle fft"}
            out.update(o.precision_metrics(ys, ref))
            return out
        # N-D: output planes k0 along the slowest axis of batch 0 equal the
        # oracle's (rank-1)-D FFT of the direct axis-0 DFT sum of the input
        n0, rest = dims[0], int(np.prod(dims[1:]))
        xs = _host(x[: 2 * n0 * rest]).astype(np.complex128).reshape(n0, rest)
        ys = _host(y[: 2 * n0 * rest]).reshape(n0, rest)
        ks = [0, 1, n0 // 3, n0 - 1]
        num = den = 0.0
        for k in ks:
            plane = _partial_dft_weights(n0, k) @ xs
            ref = o.fft_nd(plane, dims[1:], 1, threads=threads) if len(dims) > 2 else o.fft(plane)
            num += float(np.sum(np.abs(ys[k] - ref) ** 2))
            den += float(np.sum(np.abs(ref) ** 2))
        return {"rel_l2": math.sqrt(num / den), "tolerance": tol,
                "sample": f"batch 0, planes k0={ks} of axis 0: direct axis-0 DFT sum, then the oracle's "
                          f"{len(dims) - 1}-D FFT"}

    return check


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, budget_s=15.0, single_s=2.0):
    """The oracle (C port of reference.rs, f64) on a bounded sample of the
    config, as effective GB/s of the config's own byte count: one thread (the
    reference is single-threaded) for about single_s, then batch-parallel on
    this GPU's share of the host cores for about budget_s of CPU work. A unit
    of work is one transform of a 1-D C2C line, one R2C + C2R round trip of a
    real line, or, for N-D transforms, the line FFTs of every axis (the
    separable driver's work per tensor, timed on contiguous lines of each axis
    length; its strided gathers are not included, so the CPU figure is an
    upper bound)."""
    import numpy as np

    from oracle import oracle as o

    nproc = os.cpu_count() or 1
    threads = min(16, nproc)  # one GPU's share of the box's cores
    dims = cfg["dims"]
    n = 1
    for d in dims:
        n *= d
    es = 8 if cfg["prec"] == "f32" else 16
    nbytes, _ = algorithmic(dict(cfg, batch=1))  # bytes of one tensor / transform

    def pool(length):  # lines of input held for the timing calls
        return max(threads, 4) if length > 65536 else 64

    # per axis length: (lines of that length per tensor, line-unit runner)
    if cfg["kind"] == "r2c_c2r":
        def runner(length):
            r = o.normal(length * pool(length), 3)

            def go(lines, th):
                spec = o.r2c_batch(r[:length * lines], length, threads=th)
                o.c2r_batch(spec, length, True, threads=th)
            return go
        axes = [(dims[0], 1)]
    else:
        def runner(length):
            x = o.complex_uniform(length * pool(length), 1, np.complex128)

            def go(lines, th):
                xs = x if lines * length <= x.size else np.resize(x, lines * length)
                o.fft_batch(xs[:lines * length], length, threads=th)
            return go
        axes = [(d, n // d) for d in dims]

    def rate(th, seconds, min_lines):
        """seconds per tensor with `th` threads, timing each axis length for
        its share of `seconds`"""
        per_tensor, lines_done = 0.0, 0
        for length, lines_per_tensor in axes:
            go = runner(length)
            lines = max(min_lines, 1)
            go(1, 1)  # warm
            done, t0 = 0, time.perf_counter()
            while True:
                go(lines, th)
                done += lines
                if time.perf_counter() - t0 >= seconds / len(axes):
                    break
            per_line = (time.perf_counter() - t0) / done
            per_tensor += per_line * lines_per_tensor
            lines_done += done
        return per_tensor, lines_done

    per1, lines1 = rate(1, single_s, 1)
    perT, linesT = rate(threads, budget_s / threads, threads)
    unit = "transform" if len(dims) == 1 else "tensor"
    return {"value": round(nbytes / perT / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "host_nproc": nproc, "cpu_model": _cpu_model(),
            "single_thread": {"us_per_" + unit: round(per1 * 1e6, 2), "value": round(nbytes / per1 / 1e9, 4),
                              "unit": "GB/s", "lines": lines1},
            "all_cores_us_per_" + unit: round(perT * 1e6, 3),
            "sample": f"1 thread: {lines1} lines in ~{single_s:.0f} s; {threads} threads: {linesT} lines in "
                      f"~{budget_s / threads:.1f} s wall (~{budget_s:.0f} s CPU work); axis lengths "
                      f"{[a for a, _ in axes]}; the oracle (C port of reference.rs, f64)"
                      + ("; N-D: per-axis line FFTs only" if len(dims) > 1 else "")}


def hbm_sweeps(info, cfg):
    """HBM sweeps of one step: the data the plan's FFT passes read and write,
    over one read + write of the step's logical data. A pass over L lines of
    length F counts L * F; a Bluestein pass reads or writes the logical N on
    the side that faces the caller and M on the workspace side (N + M over
    two). A single-pass transform counts 1.0."""
    n = 1
    for d in cfg["dims"]:
        n *= d
    if cfg["kind"] == "r2c_c2r":
        logical = n // 2 * cfg["batch"] * 2          # half-length complex lines, both directions
    else:
        logical = n * cfg["batch"] * len(info["plans"])
    moved = 0.0
    for plan in info["plans"]:
        for p in plan.get("passes", []):
            if "lines" not in p or "fft_len" not in p:
                continue
            lines, m, k = p["lines"], p["fft_len"], p["kernel"]
            if k == "bluestein_single":
                moved += lines * n
            elif k in ("bluestein_columns", "bluestein_columns_out"):
                # a column pass over the chunk's M-point lines: the caller-facing
                # side holds N of every M points
                moved += lines * m * 0.5 * (1 + n / _plan_m(plan))
            else:
                moved += lines * m
    return round(moved / logical, 3) if logical else None


def _plan_m(plan):
    """Bluestein convolution length of a 1-D plan (its axes entry)."""
    for ax in plan.get("axes", []):
        if ax.get("convolution_len"):
            return ax["convolution_len"]
    return 1


COPY_BYTES = 1 << 30  # plain_copy_bandwidth(): 1 GiB read + 1 GiB written per launch
CALIBRATION_KERNEL = "k_copy16"


def rocprof_summary(dirs, workload_kernel="vkfx"):
    """Markdown summary of rocprofv3 CSV output directories: kernel stats
    (--kernel-trace --stats), the library's kernels per dispatch shape (name,
    grid size) with their mean durations and scratch bytes from the kernel
    trace, and FETCH_SIZE / WRITE_SIZE (--pmc) per dispatch shape, scaled by
    what the same counter reads for the 1 GiB plain copy that
    plain_copy_bandwidth() runs in the same process."""
    import csv
    import glob
    lines = []
    traffic = {}
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)):
            lines.append(f"### kernel stats ({os.path.basename(f)})\n")
            lines.append("| kernel | calls | avg us | min us | max us | % |")
            lines.append("|---|---|---|---|---|---|")
            for r in list(csv.DictReader(open(f)))[:8]:
                lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                             f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {r['Percentage']} |")
            lines.append("")
        for f in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
            shapes = {}
            for r in csv.DictReader(open(f)):
                if workload_kernel not in r["Kernel_Name"] or CALIBRATION_KERNEL in r["Kernel_Name"]:
                    continue
                key = (r["Kernel_Name"], int(r["Grid_Size_X"]))
                dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                shapes.setdefault(key, []).append((dur, int(r["Scratch_Size"]), int(r["VGPR_Count"])))
            if shapes:
                lines.append(f"### library kernels per dispatch shape ({os.path.basename(f)})\n")
                lines.append("| kernel | grid threads | calls | avg us | min us | max us | VGPRs | scratch B/lane |")
                lines.append("|---|---|---|---|---|---|---|---|")
                for (k, g), v in sorted(shapes.items(), key=lambda kv: -sum(x[0] for x in kv[1])):
                    ds = [x[0] for x in v]
                    lines.append(f"| `{k[:110]}` | {g} | {len(v)} | {sum(ds) / len(ds):.2f} | {min(ds):.2f} | "
                                 f"{max(ds):.2f} | {v[0][2]} | {v[0][1]} |")
                lines.append("")
                for (k, g), v in shapes.items():
                    ds = [x[0] for x in v]
                    lines.append(f"kernel_avg_us `{k[:90]}` grid={g}: {sum(ds) / len(ds):.4f}")
                lines.append("")
        for f in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            per = {}
            for r in csv.DictReader(open(f)):
                key = (r["Kernel_Name"], int(r["Grid_Size"]), r["Counter_Name"])
                per.setdefault(key, []).append(float(r["Counter_Value"]))
            for (k, g, c), v in per.items():
                if CALIBRATION_KERNEL in k:
                    traffic.setdefault(c, {}).setdefault("copy", []).append((k, g, max(v)))
                elif workload_kernel in k:
                    traffic.setdefault(c, {}).setdefault("fft", []).append((k, g, sum(v) / len(v)))
    if traffic:
        lines.append("### HBM traffic per launch (rocprofv3 --pmc, KiB per dispatch)\n")
        lines.append("| counter | kernel | grid threads | raw KiB/launch | plain-copy raw KiB (1 GiB moved) | "
                     "scaled bytes/launch |")
        lines.append("|---|---|---|---|---|---|")
        result = {}
        for c, tags in sorted(traffic.items()):
            copy = [v for _, _, v in tags.get("copy", [])]
            ref = max(copy) if copy else None
            for k, g, v in tags.get("fft", []):
                scaled = v / ref * COPY_BYTES if ref else None
                lines.append(f"| {c} | `{k[:90]}` | {g} | {v:.1f} | {ref if ref else 'n/a'} | "
                             f"{'%.4g' % scaled if scaled else 'n/a'} |")
                result.setdefault((k, g), {})[c] = scaled
        lines.append("")
        for (k, g), cs in result.items():
            if cs.get("FETCH_SIZE") and cs.get("WRITE_SIZE"):
                lines.append(f"traffic_bytes_per_launch `{k[:90]}` grid={g}: {cs['FETCH_SIZE'] + cs['WRITE_SIZE']:.6g}")
    return "\n".join(lines)


def profiled_traffic(workload, label, fft_len, grid_threads=None):
    """HBM bytes per launch of the kernel that runs pass `label` with line
    length `fft_len` over `grid_threads` threads, from the committed
    rocprofv3 summary profiles/<workload>.md: (bytes, kernel name), or
    (None, None). The kernel is matched by its IO policy, the length of a
    fixed shape and the dispatch's grid size."""
    import re
    path = os.path.join(ROOT, "profiles", f"{workload}.md")
    if not os.path.exists(path):
        return None, None
    ios = PASS_IO.get(label, [])
    found = []
    for line in open(path):
        if not line.startswith("traffic_bytes_per_launch"):
            continue
        name = line[line.index("`") + 1:line.rindex("`")]
        val = float(line.rsplit(":", 1)[1])
        g = re.search(r"grid=(\d+)", line[line.rindex("`"):])
        if not any(re.search(r"vkfx::%s[,<>]" % io, name) for io in ios):
            continue
        m = re.search(r"Shape<(\d+),", name)
        if m and int(m.group(1)) != fft_len:
            continue
        if g and grid_threads and int(g.group(1)) != grid_threads:
            continue
        found.append((val, name))
    if len(found) != 1:
        return None, None
    return found[0]


def summarize(name, cfg, r, steps, warmup, threads, with_cpu):
    """One result record of a configuration from run_gpu's measurements."""
    import statistics
    nbytes, flops = algorithmic(cfg)
    ms = r["ms_mean"]
    med = statistics.median(r["block_ms"])
    value = nbytes / (ms * 1e-3) / 1e9
    dom = dominant_kernel(r["kernels"], r["info"]["plans"], cfg)
    out = {
        "metric": METRICS[name],
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if cfg["prec"] == "f32" else "f64",
        "data": "synthetic, torch-seeded: " + ("normal(0,1) reals" if cfg["kind"] == "r2c_c2r"
                                               else "uniform[-1,1) re/im"),
        "config": {"workload": cfg["workload"], "dims": cfg["dims"], "batch": cfg["batch"],
                   "buffer_pairs": r["info"]["pairs"]},
        "ms_per_step_median": round(med, 5),
        "ms_per_step_min": round(min(r["block_ms"]), 5),
        "ms_per_step_max": round(max(r["block_ms"]), 5),
        "median_protocol": f"median over {MEDIAN_BLOCKS} host-clocked blocks of {r['block_steps']} step(s)",
        "value_at_median": round(nbytes / (med * 1e-3) / 1e9, 2),
        "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "gflops": round(flops / (ms * 1e-3) / 1e9, 1),
        "hbm_sweeps": hbm_sweeps(r["info"], cfg),
        "accuracy": r["info"].get("accuracy"),
        "roofline": roofline_of(dom, cfg["workload"]),
        "kernels": [[{k: (round(v, 5) if isinstance(v, float) else v) for k, v in rec.items()} for rec in recs]
                    for recs in r["kernels"]],
        "cpu_baseline": None,
    }
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c1", choices=sorted(CONFIGS))
    ap.add_argument("--all", action="store_true", help="one line per benchmark configuration")
    ap.add_argument("--rotate", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle check of the timed output")
    ap.add_argument("--headline-only", action="store_true", help="skip the other configurations")
    ap.add_argument("--batch", type=int, default=0, help="override the config's batch (tuning runs)")
    ap.add_argument("--index-build", action="store_true",
                    help="time the identity-arithmetic build (data movement only); implies --no-check --no-cpu")
    ap.add_argument("--profile-region", action="store_true",
                    help="bracket the kernel-timing run with roctxProfilerResume/Pause (rocprofv3 --selected-regions)")
    ap.add_argument("--rocprof-summary", nargs="+", metavar="DIR",
                    help="print a markdown summary of rocprofv3 CSV output directories and exit")
    args = ap.parse_args()
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary))
        return
    _ROCTX["on"] = args.profile_region
    if args.index_build:
        _INDEX_BUILD["on"] = True
        args.no_check = args.no_cpu = True
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)
    threads = min(16, os.cpu_count() or 1)
    names = list(CONFIGS) if args.all else [args.config]
    steps = max(20, args.steps)
    warmup = max(3, args.warmup)
    copy_gbs = plain_gbs = None
    lines_out = []
    for name in names:
        cfg = dict(CONFIGS[name])
        if args.batch:
            cfg["batch"] = args.batch
            cfg["workload"] += f"_batch_override_{args.batch}"
        # the default line (C1) keeps exactly --warmup steps; --all lines and
        # the other configurations warm up for at least 50 ms as the rows do
        warm_ms = 0.0 if (not args.all and name == "c1") else 50.0
        r = run_gpu(cfg, steps, warmup, args.rotate, check=None if args.no_check else make_check(cfg, threads),
                    warm_ms=warm_ms)
        if copy_gbs is None:
            copy_gbs = copy_bandwidth()
            plain_gbs = plain_copy_bandwidth()
        out = summarize(name, cfg, r, steps, warmup, threads, not args.no_cpu)
        if args.index_build:
            out["build"] = "index (identity arithmetic: data movement only; not the product)"
        out["hbm_copy_gbs"] = round(copy_gbs, 1)
        out["hbm_plain_copy_gbs"] = round(plain_gbs, 1)
        out["pct_of_copy"] = round(100 * out["value"] / copy_gbs, 2)
        out["device"] = r["info"]["device"]
        if warm_ms:
            out["warmup_steps_run"] = r["info"]["warmup_steps_run"]
        print(f"# {name}: {out['ms_per_step']} ms mean, {out['ms_per_step_median']} ms median, "
              f"{out['value']} GB/s", file=sys.stderr, flush=True)
        lines_out.append((name, out))
    if not args.all and args.config == "c1" and not args.headline_only:
        # every other configuration beside the headline, same process and protocol
        table = {}
        for name in CONFIGS:
            if name == "c1":
                continue
            cfg = dict(CONFIGS[name])
            # at least 50 steps, after at least 50 ms of warmup work: the mean
            # of a short region right after a short warmup weighs the first
            # steps' ramp (C5a: 0.255 ms at 20 steps, 0.234 at 200)
            ksteps = max(steps, 50)
            r = run_gpu(cfg, ksteps, warmup, args.rotate, check=None if args.no_check else make_check(cfg, threads),
                        warm_ms=50.0)
            row = summarize(name, cfg, r, ksteps, warmup, threads, False)
            row["warmup_steps_run"] = r["info"]["warmup_steps_run"]
            acc = row.pop("accuracy") or {}
            for k in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "data", "unit"):
                row.pop(k, None)
            row["workload"] = row.pop("config")["workload"]
            row["rel_l2"] = acc.get("rel_l2")
            row["accuracy_sample"] = acc.get("sample")
            row["baseline_config"] = name in BASELINE_CONFIGS
            table[name] = row
            print(f"# {name}: {row['ms_per_step']} ms mean, {row['ms_per_step_median']} ms median, "
                  f"{row['value']} GB/s", file=sys.stderr, flush=True)
        lines_out[0][1]["configs"] = table
    if not args.no_cpu:
        for name, out in lines_out:
            out["cpu_baseline"] = cpu_baseline(CONFIGS[name], 15.0 if name == "c1" else 6.0,
                                               2.0 if name == "c1" else 1.0)
            for other, row in (out.get("configs") or {}).items():
                cb = cpu_baseline(CONFIGS[other], 4.0, 1.0)
                row["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
                row["cpu_baseline"]["single_thread_gbs"] = cb["single_thread"]["value"]
    for _, out in lines_out:
        print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
