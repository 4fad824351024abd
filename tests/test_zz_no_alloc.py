"""vkfx_execute_noalloc through the C ABI: the plan's passes run with the
library's static device scratch in place of the plan's workspace. Its output
must equal vkfx_execute's on the same plan and input bit for bit (the same
kernels), on calls in a row whose later plans are smaller (each call finds
the previous call's data in the scratch), and a plan whose workspace exceeds
the scratch is refused before anything is launched."""
import numpy as np
import pytest

import vkfft_amd as vk
from oracle import oracle as o

pytestmark = pytest.mark.gpu

F32 = vk.Precision.F32
SCRATCH_BYTES = 64 << 20


def _ir(n, batch, kind=vk.TransformKind.ComplexToComplex):
    cfg = vk.FftConfig.new([n]).with_batch_count(batch).with_transform(kind)
    return vk.TransformIr.build(cfg, vk.Direction.Forward)


def _run(plan, x, noalloc):
    import torch
    y = torch.full((plan.out_bytes // 4,), float("nan"), device="cuda", dtype=torch.float32)
    s = torch.cuda.current_stream().cuda_stream
    if noalloc:
        plan.execute_noalloc(x.data_ptr(), y.data_ptr(), s)
    else:
        plan.execute(x.data_ptr(), y.data_ptr(), 0, s)
    torch.cuda.synchronize()
    return y


def test_noalloc_matches_execute_on_calls_in_a_row(hip_ctx):
    import torch
    gen = torch.Generator(device="cuda").manual_seed(77)
    # the second call of each pair has a smaller input than the first
    cases = [(1 << 16, 64, vk.TransformKind.ComplexToComplex),   # four-step, 32 MiB of scratch
             (1 << 16, 8, vk.TransformKind.ComplexToComplex),    # four-step, 4 MiB
             (65537, 6, vk.TransformKind.ComplexToComplex),      # Bluestein, three passes
             (65537, 2, vk.TransformKind.ComplexToComplex),
             (1 << 20, 4, vk.TransformKind.RealToComplex),       # real four-step
             (1 << 20, 2, vk.TransformKind.RealToComplex)]
    for n, batch, kind in cases:
        plan = hip_ctx.plan(_ir(n, batch, kind))
        assert 0 < plan.workspace_bytes <= SCRATCH_BYTES, (n, batch, plan.workspace_bytes)
        print(f"noalloc case n={n} batch={batch} kind={kind.name} work={plan.workspace_bytes}", flush=True)
        x = torch.rand(plan.in_bytes // 4, device="cuda", generator=gen, dtype=torch.float32) * 2 - 1
        y_ref = _run(plan, x, noalloc=False)
        for _ in range(2):
            y = _run(plan, x, noalloc=True)
            assert torch.equal(y, y_ref), (n, batch, kind)
        # and the oracle on the first line, to the parity tolerance
        xh = x.cpu().numpy()
        yh = y.cpu().numpy().view(np.complex64)
        if kind == vk.TransformKind.RealToComplex:
            ref = o.r2c_batch(xh[:n].astype(np.float64), n, threads=8)
            assert o.rel_l2(yh[: n // 2 + 1], ref) <= 1e-5
        else:
            ref = o.fft(xh[: 2 * n].view(np.complex64).astype(np.complex128))
            assert o.rel_l2(yh[:n], ref) <= 1e-5


def test_noalloc_refuses_a_workspace_beyond_the_scratch(hip_ctx):
    import torch
    plan = hip_ctx.plan(_ir(1 << 16, 512))
    assert plan.workspace_bytes > SCRATCH_BYTES
    x = torch.zeros(plan.in_bytes // 4, device="cuda", dtype=torch.float32)
    y = torch.full((plan.out_bytes // 4,), 7.0, device="cuda", dtype=torch.float32)
    with pytest.raises(vk.VkFftError) as e:
        plan.execute_noalloc(x.data_ptr(), y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert e.value.status == -6 and "static scratch" in str(e.value)
    torch.cuda.synchronize()
    assert bool(torch.all(y == 7.0))  # nothing ran


def test_noalloc_without_workspace(hip_ctx):
    import torch
    plan = hip_ctx.plan(_ir(1024, 64))
    assert plan.workspace_bytes == 0
    x = torch.rand(plan.in_bytes // 4, device="cuda", dtype=torch.float32)
    assert torch.equal(_run(plan, x, True), _run(plan, x, False))
