"""Shared test setup: import paths, the `gpu` marker and a GPU context fixture."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vkfft-rs_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def hip_ctx():
    """One HipExecutionContext for the whole GPU session. On a machine with a
    GPU a missing library or a context failure is an error, not a skip."""
    if not os.path.exists("/dev/kfd"):
        pytest.skip("no GPU in this container")
    # torch ships its own libamdhip64.so.7; initialising torch first makes the
    # library bind to that same runtime (one HIP runtime per process).
    import torch
    torch.cuda.init()
    import vkfft_amd as vk
    ctx = vk.HipExecutionContext(0)
    yield ctx
    ctx.close()
