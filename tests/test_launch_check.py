"""Host-side launch validation (csrc/launch_check.cpp): the rules launch()
applies before any dispatch, built with g++ beside a driver of accepted and
rejected launches (tests/host/launch_check_driver.cpp). Covers the Rader
stage scratch region (2 G LS elements), Rader stages on kernels that have no
scratch region (fixed shapes, HBM-direct and edge kernels) or without the
KF_RADER instantiation, and the ordinary block / LDS / direction checks."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "vkfft-rs_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include"),
                    reason="needs g++ and the ROCm headers")
def test_launch_check_rejections(tmp_path):
    exe = str(tmp_path / "launch_check")
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I", CSRC,
           os.path.join(HERE, "host", "launch_check_driver.cpp"), os.path.join(CSRC, "launch_check.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout[-2000:]
    assert r.stdout.startswith("ok "), r.stdout
