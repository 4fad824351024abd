"""Host sanitizers on the planner restatement: tests/asan/planner_asan.cpp
linked with csrc/planner.cpp under AddressSanitizer and
UndefinedBehaviorSanitizer (g++ on the host sources only), run over every
length to 20000 and a sample beyond, both precisions, strided and contiguous
axes, recursive-Rader tuning and three shared-memory sizes."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "vkfft-rs_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_planner_under_asan_and_ubsan(tmp_path):
    exe = str(tmp_path / "planner_asan")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-I", CSRC, os.path.join(HERE, "asan", "planner_asan.cpp"),
           os.path.join(CSRC, "planner.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert r.stdout.startswith("ok "), r.stdout
