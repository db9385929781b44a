"""Host-side native code under sanitizers (CPU only).

The file offloader (slideformer_amd/csrc/disk_offload.hip) and the copy pool of
the streaming pipeline (slideformer_amd/csrc/copy_pool.h) are plain host C++;
each is compiled here with g++ together with a driver that hammers it from
several threads, once under AddressSanitizer + UndefinedBehaviorSanitizer and
once under ThreadSanitizer.  No GPU code is built or run."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "slideformer_amd", "csrc", "disk_offload.hip")
DRIVER = os.path.join(REPO, "tests", "native", "disk_offload_driver.cpp")


@pytest.mark.parametrize("sanitize", ["address,undefined", "thread"])
def test_disk_offload_under_sanitizer(sanitize, tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "driver"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-pthread", f"-fsanitize={sanitize}", "-fno-omit-frame-pointer",
           "-I", os.path.join(REPO, "include"), "-x", "c++", SRC, "-x", "none", DRIVER, "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True)
    work = tmp_path / "files"
    work.mkdir()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", TSAN_OPTIONS="halt_on_error=1")
    res = subprocess.run([str(exe), str(work)], capture_output=True, text=True, env=env, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "disk offload driver ok" in res.stdout
    assert list(work.iterdir()) == []  # every offload file removed by la_disk_destroy


POOL_DRIVER = os.path.join(REPO, "tests", "native", "copy_pool_driver.cpp")


@pytest.mark.parametrize("sanitize", ["address,undefined", "thread"])
def test_copy_pool_under_sanitizer(sanitize, tmp_path):
    """The host copy pool of the streaming pipeline (slideformer_amd/csrc/copy_pool.h),
    many fork-join rounds on pools of 1-8 threads, under ASan+UBSan and TSan."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "pool_driver"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-pthread", f"-fsanitize={sanitize}", "-fno-omit-frame-pointer",
           "-I", os.path.join(REPO, "slideformer_amd", "csrc"), POOL_DRIVER, "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", TSAN_OPTIONS="halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "copy pool driver ok" in res.stdout
