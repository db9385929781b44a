"""CPU checks of bench.py's own logic: the multi-GPU refusal, the HBM-traffic
arithmetic from rocprofv3 counters, and the committed traffic profile it falls
back to.  Nothing here touches a GPU."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402

KERNEL = "void (anonymous namespace)::la_adamw_kernel<float, (anonymous namespace)::bf16_t, float>(StepArgs)"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True)
    assert r.returncode == 2 and "one GPU only" in r.stderr and r.stdout == ""


def _csv(tmp_path, rows):
    path = tmp_path / "c_counter_collection.csv"
    lines = ["Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"]
    lines += [f'{i},"{k}",{c},{v}' for i, (k, c, v) in enumerate(rows)]
    path.write_text("\n".join(lines) + "\n")
    return str(path)


def test_traffic_from_sized_request_counters(tmp_path):
    """Two dispatches of the update kernel among other kernels' rows: the mean
    per dispatch, and bytes = 128/64/32 x the sized read requests + 64 x the
    64-byte writes + 32 x the other writes (the C2 counts of one launch)."""
    rd = bench.READ_COUNTERS
    rows = []
    for r64 in (400, 440):
        rows += [(KERNEL, rd[0], 23_856_000), (KERNEL, rd[1], r64), (KERNEL, rd[2], 0)]
        rows += [("la_sqnorm_kernel<bf16_t, false>(NormArgs)", rd[0], 3_408_000)]
    vals, n = bench.update_kernel_counters(_csv(tmp_path, rows), rd)
    assert n == 2 and vals[rd[1]] == 420
    w = bench.WRITE_COUNTERS
    wvals, _ = bench.update_kernel_counters(_csv(tmp_path, [(KERNEL, w[0], 47_712_010), (KERNEL, w[1], 47_712_000)]),
                                           w)
    vals.update(wvals)
    read, write = bench.traffic_bytes(vals)
    assert read == 23_856_000 * 128 + 420 * 64
    assert write == 47_712_000 * 64 + 10 * 32
    assert bench.update_kernel_counters(_csv(tmp_path, rows), w) == f"no {w[0]} for the update kernel"


def test_committed_traffic_profile_is_read():
    value, source = bench.read_traffic()
    assert value == pytest.approx(28 * sum(bench.LLAMA8B_LAYER), rel=1e-4)
    assert "kernel build" in source


@pytest.mark.parametrize("env", [{"ROCP_TOOL_LIBRARIES": "x"}, {"ROCPROF_OUTPUT_PATH": "/tmp/la_prof"},
                                 {"LD_PRELOAD": "librocprofiler-sdk-tool.so"}])
def test_profiler_environment_is_detected(env, monkeypatch):
    for k in ("ROCP_TOOL_LIBRARIES", "ROCPROF_OUTPUT_PATH", "LD_PRELOAD"):
        monkeypatch.delenv(k, raising=False)
    assert not bench.under_profiler()
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    assert bench.under_profiler()


def test_default_run_under_a_profiler_reaches_the_device_check():
    """`rocprofv3 ... -- python3 bench.py` with the default --traffic live: the
    run skips its own counter passes and goes on to the device.  Here, on a
    host without a GPU, it must end at the device check (rc 1), not with a
    traceback.  The profiler is marked by ROCPROF_OUTPUT_PATH, which only the
    profiler's own tool reads: a ROCP_TOOL_LIBRARIES naming no library makes
    the ROCm runtime abort when torch starts it."""
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible: this checks the path up to the device check on a host without one")
    env = dict(os.environ, ROCPROF_OUTPUT_PATH="/tmp/la_prof_unused")
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--steps", "1", "--cpu-budget", "0"],
                       capture_output=True, text=True, env=env, timeout=300)
    assert "Traceback" not in r.stderr, r.stderr
    assert r.returncode == 1 and "needs a HIP device" in r.stderr, (r.returncode, r.stderr)
    assert "running under a profiler" in r.stderr and r.stdout == ""
