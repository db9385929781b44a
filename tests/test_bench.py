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
