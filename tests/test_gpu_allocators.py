"""The library under torch's other caching-allocator configurations.

Every C-ABI entry point that launches asks the HIP runtime what each array is
(hipPointerGetAttributes) and refuses anything but device memory.  torch can
hand out device memory through its default caching allocator (hipMalloc) or
through the stream-ordered hipMallocAsync backend, chosen by
PYTORCH_HIP_ALLOC_CONF before the first GPU call; the reference's launch
scripts name the latter, and expandable segments, as options.  Each
configuration runs tests/alloc_child.py in a fresh process: a clipped
step_with_grad_views of three tensors (twice), a flat step_chunk with the bf16
copy, and a streamed step_chunk on a host-resident master with device grads
and moments.  Every result must equal the CPU checker's bit for bit, and so
the other configuration's too.

Expandable segments (virtual address ranges mapped onto physical pieces with
hipMemCreate / hipMemMap) are not offered by torch's ROCm build on this
platform: with expandable_segments:True it warns and keeps its default
segments.  The library's handling of such memory is checked without torch,
by tests/native/device_from_c.c mapping every array itself
(test_gpu_parity.py::test_plain_c_program_runs_the_step[vmm])."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHILD = os.path.join(REPO, "tests", "alloc_child.py")
CONFIGS = [("default", None, "native"),
           # the ROCm build of torch names this backend "cudaMallocAsync" (and runs
           # hipMallocAsync under it); "backend:hipMallocAsync" parses at import but is
           # refused at the first allocation as a mismatch with that name
           ("hipMallocAsync", "backend:cudaMallocAsync", "cudaMallocAsync")]
A_SIZES = [10_007, 4096, 333]
LR, BETAS, EPS, WD = 1e-3, (0.9, 0.999), 1e-8, 0.01


def _inputs(rng):
    def f32(n, std, absval=False):
        x = rng.normal(0, std, n).astype(np.float32)
        return np.abs(x) if absval else x

    def bf16(n, std):
        return O.f32_to_bf16(rng.normal(0, std, n).astype(np.float32))

    inp = {"a_count": np.int64(len(A_SIZES))}
    for i, n in enumerate(A_SIZES):
        inp[f"a_p{i}"], inp[f"a_g{i}"] = f32(n, 0.02), bf16(n, 1e-2)
    for key, n in (("b", 100_003), ("c", 3_000_001)):
        inp[f"{key}_p"], inp[f"{key}_g"] = f32(n, 0.02), bf16(n, 1e-3)
        inp[f"{key}_m"], inp[f"{key}_v"] = f32(n, 1e-3), f32(n, 1e-6, absval=True)
    return inp


def _expected(inp, coef):
    """The CPU checker's replay of the child's calls, in the child's order."""
    want = {}
    orc = O.OracleAdam(LR, BETAS, EPS, WD, True)
    ps = [inp[f"a_p{i}"].copy() for i in range(len(A_SIZES))]
    ms = [np.zeros(n, np.float32) for n in A_SIZES]
    vs = [np.zeros(n, np.float32) for n in A_SIZES]
    for step in (1, 2):
        for i in range(len(A_SIZES)):
            orc.update(step, LR, BETAS[0], BETAS[1], EPS, WD, True, ps[i], inp[f"a_g{i}"], ms[i], vs[i],
                       g16="bf16", clip_coef=coef)
    for i in range(len(A_SIZES)):
        want[f"a_p{i}"], want[f"a_m{i}"], want[f"a_v{i}"] = ps[i], ms[i], vs[i]
    for key in ("b", "c"):
        p, m, v = inp[f"{key}_p"].copy(), inp[f"{key}_m"].copy(), inp[f"{key}_v"].copy()
        out = np.zeros(p.size, np.uint16)
        O.OracleAdam(LR, BETAS, EPS, WD, True).update(1, LR, BETAS[0], BETAS[1], EPS, WD, True, p,
                                                      inp[f"{key}_g"], m, v, g16="bf16", p_bf16_out=out)
        want.update({f"{key}_p": p, f"{key}_m": m, f"{key}_v": v, f"{key}_out": out})
    return want


def _as_bits(a):
    return a.view(np.uint32) if a.dtype in (np.float32, np.int32) else a.view(np.uint16)


def test_every_allocator_configuration_gives_the_checker_bits(tmp_path, hip_device):
    inp = _inputs(np.random.default_rng(909))
    src = tmp_path / "in.npz"
    np.savez(src, **inp)
    g_all = np.concatenate([inp[f"a_g{i}"] for i in range(len(A_SIZES))])
    c_ref, n_ref = O.clip_coef(O.grad_sqnorm(g_all, "bf16"), 0.5)
    assert c_ref < 1.0
    want = _expected(inp, float(np.float32(c_ref)))
    results = {}
    for name, conf, backend in CONFIGS:
        env = dict(os.environ)
        env.pop("PYTORCH_CUDA_ALLOC_CONF", None)
        env.pop("PYTORCH_HIP_ALLOC_CONF", None)
        if conf is not None:
            env["PYTORCH_HIP_ALLOC_CONF"] = conf
        dst = tmp_path / f"out_{name}.npz"
        print(f"allocator configuration {name}: PYTORCH_HIP_ALLOC_CONF={conf}", flush=True)
        r = subprocess.run([sys.executable, CHILD, str(src), str(dst)], capture_output=True, text=True,
                           timeout=240, env=env, cwd=REPO)
        assert r.returncode == 0, (name, r.returncode, r.stdout[-2000:], r.stderr[-4000:])
        assert f"ALLOC_CHILD_OK backend={backend}" in r.stdout, (name, r.stdout)
        got = dict(np.load(dst))
        assert got["a_coef"].view(np.float32)[0] == np.float32(c_ref), name
        assert got["a_norm"].view(np.float32)[0] == np.float32(n_ref), name
        for key, w in want.items():
            g = got[key]
            assert np.array_equal(_as_bits(g), _as_bits(w)), (name, key)
        results[name] = got
    for name in results:
        for key in results["default"]:
            assert np.array_equal(results[name][key], results["default"][key]), (name, key)
