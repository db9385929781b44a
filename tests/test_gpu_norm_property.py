"""Randomised parity of the grad norm and clip (la_grad_sqnorm, la_grad_norm_clip,
la_grad_norm_clip_noalloc, la_clip_coef) with the CPU checker.

Each example draws 1-6 grad buffers (dtype, 0 to 2.5 M elements, element
offset 0-7 inside its allocation, value scale 1e-20 to 1e10, so fp16 grads
may hold inf) and a max norm.
The buffers' squares are accumulated in order into one float64 sum, as a
sliding-order global clip does: every buffer but the last through
la_grad_sqnorm with accumulate, the last through la_grad_norm_clip, which
also writes the coefficient.  The sum must be within 1e-12 (relative) of the
exact one (the checker's compensated float64 sum, itself pinned to math.fsum
by the CPU tests); the coefficient and the norm must be bit-identical to the
checker's clip of the sum the device produced (the torch clip_grad_norm_
formula); la_clip_coef on that sum and the no-workspace variant run over the
same sequence must give the same bits.  The same buffers then go through
la_grad_norm_multi in runs of one dtype, to the same bar (with bit equality
when every run holds one buffer).  Examples are drawn from a fixed seed."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from hypothesis import given
from hypothesis import strategies as st

from oracle import oracle as O
from slideformer_amd import _lib
from tests import _hip as H
from tests._props import property_test

pytestmark = pytest.mark.gpu

KIND16 = {"bf16": "bf16", "f16": "f16", "f32": None}


@st.composite
def buffer(draw):
    return dict(kind=draw(st.sampled_from(["bf16", "f32", "f16"])),
                n=draw(st.one_of(st.integers(0, 100), st.integers(101, 70_000), st.integers(70_001, 2_500_000))),
                off=draw(st.integers(0, 7)),
                scale=draw(st.floats(-20, 10).map(lambda e: 10.0 ** e)),
                seed=draw(st.integers(0, 2**31 - 1)))


@st.composite
def cases(draw):
    return dict(buffers=draw(st.lists(buffer(), min_size=1, max_size=6)),
                max_norm=draw(st.sampled_from([1e-3, 0.5, 1.0, 1e6])))


def _bits(x: np.ndarray, kind: str) -> np.ndarray:
    return H.to_np_bits(torch.from_numpy(x.astype(np.float32)).to(H.TD[kind]), kind)


@property_test(200)
@given(c=cases())
def test_accumulated_norm_and_clip_equal_checker(c, hip_device):
    print(f"norm property case: {c}", flush=True)
    L = _lib.load()
    st_ = torch.cuda.current_stream(hip_device).cuda_stream
    exact = 0.0
    grads = []
    for b in c["buffers"]:
        rng = np.random.default_rng(b["seed"])
        bits = _bits(rng.normal(0, b["scale"], b["n"] + b["off"]), b["kind"])
        view = bits.view(np.float32) if b["kind"] == "f32" else bits
        exact += O.grad_sqnorm(view[b["off"]:], KIND16[b["kind"]])
        grads.append(H.to_dev_bits(bits, b["kind"], hip_device)[b["off"]:])
    # sized for all buffers together: la_grad_norm_multi's stage 1 reads them in one grid
    ws = torch.zeros(max(1, L.la_grad_sqnorm_workspace(sum(g.numel() for g in grads)) // 8), dtype=torch.float64,
                     device=hip_device)
    sq = torch.full((1,), 12345.0, dtype=torch.float64, device=hip_device)   # overwritten by the first call
    coef = torch.zeros(1, device=hip_device)
    norm = torch.zeros(1, device=hip_device)
    sq_na = torch.full((1,), -1.0, dtype=torch.float64, device=hip_device)
    coef_na = torch.zeros(1, device=hip_device)
    norm_na = torch.zeros(1, device=hip_device)
    last = len(grads) - 1
    for k, (b, g) in enumerate(zip(c["buffers"], grads)):
        code = H.CODE[b["kind"]]
        acc = int(k > 0)
        if k < last:
            rc = L.la_grad_sqnorm(code, g.data_ptr(), g.numel(), ws.data_ptr(), ws.numel() * 8, sq.data_ptr(),
                                  acc, st_)
            assert rc == 0, L.la_strerror(rc)
            rc = L.la_grad_norm_clip_noalloc(code, g.data_ptr(), g.numel(), sq_na.data_ptr(), acc, c["max_norm"],
                                             coef_na.data_ptr(), norm_na.data_ptr(), st_)
        else:
            rc = L.la_grad_norm_clip(code, g.data_ptr(), g.numel(), ws.data_ptr(), ws.numel() * 8, sq.data_ptr(),
                                     acc, c["max_norm"], coef.data_ptr(), norm.data_ptr(), st_)
            assert rc == 0, L.la_strerror(rc)
            rc = L.la_grad_norm_clip_noalloc(code, g.data_ptr(), g.numel(), sq_na.data_ptr(), acc, c["max_norm"],
                                             coef_na.data_ptr(), norm_na.data_ptr(), st_)
        assert rc == 0, L.la_strerror(rc)
    torch.cuda.synchronize()
    got = float(sq.item())
    if math.isinf(exact):                     # fp16 values beyond 65504 are inf
        assert got == exact
    else:
        assert abs(got - exact) <= 1e-12 * exact, (got, exact)
    c_ref, n_ref = O.clip_coef(got, c["max_norm"])
    assert coef.cpu().numpy()[0] == np.float32(c_ref) and norm.cpu().numpy()[0] == np.float32(n_ref)
    coef2, norm2 = H.clip_coef(sq, c["max_norm"])
    assert coef2.item() == coef.item() and norm2.item() == norm.item()
    # the no-workspace sequence: the same partial order, so the same bits
    assert sq_na.item() == got and coef_na.item() == coef.item() and norm_na.item() == norm.item()

    # the multi-buffer norm over runs of one dtype (as LayerAdam.clip_grad_norm
    # groups them): its own summation order, so within 1e-12 of the exact sum,
    # and the clip of its sum bit-exact; a run of one buffer is the single-buffer
    # computation, so with every run of length one the bits equal the sequence above
    runs = []
    for b, g in zip(c["buffers"], grads):
        if runs and runs[-1][0][0] == b["kind"] and len(runs[-1]) < _lib.LA_NORM_MULTI_MAX:
            runs[-1].append((b["kind"], g))
        else:
            runs.append([(b["kind"], g)])
    sq_m = torch.full((1,), 777.0, dtype=torch.float64, device=hip_device)
    coef_m = torch.zeros(1, device=hip_device)
    norm_m = torch.zeros(1, device=hip_device)
    for i, run in enumerate(runs):
        bufs = (_lib.LaGradBuffer * len(run))()
        for q, (_, g) in zip(bufs, run):
            q.g, q.n = g.data_ptr(), g.numel()
        last = i == len(runs) - 1
        rc = L.la_grad_norm_multi(H.CODE[run[0][0]], bufs, len(run), ws.data_ptr(), ws.numel() * 8, sq_m.data_ptr(),
                                  int(i > 0), c["max_norm"], coef_m.data_ptr() if last else None,
                                  norm_m.data_ptr() if last else None, st_)
        assert rc == 0, L.la_strerror(rc)
    torch.cuda.synchronize()
    got_m = float(sq_m.item())
    if math.isinf(exact):
        assert got_m == exact
    else:
        assert abs(got_m - exact) <= 1e-12 * exact, (got_m, exact)
    c_ref, n_ref = O.clip_coef(got_m, c["max_norm"])
    assert coef_m.cpu().numpy()[0] == np.float32(c_ref) and norm_m.cpu().numpy()[0] == np.float32(n_ref)
    if all(len(run) == 1 for run in runs):
        assert got_m == got and coef_m.item() == coef.item() and norm_m.item() == norm.item()


@pytest.mark.parametrize("kind", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("count", [1, 2, 31, 32])
def test_multi_norm_of_many_small_buffers(kind, count, hip_device):
    """Up to LA_NORM_MULTI_MAX buffers in one call: sizes 0-5000 (most far below
    one workgroup's share), each at an element offset 0-7 of its allocation.
    The sum is within 1e-12 of the exact one, the clip bit-exact to the
    checker's clip of that sum; a second identical call gives the same bits."""
    print(f"multi norm: {kind} x {count}", flush=True)
    L = _lib.load()
    rng = np.random.default_rng(count * 7 + len(kind))
    bufs = (_lib.LaGradBuffer * count)()
    keep, exact = [], 0.0
    for q in bufs:
        n, off = int(rng.integers(0, 5000)), int(rng.integers(0, 8))
        bits = _bits(rng.normal(0, 1e-2, n + off), kind)
        view = bits.view(np.float32) if kind == "f32" else bits
        exact += O.grad_sqnorm(view[off:], KIND16[kind])
        g = H.to_dev_bits(bits, kind, hip_device)[off:]
        keep.append(g)
        q.g, q.n = g.data_ptr(), g.numel()
    total = sum(g.numel() for g in keep)
    ws = torch.zeros(max(1, L.la_grad_sqnorm_workspace(total) // 8), dtype=torch.float64, device=hip_device)
    out = []
    for _ in range(2):
        sq = torch.zeros(1, dtype=torch.float64, device=hip_device)
        coef = torch.zeros(1, device=hip_device)
        norm = torch.zeros(1, device=hip_device)
        rc = L.la_grad_norm_multi(H.CODE[kind], bufs, count, ws.data_ptr(), ws.numel() * 8, sq.data_ptr(), 0, 1.0,
                                  coef.data_ptr(), norm.data_ptr(), torch.cuda.current_stream(hip_device).cuda_stream)
        assert rc == 0, L.la_strerror(rc)
        torch.cuda.synchronize()
        out.append((sq.item(), coef.item(), norm.item()))
    got = out[0][0]
    assert abs(got - exact) <= 1e-12 * exact
    c_ref, n_ref = O.clip_coef(got, 1.0)
    assert out[0][1] == np.float32(c_ref) and out[0][2] == np.float32(n_ref)
    assert out[0] == out[1]


def test_clip_grad_norm_over_many_tensors_of_mixed_dtype(hip_device):
    """LayerAdam.clip_grad_norm over 75 grad tensors (more than two
    la_grad_norm_multi calls' worth, three dtypes, empty ones among them):
    the norm is the exact float64 norm rounded to fp32 (within one ulp, since
    the device's float64 sum may differ from the exact one in its last bits)
    and the coefficient follows from it as torch's clip_grad_norm_ computes."""
    from slideformer_amd import LayerAdam

    rng = np.random.default_rng(75)
    kinds = ["bf16"] * 40 + ["f32"] * 20 + ["bf16"] * 5 + ["f16"] * 10
    grads, exact = [], 0.0
    for k, kind in enumerate(kinds):
        n = 0 if k % 17 == 3 else int(rng.integers(1, 20_000))
        bits = _bits(rng.normal(0, 3e-3, n), kind)
        view = bits.view(np.float32) if kind == "f32" else bits
        exact += O.grad_sqnorm(view, KIND16[kind])
        grads.append(H.to_dev_bits(bits, kind, hip_device))
    adam = LayerAdam()
    coef, norm = adam.clip_grad_norm(grads, 0.05)
    torch.cuda.synchronize()
    want = np.float32(math.sqrt(exact))
    assert abs(float(norm.item()) - float(want)) <= float(np.spacing(want))
    c_ref, n_ref = O.clip_coef(float(norm.item()) ** 2, 0.05)
    assert abs(coef.item() - c_ref) <= 2 * float(np.spacing(np.float32(c_ref)))
    assert 0.0 < coef.item() < 1.0


def test_accumulator_takes_lists_of_per_tensor_grads(hip_device):
    """GradNormAccumulator.add with a layer's per-tensor grads (a list: runs of
    one dtype through la_grad_norm_multi) and with single buffers, in sliding
    order: the norm is the exact one rounded to fp32 (within one ulp)."""
    from slideformer_amd import LayerAdam

    rng = np.random.default_rng(41)
    adam = LayerAdam()
    acc = adam.grad_norm_begin(hip_device)
    exact = 0.0
    for layer in range(5):
        kinds = ["bf16"] * 7 + ["f32"] * 3 if layer % 2 else ["bf16"] * 40
        grads = []
        for kind in kinds:
            bits = _bits(rng.normal(0, 1e-3, int(rng.integers(0, 9000))), kind)
            view = bits.view(np.float32) if kind == "f32" else bits
            exact += O.grad_sqnorm(view, KIND16[kind])
            grads.append(H.to_dev_bits(bits, kind, hip_device))
        acc.add(grads if layer != 3 else grads[0])
        if layer == 3:
            for g in grads[1:]:
                acc.add(g)
    acc.add([])                                   # nothing to add
    coef, norm = acc.finish(1e-3)
    torch.cuda.synchronize()
    want = np.float32(math.sqrt(exact))
    assert abs(float(norm.item()) - float(want)) <= float(np.spacing(want))
    assert 0.0 < coef.item() < 1.0
