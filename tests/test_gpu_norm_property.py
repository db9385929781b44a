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
same sequence must give the same bits.  Examples are drawn from a fixed seed."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import oracle as O
from slideformer_amd import _lib
from tests import _hip as H

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


@settings(max_examples=60, deadline=None, derandomize=True, suppress_health_check=list(HealthCheck))
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
    ws = torch.zeros(max(1, L.la_grad_sqnorm_workspace(max(g.numel() for g in grads)) // 8), dtype=torch.float64,
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
