"""Randomised parity of the device entry point (la_adam_update) with the CPU checker.

Each example draws a dtype triple the reference registers, the optimizer's
mode (AdamW or L2) and a sequence of 1-4 calls.  Every call draws its own
hyper-parameters (lr, betas, eps, weight decay, bias correction), its step
number (repeated, skipped, going back, or the next one, so every branch of
the reference's beta-power state machine, cpu_adam.h:57-89, is taken, also
when the betas change between calls), its size (0 to 70,000 elements), the
element offset of each stream within its buffer (0-7, so the alignment
phases agree or disagree), whether the bf16 copy is written and a clip
coefficient.  Value scales are log-uniform over 1e-30 to 1e6, so denormal
moments, underflowing squares and overflowing ones come up.  Every bit of p,
m, v and the copy must equal the checker's, NaN as a class.  Examples are
drawn from a fixed seed."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given
from hypothesis import strategies as st

from oracle import oracle as O
from tests import _golden as G
from tests import _hip as H
from tests._props import property_test

pytestmark = pytest.mark.gpu

TRIPLES = [("f32", "bf16", "f32"), ("f32", "f32", "f32"), ("f32", "f16", "f32"),
           ("bf16", "bf16", "f32"), ("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"),
           ("f16", "f16", "f32"), ("f16", "f32", "f32"), ("f16", "f16", "f16")]
KIND16 = {"bf16": "bf16", "f16": "f16", "f32": None}


def _bits(x: np.ndarray, kind: str) -> np.ndarray:
    """float32 values -> the stream's bits (round to nearest even for 16-bit kinds)."""
    return H.to_np_bits(torch.from_numpy(x.astype(np.float32)).to(H.TD[kind]), kind)


def _view(bits_arr, kind):
    return bits_arr.view(np.float32) if kind == "f32" else bits_arr


betas = st.sampled_from([0.0, 0.5, 0.8, 0.9, 0.95, 0.99, 0.999, 0.9999, 0.99999])
scale = st.floats(-30, 6).map(lambda e: 10.0 ** e)


@st.composite
def call(draw):
    return dict(
        step=draw(st.integers(1, 12)),
        lr=draw(st.sampled_from([0.0, 1e-6, 1e-4, 1e-3, 3e-3, 0.1, 1.0])),
        b1=draw(betas), b2=draw(betas),
        eps=draw(st.sampled_from([0.0, 1e-12, 1e-8, 1e-6, 1e-3])),
        wd=draw(st.sampled_from([0.0, 0.01, 0.1, 0.5])),
        bc=draw(st.booleans()),
        n=draw(st.one_of(st.integers(0, 40), st.integers(41, 2100), st.integers(2101, 70_000))),
        offs=draw(st.lists(st.integers(0, 7), min_size=5, max_size=5)),
        with_out=draw(st.booleans()),
        coef=draw(st.sampled_from([None, 1.0, 0.5, 1e-3])),
        sg=draw(scale), seed=draw(st.integers(0, 2**31 - 1)),
    )


@st.composite
def cases(draw):
    return dict(triple=draw(st.sampled_from(TRIPLES)), adamw=draw(st.booleans()),
                sp=draw(scale), sm=draw(scale), sv=draw(scale),
                calls=draw(st.lists(call(), min_size=1, max_size=4)), seed=draw(st.integers(0, 2**31 - 1)))


@property_test(500)
@given(c=cases())
def test_device_update_equals_checker_on_random_calls(c, hip_device):
    print(f"update property case: {c}", flush=True)
    pk, gk, sk = c["triple"]
    rng = np.random.default_rng(c["seed"])
    size = max(k["n"] for k in c["calls"]) + 8
    # the state lives in one buffer per stream for the whole sequence
    ph = _bits(rng.normal(0, c["sp"], size), pk)
    mh = _bits(rng.normal(0, c["sm"], size), sk)
    vh = _bits(np.abs(rng.normal(0, c["sv"], size)), sk)
    oh = np.zeros(size, np.uint16)
    pd, md, vd = (H.to_dev_bits(b, k, hip_device) for b, k in ((ph, pk), (mh, sk), (vh, sk)))
    od = torch.zeros(size, dtype=torch.bfloat16, device=hip_device)
    first = c["calls"][0]
    hip = H.HipAdam(first["lr"], (first["b1"], first["b2"]), first["eps"], first["wd"], c["adamw"])
    orc = O.OracleAdam(first["lr"], (first["b1"], first["b2"]), first["eps"], first["wd"], c["adamw"])
    for k in c["calls"]:
        n, (op, og, om, ov, oo) = k["n"], k["offs"]
        crng = np.random.default_rng(k["seed"])
        gh = _bits(crng.normal(0, k["sg"], size), gk)
        gd = H.to_dev_bits(gh, gk, hip_device)
        coef = None if k["coef"] is None else torch.tensor([k["coef"]], device=hip_device)
        args = (k["step"], k["lr"], k["b1"], k["b2"], k["eps"], k["wd"], k["bc"])
        hip.update(*args, pd[op:op + n], gd[og:og + n], md[om:om + n], vd[ov:ov + n],
                   out=od[oo:oo + n] if k["with_out"] else None, coef=coef)
        orc.update(*args, _view(ph, pk)[op:op + n], _view(gh, gk)[og:og + n], _view(mh, sk)[om:om + n],
                   _view(vh, sk)[ov:ov + n], p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk],
                   p_bf16_out=oh[oo:oo + n] if k["with_out"] else None, clip_coef=k["coef"])
    torch.cuda.synchronize()
    for dev, want, kind in ((pd, ph, pk), (md, mh, sk), (vd, vh, sk), (od, oh, "bf16")):
        got = H.to_np_bits(dev, kind)
        bad = np.flatnonzero(~G.same_bits(got, want, kind))
        assert bad.size == 0, (kind, bad[:8], got[bad[:8]], want[bad[:8]])
