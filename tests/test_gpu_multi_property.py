"""Randomised parity of the batched per-tensor entry point (la_adam_update_multi).

`step(layer)` and `step_with_grad_views` make one adam_update call per tensor
(layer_adam.py:314-327,397-410); la_adam_update_multi does those calls in one
launch per 16 tensors, with per-tensor scalars (the first call of a step
multiplies the beta powers, the later ones of the same step take pow,
cpu_adam.h:57-89) and per-tensor scalar tails.  Each example draws a dtype
triple, the optimizer's mode, 1-3 steps (numbers drawn, so repeated and
skipped steps occur) with their own hyper-parameters, and 1-40 tensors
(counts around the 16 segments of one launch).  Each tensor has 0 to 300,000
elements, each of its streams sits at its own element offset inside its
buffer (phases that agree or not), and it has a bf16 copy or none; each call
has a clip coefficient or none.  Half the examples run on the small-grid
test build of the library (64 waves per launch at most), where a batch holds
at most 32 runs, tensors of more than 32 runs (8192 elements) take their own
grid-stride launch, and the update kernel's grid-stride loop runs (the product
build splits batches and strides only above 2^33 elements).  Every
bit of every tensor's p, m, v and copy must equal the CPU checker replaying
the same calls one tensor at a time, NaN as a class.  Examples are drawn
from a fixed seed."""
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
    return H.to_np_bits(torch.from_numpy(x.astype(np.float32)).to(H.TD[kind]), kind)


def _view(bits_arr, kind):
    return bits_arr.view(np.float32) if kind == "f32" else bits_arr


@st.composite
def tensor(draw):
    return dict(n=draw(st.one_of(st.integers(0, 20), st.integers(21, 3000), st.integers(3001, 300_000))),
                offs=draw(st.lists(st.integers(0, 7), min_size=5, max_size=5)),
                with_out=draw(st.booleans()))


@st.composite
def step(draw):
    return dict(step=draw(st.integers(1, 6)),
                lr=draw(st.sampled_from([1e-5, 1e-3, 0.1])),
                b1=draw(st.sampled_from([0.8, 0.9])), b2=draw(st.sampled_from([0.95, 0.999])),
                eps=draw(st.sampled_from([1e-8, 1e-6])), wd=draw(st.sampled_from([0.0, 0.01, 0.1])),
                bc=draw(st.booleans()), coef=draw(st.sampled_from([None, 1.0, 0.37])),
                seed=draw(st.integers(0, 2**31 - 1)))


@st.composite
def cases(draw):
    k = draw(st.sampled_from([1, 2, 5, 15, 16, 17, 31, 32, 33, 40]))
    return dict(triple=draw(st.sampled_from(TRIPLES)), adamw=draw(st.booleans()),
                small_grid=draw(st.booleans()),
                tensors=draw(st.lists(tensor(), min_size=k, max_size=k)),
                steps=draw(st.lists(step(), min_size=1, max_size=3)), seed=draw(st.integers(0, 2**31 - 1)))


@property_test(200)
@given(c=cases())
def test_multi_update_equals_checker_on_random_layers(c, hip_device):
    print(f"multi property case: {c}", flush=True)
    pk, gk, sk = c["triple"]
    rng = np.random.default_rng(c["seed"])
    host, dev = [], []
    for t in c["tensors"]:
        size = t["n"] + 8
        ph = _bits(rng.normal(0, 0.02, size), pk)
        mh = _bits(rng.normal(0, 1e-3, size), sk)
        vh = _bits(np.abs(rng.normal(0, 1e-6, size)), sk)
        oh = np.zeros(size, np.uint16)
        host.append([ph, mh, vh, oh])
        dev.append([H.to_dev_bits(ph, pk, hip_device), H.to_dev_bits(mh, sk, hip_device),
                    H.to_dev_bits(vh, sk, hip_device), torch.zeros(size, dtype=torch.bfloat16, device=hip_device)])
    s0 = c["steps"][0]
    lib = H.load_small_grid() if c["small_grid"] else None
    hip = H.HipAdam(s0["lr"], (s0["b1"], s0["b2"]), s0["eps"], s0["wd"], c["adamw"], lib=lib)
    orc = O.OracleAdam(s0["lr"], (s0["b1"], s0["b2"]), s0["eps"], s0["wd"], c["adamw"])
    for s in c["steps"]:
        srng = np.random.default_rng(s["seed"])
        grads = [_bits(srng.normal(0, 1e-3, t["n"] + 8), gk) for t in c["tensors"]]
        gdev = [H.to_dev_bits(g, gk, hip_device) for g in grads]
        coef = None if s["coef"] is None else torch.tensor([s["coef"]], device=hip_device)
        args = (s["step"], s["lr"], s["b1"], s["b2"], s["eps"], s["wd"], s["bc"])
        segs = []
        for t, (pd, md, vd, od), gd in zip(c["tensors"], dev, gdev):
            n, (op, og, om, ov, oo) = t["n"], t["offs"]
            segs.append((pd[op:op + n], gd[og:og + n], md[om:om + n], vd[ov:ov + n],
                         od[oo:oo + n] if t["with_out"] else None))
        hip.update_multi(*args, segs, coef=coef)
        for t, (ph, mh, vh, oh), gh in zip(c["tensors"], host, grads):
            n, (op, og, om, ov, oo) = t["n"], t["offs"]
            orc.update(*args, _view(ph, pk)[op:op + n], _view(gh, gk)[og:og + n], _view(mh, sk)[om:om + n],
                       _view(vh, sk)[ov:ov + n], p16=KIND16[pk], g16=KIND16[gk], s16=KIND16[sk],
                       p_bf16_out=oh[oo:oo + n] if t["with_out"] else None, clip_coef=s["coef"])
    torch.cuda.synchronize()
    for k, (d, h) in enumerate(zip(dev, host)):
        for dt, want, kind in zip(d, h, (pk, sk, sk, "bf16")):
            got = H.to_np_bits(dt, kind)
            bad = np.flatnonzero(~G.same_bits(got, want, kind))
            assert bad.size == 0, (k, kind, bad[:8], got[bad[:8]], want[bad[:8]])
