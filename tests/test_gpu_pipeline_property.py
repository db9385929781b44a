"""Randomised check of the host<->HBM pipeline against the resident path.

Each example draws a dtype triple the reference registers, a size, a chunk
size and slot count, which of p, m, v, g and the bf16 copy live in host memory
(each page-locked or pageable, so the staging twins come and go), a clip
coefficient or none, and whether the calls return once queued
(overlap_host_chunks).  Two steps run through the pipeline; the same two steps
run on HBM-resident copies through the device entry point, with the same call
sequence on an optimizer of its own (same beta-power states).  Every bit of p,
m, v and the bf16 copy must agree.  The resident path is itself pinned to the
CPU checker by the parity tests.  Examples are drawn from a fixed seed."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import given
from hypothesis import strategies as st

from slideformer_amd import LayerAdam
from slideformer_amd.layer_adam import SUPPORTED_TRIPLES, HostStreamer
from tests import _hip as H
from tests._props import property_test

pytestmark = pytest.mark.gpu

TRIPLES = sorted(SUPPORTED_TRIPLES, key=str)
KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


@st.composite
def cases(draw):
    return dict(
        triple=draw(st.sampled_from(TRIPLES)),
        n=draw(st.one_of(st.integers(1, 64), st.integers(65, 5000), st.integers(5001, 120_000))),
        chunk=16 * draw(st.integers(1, 300)),
        slots=draw(st.integers(1, 4)),
        host=draw(st.lists(st.booleans(), min_size=5, max_size=5)),      # p, m, v, g, out on the host
        pinned=draw(st.lists(st.booleans(), min_size=5, max_size=5)),
        with_out=draw(st.booleans()),
        coef=draw(st.sampled_from([None, 0.25, 1.0])),
        overlap=draw(st.booleans()),
        seed=draw(st.integers(0, 2**31 - 1)),
    )


def _place(t, host, pinned, dev):
    if not host:
        return t.to(dev)
    return t.pin_memory() if pinned else t.clone()


@property_test(200)
@given(c=cases())
def test_pipeline_equals_resident_on_random_layouts(c, hip_device):
    print(f"pipeline property case: {c}", flush=True)
    dev = hip_device
    pdt, gdt, sdt = c["triple"]
    n, rng = c["n"], np.random.default_rng(c["seed"])
    if not any(c["host"][:4]) and not (c["with_out"] and c["host"][4]):
        c["host"][0] = True                       # at least one array streams
    hp, hm, hv, hg, ho = c["host"]
    pp, pm, pv, pg, po = c["pinned"]
    p0 = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(pdt)
    m0 = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(sdt)
    v0 = torch.from_numpy(np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)).to(sdt)
    grads = [torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(gdt) for _ in range(2)]
    coef = None if c["coef"] is None else torch.tensor([c["coef"]], device=dev)

    streamed = LayerAdam(lr=1e-3, weight_decay=0.01, overlap_host_chunks=c["overlap"])
    streamed._streamers[dev] = HostStreamer(dev, chunk_elems=c["chunk"], slots=c["slots"])
    resident = LayerAdam(lr=1e-3, weight_decay=0.01)
    p_s, m_s, v_s = _place(p0, hp, pp, dev), _place(m0, hm, pm, dev), _place(v0, hv, pv, dev)
    p_r, m_r, v_r = p0.to(dev), m0.to(dev), v0.to(dev)
    out_s = out_r = None
    if c["with_out"]:
        out_s = _place(torch.zeros(n, dtype=torch.bfloat16), ho, po, dev)
        out_r = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    keep = []
    for step, g in enumerate(grads, start=1):
        g_s = _place(g, hg, pg, dev)
        keep.append(g_s)
        group = dict(streamed.defaults, step=step)
        streamed.step_chunk(p_s, g_s, m_s, v_s, group, bf16_out=out_s, clip_coef=coef)
        resident.step_chunk(p_r, g.to(dev), m_r, v_r, dict(resident.defaults, step=step), bf16_out=out_r,
                            clip_coef=coef)
    streamed.synchronize()
    torch.cuda.synchronize()
    for a, b, k in ((p_s, p_r, KIND[pdt]), (m_s, m_r, KIND[sdt]), (v_s, v_r, KIND[sdt])):
        assert np.array_equal(H.to_np_bits(a, k), H.to_np_bits(b, k)), (c, k)
    if c["with_out"]:
        assert np.array_equal(H.to_np_bits(out_s, "bf16"), H.to_np_bits(out_r, "bf16")), c
