"""The clipped step under HIP graph capture, through the C-ABI.

la_grad_norm_clip_noalloc needs no workspace, so a caller that cannot
allocate inside a captured region (graph capture) can still clip: the grad
norm, the clip coefficient and the fused update are captured once and
replayed.  The scalars of la_adamw_step are fixed at capture time (the host
state machine does not run on replay), so each replay is one more step with
the same scalars.  Every replay is checked bit for bit against the same
sequence run eagerly (la_grad_norm_clip with a workspace, then la_adamw_step
with the same scalars), with eager work and synchronisations of the program
in between.  Nothing in the captured region clears memory with a memset."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from slideformer_amd import _lib
from tests import _hip as H

pytestmark = pytest.mark.gpu


def test_norm_clip_and_update_captured_and_replayed(hip_device):
    L = _lib.load()
    dev = hip_device
    n = 1_000_003                     # a scalar tail of 3 elements
    gen = torch.Generator(device=dev)
    gen.manual_seed(90)
    p0 = torch.randn(n, generator=gen, device=dev) * 0.02
    m0 = torch.randn(n, generator=gen, device=dev) * 1e-4
    v0 = torch.rand(n, generator=gen, device=dev) * 1e-8
    g = (torch.randn(n, generator=gen, device=dev) * 3e-3).bfloat16()
    assert L.la_create(91, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0) == 0
    sc = _lib.LaScalars()
    assert L.la_scalars(91, 1, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, ctypes.byref(sc)) == 0

    # graph side: its own buffers, the scratch of the no-allocation norm
    p, m, v = p0.clone(), m0.clone(), v0.clone()
    out = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    sq = torch.zeros(1, dtype=torch.float64, device=dev)
    coef = torch.zeros(1, device=dev)
    norm = torch.zeros(1, device=dev)

    def step(stream):
        rc = L.la_grad_norm_clip_noalloc(_lib.LA_BF16, g.data_ptr(), n, sq.data_ptr(), 0, 1.0, coef.data_ptr(),
                                         norm.data_ptr(), stream)
        assert rc == 0, L.la_strerror(rc)
        rc = L.la_adamw_step(ctypes.byref(sc), _lib.LA_F32, p.data_ptr(), _lib.LA_BF16, g.data_ptr(), _lib.LA_F32,
                             m.data_ptr(), v.data_ptr(), n, out.data_ptr(), coef.data_ptr(), stream)
        assert rc == 0, L.la_strerror(rc)

    # one eager call first: the library looks up its scratch address on this device
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step(side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    p.copy_(p0)
    m.copy_(m0)
    v.copy_(v0)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    # capture records the work, it does not run it
    assert torch.equal(p, p0)

    # eager side: the same sequence with a workspace, on copies
    pe, me, ve = p0.clone(), m0.clone(), v0.clone()
    oe = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(L.la_grad_sqnorm_workspace(n) // 8, dtype=torch.float64, device=dev)
    sqe = torch.zeros(1, dtype=torch.float64, device=dev)
    ce = torch.zeros(1, device=dev)
    ne = torch.zeros(1, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    for replay in range(4):
        print(f"graph replay {replay}", flush=True)
        graph.replay()
        assert L.la_grad_norm_clip(_lib.LA_BF16, g.data_ptr(), n, ws.data_ptr(), ws.numel() * 8, sqe.data_ptr(),
                                   0, 1.0, ce.data_ptr(), ne.data_ptr(), st) == 0
        assert L.la_adamw_step(ctypes.byref(sc), _lib.LA_F32, pe.data_ptr(), _lib.LA_BF16, g.data_ptr(),
                               _lib.LA_F32, me.data_ptr(), ve.data_ptr(), n, oe.data_ptr(), ce.data_ptr(), st) == 0
        # eager work of the program between replays
        junk = torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert 0.0 < coef.item() < 1.0
        for a, b in ((sq, sqe), (coef, ce), (norm, ne)):
            assert np.array_equal(a.cpu().numpy().view(np.uint8), b.cpu().numpy().view(np.uint8)), replay
        for a, b, k in ((p, pe, "f32"), (m, me, "f32"), (v, ve, "f32"), (out, oe, "bf16")):
            assert np.array_equal(H.to_np_bits(a, k), H.to_np_bits(b, k)), (replay, k)
    assert not torch.equal(p, p0)
    del graph
    L.la_destroy(91)
