"""The reference LayerAdam's native call pattern on slideformer_amd.cpu_adam_compat,
the stand-in for its pybind module cpu_adam, on the GPU.

The calls are the ones the unchanged reference makes: create_adam(0, ..., True)
(layer_adam.py:62-72); per-tensor adam_update on host tensors as step(layer)
makes them (layer_adam.py:314-327); the runtime's chunked step_chunk calls on
slices of flat host buffers with bf16 grads (layer_adam.py:448-461,
transformer_layer.py:470-476); then the same calls on device tensors, an
unregistered dtype triple, and destroy_adam.  Every result is bit-exact with the
CPU checker replaying the same call sequence (one optimizer id, so the
beta-power state machine takes the same multiply and pow paths)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slideformer_amd import cpu_adam_compat as C
from tests import _hip as H

pytestmark = pytest.mark.gpu

LR, B1, B2, EPS, WD = 1e-3, 0.9, 0.999, 1e-8, 0.01


def _same(t, ref):
    return np.array_equal(H.to_np_bits(t, "f32"), ref.view(np.uint32))


def test_reference_call_pattern_on_host_then_device_tensors(hip_device):
    rng = np.random.default_rng(2024)
    assert C.create_adam(0, LR, B1, B2, EPS, WD, True, True) == 0
    orc = O.OracleAdam(LR, (B1, B2), EPS, WD, True)
    try:
        # step(layer): one call per parameter, fp32 grads (p.grad.data), pageable host state
        sizes = [4096 * 3 + 5, 768, 17]
        ps = [rng.normal(0, 0.02, k).astype(np.float32) for k in sizes]
        p_t = [torch.from_numpy(x.copy()) for x in ps]
        m_t = [torch.zeros(k) for k in sizes]
        v_t = [torch.zeros(k) for k in sizes]
        ms = [np.zeros(k, np.float32) for k in sizes]
        vs = [np.zeros(k, np.float32) for k in sizes]
        for step in (1, 2):
            for i, k in enumerate(sizes):
                g = rng.normal(0, 1e-3, k).astype(np.float32)
                print(f"cpu_adam stand-in: host per-tensor step {step} tensor {i} n {k}", flush=True)
                assert C.adam_update(0, step, LR, B1, B2, EPS, WD, True, p_t[i], torch.from_numpy(g.copy()),
                                     m_t[i], v_t[i]) == 0
                orc.update(step, LR, B1, B2, EPS, WD, True, ps[i], g, ms[i], vs[i])
        for i in range(len(sizes)):
            assert _same(p_t[i], ps[i]) and _same(m_t[i], ms[i]) and _same(v_t[i], vs[i]), i

        # the runtime's chunk calls: slices of flat host buffers, bf16 grads
        n, chunk = 100_003, 30_000
        P = rng.normal(0, 0.02, n).astype(np.float32)
        Pt, Mt, Vt = torch.from_numpy(P.copy()), torch.zeros(n), torch.zeros(n)
        M, V = np.zeros(n, np.float32), np.zeros(n, np.float32)
        for step in (3, 4):
            g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
            gb = H.to_np_bits(g, "bf16")
            for cs in range(0, n, chunk):
                ce = min(n, cs + chunk)
                print(f"cpu_adam stand-in: host chunk step {step} [{cs}:{ce}]", flush=True)
                C.adam_update(0, step, LR, B1, B2, EPS, WD, True, Pt[cs:ce], g[cs:ce], Mt[cs:ce], Vt[cs:ce])
                orc.update(step, LR, B1, B2, EPS, WD, True, P[cs:ce], gb[cs:ce], M[cs:ce], V[cs:ce], g16="bf16")
        assert _same(Pt, P) and _same(Mt, M) and _same(Vt, V)

        # the same flat state moved to the device: asynchronous calls on the current stream
        Pd, Md, Vd = Pt.to(hip_device), Mt.to(hip_device), Vt.to(hip_device)
        for step in (5, 6):
            g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
            gb = H.to_np_bits(g, "bf16")
            gd = g.to(hip_device)
            if step == 6:
                # an unregistered triple (bf16 params, f16 grads, f32 state): the
                # state advances, then the reference's error
                with pytest.raises(RuntimeError, match="is not supported on current hardware"):
                    C.adam_update(0, step, LR, B1, B2, EPS, WD, True, Pd[:16].bfloat16(), gd[:16].half(),
                                  Md[:16], Vd[:16])
                e = np.zeros(0, np.float32)
                orc.update(step, LR, B1, B2, EPS, WD, True, e, e.copy(), e.copy(), e.copy())
            for cs in range(0, n, chunk):
                ce = min(n, cs + chunk)
                print(f"cpu_adam stand-in: device chunk step {step} [{cs}:{ce}]", flush=True)
                C.adam_update(0, step, LR, B1, B2, EPS, WD, True, Pd[cs:ce], gd[cs:ce], Md[cs:ce], Vd[cs:ce])
                orc.update(step, LR, B1, B2, EPS, WD, True, P[cs:ce], gb[cs:ce], M[cs:ce], V[cs:ce], g16="bf16")
        torch.cuda.synchronize()
        assert _same(Pd, P) and _same(Md, M) and _same(Vd, V)

        # a host master beside device moments is refused before anything runs
        before = H.to_np_bits(Pt, "f32")
        with pytest.raises(RuntimeError, match="all be in host memory or all on one"):
            C.adam_update(0, 7, LR, B1, B2, EPS, WD, True, Pt, gd, Md, Vd)
        torch.cuda.synchronize()
        assert np.array_equal(H.to_np_bits(Pt, "f32"), before) and _same(Md, M) and _same(Vd, V)
    finally:
        assert C.destroy_adam(0) == 0
    # the id is gone: a further update is an error, not a null dereference
    with pytest.raises(RuntimeError, match="invalid argument"):
        C.adam_update(0, 8, LR, B1, B2, EPS, WD, True, *[torch.zeros(4, device=hip_device) for _ in range(4)])
