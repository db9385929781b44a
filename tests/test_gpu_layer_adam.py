"""The LayerAdam API (drop-in for optimizer/layer_adam/layer_adam.py) on the MI355X."""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slideformer_amd import LayerAdam
from tests import _hip as H

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("where", ["device", "host"])
@pytest.mark.parametrize("gdtype", [torch.float32, torch.bfloat16])
def test_known_answer_vs_torch_adamw(gdtype, where, hip_device):
    """The reference's only numeric test, test_shared_data_parallel.py:53-93, single
    process: sizes (19, 3, 0) in chunks of 5, five steps, lr change at step 3.
    The reference calls step_chunk on CPU tensors (:70-73); "host" does the
    same here (streamed through HBM), "device" keeps everything in HBM."""
    adam = LayerAdam(lr=0.01, betas=(0.8, 0.95), eps=1e-6, weight_decay=0.1)
    chunk = 5
    at = hip_device if where == "device" else "cpu"
    for layer, size in enumerate((19, 3, 0)):
        initial = torch.linspace(-0.5, 0.5, size)
        params = initial.clone().to(at)
        first = torch.zeros(size, device=at)
        second = torch.zeros(size, device=at)
        reference = torch.nn.Parameter(initial.clone())
        tadam = torch.optim.AdamW([reference], lr=0.01, betas=(0.8, 0.95), eps=1e-6,
                                  weight_decay=0.1, foreach=False)
        for step in range(1, 6):
            grads = ((torch.arange(size) * 0.13 + step * 0.2).sin() * 0.1).to(gdtype)
            gd = grads.to(at)
            lr = 0.01 if step < 3 else 0.003
            tadam.param_groups[0]["lr"] = lr
            for start in range(0, size, chunk):
                end = min(start + chunk, size)
                adam.step_chunk(params[start:end], gd[start:end], first[start:end], second[start:end],
                                dict(adam.defaults, step=step, lr=lr))
            reference.grad = grads.float()
            tadam.step()
            torch.testing.assert_close(params.cpu(), reference.detach(), rtol=1e-6, atol=1e-7)
            st = tadam.state[reference]
            torch.testing.assert_close(first.cpu(), st["exp_avg"])
            torch.testing.assert_close(second.cpu(), st["exp_avg_sq"])


def _oracle_layer_step(orc, step, pieces, grads, ms, vs):
    for p, g, m, v in zip(pieces, grads, ms, vs):
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p, g, m, v,
                   g16="bf16" if g.dtype == np.uint16 else None)


def test_step_per_tensor_and_grad_views(hip_device):
    """step(layer_idx) and step_with_grad_views call adam_update once per tensor
    (layer_adam.py:299-327, 391-422), which matters for the scalar tails."""
    shapes = [(37, 5), (5,), (64, 3), (1,)]
    rng = np.random.default_rng(0)
    init = [rng.normal(0, 0.02, int(np.prod(s))).astype(np.float32) for s in shapes]
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).view(s).to(hip_device)) for x, s in zip(init, shapes)]
    assert adam.add_layer_params(0, params) == 0
    assert adam.add_layer_params(1, []) == -1
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    hp = [x.copy() for x in init]
    hm = [np.zeros_like(x) for x in init]
    hv = [np.zeros_like(x) for x in init]
    for step in range(1, 4):
        grads = [torch.from_numpy(rng.normal(0, 1e-3, x.size).astype(np.float32)) for x in init]
        if step % 2:
            # p.grad must have the param's dtype: the (f32, f32, f32) triple
            gbits = [g.numpy().copy() for g in grads]
            for p, g, s in zip(params, grads, shapes):
                p.grad = g.view(s).to(hip_device)
            adam.step(0)
        else:
            # grad views carry the runtime's bf16 grads (transformer_layer.py:225,232)
            grads = [g.bfloat16() for g in grads]
            gbits = [H.to_np_bits(g, "bf16") for g in grads]
            adam.step_with_grad_views(0, {p: g.view(s).to(hip_device) for p, g, s in zip(params, grads, shapes)})
        _oracle_layer_step(orc, step, hp, gbits, hm, hv)
    torch.cuda.synchronize()
    assert adam.param_groups[0]["step"] == 3
    for p, x, m, v in zip(params, hp, hm, hv):
        assert np.array_equal(H.to_np_bits(p.data.reshape(-1), "f32"), x.view(np.uint32))
        st = adam.state[p]
        assert np.array_equal(H.to_np_bits(st["exp_avg"].reshape(-1), "f32"), m.view(np.uint32))
        assert np.array_equal(H.to_np_bits(st["exp_avg_sq"].reshape(-1), "f32"), v.view(np.uint32))


@pytest.mark.parametrize("where", ["device", "host"])
def test_step_per_tensor_with_clip_coef(where, hip_device):
    """step(layer) and step_with_grad_views with the keyword-only clip_coef:
    the layer's grads go through clip_grad_norm (one la_grad_norm_multi call)
    and every tensor's update scales its grads by the coefficient, bit-exact
    with the checker fed the same coefficient.  On host tensors the per-tensor
    calls stream through HBM with the device coefficient."""
    shapes = [(37, 5), (5,), (64, 3), (1,), (300, 7)]
    rng = np.random.default_rng(12)
    init = [rng.normal(0, 0.02, int(np.prod(s))).astype(np.float32) for s in shapes]
    at = hip_device if where == "device" else "cpu"
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).view(s).to(at)) for x, s in zip(init, shapes)]
    adam.add_layer_params(0, params)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    hp = [x.copy() for x in init]
    hm = [np.zeros_like(x) for x in init]
    hv = [np.zeros_like(x) for x in init]
    for step in range(1, 4):
        grads = [torch.from_numpy(rng.normal(0, 1e-2, x.size).astype(np.float32)) for x in init]
        if step % 2:
            gbits = [g.numpy().copy() for g in grads]
            for p, g, s in zip(params, grads, shapes):
                p.grad = g.view(s).to(at)
            coef, _ = adam.clip_grad_norm([g.to(hip_device) for g in grads], 1e-2)
            adam.step(0, clip_coef=coef)
        else:
            grads = [g.bfloat16() for g in grads]
            gbits = [H.to_np_bits(g, "bf16") for g in grads]
            coef, _ = adam.clip_grad_norm([g.to(hip_device) for g in grads], 1e-2)
            adam.step_with_grad_views(0, {p: g.view(s).to(at) for p, g, s in zip(params, grads, shapes)},
                                      clip_coef=coef)
        c = float(coef.item())
        assert 0.0 < c < 1.0
        for x, g, m, v in zip(hp, gbits, hm, hv):
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, x, g, m, v,
                       g16="bf16" if g.dtype == np.uint16 else None, clip_coef=c)
    torch.cuda.synchronize()
    for p, x, m, v in zip(params, hp, hm, hv):
        assert np.array_equal(H.to_np_bits(p.data.reshape(-1), "f32"), x.view(np.uint32))
        st = adam.state[p]
        assert np.array_equal(H.to_np_bits(st["exp_avg"].reshape(-1), "f32"), m.view(np.uint32))
        assert np.array_equal(H.to_np_bits(st["exp_avg_sq"].reshape(-1), "f32"), v.view(np.uint32))


def test_host_tensors_are_staged_through_hbm(hip_device):
    """The reference's layout (fp32 master + bf16 grads in host RAM) still works:
    the update runs on the GPU in 16 Mi-element pieces and the call returns after
    completion.  Bit-exact with the oracle across a piece boundary."""
    from slideformer_amd.layer_adam import HOST_STAGE_ELEMS
    n = HOST_STAGE_ELEMS + 21
    rng = np.random.default_rng(5)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32))
    m = torch.zeros(n)
    v = torch.zeros(n)
    out = torch.empty(n, dtype=torch.bfloat16)
    ph, mh, vh = p.numpy().copy(), m.numpy().copy(), v.numpy().copy()
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        adam.step_chunk(p, g, m, v, dict(adam.defaults, step=step), bf16_out=out)
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16")
    assert np.array_equal(p.numpy().view(np.uint32), ph.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mh.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vh.view(np.uint32))
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), O.f32_to_bf16(ph))


def test_clip_grad_norm_and_side_stream(hip_device):
    n = 3_000_017
    rng = np.random.default_rng(8)
    adam = LayerAdam(lr=1e-5, weight_decay=0.01)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(hip_device)
    m = torch.zeros(n, device=hip_device)
    v = torch.zeros(n, device=hip_device)
    g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16().to(hip_device)
    ph = p.cpu().numpy().copy()
    mh = np.zeros(n, np.float32)
    vh = np.zeros(n, np.float32)
    side = torch.cuda.Stream(device=hip_device)
    side.wait_stream(torch.cuda.current_stream(hip_device))
    with torch.cuda.stream(side):
        coef, norm = adam.clip_grad_norm([g[:1000], g[1000:]], 1.0, stream=side)
        adam.step_chunk(p, g, m, v, dict(adam.defaults, step=1), clip_coef=coef, stream=side)
    side.synchronize()
    sq = O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16")
    c_ref, n_ref = O.clip_coef(sq, 1.0)
    assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref) and c_ref < 1
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    orc.update(1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16",
               clip_coef=float(coef.item()))
    assert np.array_equal(H.to_np_bits(p, "f32"), ph.view(np.uint32))
    assert np.array_equal(H.to_np_bits(m, "f32"), mh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(v, "f32"), vh.view(np.uint32))


def test_errors(hip_device):
    adam = LayerAdam()
    a = torch.zeros(10, device=hip_device)
    with pytest.raises(RuntimeError, match="params must be contiguous"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, torch.zeros(10, 2, device=hip_device).t(),
                         a, a, a)
    with pytest.raises(RuntimeError, match="is not supported on current hardware"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a, a.bfloat16(), a.bfloat16())
    with pytest.raises(RuntimeError, match="unsupported device type: meta"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a.to("meta"), a, a)
    with pytest.raises(RuntimeError, match="size mismatch"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a[:5], a, a)


# ---------------------------------------------------------------------------
# host-state streaming (native chunk pipeline)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("chunk,slots,pinned,g_host,out_host", [
    (1024, 2, True, False, False),     # many chunks, slot reuse, device grads + device bf16 copy
    (4096, 3, True, True, True),       # the runtime's layout: grads and copy on the host
    (16 * 1024 + 16, 1, False, True, False),  # pageable host memory, a single slot
])
def test_pipeline_matches_oracle(chunk, slots, pinned, g_host, out_host, hip_device):
    from slideformer_amd.layer_adam import HostStreamer
    print(f"pipeline chunk={chunk} slots={slots} pinned={pinned} g_host={g_host} out_host={out_host}", flush=True)
    n = 100_003
    rng = np.random.default_rng(chunk + slots)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32))
    m = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32))
    v = torch.from_numpy(np.abs(rng.normal(0, 1e-6, n)).astype(np.float32))
    if pinned:
        p, m, v = p.pin_memory(), m.pin_memory(), v.pin_memory()
    ph, mh, vh = p.numpy().copy(), m.numpy().copy(), v.numpy().copy()
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=chunk, slots=slots)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    out = torch.empty(n, dtype=torch.bfloat16, device="cpu" if out_host else hip_device)
    for step in (1, 2, 3):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        gd = g if g_host else g.to(hip_device)
        adam.step_chunk(p, gd, m, v, dict(adam.defaults, step=step), bf16_out=out)
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16")
        st = adam.last_stream_stats
        assert st.chunks == -(-n // (chunk // 16 * 16))
        assert st.h2d_bytes == n * (12 + (2 if g_host else 0))
        assert st.d2h_bytes == n * (12 + (2 if out_host else 0))
    torch.cuda.synchronize()
    assert np.array_equal(p.numpy().view(np.uint32), ph.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mh.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(ph))


def test_pipeline_with_clip_and_odd_tail(hip_device):
    """Host state, device grads with a device clip coefficient; n with a scalar
    tail in the last chunk only."""
    from slideformer_amd.layer_adam import HostStreamer
    n = 3 * 2048 + 13
    rng = np.random.default_rng(77)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).pin_memory()
    m = torch.zeros(n).pin_memory()
    v = torch.zeros(n).pin_memory()
    ph, mh, vh = p.numpy().copy(), m.numpy().copy(), v.numpy().copy()
    adam = LayerAdam(lr=1e-5, weight_decay=0.01)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=2048, slots=2)
    g = torch.from_numpy(rng.normal(0, 1e-1, n).astype(np.float32)).bfloat16()
    gd = g.to(hip_device)
    coef, _ = adam.clip_grad_norm([gd], 1.0)
    adam.step_chunk(p, gd, m, v, dict(adam.defaults, step=1), clip_coef=coef)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    orc.update(1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16",
               clip_coef=float(coef.item()))
    assert float(coef.item()) < 1.0
    assert np.array_equal(p.numpy().view(np.uint32), ph.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mh.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vh.view(np.uint32))


def test_global_norm_in_sliding_order(hip_device):
    """Per-layer grads added one at a time (last layer first), one coefficient:
    equal to the oracle's norm over all buffers."""
    rng = np.random.default_rng(21)
    sizes = [7, 4096 + 3, 100_000, 1]
    grads = [torch.from_numpy(rng.normal(0, 1e-2, k).astype(np.float32)).bfloat16() for k in sizes]
    adam = LayerAdam()
    acc = adam.grad_norm_begin(hip_device)
    for g in reversed(grads):
        acc.add(g.to(hip_device))
    coef, norm = acc.finish(1.0)
    sq = sum(O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16") for g in grads)
    assert abs(acc.sqnorm.item() - sq) <= 1e-12 * sq
    c_ref, n_ref = O.clip_coef(acc.sqnorm.item(), 1.0)
    assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)
    empty = adam.grad_norm_begin(hip_device)
    c0, n0 = empty.finish(1.0)
    assert c0.item() == 1.0 and n0.item() == 0.0


def test_runtime_chunk_protocol_with_update_thread(hip_device):
    """The runtime's protocol (transformer_layer.py:343-422, 453-493) on device
    tensors: a producer publishes (cs, ce, event) per 32 Mi-element-style chunk
    (here 4096) into a queue, an update thread waits on each event and calls
    step_chunk on its own stream, writing the bf16 copy into a cache-unit
    buffer; update_finished is set at the end.  Bit-exact with the oracle."""
    import queue
    import threading

    n, chunk = 3 * 4096 + 5, 4096
    rng = np.random.default_rng(31)
    p_h = rng.normal(0, 0.02, n).astype(np.float32)
    m_h = np.zeros(n, np.float32)
    v_h = np.zeros(n, np.float32)
    adam = LayerAdam(lr=1e-5, weight_decay=0.01)
    p = torch.from_numpy(p_h.copy()).to(hip_device)
    adam.add_layer_params(0, [torch.nn.Parameter(p)])
    cache_unit = torch.zeros(n, dtype=torch.bfloat16, device=hip_device)
    produce = torch.cuda.Stream(device=hip_device)
    update_stream = torch.cuda.Stream(device=hip_device)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        g32 = rng.normal(0, 1e-3, n).astype(np.float32)
        grad = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
        q: "queue.Queue" = queue.Queue()
        finished = threading.Event()
        errors = []

        def update_thread():
            try:
                group = adam.begin_chunk_step(0)
                while True:
                    item = q.get()
                    if item is None:
                        break
                    cs, ce, ev = item
                    update_stream.wait_event(ev)
                    adam.step_chunk(p[cs:ce], grad[cs:ce], adam.exp_avg_flat[0][cs:ce],
                                    adam.exp_avg_sq_flat[0][cs:ce], group, bf16_out=cache_unit[cs:ce],
                                    stream=update_stream)
                adam.end_chunk_step(0)
                update_stream.synchronize()
            except Exception as exc:  # surfaced to the main thread like Future.result()
                errors.append(exc)
            finally:
                finished.set()

        t = threading.Thread(target=update_thread)
        t.start()
        g_src = torch.from_numpy(g32).bfloat16()
        with torch.cuda.stream(produce):
            for cs in range(0, n, chunk):
                ce = min(cs + chunk, n)
                grad[cs:ce].copy_(g_src[cs:ce].to(hip_device, non_blocking=False))
                ev = torch.cuda.Event()
                ev.record(produce)
                q.put((cs, ce, ev))
        q.put(None)
        finished.wait(timeout=60)
        t.join(timeout=60)
        assert not errors, errors
        g_bits = H.to_np_bits(g_src, "bf16")
        for cs in range(0, n, chunk):
            ce = min(cs + chunk, n)
            orc.update(step, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p_h[cs:ce], g_bits[cs:ce], m_h[cs:ce],
                       v_h[cs:ce], g16="bf16")
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p, "f32"), p_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(adam.exp_avg_flat[0], "f32"), m_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(adam.exp_avg_sq_flat[0], "f32"), v_h.view(np.uint32))
    assert np.array_equal(H.to_np_bits(cache_unit, "bf16"), O.f32_to_bf16(p_h))


@pytest.mark.parametrize("moments_in_hbm,pinned", [(False, False), (True, False), (True, True)])
def test_runtime_protocol_on_host_state_with_shared_grad_buffer(moments_in_hbm, pinned, hip_device):
    """The runtime's host-side protocol end to end, with injected delays as in
    the reference's own test (test_shared_data_parallel.py:69,82): layers in
    sliding order share ONE page-locked grad buffer (transformer_layer.py:206,
    the shared cpu_grad_tensor); a producer copies each layer's device grads
    into it chunk by chunk, recording an event per chunk (:343-422), but
    starts a layer only after the previous layer's update_finished (:348-351);
    an update thread waits on each event and calls step_chunk on the host
    master chunk, the shared grad chunk and the moments (:453-493), with
    overlap_host_chunks=True, then end_chunk_step and update_finished.  Three
    steps, bit-exact with the oracle; host moments or moments in HBM;
    pageable or page-locked masters."""
    import queue
    import threading
    import time

    sizes, chunk = [20_000, 7, 13_003], 4096
    rng = np.random.default_rng(41 + 2 * int(moments_in_hbm) + int(pinned))
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, overlap_host_chunks=True,
                     moments_device=hip_device if moments_in_hbm else None)
    from slideformer_amd.layer_adam import HostStreamer
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=2048, slots=3)
    masters, host = [], []
    for i, k in enumerate(sizes):
        p0 = rng.normal(0, 0.02, k).astype(np.float32)
        t = torch.from_numpy(p0.copy())
        masters.append(t.pin_memory() if pinned else t)
        host.append([p0.copy(), np.zeros(k, np.float32), np.zeros(k, np.float32)])
        adam.add_layer_params(i, [torch.nn.Parameter(masters[i])])
    shared_grad = torch.empty(max(sizes), dtype=torch.bfloat16, pin_memory=True)
    producer = torch.cuda.Stream(device=hip_device)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    finished_prev = threading.Event()
    finished_prev.set()
    errors = []
    for step in range(1, 4):
        for i in reversed(range(len(sizes))):                      # sliding order
            k = sizes[i]
            g_dev = (torch.from_numpy(rng.normal(0, 1e-3, k).astype(np.float32))).bfloat16().to(hip_device)
            g_bits = H.to_np_bits(g_dev, "bf16")
            q: "queue.Queue" = queue.Queue()
            finished = threading.Event()

            def update_thread(i=i, q=q, finished=finished):
                try:
                    group = adam.begin_chunk_step(i)
                    while True:
                        item = q.get()
                        if item is None:
                            break
                        cs, ce, ev = item
                        ev.synchronize()
                        adam.step_chunk(masters[i][cs:ce], shared_grad[cs:ce], adam.exp_avg_flat[i][cs:ce],
                                        adam.exp_avg_sq_flat[i][cs:ce], group)
                        time.sleep(float(rng.uniform(0, 0.002)))
                    adam.end_chunk_step(i)
                except Exception as exc:
                    errors.append(exc)
                finally:
                    finished.set()

            # the next layer's D2H into the shared buffer waits for the previous update
            assert finished_prev.wait(timeout=60)
            t = threading.Thread(target=update_thread)
            t.start()
            with torch.cuda.stream(producer):
                for cs in range(0, k, chunk):
                    ce = min(cs + chunk, k)
                    shared_grad[cs:ce].copy_(g_dev[cs:ce], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(producer)
                    q.put((cs, ce, ev))
                    time.sleep(float(rng.uniform(0, 0.002)))
            q.put(None)
            t.join(timeout=60)
            assert not t.is_alive()
            assert not errors, errors
            finished_prev = finished
            for cs in range(0, k, chunk):
                ce = min(cs + chunk, k)
                orc.update(adam.param_groups[i]["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True,
                           host[i][0][cs:ce], g_bits[cs:ce], host[i][1][cs:ce], host[i][2][cs:ce], g16="bf16")
    torch.cuda.synchronize()
    for i in range(len(sizes)):
        assert np.array_equal(masters[i].numpy().view(np.uint32), host[i][0].view(np.uint32)), i
        assert np.array_equal(H.to_np_bits(adam.exp_avg_flat[i], "f32"), host[i][1].view(np.uint32)), i
        assert np.array_equal(H.to_np_bits(adam.exp_avg_sq_flat[i], "f32"), host[i][2].view(np.uint32)), i


@pytest.mark.parametrize("fraction,prefetch", [(1.0, True), (0.3, False)])
def test_nvme_offload_in_sliding_order(fraction, prefetch, hip_device, tmp_path):
    """Host state with the moments offloaded to files between layer steps
    (layer_adam.py:92-106, 200-247): layers stepped last-to-first for two
    iterations with the runtime's chunk calls; prefetch loads layer i-1 while
    layer i is stepped.  Bit-exact with the oracle."""
    sizes = [5000, 4096 + 7, 300, 10_001]
    L_ = len(sizes)
    rng = np.random.default_rng(int(fraction * 10) + prefetch)
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, num_layer=L_, nvme_offload_fraction=fraction,
                     offload_dir=str(tmp_path), prefetch=prefetch)
    p_host = [rng.normal(0, 0.02, k).astype(np.float32) for k in sizes]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy())) for x in p_host]
    for i, p in enumerate(params):
        adam.add_layer_params(i, [p])
    m_h = [np.zeros(k, np.float32) for k in sizes]
    v_h = [np.zeros(k, np.float32) for k in sizes]
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for it in range(2):
        for idx in range(L_ - 1, -1, -1):
            g = torch.from_numpy(rng.normal(0, 1e-3, sizes[idx]).astype(np.float32)).bfloat16()
            group = adam.begin_chunk_step(idx)
            # prefetch=False: begin_chunk_step itself fences the layer's read
            assert adam.exp_avg_flat[idx].untyped_storage().nbytes() == sizes[idx] * 4
            adam.step_chunk(params[idx].data, g.to(hip_device), adam.exp_avg_flat[idx],
                            adam.exp_avg_sq_flat[idx], group)
            adam.end_chunk_step(idx)
            orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p_host[idx], H.to_np_bits(g, "bf16"),
                       m_h[idx], v_h[idx], g16="bf16")
    adam.offloader.sync_write_events()
    for idx in range(L_):
        assert np.array_equal(params[idx].data.numpy().view(np.uint32), p_host[idx].view(np.uint32))
        adam._load_layer(idx)
        adam.offloader.sync_read_events()
        assert np.array_equal(adam.exp_avg_flat[idx].numpy().view(np.uint32), m_h[idx].view(np.uint32))
        if fraction > 0.5:
            assert np.array_equal(adam.exp_avg_sq_flat[idx].numpy().view(np.uint32), v_h[idx].view(np.uint32))
        else:
            assert adam.exp_avg_sq_flat[idx].untyped_storage().nbytes() == sizes[idx] * 4
            assert np.array_equal(adam.exp_avg_sq_flat[idx].numpy().view(np.uint32), v_h[idx].view(np.uint32))


def test_page_locked_empty_is_exact_and_page_locked(hip_device):
    """_lib.page_locked_empty: one hipHostMalloc of exactly the bytes asked for
    (torch's pinned allocator would round 872 MB up to 1 GiB), seen as
    page-locked by torch and by the pipeline, usable as a copy source and
    target, and released with its last tensor."""
    import gc

    from slideformer_amd import _lib
    n = 218_112_000 // 64 + 5                       # not a power of two
    t = _lib.page_locked_empty(n, torch.float32)
    assert t.numel() == n and t.untyped_storage().nbytes() == 4 * n and _lib.is_page_locked(t)
    assert _lib.is_page_locked(t[n // 2:]) and not _lib.is_page_locked(torch.empty(n))
    t.copy_(torch.arange(n, dtype=torch.float32))
    d = t.to(hip_device, non_blocking=True)
    back = _lib.page_locked_empty(n, torch.float32)
    back.copy_(d * 2, non_blocking=True)
    torch.cuda.synchronize()
    assert torch.equal(back, torch.arange(n, dtype=torch.float32) * 2)
    assert _lib.page_locked_empty(0, torch.bfloat16).numel() == 0
    del t, back
    gc.collect()
    # the same amount again, many times over: the earlier buffers were released
    for _ in range(8):
        x = _lib.page_locked_empty(1 << 28, torch.uint8)   # 256 MiB
        assert _lib.is_page_locked(x)
        del x
        gc.collect()


def test_pinned_host_state_layer_step(hip_device):
    """pin_host_state=True: add_layer_params allocates page-locked host moments;
    step(layer) on host params streams them; bit-exact with the oracle."""
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, pin_host_state=True)
    rng = np.random.default_rng(41)
    x = rng.normal(0, 0.02, 50_003).astype(np.float32)
    p = torch.nn.Parameter(torch.from_numpy(x.copy()))
    adam.add_layer_params(0, [p])
    from slideformer_amd import _lib
    assert _lib.is_page_locked(adam.exp_avg_flat[0]) and _lib.is_page_locked(adam.exp_avg_sq_flat[0])
    m_h, v_h = np.zeros_like(x), np.zeros_like(x)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        g = rng.normal(0, 1e-3, x.size).astype(np.float32)
        p.grad = torch.from_numpy(g.copy())
        adam.step(0)
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, x, g, m_h, v_h)
    assert np.array_equal(p.data.numpy().view(np.uint32), x.view(np.uint32))
    assert np.array_equal(adam.exp_avg_flat[0].numpy().view(np.uint32), m_h.view(np.uint32))
    assert np.array_equal(adam.exp_avg_sq_flat[0].numpy().view(np.uint32), v_h.view(np.uint32))


@pytest.mark.parametrize("pinned_p, g_host, out_host", [
    (False, False, False),   # the reference's layout for moments: every state array pageable
    (True, True, True),      # pinned master, pageable moments, pageable host grads and copy
])
def test_pageable_state_staged_through_page_locked_twins(pinned_p, g_host, out_host, hip_device):
    """Pageable host arrays are copied by the native host threads through the
    page-locked twins of the slots (la_pipeline_set_host_staging): same bits as
    the runtime's own bounce path and as the oracle, over 7 chunks in 3 slots;
    the staged byte count covers exactly the pageable arrays."""
    from slideformer_amd.layer_adam import HostStreamer
    n, chunk, slots = 7 * 4096 - 5, 4096, 3
    rng = np.random.default_rng(90 + pinned_p)
    p0 = rng.normal(0, 0.02, n).astype(np.float32)
    m0 = rng.normal(0, 1e-3, n).astype(np.float32)
    v0 = np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)
    g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
    results = []
    for stage in (True, False):
        print(f"staged={stage} pinned_p={pinned_p} g_host={g_host} out_host={out_host}", flush=True)
        p = torch.from_numpy(p0.copy())
        if pinned_p:
            p = p.pin_memory()
        m, v = torch.from_numpy(m0.copy()), torch.from_numpy(v0.copy())
        assert not m.is_pinned() and not v.is_pinned()
        gd = g.clone() if g_host else g.to(hip_device)
        out = torch.empty(n, dtype=torch.bfloat16, device="cpu" if out_host else hip_device)
        adam = LayerAdam(lr=1e-3, weight_decay=0.01)
        adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=chunk, slots=slots, host_threads=3,
                                                   stage_pageable=stage)
        for step in (1, 2):
            adam.step_chunk(p, gd, m, v, dict(adam.defaults, step=step), bf16_out=out)
            st = adam.last_stream_stats
            assert st.chunks == 7
            if stage:
                per_elem = (0 if pinned_p else 8) + 16 + (2 if g_host else 0) + (2 if out_host else 0)
                assert st.staged_bytes == n * per_elem
            else:
                assert st.staged_bytes == 0
        results.append([H.to_np_bits(t, k) for t, k in ((p, "f32"), (m, "f32"), (v, "f32"), (out, "bf16"))])
    for a, b in zip(*results):
        assert np.array_equal(a, b)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    ph, mh, vh = p0.copy(), m0.copy(), v0.copy()
    for step in (1, 2):
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16")
    assert np.array_equal(results[0][0], ph.view(np.uint32))
    assert np.array_equal(results[0][1], mh.view(np.uint32))
    assert np.array_equal(results[0][2], vh.view(np.uint32))
    assert np.array_equal(results[0][3], O.f32_to_bf16(ph))


@pytest.mark.parametrize("pinned", [True, False])
def test_overlapped_host_chunks_in_the_runtime_protocol(pinned, hip_device):
    """LayerAdam(overlap_host_chunks=True) in the runtime's protocol on host
    state (transformer_layer.py:453-493): begin_chunk_step, one step_chunk per
    5000-element chunk with host grads, end_chunk_step.  The step_chunk calls
    return once queued and stream on behind each other through a 2048-element
    pipeline of 3 slots; end_chunk_step completes them.  Then two steps are
    queued back to back on the same bytes without end_chunk_step in between,
    which makes the second call settle the first.  Bit-exact with the oracle
    after every step, page-locked (no staging) and pageable (staged) state."""
    from slideformer_amd.layer_adam import HostStreamer
    n, call = 23_456, 5000
    rng = np.random.default_rng(60 + int(pinned))
    p0 = rng.normal(0, 0.02, n).astype(np.float32)
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, pin_host_state=pinned, overlap_host_chunks=True)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=2048, slots=3)
    master = torch.from_numpy(p0.copy())
    if pinned:
        master = master.pin_memory()
    adam.add_layer_params(0, [torch.nn.Parameter(master)])
    m, v = adam.exp_avg_flat[0], adam.exp_avg_sq_flat[0]
    from slideformer_amd import _lib
    assert _lib.is_page_locked(m) == pinned and master.is_pinned() == pinned
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    ph, mh, vh = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)

    def check():
        assert np.array_equal(master.numpy().view(np.uint32), ph.view(np.uint32))
        assert np.array_equal(m.numpy().view(np.uint32), mh.view(np.uint32))
        assert np.array_equal(v.numpy().view(np.uint32), vh.view(np.uint32))

    for _ in range(3):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16().pin_memory()
        gb = H.to_np_bits(g, "bf16")
        group = adam.begin_chunk_step(0)
        for cs in range(0, n, call):
            ce = min(n, cs + call)
            adam.step_chunk(master[cs:ce], g[cs:ce], m[cs:ce], v[cs:ce], group)
            assert adam.last_stream_stats is None          # returned once queued
            orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[cs:ce], gb[cs:ce], mh[cs:ce],
                       vh[cs:ce], g16="bf16")
        adam.end_chunk_step(0)
        check()
    # two whole-buffer steps queued back to back: the second call touches the
    # first one's bytes and settles it before streaming
    gs = [torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16().pin_memory() for _ in range(2)]
    for g in gs:
        group = adam.begin_chunk_step(0)
        adam.step_chunk(master, g, m, v, group)
        orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh,
                   g16="bf16")
    adam.synchronize()
    check()


@pytest.mark.parametrize("pinned", [True, False])
def test_overlapped_calls_keep_device_temporaries_alive(pinned, hip_device):
    """overlap_host_chunks=True with the device inputs of each call as
    temporaries the caller drops at once: per-chunk grads moved to the device
    by the call expression, a clip coefficient recomputed every step and a
    bf16 copy allocated per chunk.  After each call the caller allocates and
    fills same-sized tensors on its stream, which would take over those blocks
    if the optimizer let them go before the pipeline's own streams were done
    with them.  Host master, moments in HBM.  Bit-exact with the oracle."""
    from slideformer_amd.layer_adam import HostStreamer
    n, call = 40_000, 7_000
    rng = np.random.default_rng(80 + int(pinned))
    p0 = rng.normal(0, 0.02, n).astype(np.float32)
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, overlap_host_chunks=True, moments_device=hip_device)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=2048, slots=3)
    master = torch.from_numpy(p0.copy())
    if pinned:
        master = master.pin_memory()
    adam.add_layer_params(0, [torch.nn.Parameter(master)])
    m, v = adam.exp_avg_flat[0], adam.exp_avg_sq_flat[0]
    assert m.is_cuda and not master.is_cuda
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    ph, mh, vh = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    copies = []
    for _ in range(3):
        g = torch.from_numpy(rng.normal(0, 1e-2, n).astype(np.float32)).bfloat16()
        gb = H.to_np_bits(g, "bf16")
        c_ref, _ = O.clip_coef(O.grad_sqnorm(gb, "bf16"), 0.05)
        group = adam.begin_chunk_step(0)
        for cs in range(0, n, call):
            ce = min(n, cs + call)
            coef, _ = adam.clip_grad_norm([g.to(hip_device)], 0.05)
            out = torch.empty(ce - cs, dtype=torch.bfloat16, device=hip_device)
            adam.step_chunk(master[cs:ce], g[cs:ce].to(hip_device), m[cs:ce], v[cs:ce], group,
                            bf16_out=out, clip_coef=coef)
            copies.append((cs, ce, out))
            del coef, out
            # fresh allocations of the same sizes on the caller's stream, filled at once
            for k in range(4):
                torch.full((ce - cs,), float("nan"), dtype=torch.bfloat16, device=hip_device)
                torch.full((1,), float("nan"), dtype=torch.float32, device=hip_device)
            orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[cs:ce], gb[cs:ce], mh[cs:ce],
                       vh[cs:ce], g16="bf16", clip_coef=float(np.float32(c_ref)))
        adam.end_chunk_step(0)
        assert not adam._streamers[hip_device]._in_flight     # released once complete
        assert np.array_equal(master.numpy().view(np.uint32), ph.view(np.uint32))
        assert np.array_equal(H.to_np_bits(m, "f32"), mh.view(np.uint32))
        assert np.array_equal(H.to_np_bits(v, "f32"), vh.view(np.uint32))
        for cs, ce, out in copies:
            assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(ph[cs:ce])), (cs, ce)
        copies.clear()


# which of p, m, v, g and the bf16 copy are in host memory (the rest in HBM)
PLACEMENTS = {
    "master+grads on host": (True, False, False, True, False),        # the runtime with moments_device
    "master+grads+copy on host": (True, False, False, True, True),
    "moments on host": (False, True, True, False, False),
    "exp_avg+copy on host": (False, True, False, False, True),
    "grads only on host": (False, False, False, True, False),
    "copy only on host": (False, False, False, False, True),
}


@pytest.mark.parametrize("pinned", [True, False])
@pytest.mark.parametrize("name", list(PLACEMENTS))
def test_pipeline_mixed_placements_match_oracle(name, pinned, hip_device):
    """la_pipeline_step with some arrays in host memory and the others in HBM
    (used in place): three steps over several chunks and a scalar tail, with
    one chunk more than the slots so that slots are reused; bit-exact with the
    oracle; only the host-resident arrays cross the link (the byte counts);
    page-locked and pageable (staged) host arrays."""
    from slideformer_amd.layer_adam import HostStreamer
    print(f"placement {name} pinned={pinned}", flush=True)
    hp, hm, hv, hg, ho = PLACEMENTS[name]
    n, chunk = 3 * 4096 + 4099, 4096
    rng = np.random.default_rng(zlib.crc32(name.encode()) + int(pinned))
    ph = rng.normal(0, 0.02, n).astype(np.float32)
    mh = rng.normal(0, 1e-3, n).astype(np.float32)
    vh = np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)

    def place(arr, host):
        t = torch.from_numpy(arr.copy())
        if host:
            return t.pin_memory() if pinned else t
        return t.to(hip_device)

    p, m, v = place(ph, hp), place(mh, hm), place(vh, hv)
    out = torch.empty(n, dtype=torch.bfloat16, device="cpu" if ho else hip_device)
    if ho and pinned:
        out = out.pin_memory()
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=chunk, slots=3)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        gb = H.to_np_bits(g, "bf16")
        gd = (g.pin_memory() if pinned else g) if hg else g.to(hip_device)
        adam.step_chunk(p, gd, m, v, dict(adam.defaults, step=step), bf16_out=out)
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, gb, mh, vh, g16="bf16")
        st = adam.last_stream_stats
        assert st.chunks == -(-n // chunk)
        assert st.h2d_bytes == n * (4 * (hp + hm + hv) + 2 * hg)
        assert st.d2h_bytes == n * (4 * (hp + hm + hv) + 2 * ho)
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p, "f32"), ph.view(np.uint32))
    assert np.array_equal(H.to_np_bits(m, "f32"), mh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(v, "f32"), vh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(ph))


def test_staged_grads_only_wait_for_the_twins_copy_in(hip_device):
    """Pageable grads are the only staged array: no copy-out is ever owed, so
    before the host threads refill a slot's page-locked twin they must wait for
    the H2D that still reads it (that H2D queues behind the slot's earlier
    copy-back).  Many 256-element chunks over 2 slots with a single host thread
    let the host run far ahead of the copy stream; every chunk's grads differ,
    and the result must equal the oracle bit for bit."""
    from slideformer_amd.layer_adam import HostStreamer
    n, chunk = 400 * 256 + 7, 256
    rng = np.random.default_rng(4242)
    ph = rng.normal(0, 0.02, n).astype(np.float32)
    mh = rng.normal(0, 1e-3, n).astype(np.float32)
    vh = np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)
    p, m, v = (torch.from_numpy(a.copy()).to(hip_device) for a in (ph, mh, vh))
    out = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    adam = LayerAdam(lr=1e-3, weight_decay=0.01)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=chunk, slots=2, host_threads=1)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2, 3):
        print(f"grads-only staging, step {step}", flush=True)
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        assert not g.is_pinned()
        adam.step_chunk(p, g, m, v, dict(adam.defaults, step=step), bf16_out=out)
        st = adam.last_stream_stats
        assert st.chunks == -(-n // chunk)
        assert st.staged_bytes == 2 * n and st.h2d_bytes == 2 * n and st.d2h_bytes == 0
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph, H.to_np_bits(g, "bf16"), mh, vh, g16="bf16")
    torch.cuda.synchronize()
    assert np.array_equal(H.to_np_bits(p, "f32"), ph.view(np.uint32))
    assert np.array_equal(H.to_np_bits(m, "f32"), mh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(v, "f32"), vh.view(np.uint32))
    assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(ph))


@pytest.mark.parametrize("pinned", [True, False])
def test_moments_in_hbm_in_the_runtime_protocol(pinned, hip_device):
    """LayerAdam(moments_device=...) under the runtime's calls
    (transformer_layer.py:453-493): the master and the grad buffer stay in
    host memory, add_layer_params allocates exp_avg / exp_avg_sq in HBM, and
    each step_chunk streams only the master and the grads.  Overlapped calls
    (overlap_host_chunks=True) of 5000 elements through a 2048 x 3 pipeline,
    then one step_with_grad_views over the layer's parameters (one call per
    tensor); bit-exact with the oracle after every step."""
    from slideformer_amd.layer_adam import HostStreamer
    sizes = [3000, 7, 9000, 1]
    n, call = sum(sizes), 5000
    rng = np.random.default_rng(90 + int(pinned))
    p0 = rng.normal(0, 0.02, n).astype(np.float32)
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, overlap_host_chunks=True, moments_device=hip_device)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=2048, slots=3)
    master = torch.from_numpy(p0.copy())
    if pinned:
        master = master.pin_memory()
    views, lo = [], 0
    for k in sizes:
        views.append(torch.nn.Parameter(master[lo:lo + k]))
        lo += k
    adam.add_layer_params(0, views)
    m, v = adam.exp_avg_flat[0], adam.exp_avg_sq_flat[0]
    assert m.device == torch.device(hip_device) and v.device == torch.device(hip_device)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    ph, mh, vh = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)

    def check():
        assert np.array_equal(master.numpy().view(np.uint32), ph.view(np.uint32))
        assert np.array_equal(H.to_np_bits(m, "f32"), mh.view(np.uint32))
        assert np.array_equal(H.to_np_bits(v, "f32"), vh.view(np.uint32))

    for _ in range(2):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
        if pinned:
            g = g.pin_memory()
        gb = H.to_np_bits(g, "bf16")
        group = adam.begin_chunk_step(0)
        for cs in range(0, n, call):
            ce = min(n, cs + call)
            adam.step_chunk(master[cs:ce], g[cs:ce], m[cs:ce], v[cs:ce], group)
            orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[cs:ce], gb[cs:ce], mh[cs:ce],
                       vh[cs:ce], g16="bf16")
        adam.end_chunk_step(0)
        check()
    # one reference adam_update per parameter, in order (layer_adam.py:391-422), on bf16 grad views
    g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).bfloat16()
    gb = H.to_np_bits(g, "bf16")
    offs = np.cumsum([0] + sizes)
    adam.step_with_grad_views(0, {prm: g[offs[i]:offs[i + 1]] for i, prm in enumerate(views)})
    step = adam.param_groups[0]["step"]
    lo = 0
    for k in sizes:
        orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[lo:lo + k], gb[lo:lo + k], mh[lo:lo + k],
                   vh[lo:lo + k], g16="bf16")
        lo += k
    check()


def test_moments_hbm_budget_splits_layers(hip_device):
    """LayerAdam(moments_device=..., moments_hbm_bytes=B): layers get HBM
    moments while B allows, later ones keep host moments; every layer steps
    bit-exact with the oracle whatever its placement (host master, host grads)."""
    sizes = [5000, 3000, 4000, 7]
    budget = 2 * 4 * (5000 + 3000)           # exactly the first two layers' m and v
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, moments_device=hip_device, moments_hbm_bytes=budget)
    rng = np.random.default_rng(70)
    masters, host = [], []
    for i, k in enumerate(sizes):
        p0 = rng.normal(0, 0.02, k).astype(np.float32)
        t = torch.from_numpy(p0.copy())
        masters.append(t)
        host.append([p0.copy(), np.zeros(k, np.float32), np.zeros(k, np.float32)])
        adam.add_layer_params(i, [torch.nn.Parameter(t)])
    assert [adam.exp_avg_flat[i].is_cuda for i in range(4)] == [True, True, False, False]
    assert adam.moments_hbm_used == budget
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for _ in range(2):
        for i in reversed(range(4)):                 # sliding order
            g = torch.from_numpy(rng.normal(0, 1e-3, sizes[i]).astype(np.float32)).bfloat16()
            group = adam.begin_chunk_step(i)
            adam.step_chunk(masters[i], g, adam.exp_avg_flat[i], adam.exp_avg_sq_flat[i], group)
            adam.end_chunk_step(i)
            orc.update(group["step"], 1e-3, 0.9, 0.999, 1e-8, 0.01, True, *host[i][:1], H.to_np_bits(g, "bf16"),
                       *host[i][1:], g16="bf16")
    for i in range(4):
        assert np.array_equal(masters[i].numpy().view(np.uint32), host[i][0].view(np.uint32)), i
        assert np.array_equal(H.to_np_bits(adam.exp_avg_flat[i], "f32"), host[i][1].view(np.uint32)), i
        assert np.array_equal(H.to_np_bits(adam.exp_avg_sq_flat[i], "f32"), host[i][2].view(np.uint32)), i


@pytest.mark.parametrize("triple", [("bf16", "bf16", "bf16"), ("f16", "f32", "f32"), ("f16", "f16", "f16")])
@pytest.mark.parametrize("moments", ["host", "hbm"])
def test_pipeline_other_triples_staged_and_overlapped(triple, moments, hip_device):
    """The streaming pipeline on the reference's other dtype triples: 16-bit
    params and states, host grads and a host bf16 copy, all pageable (staged),
    overlapped calls of 3000 elements through 1024-element chunks in 2 slots;
    the moments on the host or in HBM (mixed element sizes per placement).
    Bit-exact with the oracle."""
    from slideformer_amd.layer_adam import HostStreamer
    pk, gk, sk = triple
    td = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    k16 = {"f32": None, "bf16": "bf16", "f16": "f16"}
    n, call = 10_007, 3000
    rng = np.random.default_rng(70)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32)).to(td[pk])
    m = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(td[sk])
    v = torch.from_numpy(np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)).to(td[sk])
    if moments == "hbm":
        m, v = m.to(hip_device), v.to(hip_device)
    out = torch.empty(n, dtype=torch.bfloat16)
    bits = lambda t, k: H.to_np_bits(t, k)
    hp, hm, hv = bits(p, pk), bits(m, sk), bits(v, sk)
    view = lambda b, k: b.view(np.float32) if k == "f32" else b
    ho = np.zeros(n, np.uint16)                      # the oracle's bf16 copy: RNE of the fp32 result
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, overlap_host_chunks=True)
    adam._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=1024, slots=2, host_threads=2)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    for step in (1, 2):
        g = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(td[gk])
        gb = bits(g, gk)
        group = dict(adam.defaults, step=step)
        for cs in range(0, n, call):
            ce = min(n, cs + call)
            adam.step_chunk(p[cs:ce], g[cs:ce], m[cs:ce], v[cs:ce], group, bf16_out=out[cs:ce])
            orc.update(step, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, view(hp, pk)[cs:ce], view(gb, gk)[cs:ce],
                       view(hm, sk)[cs:ce], view(hv, sk)[cs:ce], p16=k16[pk], g16=k16[gk], s16=k16[sk],
                       p_bf16_out=ho[cs:ce])
        adam.synchronize()
    assert np.array_equal(bits(p, pk), hp)
    assert np.array_equal(bits(m, sk), hm)
    assert np.array_equal(bits(v, sk), hv)
    assert np.array_equal(H.to_np_bits(out, "bf16"), ho)


def test_async_pipeline_calls_with_changing_layouts(hip_device):
    """Raw la_pipeline_step calls with synchronize = 0 on disjoint ranges of
    pageable host state, one workspace and one staging buffer for all, but
    alternating slot layouts (grads on the device / on the host, fp32 / bf16
    grads): each layout change settles the earlier calls, whose slots would
    otherwise overlap the new ones.  la_pipeline_sync completes the last.
    Bit-exact with the oracle."""
    import ctypes

    from slideformer_amd import _lib
    from slideformer_amd.layer_adam import HostStreamer

    L = _lib.load()
    chunk, slots, n, part = 1024, 3, 6 * 2600, 2600
    s_ = HostStreamer(hip_device, chunk_elems=chunk, slots=slots)
    F32, BF16 = _lib.LA_F32, _lib.LA_BF16
    STATE = _lib.LA_ON_HOST_P | _lib.LA_ON_HOST_M | _lib.LA_ON_HOST_V
    need = max(L.la_pipeline_workspace_bytes(chunk, slots, F32, gc, F32, STATE | gh)
               for gc in (F32, BF16) for gh in (0, _lib.LA_ON_HOST_G))
    ws = torch.empty(need + 256, dtype=torch.uint8, device=hip_device)
    wbase = (ws.data_ptr() + 255) // 256 * 256
    stg = torch.empty(need + 256, dtype=torch.uint8, pin_memory=True)
    sbase = (stg.data_ptr() + 255) // 256 * 256
    assert L.la_pipeline_set_host_staging(s_.handle, sbase, need, 2) == 0
    rng = np.random.default_rng(80)
    p = torch.from_numpy(rng.normal(0, 0.02, n).astype(np.float32))
    m, v = torch.zeros(n), torch.zeros(n)
    ph, mh, vh = p.numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    L.la_create(81, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 0)
    orc = O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True)
    st = torch.cuda.current_stream(hip_device).cuda_stream
    layouts = [(BF16, False), (F32, True), (BF16, True), (F32, False), (BF16, False), (F32, True)]
    keep = []
    for i, (gc, on_host) in enumerate(layouts):
        lo, hi = i * part, (i + 1) * part
        g32 = rng.normal(0, 1e-3, part).astype(np.float32)
        g = torch.from_numpy(g32)
        if gc == BF16:
            g = g.bfloat16()
        gbits = H.to_np_bits(g, "bf16" if gc == BF16 else "f32")
        if not on_host:
            g = g.to(hip_device)
        keep.append(g)
        sc = _lib.LaScalars()
        assert L.la_scalars(81, 1, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, ctypes.byref(sc)) == 0
        rc = L.la_pipeline_step(s_.handle, ctypes.byref(sc), F32, p[lo:hi].data_ptr(), gc, g.data_ptr(), F32,
                                m[lo:hi].data_ptr(), v[lo:hi].data_ptr(), hi - lo, None,
                                STATE | (_lib.LA_ON_HOST_G if on_host else 0), None, wbase, need, st, 0, None)
        assert rc == 0, rc
        orc.update(1, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, ph[lo:hi], g32 if gc == F32 else gbits, mh[lo:hi],
                   vh[lo:hi], g16="bf16" if gc == BF16 else None)
    assert L.la_pipeline_sync(s_.handle) == 0
    assert np.array_equal(p.numpy().view(np.uint32), ph.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), mh.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), vh.view(np.uint32))
    L.la_destroy(81)


def test_host_staging_rejects_bad_buffers(hip_device):
    """la_pipeline_set_host_staging accepts only 256-byte aligned page-locked
    memory; a staging buffer smaller than a call needs fails the call before any
    transfer, and the host state is left untouched."""
    import ctypes

    from slideformer_amd import _lib
    from slideformer_amd.layer_adam import HostStreamer

    L = _lib.load()
    s = HostStreamer(hip_device, chunk_elems=1024, slots=2)
    pageable = torch.empty(1 << 20, dtype=torch.uint8)
    pinned = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
    base = (pinned.data_ptr() + 255) // 256 * 256
    assert L.la_pipeline_set_host_staging(s.handle, pageable.data_ptr(), 1 << 19, 2) == _lib.LA_EINVAL
    assert L.la_pipeline_set_host_staging(s.handle, base + 16, 4096, 2) == _lib.LA_EINVAL
    assert L.la_pipeline_set_host_staging(s.handle, base, 4096, -1) == _lib.LA_EINVAL
    assert L.la_pipeline_set_host_staging(s.handle, base, 4096, 2) == _lib.LA_OK   # too small for a call
    n = 4096
    p, m, v = torch.randn(n), torch.zeros(n), torch.zeros(n)
    p_before = p.clone()
    g = torch.zeros(n, dtype=torch.bfloat16, device=hip_device)
    L.la_create(78, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0)
    sc = _lib.LaScalars()
    assert L.la_scalars(78, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, ctypes.byref(sc)) == 0
    STATE = _lib.LA_ON_HOST_P | _lib.LA_ON_HOST_M | _lib.LA_ON_HOST_V
    ws = s.workspace(_lib.LA_F32, _lib.LA_BF16, _lib.LA_F32, STATE)
    wbase = (ws.data_ptr() + 255) // 256 * 256
    st = torch.cuda.current_stream(hip_device).cuda_stream
    rc = L.la_pipeline_step(s.handle, ctypes.byref(sc), _lib.LA_F32, p.data_ptr(), _lib.LA_BF16, g.data_ptr(),
                            _lib.LA_F32, m.data_ptr(), v.data_ptr(), n, None, STATE, None, wbase,
                            ws.numel() - (wbase - ws.data_ptr()), st, 1, None)
    assert rc == _lib.LA_EINVAL
    assert torch.equal(p, p_before) and not m.any() and not v.any()
    assert L.la_pipeline_set_host_staging(s.handle, None, 0, 0) == _lib.LA_OK
    L.la_destroy(78)


def test_clip_grad_norm_on_two_streams_at_once(hip_device):
    """Two clip_grad_norm calls in flight on two streams share no scratch: each
    coefficient equals the oracle's for its own grads."""
    rng = np.random.default_rng(31)
    sets = [[torch.from_numpy(rng.normal(0, s, k).astype(np.float32)).bfloat16().to(hip_device)
             for k in (1_000_003, 77, 2_500_000)] for s in (1e-3, 5e-2)]
    adam = LayerAdam()
    a, b = torch.cuda.Stream(device=hip_device), torch.cuda.Stream(device=hip_device)
    for s_ in (a, b):
        s_.wait_stream(torch.cuda.current_stream(hip_device))
    results = []
    for rep in range(3):
        ca, na = adam.clip_grad_norm(sets[0], 1.0, stream=a)
        cb, nb = adam.clip_grad_norm(sets[1], 1.0, stream=b.cuda_stream)   # raw handle
        results.append((ca, na, cb, nb))
    torch.cuda.synchronize()
    for grads, (ci, ni) in zip(sets, ((0, 1), (2, 3))):
        sq = sum(O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16") for g in grads)
        c_ref, n_ref = O.clip_coef(sq, 1.0)
        for r in results:
            assert r[ci].item() == np.float32(c_ref) and r[ni].item() == np.float32(n_ref)


def test_grad_norm_accumulator_on_side_streams(hip_device):
    """GradNormAccumulator driven on side streams (a torch stream, then a raw
    handle), dropped right after finish(): its scratch is recorded on those
    streams, so allocations made meanwhile on the current stream do not take it
    over; the coefficient equals the oracle's."""
    rng = np.random.default_rng(33)
    grads = [torch.from_numpy(rng.normal(0, 1e-2, k).astype(np.float32)).bfloat16().to(hip_device)
             for k in (3_000_001, 5, 400_000)]
    adam = LayerAdam()
    side = torch.cuda.Stream(device=hip_device)
    side.wait_stream(torch.cuda.current_stream(hip_device))
    outs = []
    for rep in range(3):
        acc = adam.grad_norm_begin(hip_device)
        for i, g in enumerate(grads):
            acc.add(g, stream=side if i % 2 == 0 else side.cuda_stream)
        outs.append(acc.finish(1.0, stream=side))
        del acc
        # allocations on the current stream while the side stream may still run
        junk = [torch.full((1 << 16,), 7.0, dtype=torch.float64, device=hip_device) for _ in range(8)]
        del junk
    torch.cuda.synchronize()
    sq = sum(O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16") for g in grads)
    c_ref, n_ref = O.clip_coef(sq, 1.0)
    for coef, norm in outs:
        assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)


def test_launch_status_ignores_an_earlier_unrelated_error(hip_device):
    """A HIP error left in the thread by an unrelated host call (here a failed
    hipSetDevice) is not reported as a failure of the next launch.  Only
    C-ABI calls run between planting the error and clearing it again."""
    import ctypes

    from slideformer_amd import _lib

    L = _lib.load()
    hip = ctypes.CDLL("libamdhip64.so")
    n = 4099
    p = torch.randn(n, device=hip_device)
    m = torch.zeros(n, device=hip_device)
    v = torch.zeros(n, device=hip_device)
    g = torch.randn(n, device=hip_device).bfloat16()
    ws = torch.zeros(L.la_grad_sqnorm_workspace(n) // 8 + 1, dtype=torch.float64, device=hip_device)
    sq = torch.zeros(1, dtype=torch.float64, device=hip_device)
    coef = torch.zeros(1, device=hip_device)
    st = torch.cuda.current_stream(hip_device).cuda_stream
    assert L.la_create(79, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0) == 0
    torch.cuda.synchronize()
    try:
        assert hip.hipSetDevice(ctypes.c_int(4096)) != 0          # invalid ordinal: fails on the host
        assert hip.hipPeekAtLastError() != 0
        rc_step = L.la_adam_update(79, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, _lib.LA_F32, p.data_ptr(), _lib.LA_BF16,
                                   g.data_ptr(), _lib.LA_F32, m.data_ptr(), v.data_ptr(), n, None, None, st)
        rc_norm = L.la_grad_norm_clip(_lib.LA_BF16, g.data_ptr(), n, ws.data_ptr(), ws.numel() * 8, sq.data_ptr(),
                                      0, 1.0, coef.data_ptr(), None, st)
        rc_coef = L.la_clip_coef(sq.data_ptr(), 1.0, coef.data_ptr(), None, st)
    finally:
        hip.hipGetLastError()                                      # leave the thread clean for torch
        L.la_destroy(79)
    assert (rc_step, rc_norm, rc_coef) == (0, 0, 0)
    torch.cuda.synchronize()
    assert torch.isfinite(p).all() and sq.item() > 0 and 0.0 < coef.item() <= 1.0


def c5_layer_sizes():
    """100B-class dense layer: hidden 12288, FFN 49152, biases, 2 LayerNorms (w, b)."""
    h, ffn = 12288, 49152
    return [h * 3 * h, 3 * h, h * h, h, h * ffn, ffn, ffn * h, h, h, h, h, h]


def test_c5_streamed_full_size_matches_resident(hip_device):
    """Config C5 at full size (1,812,099,072 params, 7.25 GB per fp32 array):
    pinned host state streamed through HBM in 256 MB chunks x 2 slots gives the
    same bits as the same step on HBM-resident copies, with one clip coefficient
    from the grad norm.  Host byte offsets pass 2^32.  Every element of the
    streamed master, moments and copy also equals the CPU checker's step over
    the whole layer."""
    from slideformer_amd.layer_adam import HostStreamer

    n = sum(c5_layer_sizes())
    assert n == 1_812_099_072 and n % 16 == 0
    print(f"C5 streamed vs resident, n={n}", flush=True)
    gen = torch.Generator(device=hip_device)
    gen.manual_seed(50)
    p_d = torch.randn(n, generator=gen, device=hip_device) * 0.02
    m_d = torch.randn(n, generator=gen, device=hip_device) * 1e-4
    v_d = torch.rand(n, generator=gen, device=hip_device) * 1e-8
    g = (torch.randn(n, generator=gen, device=hip_device) * 5e-4).bfloat16()
    # the CPU checker's copy of the whole layer
    p_o, m_o, v_o = (H.to_np_bits(t, "f32").view(np.float32) for t in (p_d, m_d, v_d))
    host = []
    for t in (p_d, m_d, v_d):
        h = torch.empty(n, dtype=torch.float32, pin_memory=True)
        h.copy_(t)
        host.append(h)
    p_h, m_h, v_h = host
    torch.cuda.synchronize()
    print("pinned host state ready", flush=True)

    resident = LayerAdam(lr=6e-6, weight_decay=0.01)
    coef, _ = resident.clip_grad_norm([g], 1.0)
    out_d = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    resident.step_chunk(p_d, g, m_d, v_d, dict(resident.defaults, step=1), bf16_out=out_d, clip_coef=coef)
    streamed = LayerAdam(lr=6e-6, weight_decay=0.01)
    streamed._streamers[hip_device] = HostStreamer(hip_device, chunk_elems=64 * 1024 * 1024, slots=2)
    out_s = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    streamed.step_chunk(p_h, g, m_h, v_h, dict(streamed.defaults, step=1), bf16_out=out_s, clip_coef=coef)
    st = streamed.last_stream_stats
    assert st.chunks == -(-n // (64 * 1024 * 1024)) == 28 and st.h2d_bytes == st.d2h_bytes == 12 * n
    print(f"streamed step {st.wall_ms:.1f} ms; comparing", flush=True)
    c = float(coef.item())
    assert 0.0 < c < 1.0
    piece = 256 * 1024 * 1024
    for hst, dev in ((p_h, p_d), (m_h, m_d), (v_h, v_d)):
        for lo in range(0, n, piece):
            hi = min(n, lo + piece)
            assert torch.equal(hst[lo:hi].to(hip_device).view(torch.int32), dev[lo:hi].view(torch.int32)), lo
    assert torch.equal(out_s.view(torch.int16), out_d.view(torch.int16))
    print("streamed == resident; the CPU checker over the whole layer", flush=True)
    out_o = np.zeros(n, np.uint16)
    orc = O.OracleAdam(6e-6, (0.9, 0.999), 1e-8, 0.01, True)
    orc.update(1, 6e-6, 0.9, 0.999, 1e-8, 0.01, True, p_o, H.to_np_bits(g, "bf16"), m_o, v_o, g16="bf16",
               p_bf16_out=out_o, clip_coef=c)
    for got, want, what in ((p_h, p_o, "p"), (m_h, m_o, "m"), (v_h, v_o, "v")):
        bad = np.flatnonzero(got.numpy().view(np.uint32) != want.view(np.uint32))[:8]
        assert bad.size == 0, (what, bad)
    bad = np.flatnonzero(H.to_np_bits(out_s, "bf16") != out_o)[:8]
    assert bad.size == 0, ("out", bad)
    del p_h, m_h, v_h, host, p_d, m_d, v_d, g, out_d, out_s, p_o, m_o, v_o, out_o
    torch._C._host_emptyCache()
    torch.cuda.empty_cache()


def test_streamed_call_beyond_2_pow_32_elements(hip_device):
    """One step_chunk over n = 2^32 + 2^20 + 13 elements with the master in
    pageable host memory (17 GB, staged through the page-locked twins) and the
    moments, grads and bf16 copy in HBM: 257 pipeline chunks whose element and
    byte offsets pass 2^32.  Same bits as the step on HBM-resident copies, and
    every element (the 13-element scalar tail included) equals the CPU
    checker's step over the whole call."""
    from slideformer_amd.layer_adam import HostStreamer

    n = (1 << 32) + (1 << 20) + 13
    print(f"streamed n={n}", flush=True)
    gen = torch.Generator(device=hip_device)
    gen.manual_seed(52)
    p_d = torch.randn(n, generator=gen, device=hip_device) * 0.02
    m_d = torch.randn(n, generator=gen, device=hip_device) * 1e-4
    v_d = torch.rand(n, generator=gen, device=hip_device) * 1e-8
    g = (torch.randn(n, generator=gen, device=hip_device) * 1e-3).bfloat16()
    # the CPU checker's copy of the whole call
    p_o, m_o, v_o = (H.to_np_bits(t, "f32").view(np.float32) for t in (p_d, m_d, v_d))
    p_h = torch.empty(n, dtype=torch.float32)                    # pageable, as the runtime allocates it
    piece = 256 * 1024 * 1024
    for lo in range(0, n, piece):
        p_h[lo:lo + piece].copy_(p_d[lo:lo + piece])
    m_s, v_s = m_d.clone(), v_d.clone()
    torch.cuda.synchronize()
    print("host master ready", flush=True)

    resident = LayerAdam(lr=1e-5, weight_decay=0.01)
    out_d = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    resident.step_chunk(p_d, g, m_d, v_d, dict(resident.defaults, step=1), bf16_out=out_d)
    streamed = LayerAdam(lr=1e-5, weight_decay=0.01)
    streamed._streamers[hip_device] = HostStreamer(hip_device)
    out_s = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
    streamed.step_chunk(p_h, g, m_s, v_s, dict(streamed.defaults, step=1), bf16_out=out_s)
    st = streamed.last_stream_stats
    assert st.chunks == -(-n // (16 * 1024 * 1024)) == 257
    assert st.h2d_bytes == st.d2h_bytes == 4 * n and st.staged_bytes == 8 * n
    print(f"streamed step {st.wall_ms:.1f} ms; comparing", flush=True)
    torch.cuda.synchronize()
    for lo in range(0, n, piece):
        assert torch.equal(p_h[lo:lo + piece].to(hip_device).view(torch.int32),
                           p_d[lo:lo + piece].view(torch.int32)), lo
    assert torch.equal(m_s.view(torch.int32), m_d.view(torch.int32))
    assert torch.equal(v_s.view(torch.int32), v_d.view(torch.int32))
    assert torch.equal(out_s.view(torch.int16), out_d.view(torch.int16))
    print("streamed == resident; the CPU checker over the whole call", flush=True)
    del p_d, m_d, v_d, out_d
    out_o = np.zeros(n, np.uint16)
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
    orc.update(1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p_o, H.to_np_bits(g, "bf16"), m_o, v_o, g16="bf16",
               p_bf16_out=out_o)
    bad = np.flatnonzero(p_h.numpy().view(np.uint32) != p_o.view(np.uint32))[:8]
    assert bad.size == 0, ("p", bad)
    for got, want, kind, what in ((m_s, m_o, "f32", "m"), (v_s, v_o, "f32", "v"), (out_s, out_o, "bf16", "out")):
        w = want.view(np.uint32) if kind == "f32" else want
        bad = np.flatnonzero(H.to_np_bits(got, kind) != w)[:8]
        assert bad.size == 0, (what, bad)
    del p_h, m_s, v_s, g, out_s, streamed, resident, p_o, m_o, v_o, out_o
    torch.cuda.empty_cache()


def test_stream_shape_options_set_the_pipeline(hip_device):
    """LayerAdam(stream_chunk_elems=, stream_slots=) streams host arrays in
    chunks of that size: 20,013 elements at 4096 take 5 chunks (the last one
    short, holding the scalar tail), bit-exact with the CPU checker."""
    n, chunk = 20_013, 4096
    rng = np.random.default_rng(77)
    p_h = rng.normal(0, 0.02, n).astype(np.float32)
    g_h = O.f32_to_bf16(rng.normal(0, 1e-3, n).astype(np.float32))
    adam = LayerAdam(lr=1e-3, weight_decay=0.01, stream_chunk_elems=chunk, stream_slots=2)
    p = torch.from_numpy(p_h.copy())
    m, v = torch.zeros(n), torch.zeros(n)
    g = torch.from_numpy(g_h.view(np.int16).copy()).view(torch.bfloat16)
    adam.step_chunk(p, g, m, v, dict(adam.defaults, step=1))
    st = adam.last_stream_stats
    assert st.chunks == 5 and st.h2d_bytes == 14 * n
    assert adam._streamers[hip_device].chunk == chunk and adam._streamers[hip_device].slots == 2
    m_h, v_h = np.zeros(n, np.float32), np.zeros(n, np.float32)
    O.OracleAdam(1e-3, (0.9, 0.999), 1e-8, 0.01, True).update(1, 1e-3, 0.9, 0.999, 1e-8, 0.01, True, p_h, g_h, m_h,
                                                              v_h, g16="bf16")
    assert np.array_equal(p.numpy().view(np.uint32), p_h.view(np.uint32))
    assert np.array_equal(m.numpy().view(np.uint32), m_h.view(np.uint32))
    assert np.array_equal(v.numpy().view(np.uint32), v_h.view(np.uint32))


def test_pipeline_rejects_bad_arguments_before_any_transfer(hip_device):
    """la_pipeline_step validates the dtype triple, device-pointer alignment,
    placement and the current device up front: the host state is left
    untouched."""
    import ctypes

    from slideformer_amd import _lib
    from slideformer_amd.layer_adam import HostStreamer

    L = _lib.load()
    s = HostStreamer(hip_device, chunk_elems=1024, slots=2)
    n = 4096
    p = torch.randn(n).pin_memory()
    m = torch.zeros(n).pin_memory()
    v = torch.zeros(n).pin_memory()
    p_before = p.clone()
    g = torch.zeros(n + 1, dtype=torch.bfloat16, device=hip_device)
    L.la_create(77, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0)
    sc = _lib.LaScalars()
    assert L.la_scalars(77, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, ctypes.byref(sc)) == 0
    STATE = _lib.LA_ON_HOST_P | _lib.LA_ON_HOST_M | _lib.LA_ON_HOST_V
    ws = s.workspace(_lib.LA_F32, _lib.LA_BF16, _lib.LA_F32, STATE)
    base = (ws.data_ptr() + 255) // 256 * 256
    st = torch.cuda.current_stream(hip_device).cuda_stream
    F32, BF16 = _lib.LA_F32, _lib.LA_BF16

    def call(gptr, s_dtype=F32, on_host=STATE, out=None, ws_bytes=ws.numel() - 256, mptr=m.data_ptr()):
        return L.la_pipeline_step(s.handle, ctypes.byref(sc), F32, p.data_ptr(), BF16, gptr, s_dtype, mptr,
                                  v.data_ptr(), n, out, on_host, None, base, ws_bytes, st, 1, None)

    # (f32, bf16, bf16) is not a registered triple
    assert call(g.data_ptr(), s_dtype=BF16) == _lib.LA_EDTYPE
    # a device grad pointer at an odd byte address
    assert call(g.data_ptr() + 1) == _lib.LA_EINVAL
    # too small a workspace
    assert call(g.data_ptr(), ws_bytes=1024) == _lib.LA_EINVAL
    # placement bits beyond the five arrays; a host bf16 copy without a pointer
    assert call(g.data_ptr(), on_host=STATE | 32) == _lib.LA_EINVAL
    assert call(g.data_ptr(), on_host=STATE | _lib.LA_ON_HOST_OUT) == _lib.LA_EINVAL
    # a device-resident exp_avg at an address that is not a whole fp32 element
    md = torch.zeros(n + 1, device=hip_device)
    assert call(g.data_ptr(), on_host=_lib.LA_ON_HOST_P | _lib.LA_ON_HOST_V, mptr=md.data_ptr() + 2) == _lib.LA_EINVAL
    assert not md.any()
    # exp_avg placed as device-resident but in host memory (page-locked, then
    # pageable): refused before any transfer, not handed to the kernel
    assert call(g.data_ptr(), on_host=_lib.LA_ON_HOST_P | _lib.LA_ON_HOST_V) == _lib.LA_EFAULT
    mh = torch.zeros(n)
    assert call(g.data_ptr(), on_host=_lib.LA_ON_HOST_P | _lib.LA_ON_HOST_V, mptr=mh.data_ptr()) == _lib.LA_EFAULT
    # another device current than the pipeline's (needs a second GPU)
    if torch.cuda.device_count() > 1:
        with torch.cuda.device((hip_device.index + 1) % torch.cuda.device_count()):
            assert call(g.data_ptr()) == _lib.LA_EINVAL
    torch.cuda.synchronize()
    assert torch.equal(p, p_before) and not m.any() and not v.any() and not mh.any()
    L.la_destroy(77)


def test_device_entry_points_refuse_host_memory(hip_device):
    """The device entry points refuse host arrays, page-locked or pageable,
    with LA_EFAULT before any launch: a host address in a kernel would fault
    the GPU.  The beta-power state still advances, as for any bad argument
    after la_scalars, and the host arrays are untouched."""
    import ctypes

    from slideformer_amd import _lib
    L = _lib.load()
    n = 4096
    st = torch.cuda.current_stream(hip_device).cuda_stream
    dev = [torch.zeros(n, device=hip_device) for _ in range(3)]
    gd = torch.zeros(n, dtype=torch.bfloat16, device=hip_device)
    L.la_create(78, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 0)
    for pinned in (True, False):
        h = torch.randn(n)
        if pinned:
            h = h.pin_memory()
        before = h.clone()
        for k in range(4):      # the host array as p, m, v or g
            arrs = [dev[0].data_ptr(), gd.data_ptr(), dev[1].data_ptr(), dev[2].data_ptr()]
            if k == 1:
                hb = h.bfloat16() if not pinned else h.bfloat16().pin_memory()
                arrs[1] = hb.data_ptr()
            else:
                arrs[k] = h.data_ptr()
            rc = L.la_adam_update(78, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, _lib.LA_F32, arrs[0], _lib.LA_BF16, arrs[1],
                                  _lib.LA_F32, arrs[2], arrs[3], n, None, None, st)
            assert rc == _lib.LA_EFAULT, (pinned, k, rc)
        # the bf16 copy and the clip coefficient on the host
        hb16 = torch.zeros(n, dtype=torch.bfloat16)
        assert L.la_adam_update(78, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, _lib.LA_F32, dev[0].data_ptr(), _lib.LA_BF16,
                                gd.data_ptr(), _lib.LA_F32, dev[1].data_ptr(), dev[2].data_ptr(), n,
                                hb16.data_ptr(), None, st) == _lib.LA_EFAULT
        coef_h = torch.ones(1)
        assert L.la_adam_update(78, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, _lib.LA_F32, dev[0].data_ptr(), _lib.LA_BF16,
                                gd.data_ptr(), _lib.LA_F32, dev[1].data_ptr(), dev[2].data_ptr(), n, None,
                                coef_h.data_ptr(), st) == _lib.LA_EFAULT
        # the grad norm and the clip coefficient on host memory
        ws = torch.zeros(64, dtype=torch.float64, device=hip_device)
        sq = torch.zeros(1, dtype=torch.float64, device=hip_device)
        assert L.la_grad_sqnorm(_lib.LA_F32, h.data_ptr(), n, ws.data_ptr(), 512, sq.data_ptr(), 0, st) == _lib.LA_EFAULT
        sq_h = torch.zeros(1, dtype=torch.float64)
        assert L.la_clip_coef(sq_h.data_ptr(), 1.0, coef_h.data_ptr(), None, st) == _lib.LA_EFAULT
        torch.cuda.synchronize()
        assert torch.equal(h, before) and not hb16.any() and coef_h.item() == 1.0
    # device arrays still work
    assert L.la_adam_update(78, 2, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, _lib.LA_F32, dev[0].data_ptr(), _lib.LA_BF16,
                            gd.data_ptr(), _lib.LA_F32, dev[1].data_ptr(), dev[2].data_ptr(), n, None, None, st) == 0
    torch.cuda.synchronize()
    L.la_destroy(78)
