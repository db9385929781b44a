"""The runtime's host-state layouts at full size, bit for bit.

SlideFormer's runtime keeps every layer's fp32 master in pageable host memory
(transformer_layer.py:192-196), lands each layer's bf16 grads in ONE
page-locked buffer shared by all layers (:206), copies them there in 32 Mi-
element chunks with an event per chunk (:26-27, :384-389), and lets an update
thread call LayerAdam.step_chunk once per chunk on the host master and the
moments (:453-493).  The smaller tests replay that protocol at a few thousand
elements; here it runs on a whole Llama-3.1-8B decoder layer, and the whole
Llama-3.1-8B-shaped model is stepped from host masters in sliding order.

Each streamed result is compared with the same calls on HBM-resident copies
(every bit of every array) and with the CPU checker replaying the same calls:
over the whole C2 layer, and in windows of the C3 segments."""
from __future__ import annotations

import queue
import threading

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slideformer_amd import LayerAdam, _lib
from tests import _hip as H

pytestmark = pytest.mark.gpu

VOCAB = 128256
LLAMA8B_LAYER = sum([4096 * 4096, 1024 * 4096, 1024 * 4096, 4096 * 4096, 14336 * 4096, 14336 * 4096,
                     4096 * 14336, 4096, 4096])
CALL_CHUNK = 32 * 1024 * 1024      # the runtime's chunk, transformer_layer.py:26-27
LR, WD = 1e-5, 0.01


def log(msg):
    print(msg, flush=True)


def device_randn(n, seed, dev, std):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    return torch.randn(n, generator=gen, device=dev) * std


def equal_on_device(a, b, piece=256 * 1024 * 1024):
    """Bitwise equality of two equal-sized arrays (either may be in host memory), compared on the device."""
    dev = b.device if b.is_cuda else a.device
    iv = torch.int32 if a.element_size() == 4 else torch.int16
    for lo in range(0, a.numel(), piece):
        hi = min(a.numel(), lo + piece)
        if not torch.equal(a[lo:hi].to(dev).view(iv), b[lo:hi].to(dev).view(iv)):
            return False
    return True


def bits_equal(got, want, kind):
    """Indices (at most 8) where a tensor's bits differ from a checker array's."""
    w = want.view(np.uint32) if kind == "f32" else want
    return np.flatnonzero(H.to_np_bits(got, kind) != w)[:8]


@pytest.mark.parametrize("moments_in_hbm", [False, True])
def test_runtime_protocol_on_a_full_c2_layer(moments_in_hbm, hip_device):
    """One Llama-3.1-8B decoder layer (218,112,000 params) through the runtime's
    host-side protocol, two steps: pageable fp32 master; one page-locked bf16
    grad buffer that a producer stream fills in 32 Mi-element chunks with an
    event per chunk; an update thread that waits for each event and calls
    step_chunk on that chunk of the master, the shared grad buffer and the
    moments (7 calls per step, the last one short), with
    overlap_host_chunks=True, the step's clip coefficient and the bf16 copy
    written into a device cache-unit buffer; then end_chunk_step.  The
    moments are pageable host arrays (the reference's allocation) or in HBM
    (moments_device).  After each step, every bit of master, moments and copy
    equals the CPU checker replaying the same seven calls over the whole
    layer, and the same calls on HBM-resident copies."""
    dev, n = hip_device, LLAMA8B_LAYER
    seed = 7100 + 10 * int(moments_in_hbm)
    p0 = device_randn(n, seed, dev, 0.02)
    master = torch.empty(n, dtype=torch.float32)          # pageable, as the runtime allocates it
    master.copy_(p0)
    assert not _lib.is_page_locked(master)
    adam = LayerAdam(lr=LR, weight_decay=WD, overlap_host_chunks=True,
                     moments_device=dev if moments_in_hbm else None)
    adam.add_layer_params(0, [torch.nn.Parameter(master)])
    m_s, v_s = adam.exp_avg_flat[0], adam.exp_avg_sq_flat[0]
    assert m_s.is_cuda == moments_in_hbm and (moments_in_hbm or not _lib.is_page_locked(m_s))
    resident = LayerAdam(lr=LR, weight_decay=WD)
    p_r = p0.clone()
    resident.add_layer_params(0, [torch.nn.Parameter(p_r)])
    m_r, v_r = resident.exp_avg_flat[0], resident.exp_avg_sq_flat[0]
    shared_grad = torch.empty(n, dtype=torch.bfloat16, pin_memory=True)   # transformer_layer.py:206
    cache_unit = torch.empty(n, dtype=torch.bfloat16, device=dev)
    out_r = torch.empty(n, dtype=torch.bfloat16, device=dev)
    producer = torch.cuda.Stream(device=dev)
    bounds = list(range(0, n, CALL_CHUNK))
    assert len(bounds) == 7 and n % CALL_CHUNK != 0 and n % 16 == 0
    # the CPU checker's copy of the whole layer
    orc = O.OracleAdam(LR, (0.9, 0.999), 1e-8, WD, True)
    p_o = H.to_np_bits(p0, "f32").view(np.float32).copy()
    m_o, v_o = np.zeros(n, np.float32), np.zeros(n, np.float32)
    out_o = np.zeros(n, np.uint16)
    del p0
    for step in (1, 2):
        g = device_randn(n, seed + step, dev, 1e-3).bfloat16()
        coef, _ = adam.clip_grad_norm([g], 1.0)
        torch.cuda.synchronize()
        c = float(coef.item())
        assert 0.0 < c < 1.0
        log(f"C2 protocol (moments {'HBM' if moments_in_hbm else 'host'}): step {step}, coef {c}")
        q: "queue.Queue" = queue.Queue()
        errors = []

        def update_thread():
            try:
                group = adam.begin_chunk_step(0)
                while True:
                    item = q.get()
                    if item is None:
                        break
                    cs, ce, ev = item
                    ev.synchronize()
                    adam.step_chunk(master[cs:ce], shared_grad[cs:ce], m_s[cs:ce], v_s[cs:ce], group,
                                    bf16_out=cache_unit[cs:ce], clip_coef=coef)
                adam.end_chunk_step(0)
            except Exception as exc:           # reported by the main thread
                errors.append(exc)

        t = threading.Thread(target=update_thread)
        t.start()
        with torch.cuda.stream(producer):
            for cs in bounds:
                ce = min(cs + CALL_CHUNK, n)
                shared_grad[cs:ce].copy_(g[cs:ce], non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(producer)
                q.put((cs, ce, ev))
        q.put(None)
        t.join(timeout=240)
        assert not t.is_alive() and not errors, errors
        group_r = resident.begin_chunk_step(0)
        g_h = H.to_np_bits(g, "bf16")
        for cs in bounds:
            ce = min(cs + CALL_CHUNK, n)
            resident.step_chunk(p_r[cs:ce], g[cs:ce], m_r[cs:ce], v_r[cs:ce], group_r, bf16_out=out_r[cs:ce],
                                clip_coef=coef)
            orc.update(step, LR, 0.9, 0.999, 1e-8, WD, True, p_o[cs:ce], g_h[cs:ce], m_o[cs:ce], v_o[cs:ce],
                       g16="bf16", p_bf16_out=out_o[cs:ce], clip_coef=c)
        resident.end_chunk_step(0)
        torch.cuda.synchronize()
        log(f"C2 protocol: compare step {step} with the resident calls and the CPU checker")
        for a, b, what in ((master, p_r, "p"), (m_s, m_r, "m"), (v_s, v_r, "v"), (cache_unit, out_r, "out")):
            assert equal_on_device(a, b), (step, what)
        for got, want, kind, what in ((master, p_o, "f32", "p"), (m_s, m_o, "f32", "m"), (v_s, v_o, "f32", "v"),
                                      (cache_unit, out_o, "bf16", "out")):
            bad = bits_equal(got, want, kind)
            assert bad.size == 0, (step, what, bad)
        del g, g_h, coef


@pytest.mark.parametrize("layout", ["moments_in_hbm", "all_on_host"])
def test_c3_whole_model_streamed_from_host_state(layout, hip_device):
    """Config C3 stepped whole from host state, in two layouts:
    - moments_in_hbm, the layout recommended for the runtime: every segment's
      fp32 master in host memory, its moments in HBM
      (LayerAdam(moments_device=...)); the masters of lm_head and layers
      31-16 (sliding order) page-locked at exact size, the other 17 segments
      pageable and staged;
    - all_on_host, the reference's own layout: master, m and v of every
      segment in host memory; those of lm_head and layers 31-12 page-locked
      at exact size (54.6 GiB: one process may page-lock at most 64 GiB on
      these hosts), the other 13 segments pageable and staged.
    bf16 grads and copies in HBM; the moments start from non-zero values.  One
    step: the global grad norm over all 34 segments in sliding order, one
    clip coefficient, then every segment stepped in sliding order (lm_head,
    L31 ... L0, embed; offload_transformer.py:265-301,
    transformer_layer.py:453-493).  Each segment's master, moments and copy
    equal, bit for bit, the same calls on HBM-resident copies; both vocab
    segments and the first and last decoder layers also equal, every element,
    the CPU checker replaying the step's calls on one optimizer id."""
    dev = hip_device
    sizes = [VOCAB * 4096] + [LLAMA8B_LAYER] * 32 + [4096 + VOCAB * 4096]
    assert sum(sizes) == 8_030_261_248 and len(sizes) == 34
    order = list(range(33, -1, -1))
    host_moments = layout == "all_on_host"
    # lm_head and layers 31-16 (segments 33, 32-17), or 31-12 (33, 32-13)
    pinned = {33} | set(range(13 if host_moments else 17, 33))
    assert not host_moments or 12 * sum(sizes[i] for i in pinned) < 55 * 2**30
    adam = LayerAdam(lr=LR, weight_decay=WD, moments_device=None if host_moments else dev)
    resident = LayerAdam(lr=LR, weight_decay=WD)
    masters = []
    log(f"C3 streamed ({layout}): host state for 34 segments")
    for idx, n in enumerate(sizes):
        p0 = device_randn(n, 8000 + idx, dev, 0.02)
        p_h = _lib.page_locked_empty(n, torch.float32) if idx in pinned else torch.empty(n, dtype=torch.float32)
        p_h.copy_(p0)
        masters.append(p_h)
        adam.pin_host_state = idx in pinned         # read by add_layer_params for host moments
        assert adam.add_layer_params(idx, [torch.nn.Parameter(p_h)]) == idx
        adam.exp_avg_flat[idx].copy_(device_randn(n, 9000 + idx, dev, 1e-5))
        adam.exp_avg_sq_flat[idx].copy_(device_randn(n, 10000 + idx, dev, 3e-5).square_())
        m_h = adam.exp_avg_flat[idx]
        assert m_h.is_cuda != host_moments and _lib.is_page_locked(p_h) == (idx in pinned)
        assert not host_moments or _lib.is_page_locked(m_h) == (idx in pinned)
        # the resident twin registers an empty stand-in: its state is made per segment at step time
        assert resident.add_layer_params(idx, [torch.nn.Parameter(torch.empty(1, device=dev))]) == idx
        del p0
    torch.cuda.synchronize()

    def grads(idx):
        return device_randn(sizes[idx], 11000 + idx, dev, 1e-3).bfloat16()

    log(f"C3 streamed ({layout}): global grad norm in sliding order")
    acc = adam.grad_norm_begin(dev)
    for idx in order:
        acc.add(grads(idx))
    coef, _ = acc.finish(1.0)
    torch.cuda.synchronize()
    c = float(coef.item())
    assert 0.0 < c < 1.0

    checked = {0, 1, 32, 33}                              # embed, layer 0, layer 31, lm_head
    for j, idx in enumerate(order):
        n = sizes[idx]
        g = grads(idx)
        # the resident replay of this segment, from the same initial values
        p_r = device_randn(n, 8000 + idx, dev, 0.02)
        m_r = adam.exp_avg_flat[idx].to(dev, copy=True)
        v_r = adam.exp_avg_sq_flat[idx].to(dev, copy=True)
        if idx in checked:      # the checker's copy of the whole segment
            p_o, m_o, v_o = (H.to_np_bits(t, "f32").view(np.float32).copy() for t in (p_r, m_r, v_r))
        out_s = torch.empty(n, dtype=torch.bfloat16, device=dev)
        out_r = torch.empty(n, dtype=torch.bfloat16, device=dev)
        group = adam.begin_chunk_step(idx)
        adam.step_chunk(masters[idx], g, adam.exp_avg_flat[idx], adam.exp_avg_sq_flat[idx], group, bf16_out=out_s,
                        clip_coef=coef)
        adam.end_chunk_step(idx)
        st = adam.last_stream_stats
        assert st.h2d_bytes == st.d2h_bytes == (12 if host_moments else 4) * n   # the host arrays crossed the link
        group_r = resident.begin_chunk_step(idx)
        resident.step_chunk(p_r, g, m_r, v_r, group_r, bf16_out=out_r, clip_coef=coef)
        resident.end_chunk_step(idx)
        torch.cuda.synchronize()
        for a, b, what in ((masters[idx], p_r, "p"), (adam.exp_avg_flat[idx], m_r, "m"),
                           (adam.exp_avg_sq_flat[idx], v_r, "v"), (out_s, out_r, "out")):
            assert equal_on_device(a, b), (idx, what)
        if idx in checked:
            log(f"C3 streamed ({layout}): segment {idx} (call {j} of the step) against the CPU checker")
            orc = O.OracleAdam(LR, (0.9, 0.999), 1e-8, WD, True)
            e = np.zeros(0, np.float32)
            for _ in range(j):          # the earlier calls of this step on the same optimizer id
                orc.update(1, LR, 0.9, 0.999, 1e-8, WD, True, e, np.zeros(0, np.uint16), e.copy(), e.copy(),
                           g16="bf16")
            out_o = np.zeros(n, np.uint16)
            orc.update(1, LR, 0.9, 0.999, 1e-8, WD, True, p_o, H.to_np_bits(g, "bf16"), m_o, v_o, g16="bf16",
                       p_bf16_out=out_o, clip_coef=c)
            for got, want, kind, what in ((masters[idx], p_o, "f32", "p"), (adam.exp_avg_flat[idx], m_o, "f32", "m"),
                                          (adam.exp_avg_sq_flat[idx], v_o, "f32", "v"), (out_s, out_o, "bf16", "out")):
                bad = bits_equal(got, want, kind)
                assert bad.size == 0, (idx, what, bad)
            del p_o, m_o, v_o, out_o
        if j % 8 == 0:
            log(f"C3 streamed ({layout}): {j + 1} of 34 segments stepped and compared")
        del g, p_r, m_r, v_r, out_s, out_r
    del adam, resident, masters, acc
    torch._C._host_emptyCache()
    torch.cuda.empty_cache()


C5_LAYER = sum([12288 * 3 * 12288, 3 * 12288, 12288 * 12288, 12288, 12288 * 49152, 49152, 49152 * 12288, 12288,
                12288, 12288, 12288, 12288])


def test_nvme_offload_of_a_c5_layer(hip_device, tmp_path):
    """The moment file offload at full size (layer_adam.py:92-106, 200-247):
    a C5 layer (1,812,099,072 params; each moment a 7.25 GB file, so file
    offsets pass 2^32 bytes) and a small layer, nvme_offload_fraction=1.0,
    prefetch=True, direct I/O (the reference's backend name 'uring'), two
    iterations in sliding order (small layer, then C5), the runtime's
    begin_chunk_step / step_chunk / end_chunk_step with device grads and the
    master in pageable host memory.  Between the steps the moments live only
    in their files (storage released).  After the last write-back every
    element of both masters and of both layers' moments, read back from the
    files, equals the CPU checker's replay."""
    dev = hip_device
    sizes = [C5_LAYER, 10_001]
    assert sizes[0] == 1_812_099_072
    adam = LayerAdam(lr=6e-6, weight_decay=0.01, num_layer=2, nvme_offload_fraction=1.0,
                     offload_dir=str(tmp_path), prefetch=True)
    assert adam.offloader.direct
    params, p_o = [], []
    for idx, n in enumerate(sizes):
        p0 = device_randn(n, 12000 + idx, dev, 0.02)
        p_h = torch.empty(n, dtype=torch.float32)
        p_h.copy_(p0)
        params.append(torch.nn.Parameter(p_h))
        p_o.append(H.to_np_bits(p0, "f32").view(np.float32))
        del p0
        assert adam.add_layer_params(idx, [params[idx]]) == idx
    # layer 0 is not the last one: its moments went to their files at registration
    assert adam.exp_avg_flat[0].untyped_storage().nbytes() == 0
    m_o = [np.zeros(n, np.float32) for n in sizes]
    v_o = [np.zeros(n, np.float32) for n in sizes]
    orc = O.OracleAdam(6e-6, (0.9, 0.999), 1e-8, 0.01, True)
    for it in range(2):
        for idx in (1, 0):                                   # sliding order: the last layer first
            n = sizes[idx]
            log(f"NVMe C5: iteration {it}, layer {idx} ({n} params)")
            g = device_randn(n, 13000 + 10 * it + idx, dev, 5e-4).bfloat16()
            group = adam.begin_chunk_step(idx)
            assert adam.exp_avg_flat[idx].untyped_storage().nbytes() == 4 * n     # read back (prefetched)
            adam.step_chunk(params[idx].data, g, adam.exp_avg_flat[idx], adam.exp_avg_sq_flat[idx], group)
            adam.end_chunk_step(idx)
            orc.update(group["step"], 6e-6, 0.9, 0.999, 1e-8, 0.01, True, p_o[idx], H.to_np_bits(g, "bf16"),
                       m_o[idx], v_o[idx], g16="bf16")
            del g
    adam.offloader.sync_write_events()
    # the C5 layer's moments were written back last and released; the small
    # layer's last release was cancelled by the prefetch that followed it (its
    # write was fenced), so its buffers still hold the bytes: write them out
    assert adam.exp_avg_flat[0].untyped_storage().nbytes() == 0
    for idx, n in enumerate(sizes):
        log(f"NVMe C5: layer {idx} against the CPU checker")
        bad = np.flatnonzero(params[idx].data.numpy().view(np.uint32) != p_o[idx].view(np.uint32))[:8]
        assert bad.size == 0, (idx, "p", bad)
        for t in (adam.exp_avg_flat[idx], adam.exp_avg_sq_flat[idx]):
            if t.untyped_storage().nbytes():
                adam.offloader.sync_write(t)
            assert t.untyped_storage().nbytes() == 0                              # in its file only
        adam._load_layer(idx)
        adam.offloader.sync_read_events()
        for t, want, what in ((adam.exp_avg_flat[idx], m_o[idx], "m"), (adam.exp_avg_sq_flat[idx], v_o[idx], "v")):
            bad = np.flatnonzero(t.numpy().view(np.uint32) != want.view(np.uint32))[:8]
            assert bad.size == 0, (idx, what, bad)
    del adam, params, p_o, m_o, v_o
