"""Whole-model workloads on the GPU: config C3 (the Llama-3.1-8B-shaped model,
stepped from page-locked host state) and config C4 (the 48-layer
Qwen2.5-14B-shaped stack with one global clip).

Both follow the runtime's order: grads land in sliding order, last segment
first (post-backward hooks, offload_transformer.py:265-301), a global grad
norm is accumulated segment by segment as they land (GradNormAccumulator),
one clip coefficient is taken, and then the segments are stepped in the same
order with begin_chunk_step / step_chunk / end_chunk_step
(transformer_layer.py:453-493).  Grads are generated per segment on the
device from fixed seeds, so a segment's grads can be made again instead of
being kept."""
from __future__ import annotations

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
QWEN14B_LAYER = sum([5120 * 5120, 5120, 5120 * 1024, 1024, 5120 * 1024, 1024, 5120 * 5120, 5120 * 13824,
                     5120 * 13824, 13824 * 5120, 5120, 5120])


def log(msg):
    print(msg, flush=True)


def seg_grad(n, seed, dev, std=1e-3, outliers=False):
    """bf16 grads N(0, std) of one segment, from its seed, on the device; with
    outliers, 0.1 % of the indices (seeded) scaled x100."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    g = (torch.randn(n, generator=gen, device=dev) * std).bfloat16()
    if outliers:
        sel = torch.randint(0, n, (n // 1000,), generator=gen, device=dev)
        g[sel] = g[sel] * 100
    return g


def oracle_sqnorm(g):
    """The CPU checker's compensated float64 sum of squares of device bf16 grads."""
    return O.grad_sqnorm(H.to_np_bits(g, "bf16"), "bf16")


def equal_on_device(a, b, piece=256 * 1024 * 1024):
    """Bitwise equality of two fp32 arrays (either may be in host memory), compared on the device."""
    dev = b.device if b.is_cuda else a.device
    for lo in range(0, a.numel(), piece):
        hi = min(a.numel(), lo + piece)
        x, y = a[lo:hi].to(dev), b[lo:hi].to(dev)
        if not torch.equal(x.view(torch.int32), y.view(torch.int32)):
            return False
    return True


def test_c3_model_sliding_order_from_page_locked_state(hip_device):
    """Config C3: the Llama-3.1-8B-shaped model, 34 segments in layer-index order
    (embed 128256 x 4096; 32 decoder layers of 218,112,000; final norm + lm_head
    4096 + 128256 x 4096), 8,030,261,248 params.  The global norm covers all 34
    segments.  Four of them are stepped in sliding order with the clip
    coefficient: lm_head, layers 31 and 30, embed.  Their fp32 master, m and v
    are in page-locked host memory (one exact-size page-locked allocation per
    array and segment) and stream through HBM in LayerAdam's default 16 Mi-element
    (64 MB) chunks; grads and bf16 copies are in HBM.  Each segment's results
    equal, bit for bit, the same step on HBM-resident copies, and windows at
    the start, across the first chunk boundary and at the end (in the short
    last chunk) equal the CPU checker's."""
    dev = hip_device
    sizes = [VOCAB * 4096] + [LLAMA8B_LAYER] * 32 + [4096 + VOCAB * 4096]
    assert sum(sizes) == 8_030_261_248 and len(sizes) == 34
    order = list(range(33, -1, -1))                       # sliding order: lm_head first
    stepped = [33, 32, 31, 0]                             # in sliding order
    seed = {idx: 3000 + idx for idx in range(34)}
    adam = LayerAdam(lr=1e-5, weight_decay=0.01, pin_host_state=True)
    resident = LayerAdam(lr=1e-5, weight_decay=0.01)

    # 1. the global norm, accumulated as the grads land
    log("C3: global grad norm over 34 segments in sliding order")
    acc = adam.grad_norm_begin(dev)
    total, kept = 0.0, {}
    for idx in order:
        g = seg_grad(sizes[idx], seed[idx], dev)
        acc.add(g)
        total += oracle_sqnorm(g)
        if idx in stepped:
            kept[idx] = g
        del g
    coef, norm = acc.finish(1.0)
    torch.cuda.synchronize()
    assert acc.count == 34
    assert abs(acc.sqnorm.item() - total) <= 1e-12 * total, (acc.sqnorm.item(), total)
    c_ref, n_ref = O.clip_coef(total, 1.0)
    assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)
    c = float(coef.item())
    assert 0.0 < c < 1.0                                  # ||g|| ~ 1e-3 * sqrt(8e9) ~ 90: clipping triggers

    # 2. state of the stepped segments: page-locked host copies and HBM twins
    #    (the optimizers hold the stepped segments only, registered in
    #    layer-index order: positions 0..3 = embed, layer 30, layer 31, lm_head)
    pos = {idx: k for k, idx in enumerate(sorted(stepped))}
    host, dev_state, outs_s, outs_r, windows = {}, {}, {}, {}, {}
    chunk = 16 * 1024 * 1024
    for idx in sorted(stepped):
        n = sizes[idx]
        log(f"C3: segment {idx} ({n} params): page-locked host state + HBM twin")
        gen = torch.Generator(device=dev)
        gen.manual_seed(4000 + idx)
        p_d = torch.randn(n, generator=gen, device=dev) * 0.02
        m_d = torch.randn(n, generator=gen, device=dev) * 1e-5
        v_d = torch.rand(n, generator=gen, device=dev) * 1e-9
        p_h = _lib.page_locked_empty(n, torch.float32)
        p_h.copy_(p_d)
        assert adam.add_layer_params(pos[idx], [torch.nn.Parameter(p_h)]) == pos[idx]
        assert resident.add_layer_params(pos[idx], [torch.nn.Parameter(p_d)]) == pos[idx]
        m_h, v_h = adam.exp_avg_flat[pos[idx]], adam.exp_avg_sq_flat[pos[idx]]
        assert _lib.is_page_locked(m_h) and _lib.is_page_locked(v_h) and _lib.is_page_locked(p_h)
        m_h.copy_(m_d)
        v_h.copy_(v_d)
        resident.exp_avg_flat[pos[idx]].copy_(m_d)
        resident.exp_avg_sq_flat[pos[idx]].copy_(v_d)
        host[idx] = (p_h, m_h, v_h)
        dev_state[idx] = (p_d, resident.exp_avg_flat[pos[idx]], resident.exp_avg_sq_flat[pos[idx]])
        outs_s[idx] = torch.empty(n, dtype=torch.bfloat16, device=dev)
        outs_r[idx] = torch.empty(n, dtype=torch.bfloat16, device=dev)
        windows[idx] = [(0, 4096), (chunk - 2048, chunk + 2048), (n - 4096, n)]
        assert n % chunk != 0                             # the last pipeline chunk is short
        del m_d, v_d
    torch.cuda.synchronize()
    init = {idx: [[t[lo:hi].cpu().numpy().copy() for t in host[idx]] for lo, hi in windows[idx]]
            for idx in stepped}

    # 3. the step, in sliding order, streamed and resident
    for idx in stepped:
        log(f"C3: step segment {idx}")
        k = pos[idx]
        p_h, m_h, v_h = host[idx]
        group = adam.begin_chunk_step(k)
        adam.step_chunk(p_h, kept[idx], m_h, v_h, group, bf16_out=outs_s[idx], clip_coef=coef)
        adam.end_chunk_step(k)
        st = adam.last_stream_stats
        assert st.chunks == -(-sizes[idx] // chunk) and st.h2d_bytes == st.d2h_bytes == 12 * sizes[idx]
        group_r = resident.begin_chunk_step(k)
        resident.step_chunk(dev_state[idx][0], kept[idx], dev_state[idx][1], dev_state[idx][2], group_r,
                            bf16_out=outs_r[idx], clip_coef=coef)
        resident.end_chunk_step(k)
    torch.cuda.synchronize()

    # 4. streamed == resident, and windows == the CPU checker
    for j, idx in enumerate(stepped):
        log(f"C3: compare segment {idx}")
        for a, b in zip(host[idx], dev_state[idx]):
            assert equal_on_device(a, b), idx
        assert torch.equal(outs_s[idx].view(torch.int16), outs_r[idx].view(torch.int16)), idx
        g = kept[idx]
        for (lo, hi), (p0, m0, v0) in zip(windows[idx], init[idx]):
            # the j-th call of step 1 on one optimizer id: replay the earlier calls' state changes
            orc_w = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.01, True)
            e = np.zeros(0, np.float32)
            for _ in range(j):
                orc_w.update(1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, e, e.copy(), e.copy(), e.copy())
            orc_w.update(1, 1e-5, 0.9, 0.999, 1e-8, 0.01, True, p0, H.to_np_bits(g[lo:hi], "bf16"), m0, v0,
                         g16="bf16", clip_coef=c)
            p_h, m_h, v_h = host[idx]
            assert np.array_equal(p_h[lo:hi].numpy().view(np.uint32), p0.view(np.uint32)), (idx, lo)
            assert np.array_equal(m_h[lo:hi].numpy().view(np.uint32), m0.view(np.uint32)), (idx, lo)
            assert np.array_equal(v_h[lo:hi].numpy().view(np.uint32), v0.view(np.uint32)), (idx, lo)
            assert np.array_equal(H.to_np_bits(outs_s[idx][lo:hi], "bf16"), O.f32_to_bf16(p0)), (idx, lo)
    del adam, resident, host, dev_state, outs_s, outs_r, kept, init, acc
    torch._C._host_emptyCache()
    torch.cuda.empty_cache()


def test_c4_stack_global_clip_over_48_layers(hip_device):
    """Config C4: 48 Qwen2.5-14B-shaped layers of 275,268,608 params
    (13,212,893,184 in all), bf16 grads N(0, 1e-3) with 0.1 % of the indices
    (seeded) x100, generated per layer on the device.  The float64 norm
    accumulated over the 48 layers in sliding order is within 1e-12 of the sum
    of the CPU checker's per-layer compensated sums, and the clip coefficient
    and norm are bit-exact.  The first and the last layer, HBM-resident, are
    then stepped with that coefficient (AdamW, wd 0.1, bf16 copy), last layer
    first, and every bit equals the CPU checker's."""
    dev = hip_device
    n, layers = QWEN14B_LAYER, 48
    assert n == 275_268_608 and n * layers == 13_212_893_184 and n % 1024 == 0
    adam = LayerAdam(lr=1e-5, weight_decay=0.1)
    log("C4: global grad norm over 48 layers in sliding order")
    acc = adam.grad_norm_begin(dev)
    total, kept = 0.0, {}
    for idx in range(layers - 1, -1, -1):
        g = seg_grad(n, 5000 + idx, dev, outliers=True)
        acc.add(g)
        total += oracle_sqnorm(g)
        if idx in (0, layers - 1):
            kept[idx] = g
        del g
    coef, norm = acc.finish(1.0)
    torch.cuda.synchronize()
    assert acc.count == layers
    assert abs(acc.sqnorm.item() - total) <= 1e-12 * total, (acc.sqnorm.item(), total)
    c_ref, n_ref = O.clip_coef(total, 1.0)
    assert coef.item() == np.float32(c_ref) and norm.item() == np.float32(n_ref)
    c = float(coef.item())
    assert 0.0 < c < 1.0

    log("C4: step the last and the first layer with the global coefficient")
    orc = O.OracleAdam(1e-5, (0.9, 0.999), 1e-8, 0.1, True)
    for k, idx in enumerate((0, layers - 1)):
        gen = torch.Generator(device=dev)
        gen.manual_seed(6000 + idx)
        p = torch.randn(n, generator=gen, device=dev) * 0.02
        assert adam.add_layer_params(k, [torch.nn.Parameter(p)]) == k
    state = {}
    for k, idx in ((1, layers - 1), (0, 0)):                # sliding order: last layer first
        p = adam.param_groups[k]["params"][0].data
        m, v = adam.exp_avg_flat[k], adam.exp_avg_sq_flat[k]
        out = torch.empty(n, dtype=torch.bfloat16, device=dev)
        p_h, m_h, v_h = H.to_np_bits(p, "f32").view(np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)
        group = adam.begin_chunk_step(k)
        adam.step_chunk(p, kept[idx], m, v, group, bf16_out=out, clip_coef=coef)
        adam.end_chunk_step(k)
        orc.update(group["step"], 1e-5, 0.9, 0.999, 1e-8, 0.1, True, p_h, H.to_np_bits(kept[idx], "bf16"), m_h, v_h,
                   g16="bf16", clip_coef=c)
        state[idx] = (p, m, v, out, p_h, m_h, v_h)
    torch.cuda.synchronize()
    for idx, (p, m, v, out, p_h, m_h, v_h) in state.items():
        log(f"C4: compare layer {idx}")
        assert np.array_equal(H.to_np_bits(p, "f32"), p_h.view(np.uint32)), idx
        assert np.array_equal(H.to_np_bits(m, "f32"), m_h.view(np.uint32)), idx
        assert np.array_equal(H.to_np_bits(v, "f32"), v_h.view(np.uint32)), idx
        assert np.array_equal(H.to_np_bits(out, "bf16"), O.f32_to_bf16(p_h)), idx
    del state, kept, adam, acc
    torch.cuda.empty_cache()
