"""A tiny model trained through LayerAdam the way the sliding-window runtime
drives it, checked bit for bit against the CPU checker.

The reference's only smoke check (multi_gpu/scripts/main_dp.py:117-124) trains
a random 2-layer model and asserts that the weights changed, stayed finite and
that the step count is right.  Here the same model shape of use runs through
the runtime's protocol on one MI355X:

- each layer's fp32 master, exp_avg and exp_avg_sq are flat and resident in
  HBM (transformer_layer.py:192-196, layer_adam.py:161-173);
- the module's parameters are views into a flat bf16 compute copy, the GPU
  cache unit (offload_transformer.py:205-219), and their ``.grad`` are views
  into a flat bf16 grad buffer (transformer_layer.py:217-238), so backward
  accumulates straight into it;
- one global clip coefficient is accumulated in sliding order, last layer
  first (offload_transformer.py:265-301);
- each layer is stepped with begin_chunk_step / step_chunk(bf16_out=compute
  copy, clip_coef=coef) / end_chunk_step over two chunks whose boundary is not
  a multiple of 16 (transformer_layer.py:453-493), so every call has a scalar
  tail.

The oracle replays exactly the same calls on host copies (same grads, same
coefficient), so master, moments and compute copy must agree bit for bit at
the end of the run; the forward pass of each step reads the compute copy the
previous step wrote, so a difference at any step would carry through.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from slideformer_amd import LayerAdam
from tests import _hip as H

pytestmark = pytest.mark.gpu

D, F, BATCH, STEPS = 128, 512, 64, 30
LR, BETAS, EPS, WD, MAX_NORM = 3e-3, (0.9, 0.999), 1e-8, 0.01, 1.0


class Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.norm = torch.nn.RMSNorm(D)
        self.up = torch.nn.Linear(D, F)
        self.down = torch.nn.Linear(F, D)

    def forward(self, x):
        return x + self.down(torch.nn.functional.gelu(self.up(self.norm(x))))


def _bind_flat(module, compute, grads):
    """Replace the module's parameters by views into `compute` (bf16) and point
    their .grad at views into `grads`; return the fp32 master in the same order."""
    pieces, off = [], 0
    for name, p in list(module.named_parameters()):
        n = p.numel()
        pieces.append(p.detach().reshape(-1).float())
        view = torch.nn.Parameter(compute[off:off + n].view(p.shape))
        view.grad = grads[off:off + n].view(p.shape)
        owner = module
        *path, leaf = name.split(".")
        for part in path:
            owner = getattr(owner, part)
        setattr(owner, leaf, view)
        off += n
    return torch.cat(pieces)


def test_tiny_model_trains_through_the_runtime_protocol_bit_exact(hip_device):
    torch.manual_seed(0)
    blocks = [Block(), Block()]
    sizes = [sum(p.numel() for p in b.parameters()) for b in blocks]
    masters, computes, gflats = [], [], []
    for b, n in zip(blocks, sizes):
        compute = torch.empty(n, dtype=torch.bfloat16, device=hip_device)
        gflat = torch.zeros(n, dtype=torch.bfloat16, device=hip_device)
        master = _bind_flat(b, compute, gflat).to(hip_device)
        compute.copy_(master)                  # the first compute copy: RNE of the master
        masters.append(master)
        computes.append(compute)
        gflats.append(gflat)
    adam = LayerAdam(lr=LR, betas=BETAS, eps=EPS, weight_decay=WD)
    for idx, master in enumerate(masters):
        assert adam.add_layer_params(idx, [torch.nn.Parameter(master)]) == idx
    initial = [m.cpu().numpy().copy() for m in masters]

    # the oracle's copy of every buffer, stepped by the same sequence of calls
    orc = O.OracleAdam(LR, BETAS, EPS, WD, True)
    host_p = [m.copy() for m in initial]
    host_m = [np.zeros(n, np.float32) for n in sizes]
    host_v = [np.zeros(n, np.float32) for n in sizes]

    gen = torch.Generator(device=hip_device)
    gen.manual_seed(1)
    x = torch.randn(BATCH, D, generator=gen, device=hip_device).bfloat16()
    target = torch.randn(BATCH, D, generator=gen, device=hip_device)
    order = [1, 0]                             # sliding order: last layer first
    losses = []
    for step in range(1, STEPS + 1):
        for gflat in gflats:
            gflat.zero_()
        y = x
        for b in blocks:
            y = b(y)
        loss = torch.nn.functional.mse_loss(y.float(), target)
        loss.backward()
        losses.append(loss.item())
        for b, gflat in zip(blocks, gflats):   # backward accumulated into the flat buffers
            base = gflat.untyped_storage().data_ptr()
            assert all(p.grad.untyped_storage().data_ptr() == base for p in b.parameters())
            assert bool(gflat.abs().sum() > 0)

        acc = adam.grad_norm_begin(hip_device)
        for idx in order:
            acc.add(gflats[idx])
        coef, _ = acc.finish(MAX_NORM)
        for idx in order:
            n = sizes[idx]
            cut = n // 2 + 5                   # chunk boundary off the 16-element grid
            group = adam.begin_chunk_step(idx)
            for cs, ce in ((0, cut), (cut, n)):
                adam.step_chunk(masters[idx][cs:ce], gflats[idx][cs:ce], adam.exp_avg_flat[idx][cs:ce],
                                adam.exp_avg_sq_flat[idx][cs:ce], group, bf16_out=computes[idx][cs:ce],
                                clip_coef=coef)
            adam.end_chunk_step(idx)

        c = float(coef.item())
        for idx in order:
            g_bits = H.to_np_bits(gflats[idx], "bf16")
            n = sizes[idx]
            cut = n // 2 + 5
            for cs, ce in ((0, cut), (cut, n)):
                orc.update(step, LR, BETAS[0], BETAS[1], EPS, WD, True, host_p[idx][cs:ce], g_bits[cs:ce],
                           host_m[idx][cs:ce], host_v[idx][cs:ce], g16="bf16", clip_coef=c)
    torch.cuda.synchronize()

    assert losses[-1] < 0.7 * losses[0], losses
    for idx in range(len(blocks)):
        p = H.to_np_bits(masters[idx], "f32")
        assert np.array_equal(p, host_p[idx].view(np.uint32)), idx
        assert np.array_equal(H.to_np_bits(adam.exp_avg_flat[idx], "f32"), host_m[idx].view(np.uint32)), idx
        assert np.array_equal(H.to_np_bits(adam.exp_avg_sq_flat[idx], "f32"), host_v[idx].view(np.uint32)), idx
        # the module computes with exactly the RNE bf16 copy of the master
        assert np.array_equal(H.to_np_bits(computes[idx], "bf16"), O.f32_to_bf16(host_p[idx])), idx
        assert np.isfinite(host_p[idx]).all() and not np.array_equal(host_p[idx], initial[idx])
        assert adam.param_groups[idx]["step"] == STEPS
