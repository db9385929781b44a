"""Child process of tests/test_gpu_allocators.py (not a test module).

Runs LayerAdam on one GPU under whatever torch caching-allocator
configuration the parent put into PYTORCH_HIP_ALLOC_CONF (the stream-ordered
hipMallocAsync backend, or the default), so that every device array the
library sees comes from that allocator:
  A. clip_grad_norm over three device grads, then step_with_grad_views twice
     with the clip coefficient (la_grad_norm_multi, la_adam_update_multi);
  B. step_chunk on flat device buffers with the bf16 copy (la_adam_update);
  C. step_chunk on a host-resident master with device grads and moments
     (la_pipeline_step: its device slots come from the allocator too).
Reads the inputs from the .npz named by argv[1], writes every result's raw
bits to the .npz named by argv[2], and prints one line naming the backend.

usage: python tests/alloc_child.py IN.npz OUT.npz
"""
from __future__ import annotations

import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)


def main() -> int:
    import torch

    from slideformer_amd import LayerAdam

    inp = np.load(sys.argv[1])
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    def f32(a):
        return torch.from_numpy(a.view(np.int32).copy()).view(torch.float32).to(dev)

    def bf16(a):
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev)

    def bits(t):
        t = t.detach().contiguous().cpu()
        return (t.view(torch.int32) if t.element_size() == 4 else t.view(torch.int16)).numpy().copy()

    out = {}
    # A: a layer of three tensors, global clip, two steps
    k = int(inp["a_count"])
    params = [torch.nn.Parameter(f32(inp[f"a_p{i}"])) for i in range(k)]
    grads = [bf16(inp[f"a_g{i}"]) for i in range(k)]
    adam = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    adam.add_layer_params(0, params)
    coef, norm = adam.clip_grad_norm(grads, 0.5)
    for _ in range(2):
        # bf16 grads of fp32 params, as the runtime hands them over (a param's
        # .grad must have the param's dtype)
        adam.step_with_grad_views(0, dict(zip(params, grads)), clip_coef=coef)
    torch.cuda.synchronize()
    out["a_coef"], out["a_norm"] = bits(coef), bits(norm)
    for i, prm in enumerate(params):
        out[f"a_p{i}"] = bits(prm.data)
        out[f"a_m{i}"] = bits(adam.state[prm]["exp_avg"])
        out[f"a_v{i}"] = bits(adam.state[prm]["exp_avg_sq"])

    # B: one flat device call with the bf16 copy
    p, g, m, v = f32(inp["b_p"]), bf16(inp["b_g"]), f32(inp["b_m"]), f32(inp["b_v"])
    copy = torch.empty(p.numel(), dtype=torch.bfloat16, device=dev)
    adam_b = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    adam_b.step_chunk(p, g, m, v, dict(adam_b.defaults, step=1), bf16_out=copy)
    torch.cuda.synchronize()
    out.update(b_p=bits(p), b_m=bits(m), b_v=bits(v), b_out=bits(copy))

    # C: host-resident master streamed through the pipeline, moments and grads in HBM
    ph = torch.from_numpy(inp["c_p"].view(np.int32).copy()).view(torch.float32)
    gc, mc, vc = bf16(inp["c_g"]), f32(inp["c_m"]), f32(inp["c_v"])
    copy_c = torch.empty(ph.numel(), dtype=torch.bfloat16, device=dev)
    adam_c = LayerAdam(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    adam_c.step_chunk(ph, gc, mc, vc, dict(adam_c.defaults, step=1), bf16_out=copy_c)
    torch.cuda.synchronize()
    out.update(c_p=ph.view(torch.int32).numpy().copy(), c_m=bits(mc), c_v=bits(vc), c_out=bits(copy_c))

    np.savez(sys.argv[2], **out)
    print(f"ALLOC_CHILD_OK backend={torch.cuda.get_allocator_backend()}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
