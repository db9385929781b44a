"""Write the golden fixtures in this directory from the reference CPU Adam.

The reference (optimizer/layer_adam/csrc/cpu_adam*.{h,cpp}) is compiled from
its own sources by ``oracle/Makefile`` (``make -C oracle ref``) into
``oracle/_ref/``; this script calls that build's ``adam_update`` /
``create_adam`` (cpu_adam.cpp:8-13) and stores inputs and outputs as raw bits.
Run it in the container that holds /root/reference:

    python tests/golden/make_golden.py

Each case is one optimizer id driven through ``steps`` steps of
``calls`` adam_update calls each (the calls of a step share its step number,
like the chunks of one layer, layer_adam.py:437-461).  Files:

  cases.npz   per case: hyper-parameters, dtype triple, p0/m0/v0, the grads of
              every call, and p/m/v after every step (all as raw integer bits).
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import torch  # noqa: E402

from oracle import oracle as O  # noqa: E402

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
BITS_DT = {"f32": np.uint32, "bf16": np.uint16, "f16": np.uint16}

GPT2_BLOCK = [("ln_1.w", 768), ("ln_1.b", 768), ("attn.c_attn.w", 768 * 2304),
              ("attn.c_attn.b", 2304), ("attn.c_proj.w", 768 * 768), ("attn.c_proj.b", 768),
              ("ln_2.w", 768), ("ln_2.b", 768), ("mlp.c_fc.w", 768 * 3072), ("mlp.c_fc.b", 3072),
              ("mlp.c_proj.w", 3072 * 768), ("mlp.c_proj.b", 768)]


def bits(t: torch.Tensor, kind: str) -> np.ndarray:
    t = t.contiguous()
    if kind == "f32":
        return t.view(torch.int32).numpy().view(np.uint32).copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def make_case(ref, name, *, triple=("f32", "bf16", "f32"), sizes=(35,), steps=3, lr=1e-3,
              betas=(0.9, 0.999), eps=1e-8, wd=0.01, adamw=True, bc=True, seed=0,
              p_std=0.02, g_std=1e-3, m0v0="zeros", lr_schedule=None, specials=False):
    """Run the reference and return a dict of arrays for one case.

    ``sizes``: one adam_update call per entry per step (chunk sizes of one layer).
    """
    rng = np.random.default_rng(seed)
    pk, gk, sk = triple
    n = int(sum(sizes))
    p = torch.from_numpy(rng.normal(0, p_std, n).astype(np.float32)).to(TORCH_DT[pk])
    if m0v0 == "zeros":
        m = torch.zeros(n, dtype=TORCH_DT[sk])
        v = torch.zeros(n, dtype=TORCH_DT[sk])
    else:
        m = torch.from_numpy(rng.normal(0, 1e-3, n).astype(np.float32)).to(TORCH_DT[sk])
        v = torch.from_numpy(np.abs(rng.normal(0, 1e-6, n)).astype(np.float32)).to(TORCH_DT[sk])
    out = {"p0": bits(p, pk), "m0": bits(m, sk), "v0": bits(v, sk)}
    ref.create_adam(0, lr, betas[0], betas[1], eps, wd, adamw, False)
    grads, lrs, ps, ms, vs = [], [], [], [], []
    for st in range(1, steps + 1):
        g32 = rng.normal(0, g_std, n).astype(np.float32)
        if specials:
            # NaN / +-Inf / zero / subnormal / huge grads at fixed spots
            g32[0::11] = 0.0
            g32[1::13] = 1e-41
            g32[2::17] = 3e4
            if st == steps:
                g32[3] = np.nan
                g32[5] = np.inf
                g32[7] = -np.inf
        g = torch.from_numpy(g32).to(TORCH_DT[gk])
        grads.append(bits(g, gk))
        lr_t = lr if lr_schedule is None else lr_schedule(st)
        lrs.append(lr_t)
        cs = 0
        for size in sizes:
            ce = cs + size
            ref.adam_update(0, st, lr_t, betas[0], betas[1], eps, wd, bc, p[cs:ce], g[cs:ce], m[cs:ce],
                            v[cs:ce])
            cs = ce
        ps.append(bits(p, pk))
        ms.append(bits(m, sk))
        vs.append(bits(v, sk))
    out.update(grads=np.stack(grads), p=np.stack(ps), m=np.stack(ms), v=np.stack(vs),
               lrs=np.array(lrs, dtype=np.float64))
    meta = dict(name=name, triple=list(triple), sizes=list(sizes), steps=steps, betas=list(betas),
                eps=eps, wd=wd, adamw=adamw, bc=bc, seed=seed)
    return meta, out


def cases(ref):
    yield make_case(ref, "tail_hot", sizes=(1, 3, 15, 16, 17, 63, 127, 129, 1000, 4099), steps=3)
    yield make_case(ref, "tail_f32", triple=("f32", "f32", "f32"), sizes=(1, 17, 129, 4099), steps=3)
    yield make_case(ref, "l2_mode", sizes=(17, 1000), adamw=False, wd=0.1, steps=3)
    yield make_case(ref, "no_decay", sizes=(33,), wd=0.0, steps=3)
    yield make_case(ref, "no_bias_correction", sizes=(33,), bc=False, steps=3)
    for trip in (("f16", "f16", "f32"), ("f16", "f32", "f32"), ("f16", "f16", "f16"),
                 ("bf16", "bf16", "f32"), ("bf16", "f32", "f32"), ("bf16", "bf16", "bf16"),
                 ("f32", "f16", "f32")):
        yield make_case(ref, "triple_" + "_".join(trip), triple=trip, sizes=(1000, 37), steps=3,
                        m0v0="warm")
    # beta-power state machine: one call per step (multiply path) for many
    # steps; several calls per step (later calls take the pow path); betas of
    # the reference's only test (test_shared_data_parallel.py:26)
    yield make_case(ref, "bc_multiply_path", sizes=(48,), steps=200, m0v0="warm")
    yield make_case(ref, "bc_pow_path", sizes=(16, 16, 19), steps=40, m0v0="warm")
    yield make_case(ref, "bc_betas_08_095", sizes=(48, 5), steps=60, betas=(0.8, 0.95), eps=1e-6,
                    wd=0.1, lr=0.01, lr_schedule=lambda s: 0.01 if s < 3 else 0.003)
    yield make_case(ref, "specials", sizes=(100, 27), steps=3, specials=True)
    # C1 (GPT-2-small block) hyper-parameters on the block's first 4096 elements
    yield make_case(ref, "c1_slice", sizes=(4096,), steps=10, lr=1e-5)


def main():
    ref = O.load_ref("avx512") or O.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref)")
    arrays, metas = {}, []
    for meta, out in cases(ref):
        metas.append(meta)
        for k, a in out.items():
            arrays[f"{meta['name']}/{k}"] = a
    arrays["__meta__"] = np.frombuffer(json.dumps(metas).encode(), dtype=np.uint8)
    path = os.path.join(HERE, "cases.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(metas)} cases, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
