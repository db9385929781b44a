"""Shared helpers: load the golden fixtures and replay a case through an updater."""
from __future__ import annotations

import json
import os
from functools import lru_cache

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = os.path.join(HERE, "golden", "cases.npz")

BITS = {"f32": np.uint32, "bf16": np.uint16, "f16": np.uint16}


@lru_cache(maxsize=1)
def load_cases():
    z = np.load(CASES, allow_pickle=False)
    metas = json.loads(bytes(z["__meta__"]).decode())
    out = []
    for meta in metas:
        arrays = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(meta["name"] + "/")}
        out.append((meta, arrays))
    return out


def case_names():
    return [m["name"] for m, _ in load_cases()]


def get_case(name):
    for meta, arrays in load_cases():
        if meta["name"] == name:
            return meta, arrays
    raise KeyError(name)


def as_f32(bits_arr: np.ndarray, kind: str) -> np.ndarray:
    """Decode raw bits to float32 (bf16/f16 widened exactly)."""
    if kind == "f32":
        return bits_arr.view(np.float32)
    if kind == "bf16":
        return (bits_arr.astype(np.uint32) << 16).view(np.float32)
    return bits_arr.view(np.float16).astype(np.float32)


def same_bits(a: np.ndarray, b: np.ndarray, kind: str) -> np.ndarray:
    """Element-wise bit equality, NaN == NaN regardless of payload."""
    eq = a == b
    fa, fb = as_f32(a, kind), as_f32(b, kind)
    return eq | (np.isnan(fa) & np.isnan(fb))


def replay(meta, arrays, update_call):
    """Replay a case.  ``update_call(step, lr, p, g, m, v, lo, hi)`` performs one
    adam_update call on elements [lo, hi) of the flat state; ``p, m, v`` are
    numpy bit arrays owned by the caller of this function, ``g`` the grads of
    the step.  Returns the per-step snapshots (p, m, v) as bit arrays."""
    p = arrays["p0"].copy()
    m = arrays["m0"].copy()
    v = arrays["v0"].copy()
    ps, ms, vs = [], [], []
    for st in range(1, meta["steps"] + 1):
        g = arrays["grads"][st - 1]
        lr = float(arrays["lrs"][st - 1])
        lo = 0
        for size in meta["sizes"]:
            update_call(st, lr, p, g, m, v, lo, lo + size)
            lo += size
        ps.append(p.copy())
        ms.append(m.copy())
        vs.append(v.copy())
    return np.stack(ps), np.stack(ms), np.stack(vs)


def mismatches(meta, arrays, got):
    """Count bit mismatches of (p, m, v) snapshots against the fixture."""
    pk, _, sk = meta["triple"]
    gp, gm, gv = got
    return (int((~same_bits(gp, arrays["p"], pk)).sum()),
            int((~same_bits(gm, arrays["m"], sk)).sum()),
            int((~same_bits(gv, arrays["v"], sk)).sum()))
