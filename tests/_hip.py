"""GPU-test helpers: drive the HIP kernels through the C-ABI on torch device tensors."""
from __future__ import annotations

import ctypes
import itertools

import numpy as np
import torch

from slideformer_amd import _lib

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
CODE = {"f32": _lib.LA_F32, "bf16": _lib.LA_BF16, "f16": _lib.LA_F16}
_ids = itertools.count(10_000)


def to_dev_bits(bits_arr: np.ndarray, kind: str, device) -> torch.Tensor:
    """numpy raw bits -> device tensor of the element type."""
    if kind == "f32":
        t = torch.from_numpy(bits_arr.view(np.int32).copy()).view(torch.float32)
    else:
        t = torch.from_numpy(bits_arr.view(np.int16).copy()).view(TD[kind])
    return t.to(device)


def to_np_bits(t: torch.Tensor, kind: str) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if kind == "f32":
        return t.view(torch.int32).numpy().view(np.uint32).copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


_small_grid = None


def load_small_grid():
    """The small-grid test build of the library (slideformer_amd.build.SMALL_GRID_LIB),
    loaded beside the product build; raises if it has not been built."""
    global _small_grid
    if _small_grid is None:
        import os

        from slideformer_amd.build import SMALL_GRID_LIB
        if not os.path.exists(SMALL_GRID_LIB):
            raise ImportError(f"{SMALL_GRID_LIB} not built; run `python -m slideformer_amd.build`")
        _small_grid = _lib._declare(ctypes.CDLL(SMALL_GRID_LIB))
    return _small_grid


class HipAdam:
    """One optimizer id of the HIP library, called through the C-ABI."""

    def __init__(self, lr, betas, eps, wd, adamw, *, lib=None):
        self.L = lib if lib is not None else _lib.load()
        self.id = next(_ids)
        _lib.check(self.L.la_create(self.id, lr, betas[0], betas[1], eps, wd, int(adamw), 0), "la_create")

    def __del__(self):
        try:
            self.L.la_destroy(self.id)
        except Exception:
            pass

    def update(self, step, lr, b1, b2, eps, wd, bc, p, g, m, v, *, out=None, coef=None, stream=None):
        kinds = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
        st = stream if stream is not None else torch.cuda.current_stream(p.device)
        rc = self.L.la_adam_update(
            self.id, int(step), lr, b1, b2, eps, wd, int(bool(bc)),
            CODE[kinds[p.dtype]], p.data_ptr(), CODE[kinds[g.dtype]], g.data_ptr(),
            CODE[kinds[m.dtype]], m.data_ptr(), v.data_ptr(), p.numel(),
            None if out is None else out.data_ptr(), None if coef is None else coef.data_ptr(),
            st.cuda_stream)
        _lib.check(rc, "la_adam_update")

    def update_multi(self, step, lr, b1, b2, eps, wd, bc, tensors, *, coef=None, stream=None):
        """One la_adam_update_multi call over [(p, g, m, v, out-or-None), ...]."""
        kinds = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
        p0, g0, m0 = tensors[0][:3]
        segs = (_lib.LaSegment * len(tensors))()
        for k, (p, g, m, v, out) in enumerate(tensors):
            segs[k].p, segs[k].g, segs[k].m, segs[k].v = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr()
            segs[k].p_bf16_out = None if out is None else out.data_ptr()
            segs[k].n = p.numel()
        st = stream if stream is not None else torch.cuda.current_stream(p0.device)
        rc = self.L.la_adam_update_multi(
            self.id, int(step), lr, b1, b2, eps, wd, int(bool(bc)), CODE[kinds[p0.dtype]], CODE[kinds[g0.dtype]],
            CODE[kinds[m0.dtype]], segs, len(tensors), None if coef is None else coef.data_ptr(), st.cuda_stream)
        _lib.check(rc, "la_adam_update_multi")


def sqnorm(g: torch.Tensor, accumulate_into: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Sum of squares of a device grad buffer in float64 (device scalar)."""
    L = _lib.load()
    kinds = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
    ws = torch.zeros(max(1, L.la_grad_sqnorm_workspace(g.numel()) // 8), dtype=torch.float64,
                     device=g.device)
    out = accumulate_into if accumulate_into is not None else torch.zeros(1, dtype=torch.float64,
                                                                         device=g.device)
    st = stream if stream is not None else torch.cuda.current_stream(g.device)
    _lib.check(L.la_grad_sqnorm(CODE[kinds[g.dtype]], g.data_ptr(), g.numel(), ws.data_ptr(),
                                ws.numel() * 8, out.data_ptr(), int(accumulate_into is not None),
                                st.cuda_stream), "la_grad_sqnorm")
    return out


def clip_coef(sq: torch.Tensor, max_norm: float):
    L = _lib.load()
    coef = torch.empty(1, dtype=torch.float32, device=sq.device)
    norm = torch.empty(1, dtype=torch.float32, device=sq.device)
    _lib.check(L.la_clip_coef(sq.data_ptr(), float(max_norm), coef.data_ptr(), norm.data_ptr(),
                              torch.cuda.current_stream(sq.device).cuda_stream), "la_clip_coef")
    return coef, norm


def norm_clip(g: torch.Tensor, max_norm: float, ws: torch.Tensor | None = None):
    """One-launch sum of squares + clip coefficient (la_grad_norm_clip)."""
    L = _lib.load()
    kinds = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
    if ws is None:
        ws = torch.zeros(max(1, L.la_grad_sqnorm_workspace(g.numel()) // 8), dtype=torch.float64,
                         device=g.device)
    sq = torch.zeros(1, dtype=torch.float64, device=g.device)
    coef = torch.empty(1, dtype=torch.float32, device=g.device)
    norm = torch.empty(1, dtype=torch.float32, device=g.device)
    _lib.check(L.la_grad_norm_clip(CODE[kinds[g.dtype]], g.data_ptr(), g.numel(), ws.data_ptr(),
                                   ws.numel() * 8, sq.data_ptr(), 0, float(max_norm), coef.data_ptr(),
                                   norm.data_ptr(), torch.cuda.current_stream(g.device).cuda_stream),
               "la_grad_norm_clip")
    return sq, coef, norm
