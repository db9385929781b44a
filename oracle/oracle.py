"""TEST INFRASTRUCTURE ONLY -- ctypes front end of the CPU checker.

Loads ``oracle/liboracle_adam.so`` (the plain-C restatement of the reference
CPU Adam, see ``layer_adam_oracle.c``) and, where it was built, the reference's
own ``cpu_adam`` compiled from its sources into ``oracle/_ref/``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only to check or time against it.  The product
(``slideformer_amd``) never imports it.
"""
from __future__ import annotations

import ctypes
import importlib
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_adam.so")
REF_DIR = os.path.join(HERE, "_ref")

F32, BF16, F16 = 0, 1, 2

_DT_CODE = {np.dtype(np.float32): F32}


class OrcState(ctypes.Structure):
    """Mirror of ``orc_adam_t`` (the Adam_Optimizer members, cpu_adam.h:91-105)."""

    _fields_ = [
        ("alpha", ctypes.c_float),
        ("betta1", ctypes.c_float),
        ("betta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("betta1_t", ctypes.c_float),
        ("betta2_t", ctypes.c_float),
        ("step", ctypes.c_uint64),
        ("bias_correction1", ctypes.c_float),
        ("bias_correction2", ctypes.c_float),
        ("adamw_mode", ctypes.c_int),
    ]


_lib = None


def build():
    """Compile liboracle_adam.so (and, where /root/reference exists, oracle/_ref)."""
    subprocess.run(["make", "-C", HERE, "-s"], check=True)
    if os.path.isdir("/root/reference/optimizer/layer_adam/csrc"):
        subprocess.run(["make", "-C", HERE, "-s", "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        f, u64, i = ctypes.c_float, ctypes.c_uint64, ctypes.c_int
        S = ctypes.POINTER(OrcState)
        L.orc_create.argtypes = [S, f, f, f, f, f, i]
        L.orc_increment_step.argtypes = [S, u64, f, f]
        L.orc_update_state.argtypes = [S, f, f, f, i]
        L.orc_scalars.argtypes = [S, ctypes.POINTER(ctypes.c_float)]
        L.orc_adam_update.argtypes = [S, u64, f, f, f, f, f, i, i, P, i, P, i, P, P, u64, P, P, i]
        L.orc_adam_update.restype = i
        L.orc_grad_sqnorm.argtypes = [i, P, u64]
        L.orc_grad_sqnorm.restype = ctypes.c_double
        L.orc_clip_coef.argtypes = [ctypes.c_double, f, ctypes.POINTER(ctypes.c_float)]
        L.orc_clip_coef.restype = f
        L.orc_f32_to_bf16.argtypes = [f]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [f]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = f
        L.orc_f32_to_bf16_array.argtypes = [P, P, u64]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def dtype_code(a: np.ndarray, is16: str | None = None) -> int:
    """float32 arrays -> F32; uint16 arrays carry bf16 or f16 bits (``is16``)."""
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:
        return {"bf16": BF16, "f16": F16}[is16 or "bf16"]
    raise TypeError(f"unsupported dtype {a.dtype}")


class OracleAdam:
    """One optimizer id of the restated reference (cpu_adam.h Adam_Optimizer)."""

    def __init__(self, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, adamw_mode=True):
        self.s = OrcState()
        lib().orc_create(ctypes.byref(self.s), lr, betas[0], betas[1], eps, weight_decay,
                         int(adamw_mode))

    def scalars(self) -> np.ndarray:
        out = (ctypes.c_float * 8)()
        lib().orc_scalars(ctypes.byref(self.s), out)
        return np.frombuffer(bytes(out), dtype=np.float32).copy()

    def update(self, step, lr, b1, b2, eps, wd, bias_correction, p, g, m, v, *,
               p16=None, g16=None, s16=None, p_bf16_out=None, clip_coef=None, body_width=16):
        """In-place step on numpy arrays (float32, or uint16 holding bf16/f16 bits)."""
        n = p.size
        assert g.size == n and m.size == n and v.size == n
        coef = None
        if clip_coef is not None:
            coef = np.array([clip_coef], dtype=np.float32)
        rc = lib().orc_adam_update(
            ctypes.byref(self.s), int(step), lr, b1, b2, eps, wd, int(bool(bias_correction)),
            dtype_code(p, p16), _ptr(p), dtype_code(g, g16), _ptr(g), dtype_code(m, s16), _ptr(m),
            _ptr(v), n, None if p_bf16_out is None else _ptr(p_bf16_out),
            None if coef is None else _ptr(coef), int(body_width))
        if rc != 0:
            raise RuntimeError(f"orc_adam_update failed: {rc}")


def grad_sqnorm(g: np.ndarray, g16: str | None = None) -> float:
    return lib().orc_grad_sqnorm(dtype_code(g, g16), _ptr(g), g.size)


def clip_coef(sqnorm: float, max_norm: float):
    norm = ctypes.c_float()
    c = lib().orc_clip_coef(sqnorm, max_norm, ctypes.byref(norm))
    return c, norm.value


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_array(_ptr(x), _ptr(y), x.size)
    return y


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# the reference itself, compiled from /root/reference by oracle/Makefile
# ---------------------------------------------------------------------------

def _cpu_flags() -> set:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("flags"):
                    return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def ref_variant() -> str | None:
    """Which reference build this host can run: the one builder.py:55-98 would pick."""
    flags = _cpu_flags()
    if {"avx512f", "avx512bw", "avx512dq", "avx512vl"} <= flags:
        return "avx512"
    if {"avx2", "fma"} <= flags:
        return "avx2"
    return None


def load_ref(variant: str | None = None):
    """Import the compiled reference ``cpu_adam`` module, or return None if absent."""
    variant = variant or ref_variant()
    if variant is None:
        return None
    name = f"cpu_adam_ref_{variant}"
    if not os.path.exists(os.path.join(REF_DIR, name + ".so")):
        return None
    import torch  # noqa: F401  (the module links libtorch)
    if REF_DIR not in sys.path:
        sys.path.insert(0, REF_DIR)
    return importlib.import_module(name)
