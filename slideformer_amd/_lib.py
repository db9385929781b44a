"""ctypes binding of ``libslideformer_amd.so`` (C-ABI declared in ``include/layer_adam.h``).

The library is loaded after ``import torch`` so that it binds to the HIP runtime
torch already loaded (both carry the soname ``libamdhip64.so.7``); device
pointers and streams from torch are then valid in it.

There is no fallback: if the library is missing, ``load()`` raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
import weakref

import numpy as np
import torch  # noqa: F401  (binds the HIP runtime before the library is loaded)

# where slideformer_amd/build.py writes the library
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libslideformer_amd.so")

# LA_ABI_VERSION of include/layer_adam.h that these bindings declare
ABI_VERSION = 9

LA_OK = 0
LA_EINVAL = -22
LA_EDTYPE = -95
LA_ENOMEM = -12
LA_ERANGE = -34
LA_EFAULT = -14

LA_F32, LA_BF16, LA_F16 = 0, 1, 2

# la_pipeline_step placement bits: a set bit = that array is in host memory
LA_ON_HOST_P, LA_ON_HOST_M, LA_ON_HOST_V, LA_ON_HOST_G, LA_ON_HOST_OUT = 1, 2, 4, 8, 16
LA_ON_HOST_ALL = 31

# la_disk_create_ex flags
LA_DISK_DIRECT = 1
# buffers per la_grad_norm_multi call
LA_NORM_MULTI_MAX = 32

# every exported symbol of include/layer_adam.h
EXPORTED = (
    "la_abi_version",
    "la_strerror",
    "la_create",
    "la_destroy",
    "la_scalars",
    "la_adamw_step",
    "la_adam_update",
    "la_adam_update_multi",
    "la_grad_sqnorm_workspace",
    "la_grad_sqnorm",
    "la_grad_norm_clip",
    "la_grad_norm_multi",
    "la_grad_norm_clip_noalloc",
    "la_clip_coef",
    "la_pipeline_workspace_bytes",
    "la_pipeline_create",
    "la_pipeline_destroy",
    "la_pipeline_sync",
    "la_pipeline_set_host_staging",
    "la_pipeline_step",
    "la_disk_create",
    "la_disk_create_ex",
    "la_disk_destroy",
    "la_disk_write_async",
    "la_disk_read_async",
    "la_disk_sync_writes",
    "la_disk_sync_reads",
)


class LaPipelineStats(ctypes.Structure):
    """Mirror of ``la_pipeline_stats_t``."""

    _fields_ = [
        ("wall_ms", ctypes.c_float),
        ("h2d_ms", ctypes.c_float),
        ("compute_ms", ctypes.c_float),
        ("d2h_ms", ctypes.c_float),
        ("h2d_bytes", ctypes.c_uint64),
        ("d2h_bytes", ctypes.c_uint64),
        ("chunks", ctypes.c_uint32),
        ("host_copy_ms", ctypes.c_float),
        ("staged_bytes", ctypes.c_uint64),
    ]


class LaSegment(ctypes.Structure):
    """Mirror of ``la_segment_t``."""

    _fields_ = [
        ("p", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("p_bf16_out", ctypes.c_void_p),
        ("n", ctypes.c_uint64),
    ]


class LaGradBuffer(ctypes.Structure):
    """Mirror of ``la_grad_buffer_t``."""

    _fields_ = [
        ("g", ctypes.c_void_p),
        ("n", ctypes.c_uint64),
    ]


class LaScalars(ctypes.Structure):
    """Mirror of ``la_scalars_t``."""

    _fields_ = [
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("one_minus_beta1", ctypes.c_float),
        ("one_minus_beta2", ctypes.c_float),
        ("bias_correction2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("step_size", ctypes.c_float),
        ("w_decay", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("decay_mode", ctypes.c_int32),
        ("beta1_t", ctypes.c_float),
        ("beta2_t", ctypes.c_float),
        ("bias_correction1", ctypes.c_float),
        ("step", ctypes.c_uint64),
    ]


_lock = threading.Lock()
_lib = None


def _declare(L):
    P = ctypes.c_void_p
    f, i, u64 = ctypes.c_float, ctypes.c_int, ctypes.c_uint64
    SP = ctypes.POINTER(LaScalars)
    L.la_abi_version.argtypes = []
    L.la_abi_version.restype = i
    L.la_strerror.argtypes = [i]
    L.la_strerror.restype = ctypes.c_char_p
    L.la_create.argtypes = [i, f, f, f, f, f, i, i]
    L.la_create.restype = i
    L.la_destroy.argtypes = [i]
    L.la_destroy.restype = i
    L.la_scalars.argtypes = [i, u64, f, f, f, f, f, i, SP]
    L.la_scalars.restype = i
    L.la_adamw_step.argtypes = [SP, i, P, i, P, i, P, P, u64, P, P, P]
    L.la_adamw_step.restype = i
    L.la_adam_update.argtypes = [i, u64, f, f, f, f, f, i, i, P, i, P, i, P, P, u64, P, P, P]
    L.la_adam_update.restype = i
    L.la_adam_update_multi.argtypes = [i, u64, f, f, f, f, f, i, i, i, i, ctypes.POINTER(LaSegment), i, P, P]
    L.la_adam_update_multi.restype = i
    L.la_grad_sqnorm_workspace.argtypes = [u64]
    L.la_grad_sqnorm_workspace.restype = u64
    L.la_grad_sqnorm.argtypes = [i, P, u64, P, u64, P, i, P]
    L.la_grad_sqnorm.restype = i
    L.la_grad_norm_clip.argtypes = [i, P, u64, P, u64, P, i, f, P, P, P]
    L.la_grad_norm_clip.restype = i
    L.la_grad_norm_multi.argtypes = [i, ctypes.POINTER(LaGradBuffer), i, P, u64, P, i, f, P, P, P]
    L.la_grad_norm_multi.restype = i
    L.la_grad_norm_clip_noalloc.argtypes = [i, P, u64, P, i, f, P, P, P]
    L.la_grad_norm_clip_noalloc.restype = i
    L.la_clip_coef.argtypes = [P, f, P, P, P]
    L.la_clip_coef.restype = i
    L.la_pipeline_workspace_bytes.argtypes = [u64, i, i, i, i, ctypes.c_uint]
    L.la_pipeline_workspace_bytes.restype = u64
    L.la_pipeline_create.argtypes = [u64, i, ctypes.POINTER(P)]
    L.la_pipeline_create.restype = i
    L.la_pipeline_destroy.argtypes = [P]
    L.la_pipeline_destroy.restype = i
    L.la_pipeline_sync.argtypes = [P]
    L.la_pipeline_sync.restype = i
    L.la_pipeline_set_host_staging.argtypes = [P, P, u64, i]
    L.la_pipeline_set_host_staging.restype = i
    L.la_pipeline_step.argtypes = [P, SP, i, P, i, P, i, P, P, u64, P, ctypes.c_uint, P, P, u64, P, i,
                                   ctypes.POINTER(LaPipelineStats)]
    L.la_pipeline_step.restype = i
    L.la_disk_create.argtypes = [ctypes.c_char_p, i, ctypes.POINTER(P)]
    L.la_disk_create.restype = i
    L.la_disk_create_ex.argtypes = [ctypes.c_char_p, i, ctypes.c_uint, ctypes.POINTER(P)]
    L.la_disk_create_ex.restype = i
    L.la_disk_destroy.argtypes = [P]
    L.la_disk_destroy.restype = i
    L.la_disk_write_async.argtypes = [P, u64, P, u64]
    L.la_disk_write_async.restype = i
    L.la_disk_read_async.argtypes = [P, u64, P, u64]
    L.la_disk_read_async.restype = i
    L.la_disk_sync_writes.argtypes = [P]
    L.la_disk_sync_writes.restype = i
    L.la_disk_sync_reads.argtypes = [P]
    L.la_disk_sync_reads.restype = i
    return L


def load(path: str | None = None):
    """Load the HIP library (once).  Raises ImportError if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = path or os.environ.get("SLIDEFORMER_AMD_LIB", LIB_PATH)
        if not os.path.exists(path):
            raise ImportError(
                f"slideformer_amd HIP library not found at {path}; build it with "
                "`python -m slideformer_amd.build` (there is no CPU fallback)")
        raw = ctypes.CDLL(path)
        raw.la_abi_version.restype = ctypes.c_int
        found = raw.la_abi_version()
        if found != ABI_VERSION:
            raise ImportError(
                f"{path} implements the C-ABI version {found}, this package needs {ABI_VERSION}; rebuild it "
                "with `python -m slideformer_amd.build`")
        _lib = _declare(raw)
        return _lib


def check(rc: int, what: str) -> None:
    if rc != LA_OK:
        msg = load().la_strerror(rc).decode()
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


_hip_runtime = None


def _hip():
    """The HIP runtime torch has loaded (the same soname resolves to it)."""
    global _hip_runtime
    with _lock:
        if _hip_runtime is None:
            rt = ctypes.CDLL("libamdhip64.so")
            rt.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
            rt.hipHostMalloc.restype = ctypes.c_int
            rt.hipHostFree.argtypes = [ctypes.c_void_p]
            rt.hipHostFree.restype = ctypes.c_int
            _hip_runtime = rt
        return _hip_runtime


# start address -> bytes of every live page_locked_empty allocation
_page_locked = {}


def _release(rt, address: int) -> None:
    with _lock:
        _page_locked.pop(address, None)
    rt.hipHostFree(address)


def is_page_locked(t: torch.Tensor) -> bool:
    """Whether a host tensor lies in page-locked memory: torch's own pinned
    blocks (``is_pinned``) or a ``page_locked_empty`` allocation, which torch
    does not recognise as pinned."""
    if t.is_cuda:
        return False
    if t.is_pinned():
        return True
    ptr = t.data_ptr()
    with _lock:
        return any(start <= ptr < start + size for start, size in _page_locked.items())


def page_locked_empty(numel: int, dtype: torch.dtype) -> torch.Tensor:
    """A host tensor of exactly ``numel`` elements in page-locked memory
    (one ``hipHostMalloc``), uninitialised.

    torch's pinned allocator (``pin_memory=True``) rounds every allocation up to
    a power of two: an 872 MB moment of a Llama-3.1-8B layer takes 1 GiB, a
    2.1 GB vocab matrix 4 GiB.  A process may page-lock only so much host
    memory (64 GiB on the MI355X hosts measured), so exact sizes fit more
    state.  The memory is released with ``hipHostFree`` once the last tensor
    that views it is gone.  torch's ``is_pinned()`` reports False for it;
    ``is_page_locked()`` knows it."""
    elem = torch.empty(0, dtype=dtype).element_size()
    nbytes = numel * elem
    rt = _hip()
    ptr = ctypes.c_void_p()
    rc = rt.hipHostMalloc(ctypes.byref(ptr), max(1, nbytes), 0)
    if rc != 0 or not ptr.value:
        raise RuntimeError(f"hipHostMalloc of {nbytes} bytes failed (hipError_t {rc})")
    raw = np.frombuffer((ctypes.c_uint8 * max(1, nbytes)).from_address(ptr.value), dtype=np.uint8)
    with _lock:
        _page_locked[ptr.value] = max(1, nbytes)
    # Not at interpreter exit: finalizers then run in no fixed order, possibly
    # before a pipeline that still copies into this memory has been drained;
    # the process's own teardown reclaims it.
    weakref.finalize(raw, _release, rt, ptr.value).atexit = False
    return torch.from_numpy(raw)[:nbytes].view(dtype)

