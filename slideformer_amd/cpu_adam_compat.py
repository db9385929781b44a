"""Stand-in for the reference's native module ``cpu_adam`` on the MI355X.

The reference builds a pybind module with three functions
(``optimizer/layer_adam/csrc/cpu_adam.cpp:8-13``, declared at
``cpu_adam.h:199-221``) and loads it with ``CPUAdamLoader().load()``
(``layer_adam.py:59``).  This module has the same three functions, with the
same names, argument order, defaults and return value (0), so a maintainer who
keeps the reference's ``LayerAdam`` unchanged can return this module from the
loader instead::

    # optimizer/layer_adam/builder.py, CPUAdamLoader.load()
    from slideformer_amd import cpu_adam_compat
    return cpu_adam_compat

``adam_update`` routes by where the four tensors live:

* all four in host memory (what the reference's ``step`` / ``step_chunk``
  pass, ``layer_adam.py:314-327,448-461``): streamed through HBM by the native
  chunk pipeline (``la_pipeline_step``) on the current HIP device; the call
  returns after completion, as the reference's CPU call does;
* all four on one HIP device: one ``la_adam_update`` launch, asynchronous on
  that device's current stream;
* anything else (host and device mixed, two devices, another device type):
  ``RuntimeError`` before any library call, so no host address ever reaches a
  device kernel.

Errors follow ``ds_adam_step`` (``cpu_adam_impl.cpp:220-270``): the
contiguity checks raise ``RuntimeError`` with the reference's messages before
the state changes; an unregistered dtype triple advances the beta-power state
and then raises the reference's "is not supported on current hardware"
message.  Two checks the reference lacks: an unknown id raises instead of
dereferencing a null optimizer, and tensors of unequal size raise instead of
reading out of bounds.
"""
from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

__all__ = ["create_adam", "adam_update", "destroy_adam"]

_DTYPE_CODE = {torch.float32: _lib.LA_F32, torch.bfloat16: _lib.LA_BF16, torch.float16: _lib.LA_F16}

# one host-state pipeline per HIP device, shared by every optimizer id; a
# pipeline object must not be used by two threads at once
_streamers = {}
_streamers_lock = threading.Lock()


def _library():
    """The HIP library (raises ImportError when it is not built)."""
    return _lib.load()


def create_adam(optimizer_id, alpha=1e-3, betta1=0.9, betta2=0.999, eps=1e-8, weight_decay=0,
                adamw_mode=True, should_log=False):
    """``create_adam_optimizer`` (cpu_adam_impl.cpp:91-129): (re)set the scalar state of an id."""
    L = _library()
    _lib.check(L.la_create(int(optimizer_id), float(alpha), float(betta1), float(betta2), float(eps),
                           float(weight_decay), int(bool(adamw_mode)), int(bool(should_log))), "create_adam")
    return 0


def destroy_adam(optimizer_id):
    """``destroy_adam_optimizer`` (cpu_adam_impl.cpp:272-277)."""
    _lib.check(_library().la_destroy(int(optimizer_id)), "destroy_adam")
    return 0


def _where(tensors):
    """'host', a HIP device, or a RuntimeError for any other combination."""
    devices = {t.device for t in tensors}
    for d in devices:
        if d.type not in ("cpu", "cuda"):
            raise RuntimeError(f"adam_update: unsupported device type {d.type}")
    if devices == {torch.device("cpu")}:
        return "host"
    if len(devices) == 1:
        return devices.pop()
    raise RuntimeError(
        "adam_update: params, grads, exp_avg and exp_avg_sq must all be in host memory or all on one "
        f"HIP device, got {sorted(str(d) for d in devices)}")


def adam_update(optimizer_id, step, lr, beta1, beta2, epsilon, weight_decay, bias_correction,
                params, grads, exp_avg, exp_avg_sq):
    """``ds_adam_step`` (cpu_adam_impl.cpp:220-270) on the MI355X; returns 0."""
    tensors = (params, grads, exp_avg, exp_avg_sq)
    for t in tensors:
        if not isinstance(t, torch.Tensor):
            raise TypeError("adam_update: params, grads, exp_avg and exp_avg_sq must be tensors")
    # cpu_adam_impl.cpp:234-237
    if not params.is_contiguous():
        raise RuntimeError("params must be contiguous")
    if not grads.is_contiguous():
        raise RuntimeError("grads must be contiguous")
    if not exp_avg.is_contiguous():
        raise RuntimeError("exp_avg must be contiguous")
    if not exp_avg_sq.is_contiguous():
        raise RuntimeError("exp_avg_sq must be contiguous")
    where = _where(tensors)
    n = params.numel()
    if grads.numel() != n or exp_avg.numel() != n or exp_avg_sq.numel() != n:
        raise RuntimeError(f"adam_update: size mismatch: params {n}, grads {grads.numel()}, "
                           f"exp_avg {exp_avg.numel()}, exp_avg_sq {exp_avg_sq.numel()}")
    if exp_avg_sq.dtype != exp_avg.dtype:
        raise RuntimeError("adam_update: exp_avg and exp_avg_sq must have the same dtype")
    if where == "host" and not torch.cuda.is_available():
        raise RuntimeError("adam_update needs a HIP device (MI355X); there is no CPU arithmetic path")

    L = _library()
    # IncrementStep + update_state come before the dtype lookup (cpu_adam_impl.cpp:241-261)
    sc = _lib.LaScalars()
    _lib.check(L.la_scalars(int(optimizer_id), int(step), float(lr), float(beta1), float(beta2),
                            float(epsilon), float(weight_decay), int(bool(bias_correction)), ctypes.byref(sc)),
               "adam_update")
    codes = [_DTYPE_CODE.get(t.dtype) for t in (params, grads, exp_avg)]
    from .layer_adam import SUPPORTED_TRIPLES, _unsupported
    if (params.dtype, grads.dtype, exp_avg.dtype) not in SUPPORTED_TRIPLES:
        raise _unsupported(params.dtype, grads.dtype, exp_avg.dtype)
    if n == 0:
        return 0
    if where == "host":
        _host_step(L, sc, codes, tensors, n)
    else:
        with torch.cuda.device(where):
            stream = torch.cuda.current_stream(where).cuda_stream
            _lib.check(L.la_adamw_step(ctypes.byref(sc), codes[0], params.data_ptr(), codes[1], grads.data_ptr(),
                                       codes[2], exp_avg.data_ptr(), exp_avg_sq.data_ptr(), n, None, None, stream),
                       "adam_update")
    return 0


def _host_step(L, sc, codes, tensors, n):
    """Host-resident p, g, m, v: streamed through HBM on the current HIP device
    (every placement bit set), complete on return."""
    from .layer_adam import HostStreamer
    device = torch.device("cuda", torch.cuda.current_device())
    params, grads, exp_avg, exp_avg_sq = tensors
    with _streamers_lock:
        streamer = _streamers.get(device)
        if streamer is None:
            streamer = _streamers[device] = HostStreamer(device)
        with torch.cuda.device(device):
            streamer.step(sc, codes[0], params, codes[1], grads, codes[2], exp_avg, exp_avg_sq, n, None,
                          _lib.LA_ON_HOST_P | _lib.LA_ON_HOST_G | _lib.LA_ON_HOST_M | _lib.LA_ON_HOST_V,
                          None, torch.cuda.current_stream(device).cuda_stream, synchronize=True)
