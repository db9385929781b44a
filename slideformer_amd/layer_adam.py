"""``LayerAdam`` for MI355X: the reference's layer-wise Adam API over a HIP kernel.

Drop-in for ``optimizer/layer_adam/layer_adam.py`` (class ``LayerAdam``,
layer_adam.py:12-484): same constructor hyper-parameters, the same
``param_groups`` / ``state`` / ``exp_avg_flat`` / ``exp_avg_sq_flat`` layout and
the same methods (``add_layer_params``, ``step``, ``step_with_grad_views``,
``begin_chunk_step`` / ``step_chunk`` / ``end_chunk_step``,
``update_learning_rate``).  The element update runs in the gfx950 kernel of
``libslideformer_amd.so`` (C-ABI ``include/layer_adam.h``); the
beta-power state machine of the reference runs on the host inside that library.

Device tensors are updated in place, asynchronously on the current HIP stream.
Host tensors (the reference's layout: fp32 master and moments in CPU RAM) are
streamed through HBM in 16 Mi-element chunks by the library's native
three-stream pipeline (H2D / update / D2H overlapped) and the call returns
after completion, as the reference's CPU call does.  Each array of a call may
be on the host or on the one device; only the host-resident ones cross the
host link (``LayerAdam(moments_device=...)`` keeps the moments in HBM beside a
host-resident master).  Pageable host arrays are copied through page-locked
staging by native host threads.  There is no CPU arithmetic path.

Additions, all keyword-only so that positional signatures are unchanged:
``bf16_out=`` (the bf16 compute copy written in the same pass), ``clip_coef=``
(a device fp32 scalar that scales the grads), ``stream=``; and
``clip_grad_norm(grads, max_norm)`` which produces that coefficient on device.
"""
from __future__ import annotations

import contextlib
import ctypes
import glob
import itertools
import math
import os
import threading
from collections import OrderedDict, defaultdict
from typing import Any, DefaultDict, Dict, Iterable, Optional, Sequence

import torch

from . import _lib, cpu_adam_compat

_DTYPE_CODE = {torch.float32: _lib.LA_F32, torch.bfloat16: _lib.LA_BF16, torch.float16: _lib.LA_F16}
_DTYPE_NAME = {torch.float32: "Float", torch.bfloat16: "BFloat16", torch.float16: "Half"}

# the (param, grad, state) triples the reference registers, cpu_adam_impl.cpp:181-189
SUPPORTED_TRIPLES = frozenset({
    (torch.float16, torch.float16, torch.float32),
    (torch.float16, torch.float32, torch.float32),
    (torch.float16, torch.float16, torch.float16),
    (torch.bfloat16, torch.bfloat16, torch.float32),
    (torch.bfloat16, torch.float32, torch.float32),
    (torch.bfloat16, torch.bfloat16, torch.bfloat16),
    (torch.float32, torch.float32, torch.float32),
    (torch.float32, torch.bfloat16, torch.float32),
    (torch.float32, torch.float16, torch.float32),
})

# Host tensors are streamed through HBM in chunks of this many elements (64 MB
# of fp32 per state array), through HOST_STAGE_SLOTS staging slots.  A multiple
# of 16, so that only the last chunk of a call holds the reference's scalar
# tail (the last n % 16 elements of the call).  Measured on MI355X over one
# Llama-3.1-8B layer: with page-locked state, 4-16 Mi-element chunks with 3-4
# slots all run at 46-47.5 GB/s each way (the concurrent-duplex limit of the
# host link); with pageable state staged by host threads, 16 Mi x 3 runs at
# 59-60 ms per layer every time, while with four slots a D2H hipMemcpyAsync
# into a page-locked twin now and then blocks the calling thread for 6-7 ms
# and the pipeline drains (8 Mi x 4 and 16 Mi x 4: 80-90 ms).
HOST_STAGE_ELEMS = 16 * 1024 * 1024
HOST_STAGE_SLOTS = 3


class HostStreamer:
    """One native chunk pipeline (``la_pipeline_t``) on one device, plus the
    device staging memory it needs (allocated here, never by the library).

    Pageable host arrays (the reference's moments are plain ``torch.zeros``,
    layer_adam.py:161-173) go through page-locked twins of the staging slots,
    copied by ``host_threads`` native threads (0 = up to 16); the copy engines
    then only see page-locked memory.  ``stage_pageable=False`` leaves pageable
    arrays to the HIP runtime's own bounce buffers instead."""

    def __init__(self, device, chunk_elems: int = HOST_STAGE_ELEMS, slots: int = HOST_STAGE_SLOTS, *,
                 host_threads: int = 0, stage_pageable: bool = True):
        self.lib = _lib.load()
        self.device = torch.device(device)
        self.chunk = chunk_elems
        self.slots = slots
        self.host_threads = host_threads
        self.stage_pageable = stage_pageable
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self.lib.la_pipeline_create(chunk_elems, slots, ctypes.byref(handle)),
                       "la_pipeline_create")
        self.handle = handle
        self._ws = {}
        self._host_ws = {}
        # every tensor of a call that returned once queued, until the pipeline
        # has completed it: the pipeline's own streams still read and write
        # them, and a temporary the caller drops (a grad moved to the device,
        # a clip coefficient of this step) must not go back to the caching
        # allocator, which could hand its memory out on the caller's stream
        self._in_flight = []

    def _bytes(self, key) -> int:
        return self.lib.la_pipeline_workspace_bytes(self.chunk, self.slots, *[int(k) for k in key])

    def workspace(self, pc, gc, sc, on_host) -> torch.Tensor:
        """Device staging for one element-type triple and placement (la_pipeline_workspace_bytes)."""
        key = (pc, gc, sc, on_host)
        ws = self._ws.get(key)
        if ws is None:
            ws = torch.empty(self._bytes(key) + 256, dtype=torch.uint8, device=self.device)
            self._ws[key] = ws
        return ws

    def _attach_host_staging(self, key, needed: bool):
        if not needed:
            _lib.check(self.lib.la_pipeline_set_host_staging(self.handle, None, 0, 0),
                       "la_pipeline_set_host_staging")
            return
        buf = self._host_ws.get(key)
        if buf is None:
            buf = torch.empty(self._bytes(key) + 256, dtype=torch.uint8, pin_memory=True)
            self._host_ws[key] = buf
        base = buf.data_ptr()
        aligned = (base + 255) // 256 * 256
        _lib.check(self.lib.la_pipeline_set_host_staging(self.handle, aligned, buf.numel() - (aligned - base),
                                                         self.host_threads),
                   "la_pipeline_set_host_staging")

    def step(self, scalars, pc, params, gc, grads, sc, exp_avg, exp_avg_sq, n, bf16_out, on_host,
             clip_coef, stream_handle, synchronize: bool = True):
        """One la_pipeline_step; ``on_host`` is its placement mask (``_placement``).
        With synchronize=False it returns once the work is queued (statistics
        then None); ``sync()`` completes it."""
        key = (pc, gc, sc, on_host)
        ws = self.workspace(*key)
        host = [t for t in (params, grads, exp_avg, exp_avg_sq, bf16_out) if t is not None and not t.is_cuda]
        self._attach_host_staging(key, self.stage_pageable and not all(_lib.is_page_locked(t) for t in host))
        base = ws.data_ptr()
        aligned = (base + 255) // 256 * 256
        stats = _lib.LaPipelineStats() if synchronize else None
        if not synchronize:
            self._in_flight.append((params, grads, exp_avg, exp_avg_sq, bf16_out, clip_coef))
        rc = self.lib.la_pipeline_step(
            self.handle, ctypes.byref(scalars), pc, params.data_ptr(), gc, grads.data_ptr(), sc,
            exp_avg.data_ptr(), exp_avg_sq.data_ptr(), n, None if bf16_out is None else bf16_out.data_ptr(),
            on_host, None if clip_coef is None else clip_coef.data_ptr(), aligned,
            ws.numel() - (aligned - base), stream_handle, int(synchronize),
            None if stats is None else ctypes.byref(stats))
        _lib.check(rc, "la_pipeline_step")
        if synchronize:
            # a synchronizing call completes every earlier call as well
            self._in_flight.clear()
        return stats

    def sync(self):
        """Wait until every queued step is complete in host memory."""
        _lib.check(self.lib.la_pipeline_sync(self.handle), "la_pipeline_sync")
        self._in_flight.clear()

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self.lib.la_pipeline_destroy(self.handle)
        except Exception:
            pass


# LayerAdam ids start far above 0: the reference's own LayerAdam, run on the
# cpu_adam stand-in of this package (cpu_adam_compat), always uses id 0
# (layer_adam.py:62), and the two must not reset each other's state
_ids = itertools.count(1 << 20)
_ids_lock = threading.Lock()


def _next_id() -> int:
    with _ids_lock:
        return next(_ids)


# torch's own accessor of the current stream's raw handle: 0.1 us against
# ~2 us for torch.cuda.current_stream(device).cuda_stream (measured on the
# MI355X host); the public call is the fallback
_raw_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(stream, device) -> int:
    if stream is None:
        if _raw_current_stream is not None:
            index = device.index if device.index is not None else torch.cuda.current_device()
            return _raw_current_stream(index)
        stream = torch.cuda.current_stream(device)
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _on_device(device):
    """``torch.cuda.device(device)``, or nothing to do when it is already current
    (the context manager costs ~1.3 us per call)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _placement(params, grads, exp_avg, exp_avg_sq, bf16_out) -> int:
    """la_pipeline_step's ``on_host`` mask: one bit per array in host memory."""
    mask = 0
    for t, bit in ((params, _lib.LA_ON_HOST_P), (exp_avg, _lib.LA_ON_HOST_M), (exp_avg_sq, _lib.LA_ON_HOST_V),
                   (grads, _lib.LA_ON_HOST_G), (bf16_out, _lib.LA_ON_HOST_OUT)):
        if t is not None and not t.is_cuda:
            mask |= bit
    return mask


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _unsupported(p, g, s) -> RuntimeError:
    # message format of cpu_adam_impl.cpp:256-260
    return RuntimeError(
        f"Adam optimizer with param type {_DTYPE_NAME.get(p, p)}, grads type {_DTYPE_NAME.get(g, g)} "
        f"and state type {_DTYPE_NAME.get(s, s)} is not supported on current hardware")


def _segments(entries):
    """The la_segment_t array of one la_adam_update_multi call over the
    (params, grads, exp_avg, exp_avg_sq) entries, or None when they cannot go
    in one: one HIP device, one registered dtype triple, contiguous, matching
    sizes, and no two tensors written by the update overlapping.  One pass;
    the array is built as six uint64 per segment (the layout of la_segment_t:
    p, g, m, v, p_bf16_out, n)."""
    p0, g0, m0, _ = entries[0]
    if not p0.is_cuda:
        return None
    pdt, gdt, sdt = p0.dtype, g0.dtype, m0.dtype
    if (pdt, gdt, sdt) not in SUPPORTED_TRIPLES:
        return None
    dev = p0.get_device()
    pe, se = p0.element_size(), m0.element_size()
    flat, spans = [], []
    for p, g, m, v in entries:
        n = p.numel()
        if (g.numel() != n or m.numel() != n or v.numel() != n
                or p.dtype != pdt or g.dtype != gdt or m.dtype != sdt or v.dtype != sdt
                or not (p.is_contiguous() and g.is_contiguous() and m.is_contiguous() and v.is_contiguous())
                or p.get_device() != dev or g.get_device() != dev or m.get_device() != dev
                or v.get_device() != dev):
            return None
        pp, mp, vp = p.data_ptr(), m.data_ptr(), v.data_ptr()
        flat += (pp, g.data_ptr(), mp, vp, 0, n)
        if n:
            spans += ((pp, pp + n * pe), (mp, mp + n * se), (vp, vp + n * se))
    spans.sort()
    for a, b in zip(spans, spans[1:]):
        if a[1] > b[0]:
            return None
    return ctypes.cast((ctypes.c_uint64 * len(flat))(*flat), ctypes.POINTER(_lib.LaSegment))


def _torch_stream(stream, device):
    """The stream a call runs on, as a torch stream object (None = current stream;
    a raw hipStream_t handle is wrapped), so that scratch tensors can be
    allocated on it and the caching allocator orders their reuse after it."""
    if stream is None:
        return torch.cuda.current_stream(device)
    if isinstance(stream, torch.cuda.Stream):
        return stream
    return torch.cuda.ExternalStream(int(stream), device=device)


_norm_elems = None


def _norm_workspace_elems(lib) -> int:
    """float64 partials for any buffer size: stage 1 never uses more workgroups than this."""
    global _norm_elems
    if _norm_elems is None:
        _norm_elems = max(1, lib.la_grad_sqnorm_workspace(1 << 62) // 8)
    return _norm_elems


def _norm_runs(lib, grads, work, nwork, sqnorm, accumulate, max_norm, cn, handle):
    """The sum of squares of ``grads`` into the float64 at ``sqnorm`` (added to
    it when ``accumulate``): runs of one dtype, at most LA_NORM_MULTI_MAX
    buffers each, one library call (two launches) per run, later runs adding
    to the earlier ones: la_grad_norm_multi for a run of several buffers,
    la_grad_sqnorm / la_grad_norm_clip for a run of one.  With ``cn`` (address
    of two fp32: coef, norm) the last call also writes the clip coefficient."""
    runs = []
    for g in grads:
        if runs and runs[-1][0].dtype == g.dtype and len(runs[-1]) < _lib.LA_NORM_MULTI_MAX:
            runs[-1].append(g)
        else:
            runs.append([g])
    for i, run in enumerate(runs):
        last = cn is not None and i == len(runs) - 1
        acc = int(accumulate or i > 0)
        code = _DTYPE_CODE[run[0].dtype]
        if len(run) == 1:
            # one buffer: the single-buffer entry points (the same bits, a smaller launch)
            g = run[0]
            if last:
                rc = lib.la_grad_norm_clip(code, g.data_ptr(), g.numel(), work, nwork * 8, sqnorm, acc, max_norm, cn,
                                           cn + 4, handle)
            else:
                rc = lib.la_grad_sqnorm(code, g.data_ptr(), g.numel(), work, nwork * 8, sqnorm, acc, handle)
            _lib.check(rc, "la_grad_sqnorm")
            continue
        flat = []
        for g in run:
            flat += (g.data_ptr(), g.numel())
        bufs = ctypes.cast((ctypes.c_uint64 * len(flat))(*flat), ctypes.POINTER(_lib.LaGradBuffer))
        rc = lib.la_grad_norm_multi(code, bufs, len(run), work, nwork * 8, sqnorm, acc, max_norm,
                                    cn if last else None, cn + 4 if last else None, handle)
        _lib.check(rc, "la_grad_norm_multi")


def _check_grads(grads, device):
    for g in grads:
        if g.device != device:
            raise RuntimeError(f"grad on {g.device}, expected {device}: all grads must be on one device")
        if not g.is_contiguous():
            raise RuntimeError("grads must be contiguous")
        if g.dtype not in _DTYPE_CODE:
            raise RuntimeError(f"unsupported grad dtype {g.dtype}")


class LayerAdam:
    """Layer-wise Adam/AdamW whose element update runs on the MI355X.

    Mirrors ``LayerAdam`` of the reference (layer_adam.py:12-106): one optimizer
    instance for all layers; each layer can be stepped on its own.
    """

    def __init__(
            self,
            lr=1e-3,
            bias_correction=True,
            betas=(0.9, 0.999),
            eps=1e-8,
            weight_decay=0,
            adamw_mode=True,
            fp32_optimizer_state=True,
            num_layer: int = 0,
            nvme_offload_fraction: float = 0.0,
            offload_dir: str = '/NVME1',
            prefetch: bool = True,
            *,
            device: Optional[torch.device] = None,
            pin_host_state: bool = False,
            overlap_host_chunks: bool = False,
            moments_device: Optional[torch.device] = None,
            moments_hbm_bytes: Optional[int] = None,
            stream_chunk_elems: int = HOST_STAGE_ELEMS,
            stream_slots: int = HOST_STAGE_SLOTS,
    ):
        """Arguments of the reference (layer_adam.py:17-30), plus keyword-only:
        ``device``: the HIP device that updates host-resident state (default: current);
        ``moments_device``: a HIP device on which ``add_layer_params`` allocates
        ``exp_avg`` / ``exp_avg_sq`` (default: beside the params, as the
        reference does).  With a host-resident master (the runtime's layout) the
        moments then stay in HBM and each step moves 6 B/param to the device
        and 4 B/param back instead of 14 and 12;
        ``moments_hbm_bytes``: with ``moments_device``, the most HBM the moments
        may take (None = no limit); layers registered once it is used up keep
        their moments beside their params, so a model whose moments do not all
        fit in HBM keeps as many layers' moments there as the budget allows;
        ``pin_host_state``: allocate host-resident moments in page-locked memory,
        at their exact size (streamed without staging copies; the reference
        allocates pageable memory, which the pipeline stages through page-locked
        buffers);
        ``overlap_host_chunks``: host-tensor updates return once queued, so that
        the runtime's one ``step_chunk`` per chunk keeps the host link busy across
        calls; ``end_chunk_step``, the end of ``step``/``step_with_grad_views`` and
        ``synchronize()`` complete them.  Between those points the tensors
        passed in, host and device alike (grads, moments in HBM, ``bf16_out``,
        ``clip_coef``), must not be read or written by the caller; the optimizer
        keeps a reference to each of them until its update is complete, so a
        temporary the caller drops is not freed early;
        ``stream_chunk_elems``, ``stream_slots``: the chunk (elements, rounded
        down to a multiple of 16) and the number of device staging slots with
        which host-resident arrays stream through HBM.  The defaults, 16 Mi
        elements (64 MB of fp32) and 3 slots, are the best or near it for
        every measured layout but one: a page-locked master with the moments in
        HBM in one call of a very large layer (1.8 B params), where 64 Mi x 3
        runs 150 ms against 180-207 ms (64 MB copies back to the host then go
        partly to a DMA engine that the other direction also uses)."""
        self.defaults = dict(
            lr=lr,
            bias_correction=bias_correction,
            betas=betas,
            eps=eps,
            weight_decay=weight_decay,
            adamw_mode=adamw_mode,
        )
        self.param_groups = []
        if moments_device is not None and torch.device(moments_device).type != 'cuda':
            raise ValueError(f"moments_device must be a HIP device, got {moments_device}")
        if moments_device is not None and nvme_offload_fraction > 0.0:
            raise ValueError("moments_device and nvme_offload_fraction > 0 exclude each other: "
                             "the file offload moves host-resident moments")
        if moments_hbm_bytes is not None and (moments_device is None or moments_hbm_bytes < 0):
            raise ValueError("moments_hbm_bytes needs moments_device and must be >= 0")
        if int(stream_chunk_elems) < 16 or not 1 <= int(stream_slots) <= 16:
            raise ValueError("stream_chunk_elems must be at least 16 and stream_slots 1..16")

        # The reference loads its CPU extension here (layer_adam.py:59); this
        # loads the HIP library and fails loudly if it is missing.  cpu_adam is
        # the module with the reference extension's three functions.
        self.lib = _lib.load()
        self.cpu_adam = cpu_adam_compat
        # The reference always uses id 0 (layer_adam.py:62), so a second
        # instance would reset the first one's beta-power state; each instance
        # here gets its own id, and a single instance behaves identically.
        self.optimizer_id = _next_id()
        # creation logged, as layer_adam.py:63-72 asks for
        self.cpu_adam.create_adam(self.optimizer_id, lr, betas[0], betas[1], eps, weight_decay,
                                  adamw_mode, True)

        self.fp32_optimizer_state = fp32_optimizer_state
        self.num_layer = num_layer
        self.device = torch.device(device) if device is not None else None
        self.pin_host_state = pin_host_state
        self.overlap_host_chunks = overlap_host_chunks
        self.moments_device = torch.device(moments_device) if moments_device is not None else None
        self.moments_hbm_bytes = moments_hbm_bytes
        self.stream_chunk_elems = int(stream_chunk_elems)
        self.stream_slots = int(stream_slots)
        self.moments_hbm_used = 0     # bytes of moments placed on moments_device so far
        self.state: DefaultDict[torch.Tensor, Any] = defaultdict(dict)

        assert 0.0 <= nvme_offload_fraction <= 1.0
        self.nvme_offload_fraction = nvme_offload_fraction
        self.prefetch = prefetch
        self.pin_memory = nvme_offload_fraction > 0.0

        self.exp_avg_flat = OrderedDict()
        self.exp_avg_sq_flat = OrderedDict()
        self._streamers: Dict[Any, HostStreamer] = {}
        # la_pipeline_stats_t of the last host-state update (timings, bytes moved)
        self.last_stream_stats = None

        if self.nvme_offload_fraction > 0.0:
            # layer_adam.py:92-101: same construction, with the native file
            # offloader of this package in place of tensornvme's
            from .nvme import DiskOffloader
            assert offload_dir is not None, "offload_dir cannot be None"
            self.offload_dir = offload_dir
            self.offloader = DiskOffloader(self.offload_dir, 16, 'uring')
            self.offload_numel = OrderedDict()
        else:
            self.offload_dir = None
            self.offloader = None

    def __del__(self):
        # overlapped host updates still write exp_avg / exp_avg_sq: finish them
        # while those buffers are certainly alive
        try:
            if getattr(self, '_streamers', None):
                self.synchronize()
        except Exception:
            pass
        if hasattr(self, 'lib') and hasattr(self, 'optimizer_id'):
            try:
                self.lib.la_destroy(self.optimizer_id)
            except Exception:
                pass
        if getattr(self, 'offloader', None) is not None:
            # layer_adam.py:117-124 removes every "offload-*" file of the
            # directory, those of other processes sharing it included; the
            # files here carry the process id, and only this process's go
            del self.offloader
            if self.offload_dir and os.path.exists(self.offload_dir):
                try:
                    for file in glob.glob(os.path.join(self.offload_dir, f"offload-{os.getpid()}-*")):
                        os.remove(file)
                except OSError:
                    pass

    # ------------------------------------------------------------------
    # layer registration (layer_adam.py:127-198)
    # ------------------------------------------------------------------
    def _get_layer_numel(self, layer_idx: int) -> int:
        return sum(p.numel() for p in self.param_groups[layer_idx]['params'])

    def add_layer_params(self, layer_idx: int, params: Iterable[torch.nn.Parameter]) -> int:
        """Register one layer; allocate its flat m/v beside the params (layer_adam.py:134-198),
        or on ``moments_device`` while its budget allows."""
        params = list(params)
        if not params:
            return -1
        layer_numel = sum(p.numel() for p in params)
        state_type = torch.float32 if self.fp32_optimizer_state else params[0].dtype
        device = params[0].device
        need = 2 * layer_numel * torch.empty(0, dtype=state_type).element_size()
        if self.moments_device is not None and (self.moments_hbm_bytes is None or
                                                self.moments_hbm_used + need <= self.moments_hbm_bytes):
            device = self.moments_device
        if self.offloader is not None and device.type != 'cpu':
            # as in the reference, the file offload moves host-resident moments
            raise RuntimeError("nvme_offload_fraction > 0 needs host-resident params and state")
        param_group = {
            'params': params,
            'layer_idx': layer_idx,
            'step': 0,
            **self.defaults,
        }
        self.param_groups.append(param_group)
        # host moments are page-locked on request: the copy engines then read and
        # write them directly, without the staging copies that pageable arrays
        # take (not with the file offload, which releases and re-allocates them);
        # at their exact size, since a process may page-lock only so much
        pin = (device.type == 'cpu' and self.pin_host_state and self.offloader is None
               and torch.cuda.is_available())
        if pin:
            self.exp_avg_flat[layer_idx] = _lib.page_locked_empty(layer_numel, state_type).zero_()
            self.exp_avg_sq_flat[layer_idx] = _lib.page_locked_empty(layer_numel, state_type).zero_()
        else:
            self.exp_avg_flat[layer_idx] = torch.zeros(layer_numel, dtype=state_type, device=device)
            self.exp_avg_sq_flat[layer_idx] = torch.zeros(layer_numel, dtype=state_type, device=device)
        if device == self.moments_device:
            self.moments_hbm_used += need
        offset = 0
        for p in params:
            size = p.numel()
            shape = p.shape
            if p not in self.state:
                self.state[p] = {}
            self.state[p]['exp_avg'] = self.exp_avg_flat[layer_idx][offset:offset + size].view(shape)
            self.state[p]['exp_avg_sq'] = self.exp_avg_sq_flat[layer_idx][offset:offset + size].view(shape)
            offset += size
        if self.offloader is not None:
            if layer_idx != self.num_layer - 1:
                self._offload_layer(layer_idx)
            else:
                self.offloader.sync_write_events()
        return layer_idx

    # NVMe hooks, layer_adam.py:200-247 (no-ops without an offloader)
    def _load_layer(self, layer_idx: int):
        if self.offloader is None:
            return
        if layer_idx < 0:
            layer_idx = self.num_layer + layer_idx
        assert layer_idx in self.exp_avg_flat
        self.offloader.async_read(self.exp_avg_flat[layer_idx])
        if self.nvme_offload_fraction > 0.5:
            self.offloader.async_read(self.exp_avg_sq_flat[layer_idx])

    def _offload_layer(self, layer_idx: int):
        if self.offloader is None:
            return
        assert layer_idx in self.exp_avg_flat
        self.offloader.async_write(self.exp_avg_flat[layer_idx])
        if self.nvme_offload_fraction > 0.5:
            self.offloader.async_write(self.exp_avg_sq_flat[layer_idx])

    def _pre_step(self, layer_idx: int):
        if self.offloader is None:
            return
        if self.prefetch:
            self.offloader.sync_read_events()
            self._load_layer(layer_idx - 1)
        else:
            self._load_layer(layer_idx)
            # layer_adam.py:234-236 returns with this read still running, and the
            # step that follows would read moments the read is still writing;
            # the read is fenced here instead
            self.offloader.sync_read_events()

    def _post_step(self, layer_idx: int):
        if self.offloader is None:
            return
        if self.prefetch:
            self.offloader.sync_write_events()
        self._offload_layer(layer_idx)

    def torch_adam_update(self, data, grad, exp_avg, exp_avg_sq, lr, beta1, beta2, eps,
                          weight_decay, bias_correction1, bias_correction2):
        """The reference's unused pure-torch formula (layer_adam.py:250-268), kept for API parity."""
        grad = grad.to(data.dtype)
        if weight_decay != 0:
            if self.defaults['adamw_mode']:
                data.mul_(1 - lr * weight_decay)
            else:
                grad = grad.add(data, alpha=weight_decay)
        exp_avg.mul_(beta1).add_(grad, alpha=1 - beta1)
        exp_avg_sq.mul_(beta2).addcmul_(grad, grad, value=1 - beta2)
        denom = (exp_avg_sq.sqrt() / math.sqrt(bias_correction2)).add_(eps)
        step_size = lr / bias_correction1
        data.addcdiv_(exp_avg, denom, value=-step_size)

    # ------------------------------------------------------------------
    # the native call (cpu_adam.adam_update -> la_adam_update)
    # ------------------------------------------------------------------
    def adam_update(self, step, lr, beta1, beta2, eps, weight_decay, bias_correction,
                    params, grads, exp_avg, exp_avg_sq, *, bf16_out=None, clip_coef=None,
                    stream=None):
        """One reference ``adam_update`` call (cpu_adam_impl.cpp:220-270) on the MI355X."""
        # contiguity checks of cpu_adam_impl.cpp:234-237
        if not params.is_contiguous():
            raise RuntimeError("params must be contiguous")
        if not grads.is_contiguous():
            raise RuntimeError("grads must be contiguous")
        if not exp_avg.is_contiguous():
            raise RuntimeError("exp_avg must be contiguous")
        if not exp_avg_sq.is_contiguous():
            raise RuntimeError("exp_avg_sq must be contiguous")
        n = params.numel()
        if grads.numel() != n or exp_avg.numel() != n or exp_avg_sq.numel() != n:
            raise RuntimeError(
                f"size mismatch: params {n}, grads {grads.numel()}, exp_avg {exp_avg.numel()}, "
                f"exp_avg_sq {exp_avg_sq.numel()}")
        if exp_avg_sq.dtype != exp_avg.dtype:
            raise RuntimeError("exp_avg and exp_avg_sq must have the same dtype")
        if bf16_out is not None:
            if bf16_out.dtype != torch.bfloat16 or bf16_out.numel() != n or not bf16_out.is_contiguous():
                raise RuntimeError("bf16_out must be a contiguous bfloat16 tensor of params.numel() elements")
        if clip_coef is not None:
            if clip_coef.dtype != torch.float32 or clip_coef.numel() < 1 or clip_coef.device.type != 'cuda':
                raise RuntimeError("clip_coef must be a float32 device tensor")

        arrays = [t for t in (params, grads, exp_avg, exp_avg_sq, bf16_out) if t is not None]
        # every array on the host or on one HIP device (the clip coefficient on that device);
        # get_device() is -1 for anything not on a HIP device
        indices = {t.get_device() for t in arrays}
        if clip_coef is not None:
            indices.add(clip_coef.get_device())
        if -1 not in indices and len(indices) == 1:
            self._device_update(step, lr, beta1, beta2, eps, weight_decay, bias_correction, params,
                                grads, exp_avg, exp_avg_sq, bf16_out, clip_coef, stream, n)
            return
        for t in arrays:
            if not t.is_cuda and t.device.type != 'cpu':
                raise RuntimeError(f"unsupported device type: {t.device.type}")
        gpu_devs = {t.device for t in arrays + ([clip_coef] if clip_coef is not None else []) if t.is_cuda}
        if len(gpu_devs) > 1:
            raise RuntimeError(f"params/grads/states must be on one device, got {sorted(map(str, gpu_devs))}")
        self._host_update(step, lr, beta1, beta2, eps, weight_decay, bias_correction, params,
                          grads, exp_avg, exp_avg_sq, bf16_out, clip_coef, stream, n,
                          gpu_devs.pop() if gpu_devs else None)

    def _codes(self, params, grads, exp_avg):
        key = (params.dtype, grads.dtype, exp_avg.dtype)
        if key not in SUPPORTED_TRIPLES:
            raise _unsupported(*key)
        return _DTYPE_CODE[params.dtype], _DTYPE_CODE[grads.dtype], _DTYPE_CODE[exp_avg.dtype]

    def _scalars(self, step, lr, beta1, beta2, eps, weight_decay, bias_correction):
        sc = _lib.LaScalars()
        _lib.check(self.lib.la_scalars(self.optimizer_id, int(step), lr, beta1, beta2, eps,
                                       weight_decay, int(bool(bias_correction)), ctypes.byref(sc)),
                   "la_scalars")
        return sc

    def _device_update(self, step, lr, beta1, beta2, eps, weight_decay, bias_correction, params,
                       grads, exp_avg, exp_avg_sq, bf16_out, clip_coef, stream, n):
        try:
            pc, gc, sc_ = self._codes(params, grads, exp_avg)
        except RuntimeError:
            # the reference advances the state machine before the dtype lookup
            self._scalars(step, lr, beta1, beta2, eps, weight_decay, bias_correction)
            raise
        with _on_device(params.device):
            rc = self.lib.la_adam_update(
                self.optimizer_id, int(step), lr, beta1, beta2, eps, weight_decay,
                int(bool(bias_correction)), pc, _ptr(params), gc, _ptr(grads), sc_, _ptr(exp_avg),
                _ptr(exp_avg_sq), n, _ptr(bf16_out), _ptr(clip_coef),
                _stream_handle(stream, params.device))
        _lib.check(rc, "la_adam_update")

    def _host_update(self, step, lr, beta1, beta2, eps, weight_decay, bias_correction, params,
                     grads, exp_avg, exp_avg_sq, bf16_out, clip_coef, stream, n, gpu):
        """Some arrays in host memory: stream those through HBM with the native
        chunk pipeline (la_pipeline_step), the others are used in place on
        ``gpu``; returns after completion, as the reference's CPU call does."""
        if not torch.cuda.is_available():
            raise RuntimeError("LayerAdam needs a HIP device (MI355X); there is no CPU arithmetic path")
        sc = self._scalars(step, lr, beta1, beta2, eps, weight_decay, bias_correction)
        pc, gc, sc_ = self._codes(params, grads, exp_avg)
        if n == 0:
            return
        device = gpu or self.device or torch.device('cuda', torch.cuda.current_device())
        with torch.cuda.device(device):
            streamer = self._streamers.get(device)
            if streamer is None:
                streamer = self._streamers[device] = HostStreamer(device, chunk_elems=self.stream_chunk_elems,
                                                                  slots=self.stream_slots)
            on_host = _placement(params, grads, exp_avg, exp_avg_sq, bf16_out)
            self.last_stream_stats = streamer.step(
                sc, pc, params, gc, grads, sc_, exp_avg, exp_avg_sq, n, bf16_out, on_host,
                clip_coef, _stream_handle(stream, device), synchronize=not self.overlap_host_chunks)

    # ------------------------------------------------------------------
    # steps (layer_adam.py:270-468)
    # ------------------------------------------------------------------
    @torch.no_grad()
    def step(self, layer_idx: int = None, closure=None, *, clip_coef=None):
        """Update one layer (or all layers) from ``p.grad`` (layer_adam.py:271-359).

        Keyword-only ``clip_coef``: a float32 device scalar (from
        ``clip_grad_norm`` or a ``GradNormAccumulator``) that scales every grad
        first, as in ``step_chunk``."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if layer_idx is not None:
            groups = [self.param_groups[layer_idx]]
        else:
            assert self.offloader is None, "with NVMe offload, layers can only be stepped one at a time, in order"
            groups = self.param_groups
        self._pre_step(layer_idx)
        for param_group in groups:
            param_group['step'] += 1
            entries = []
            for p in param_group['params']:
                g = p.grad
                if g is None:
                    continue
                state = self.state[p]
                assert p.numel() == g.numel(), "params and grads must have the same size"
                entries.append((p, g, state['exp_avg'], state['exp_avg_sq']))
            self._update_tensors(param_group, entries, clip_coef)
        self.synchronize()
        self._post_step(layer_idx)
        return loss

    @torch.no_grad()
    def step_with_grad_views(self, layer_idx: int = None,
                             grad_views: Dict[torch.nn.Parameter, torch.Tensor] = None, closure=None, *,
                             clip_coef=None):
        """Like ``step`` but with grads from a ``{param: grad_view}`` dict
        (layer_adam.py:362-428); ``clip_coef`` as in ``step``."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if layer_idx is not None:
            groups = [self.param_groups[layer_idx]]
        else:
            assert self.offloader is None, "with NVMe offload, layers can only be stepped one at a time, in order"
            groups = self.param_groups
        self._pre_step(layer_idx)
        for param_group in groups:
            param_group['step'] += 1
            entries = []
            for p in param_group['params']:
                grad = grad_views.get(p) if grad_views else None
                if grad is None:
                    print(f"Warning: no grad view for parameter {p}, skipping update")
                    continue
                state = self.state[p]
                assert p.numel() == grad.numel(), "params and grads must have the same size"
                entries.append((p, grad, state['exp_avg'], state['exp_avg_sq']))
            self._update_tensors(param_group, entries, clip_coef)
        self.synchronize()
        self._post_step(layer_idx)
        return loss

    def synchronize(self):
        """Complete every host-tensor update still in flight (they are only in
        flight with ``overlap_host_chunks=True``)."""
        if self.overlap_host_chunks:
            for streamer in self._streamers.values():
                with torch.cuda.device(streamer.device):
                    streamer.sync()

    def _update_tensors(self, param_group, entries, clip_coef=None):
        """The per-tensor adam_update calls of step(layer) / step_with_grad_views
        (layer_adam.py:314-327, 397-410), in order.  Device tensors on one device
        with one registered dtype triple that pass every per-call check and do not
        overlap go to the library as one la_adam_update_multi call: the same
        results and the same beta-power state as separate calls, in one or two
        launches.  Anything else takes the per-call path, which raises the
        reference's errors where the reference raises them."""
        beta1, beta2 = param_group['betas']
        hp = (param_group['step'], param_group['lr'], beta1, beta2, param_group['eps'],
              param_group['weight_decay'], param_group['bias_correction'])
        segs = _segments(entries) if len(entries) > 1 else None
        if segs is not None and clip_coef is not None:
            p0 = entries[0][0]
            if (clip_coef.dtype != torch.float32 or clip_coef.numel() < 1 or not clip_coef.is_cuda
                    or clip_coef.get_device() != p0.get_device()):
                segs = None                  # the per-call path raises the reference-style error
        if segs is not None:
            p0, g0, m0, _ = entries[0]
            with _on_device(p0.device):
                rc = self.lib.la_adam_update_multi(
                    self.optimizer_id, int(hp[0]), hp[1], hp[2], hp[3], hp[4], hp[5], int(bool(hp[6])),
                    _DTYPE_CODE[p0.dtype], _DTYPE_CODE[g0.dtype], _DTYPE_CODE[m0.dtype], segs, len(entries),
                    _ptr(clip_coef), _stream_handle(None, p0.device))
            _lib.check(rc, "la_adam_update_multi")
            return
        for p, g, m, v in entries:
            self.adam_update(*hp, p, g, m, v, clip_coef=clip_coef)

    @torch.no_grad()
    def begin_chunk_step(self, layer_idx: int):
        """Start a chunked step: step += 1, NVMe prefetch (layer_adam.py:431-439)."""
        param_group = self.param_groups[layer_idx]
        param_group['step'] += 1
        self._pre_step(layer_idx)
        return param_group

    @torch.no_grad()
    def step_chunk(self, param_flat, grad_flat, exp_avg_flat, exp_avg_sq_flat, param_group, *,
                   bf16_out=None, clip_coef=None, stream=None):
        """Update one [cs:ce] chunk of flat tensors (layer_adam.py:442-461).

        ``bf16_out``: optional bf16 tensor receiving the compute copy of the
        updated params.  ``clip_coef``: optional device fp32 scalar multiplying
        the grads (see ``clip_grad_norm``).  Device tensors: asynchronous on
        ``stream`` (default: current stream).  Host tensors: returns after
        completion, or, with ``overlap_host_chunks=True``, once queued
        (``end_chunk_step`` completes the chunks).
        """
        self.adam_update(param_group['step'], param_group['lr'], param_group['betas'][0],
                         param_group['betas'][1], param_group['eps'], param_group['weight_decay'],
                         param_group['bias_correction'], param_flat, grad_flat, exp_avg_flat,
                         exp_avg_sq_flat, bf16_out=bf16_out, clip_coef=clip_coef, stream=stream)

    @torch.no_grad()
    def end_chunk_step(self, layer_idx: int):
        """End a chunked step: every chunk complete, then NVMe write-back (layer_adam.py:464-468)."""
        self.synchronize()
        self._post_step(layer_idx)

    def update_learning_rate(self, new_lr):
        """Set ``lr`` in the defaults and every param group (layer_adam.py:470-484)."""
        self.defaults['lr'] = new_lr
        for param_group in self.param_groups:
            param_group['lr'] = new_lr

    # ------------------------------------------------------------------
    # grad-norm clip (new; the reference has no clipping)
    # ------------------------------------------------------------------
    @torch.no_grad()
    def clip_grad_norm(self, grads: Sequence[torch.Tensor], max_norm: float, *, stream=None):
        """Global L2 norm of device grads and the clip coefficient, both on device.

        Returns ``(coef, norm)``: fp32 device scalars with
        ``coef = min(1, max_norm / (norm + 1e-6))`` (torch.nn.utils.clip_grad_norm_
        convention), one-element views of this call's scratch.  Pass ``coef`` as
        ``clip_coef=`` to ``step_chunk``.  The grads go to the library in runs of
        one dtype, up to 32 tensors per la_grad_norm_multi call (two launches
        each).  Nothing is synchronised with the host.
        """
        grads = [g for g in grads if g is not None]
        if not grads:
            raise RuntimeError("clip_grad_norm needs at least one grad tensor")
        device = grads[0].device
        if device.type != 'cuda':
            raise RuntimeError("clip_grad_norm works on device tensors")
        _check_grads(grads, device)
        nwork = _norm_workspace_elems(self.lib)
        with _on_device(device):
            s = _torch_stream(stream, device)
            handle = s.cuda_stream
            # scratch of this call only, one allocation on the stream it is used
            # on, so calls on different streams share nothing: the partials,
            # the float64 sum, then coef and norm as two fp32 in one more slot
            if stream is None:
                buf = torch.empty(nwork + 2, dtype=torch.float64, device=device)
            else:
                with torch.cuda.stream(s):
                    buf = torch.empty(nwork + 2, dtype=torch.float64, device=device)
            base = buf.data_ptr()
            work, sqnorm, cn = base, base + nwork * 8, base + (nwork + 1) * 8
            pair = buf[nwork + 1:].view(torch.float32)
            coef, norm = pair[0:1], pair[1:2]
            # the first run of buffers overwrites the sum, the last one writes the coefficient
            _norm_runs(self.lib, grads, work, nwork, sqnorm, False, float(max_norm), cn, handle)
        return coef, norm

    def grad_norm_begin(self, device=None) -> "GradNormAccumulator":
        """Start a global grad norm over buffers that become ready one at a time.

        In the runtime's sliding order (post-backward hooks, offload_transformer.py:265-301)
        the last layer's grads exist long before the first layer's.  Call
        ``acc.add(grad_flat)`` as each layer's grads land (asynchronous, on the
        given stream), then ``coef, norm = acc.finish(max_norm)`` once every
        buffer was added, and pass ``coef`` to each layer's ``step_chunk``."""
        device = torch.device(device) if device is not None else (
            self.device or torch.device('cuda', torch.cuda.current_device()))
        return GradNormAccumulator(device)


class GradNormAccumulator:
    """Float64 sum of squares accumulated over several device buffers
    (la_grad_sqnorm, or la_grad_norm_multi for a list of them, with
    accumulate), then one clip coefficient (la_clip_coef).

    One accumulator is one running sum: its ``add`` and ``finish`` calls must be
    ordered, i.e. on one stream or synchronised between streams.  Its scratch
    is allocated once, at the size any buffer needs, and is marked as used by
    every stream a launch runs on (``record_stream``), so that the caching
    allocator does not hand it out again before those launches are done, even
    if the accumulator is dropped early."""

    def __init__(self, device):
        self.lib = _lib.load()
        self.device = torch.device(device)
        self.sqnorm = torch.zeros(1, dtype=torch.float64, device=self.device)
        self.work = torch.empty(_norm_workspace_elems(self.lib), dtype=torch.float64, device=self.device)
        self.count = 0

    @torch.no_grad()
    def add(self, grad, *, stream=None) -> None:
        """Add one grad buffer, or a sequence of them (a layer's per-tensor
        grads: two launches for up to 32 tensors of one dtype)."""
        grads = [grad] if isinstance(grad, torch.Tensor) else [g for g in grad if g is not None]
        if not grads:
            return
        _check_grads(grads, self.device)
        with _on_device(self.device):
            s = _torch_stream(stream, self.device)
            _norm_runs(self.lib, grads, _ptr(self.work), self.work.numel(), _ptr(self.sqnorm), self.count > 0,
                       0.0, None, s.cuda_stream)
            self.work.record_stream(s)
            self.sqnorm.record_stream(s)
        self.count += 1

    @torch.no_grad()
    def finish(self, max_norm: float, *, stream=None):
        """``(coef, norm)`` as fp32 device scalars, allocated on the stream that
        writes them; no host synchronisation."""
        with torch.cuda.device(self.device):
            s = _torch_stream(stream, self.device)
            with torch.cuda.stream(s):
                coef = torch.empty(1, dtype=torch.float32, device=self.device)
                norm = torch.empty(1, dtype=torch.float32, device=self.device)
            # with nothing added, sqnorm is still the zero it was created as: coef = 1
            _lib.check(self.lib.la_clip_coef(_ptr(self.sqnorm), float(max_norm), _ptr(coef), _ptr(norm),
                                             s.cuda_stream), "la_clip_coef")
            self.sqnorm.record_stream(s)
        return coef, norm
