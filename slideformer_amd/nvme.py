"""File offload of LayerAdam's host moment buffers (the NVMe path).

``DiskOffloader`` has the interface of tensornvme's class as the reference's
LayerAdam uses it (layer_adam.py:92-106 construction, :200-247 use):
``async_write(t)`` queues the buffer's bytes to its file and, once
``sync_write_events()`` has seen the write land, releases the tensor's
storage; ``async_read(t)`` re-allocates the storage and queues the read,
complete after ``sync_read_events()``.  Views into the buffer (LayerAdam's
per-parameter ``state`` views) stay valid across the release/re-allocation
because they share the storage object.  The I/O runs on the native worker
pool of ``libslideformer_amd.so`` (``la_disk_*``).

``backend`` names tensornvme's I/O engine in the reference (it passes
``'uring'``, layer_adam.py:101).  io_uring itself is not used here: the pool's
threads issue positioned reads and writes.  The name selects how they reach
the file:
  * ``'uring'``, ``'aio'``, ``'direct'``: direct I/O (``O_DIRECT``).  The
    moments leave host RAM for real, instead of staying in it as cached
    pages, and the rates are the device's.  If the directory's file system
    refuses ``O_DIRECT``, buffered I/O is used instead, with a warning
    (``self.direct`` tells which);
  * ``'pthread'``, ``'buffered'``: buffered I/O through the page cache.
"""
from __future__ import annotations

import ctypes
import errno
import os
import warnings
from typing import Dict, List, Set

import torch

from . import _lib


class DiskOffloader:
    DIRECT_BACKENDS = ('uring', 'aio', 'direct')
    BUFFERED_BACKENDS = ('pthread', 'buffered')

    def __init__(self, dir_name: str, n_entries: int = 16, backend: str = 'uring'):
        # `n_entries` bounds the size of the native thread pool
        if backend not in self.DIRECT_BACKENDS + self.BUFFERED_BACKENDS:
            raise ValueError(f"unknown backend {backend!r}; one of {self.DIRECT_BACKENDS + self.BUFFERED_BACKENDS}")
        self.lib = _lib.load()
        self.dir_name = os.path.abspath(dir_name)
        os.makedirs(self.dir_name, exist_ok=True)
        self.backend = backend
        threads = max(1, min(int(n_entries), 16))
        handle = ctypes.c_void_p()
        self.direct = backend in self.DIRECT_BACKENDS
        rc = self.lib.la_disk_create_ex(self.dir_name.encode(), threads, _lib.LA_DISK_DIRECT if self.direct else 0,
                                        ctypes.byref(handle))
        if self.direct and rc == -errno.EINVAL:
            warnings.warn(f"{self.dir_name}: the file system does not take O_DIRECT; offloading through the "
                          "page cache instead", RuntimeWarning, stacklevel=2)
            self.direct = False
            rc = self.lib.la_disk_create_ex(self.dir_name.encode(), threads, 0, ctypes.byref(handle))
        if rc != 0:
            raise OSError(-rc, f"la_disk_create({self.dir_name}) failed: {os.strerror(-rc) if rc < 0 else rc}")
        self.handle = handle
        self._nbytes: Dict[int, int] = {}
        self._pending_writes: List[torch.Tensor] = []
        self._pending_reads: List[torch.Tensor] = []
        # keys with a native write not yet fenced by la_disk_sync_writes (a
        # cancelled release leaves its write running)
        self._writing: Set[int] = set()

    @staticmethod
    def _check_tensor(t: torch.Tensor):
        if t.device.type != 'cpu':
            raise RuntimeError("DiskOffloader moves host tensors only")
        if not t.is_contiguous() or t.storage_offset() != 0:
            raise RuntimeError("DiskOffloader needs a whole contiguous buffer")

    def _io_error(self, rc: int, what: str):
        if rc != 0:
            raise OSError(-rc if rc < 0 else rc, f"{what} failed: {os.strerror(-rc) if rc < 0 else rc}")

    def async_write(self, tensor: torch.Tensor) -> None:
        self._check_tensor(tensor)
        nbytes = tensor.numel() * tensor.element_size()
        if tensor.untyped_storage().nbytes() < nbytes:
            raise RuntimeError("async_write of a buffer whose storage was already released")
        key = id(tensor)
        if key in self._writing:
            # An earlier write of this buffer is still running (async_read
            # cancelled its release, and the buffer may have changed since).
            # The pool's workers take pieces in parallel, so an old piece could
            # land after the new one: fence the old write first.
            rc = self.lib.la_disk_sync_writes(self.handle)
            self._writing.clear()
            self._io_error(rc, "la_disk_sync_writes")
        self._nbytes[key] = nbytes
        self._io_error(self.lib.la_disk_write_async(self.handle, key, tensor.data_ptr(), nbytes),
                       "la_disk_write_async")
        self._writing.add(key)
        self._pending_writes.append(tensor)

    def async_read(self, tensor: torch.Tensor) -> None:
        """Bring the buffer back.  A buffer whose storage was never released
        (never written, or written but not yet fenced by sync_write_events)
        still holds the current bytes, so nothing is read; a pending release
        of it is cancelled."""
        self._check_tensor(tensor)
        if any(tensor is w for w in self._pending_writes):
            self._pending_writes = [w for w in self._pending_writes if w is not tensor]
            return
        nbytes = self._nbytes.get(id(tensor))
        storage = tensor.untyped_storage()
        if nbytes is None or storage.nbytes() >= nbytes:
            return
        storage.resize_(nbytes)
        self._io_error(self.lib.la_disk_read_async(self.handle, id(tensor), tensor.data_ptr(), nbytes),
                       "la_disk_read_async")
        self._pending_reads.append(tensor)

    def sync_write_events(self) -> None:
        rc = self.lib.la_disk_sync_writes(self.handle)
        self._writing.clear()
        written, self._pending_writes = self._pending_writes, []
        self._io_error(rc, "la_disk_sync_writes")
        for t in written:
            t.untyped_storage().resize_(0)  # the bytes live in the file now

    def sync_read_events(self) -> None:
        rc = self.lib.la_disk_sync_reads(self.handle)
        self._pending_reads = []
        self._io_error(rc, "la_disk_sync_reads")

    def sync_write(self, tensor: torch.Tensor) -> None:
        self.async_write(tensor)
        self.sync_write_events()

    def sync_read(self, tensor: torch.Tensor) -> None:
        self.async_read(tensor)
        self.sync_read_events()

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                self.lib.la_disk_destroy(self.handle)
                self.handle = None
        except Exception:
            pass
