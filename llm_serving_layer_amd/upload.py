"""
Per-step host-to-device uploads of index metadata and plans.

A serving loop uploads a few tens of KiB every step: the batch's index
arrays and the backend's launch plan. Queued as ``tensor.to(device,
non_blocking=True)`` each becomes a copy-engine transfer, and the kernel
after it waits for the copy engine's completion signal: on MI355X that
hand-off put ~25 us on the GPU timeline per upload, about 12% of a batch-256
decode step when the host keeps ahead of the GPU.

``PinnedUploader`` copies with the library's ``pkv_upload_pinned`` instead:
a kernel on the launch stream reads the pinned host buffer through its
device mapping, so the upload is ordered like any other kernel and costs a
few microseconds. The pinned buffers form a ring; a buffer is refilled only
after the kernel that last read it has run (an event recorded behind that
kernel), so a host that runs several steps ahead of the GPU never
overwrites metadata a queued step still has to read. Under graph capture
an upload falls back to a fresh pinned tensor copied with ``to()``.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native

__all__ = ["PinnedUploader", "uploader"]

try:  # torch's current stream as a raw handle, without building a Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream
except AttributeError:  # pragma: no cover - older torch
    _raw_stream = None

_UPLOADERS: dict = {}


def uploader(device) -> "PinnedUploader":
    """The uploader of ``device`` (one per device, created on first use)."""
    device = torch.device(device)
    up = _UPLOADERS.get(device.index)
    if up is None:
        up = _UPLOADERS[device.index] = PinnedUploader(device)
    return up


class PinnedUploader:
    """A ring of pinned host buffers uploaded by a kernel on the launch stream."""

    def __init__(self, device: torch.device, slots: int = 8):
        self.device = torch.device(device)
        self._lib = _native.load()
        self._bufs: list = [None] * slots
        self._events = [torch.cuda.Event() for _ in range(slots)]
        self._pending = [False] * slots
        self._next = 0

    def buffer(self, nbytes: int) -> torch.Tensor:
        """The next ring buffer as ``nbytes`` pinned bytes, free to fill: the
        upload that last read it has run."""
        i = self._next
        if self._pending[i]:
            self._events[i].synchronize()
            self._pending[i] = False
        buf = self._bufs[i]
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 2 * (buf.numel() if buf is not None else 0), 1 << 16)
            buf = self._bufs[i] = torch.empty(size, dtype=torch.uint8, pin_memory=True)
        return buf[:nbytes]

    def send(self, host: torch.Tensor) -> torch.Tensor:
        """Upload the bytes of ``host`` (the view ``buffer`` returned, now
        filled) on torch's current stream; returns the device copy."""
        i = self._next
        self._next = (i + 1) % len(self._bufs)
        n = host.numel()
        if torch.cuda.is_current_stream_capturing():
            # a captured upload is replayed later: it must own its source
            return host.clone().pin_memory().to(self.device, non_blocking=True)
        dev = torch.empty(n, dtype=torch.uint8, device=self.device)
        idx = self.device.index if self.device.index is not None else 0
        stream = (_raw_stream(idx) if _raw_stream is not None
                  else torch.cuda.current_stream(self.device).cuda_stream)
        rc = self._lib.pkv_upload_pinned(dev.data_ptr(), host.data_ptr(), n, stream)
        _native.check(rc, "upload")
        self._events[i].record(torch.cuda.current_stream(self.device))
        self._pending[i] = True
        return dev

    def array(self, a: np.ndarray) -> torch.Tensor:
        """A device copy of the host array ``a`` (int32 or int64), same dtype."""
        a = np.ascontiguousarray(a)
        dtype = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}[a.dtype]
        host = self.buffer(a.nbytes)
        host.numpy()[:] = a.view(np.uint8).reshape(-1)
        return self.send(host).view(dtype)
