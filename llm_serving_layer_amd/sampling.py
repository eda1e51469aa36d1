"""
The scheduler step's sampling and timing points on the device.

The reference scheduler ends every step with ``logits = model.forward_varlen(
tokens, meta, backend)`` and ``torch.argmax(logits, dim=-1).tolist()``
(serving/scheduler/scheduler.py:743-757), and times GPU work with events on
the stream rather than the host clock, because ``forward_varlen`` returns a
device tensor (docs/ADR.md:954-989, ADR-023). Here:

* ``greedy(logits)`` is that argmax on the device through the library's
  ``pkv_argmax_rows`` kernel (one int64 per row comes back, not the logits);
* ``StepTimer`` brackets a step with HIP events on torch's current stream
  (where the backend launches) and reads the elapsed time only at a declared
  synchronisation point;
* ``greedy_step`` is the forward-and-sample part of ``Scheduler.step``:
  metadata, tokens, forward, greedy pick, and one device-to-host copy of the
  picked ids, the step's only synchronisation.
"""

from __future__ import annotations

import torch

from . import _native
from .assembly import ScheduledSeq, build_batch_meta, build_token_tensor
from .backend import _DTYPES, _current_stream

__all__ = ["greedy", "StepTimer", "greedy_step"]


def rows_for_kernel(logits: torch.Tensor) -> torch.Tensor:
    """
    ``logits`` itself when the argmax kernel can read it in place -- unit
    element stride and rows that do not overlap (row stride >= vocab, or a
    single row) -- else a contiguous copy. A view whose rows overlap (an
    ``expand`` has row stride 0) would otherwise make the kernel read rows
    1..n-1 past the end of the allocation.
    """
    n, vocab = logits.shape
    unit = logits.stride(1) == 1 or vocab == 1
    apart = n <= 1 or logits.stride(0) >= vocab
    return logits if unit and apart else logits.contiguous()


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """
    ``torch.argmax(logits, dim=-1)`` for a (n_rows, vocab) f16, bf16 or f32
    device tensor whose rows are contiguous: an int64 device tensor of
    n_rows greedy ids (torch's order: a NaN beats every number, of equal
    values the first wins). Asynchronous on torch's current stream.
    """
    if logits.dim() != 2:
        raise ValueError(f"logits must be (n_rows, vocab), got shape {tuple(logits.shape)}")
    if logits.device.type != "cuda":
        raise ValueError(f"logits must be on the GPU, got {logits.device}")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"logits dtype {logits.dtype} is not float16, bfloat16 or float32")
    n, vocab = logits.shape
    if vocab == 0:
        raise ValueError("argmax of an empty row: vocab is 0")
    logits = rows_for_kernel(logits)
    out = torch.empty(n, dtype=torch.int64, device=logits.device)
    if n == 0:
        return out
    lib = _native.load()
    # (one row: its stride is never used, and may be anything, e.g. 0)
    row_stride = logits.stride(0) if n > 1 else vocab
    rc = lib.pkv_argmax_rows(logits.data_ptr(), n, vocab, row_stride,
                             _DTYPES[logits.dtype], out.data_ptr(),
                             _current_stream(logits.device))
    _native.check(rc, "greedy argmax")
    return out


class StepTimer:
    """
    GPU time of a step from two HIP events on torch's current stream of
    ``device``: ``start()`` and ``stop()`` only record; ``elapsed_ms()``
    waits for the stop event (the declared synchronisation point) and
    returns the milliseconds between them. ``history`` keeps every step read.
    """

    def __init__(self, device="cuda:0"):
        self.device = torch.device(device)
        self._start = torch.cuda.Event(enable_timing=True)
        self._stop = torch.cuda.Event(enable_timing=True)
        self._armed = False
        self.history: list[float] = []

    def start(self) -> None:
        self._start.record(torch.cuda.current_stream(self.device))
        self._armed = True

    def stop(self) -> None:
        if not self._armed:
            raise RuntimeError("StepTimer.stop() without start()")
        self._stop.record(torch.cuda.current_stream(self.device))
        self._armed = False

    def elapsed_ms(self) -> float:
        self._stop.synchronize()
        ms = self._start.elapsed_time(self._stop)
        self.history.append(ms)
        return ms


def greedy_step(model, scheduled: list[ScheduledSeq], backend, page_size: int,
                timer: StepTimer | None = None) -> list[int]:
    """
    The forward-and-sample part of the reference's ``Scheduler.step``
    (serving/scheduler/scheduler.py:743-757): block tables already grown by
    the caller, then metadata and token ids for ``scheduled`` (in that
    order), ``model.forward_varlen(tokens, meta, backend)`` -> (n_seqs,
    vocab) device logits, the greedy id of every sequence on the device, and
    ONE device-to-host copy of those ids, which is also where a ``timer``'s
    stop event is known to have passed.
    """
    meta = build_batch_meta(scheduled, device=backend.device, page_size=page_size)
    tokens = build_token_tensor(scheduled, device=backend.device)
    if timer is not None:
        timer.start()
    logits = model.forward_varlen(tokens, meta, backend)
    if tuple(logits.shape[:1]) != (len(scheduled),):
        raise ValueError(f"forward_varlen returned {tuple(logits.shape)} logits for "
                         f"{len(scheduled)} sequences")
    ids = greedy(logits)
    if timer is not None:
        timer.stop()
    return ids.tolist()
