"""
A running decode batch, stepped one token at a time on the host.

The reference's scheduler runs every decode step the same way: grow each
running sequence's block table by the token it is about to write
(``blocks.append(1)``, serving/scheduler/scheduler.py:749), then describe
the whole batch again with ``build_batch_meta`` (serving/engine_iface/
batch.py:190-318), a Python loop over sequences and pages that the
reference's own risk register names as a threat to step time (R22,
docs/RISK_REGISTER.md:271-284).

``DecodeStepper`` keeps the batch's index arrays between steps and brings
them up to date with array operations. Each step:

* grows every sequence by one token: the sequences whose last page is full
  take one fresh page each, from ONE ``allocate`` call. The allocator hands
  out its FIFO free list in order, so every sequence receives exactly the
  page it would have received from ``append(1)`` called sequence by
  sequence, and the ``SequenceBlocks`` objects are left as those calls
  leave them (``block_ids``, ``num_tokens``);
* updates the CSR triple in place (the new page ids are inserted at the
  end of their sequences' lists; ``kv_indptr`` shifts by the running count
  of insertions), ``kv_lens``, ``positions``, ``kv_last_page_len`` and
  ``slot_mapping``;
* uploads every index array and the int64 positions with one pinned
  host-to-device copy, and returns a ``BatchMeta`` that carries the host
  arrays, so the backend plans the step without reading the device back.

The result equals ``build_batch_meta`` over the same sequences, each
contributing one token, field for field (tested), without its per-sequence
loop. While a stepper runs it owns its sequences' growth: a sequence
leaving or joining the batch (finished, preempted, admitted) means a new
stepper (one ``build_batch_meta``-sized pass).
"""

from __future__ import annotations

import numpy as np
import torch

from .assembly import _upload
from .contract import MIRRORED, BatchMeta, HostMirror
from .paging import SequenceBlocks

__all__ = ["DecodeStepper"]


class DecodeStepper:
    """One token per sequence per step for a fixed set of running sequences."""

    def __init__(self, seqs: list[SequenceBlocks], device, page_size: int,
                 dtype_index: torch.dtype = torch.int32):
        if not seqs:
            raise ValueError("DecodeStepper needs at least one sequence")
        if page_size <= 0:
            raise ValueError(f"page_size must be positive, got {page_size}")
        alloc = seqs[0]._alloc
        for i, s in enumerate(seqs):
            if s.is_freed:
                raise ValueError(f"seq {i} (seq_id={s.seq_id}) has been freed; its pages may "
                                 "belong to another sequence")
            if s.block_size != page_size:
                raise ValueError(f"seq {i} (seq_id={s.seq_id}) has block_size={s.block_size} "
                                 f"but the batch declares page_size={page_size}")
            if s._alloc is not alloc:
                raise ValueError("every sequence of a DecodeStepper must draw its pages from "
                                 "one allocator")
            if s.num_tokens > s.capacity:
                raise ValueError(f"seq {i} (seq_id={s.seq_id}) claims {s.num_tokens} tokens "
                                 f"but its {s.num_blocks} blocks hold {s.capacity}")
        n = len(seqs)
        self.seqs = list(seqs)
        self.device = torch.device(device)
        self.page_size = page_size
        self.dtype_index = dtype_index
        self._alloc = alloc
        self._kv = np.fromiter((s.num_tokens for s in seqs), np.int64, n)
        self._nblk = np.fromiter((len(s.block_ids) for s in seqs), np.int64, n)
        self._indptr = np.zeros(n + 1, np.int64)
        np.cumsum(self._nblk, out=self._indptr[1:])
        self._indices = np.fromiter((b for s in seqs for b in s.block_ids), np.int64,
                                    int(self._indptr[-1]))
        # one token per sequence: these never change
        self._ones = np.ones(n, np.int64)
        self._ar = np.arange(n + 1, dtype=np.int64)
        self.steps = 0

    @property
    def n_seqs(self) -> int:
        return len(self.seqs)

    def step(self) -> BatchMeta:
        """Grow every sequence by one token and describe the step."""
        bs = self.page_size
        kv = self._kv
        full = kv >= self._nblk * bs            # the new token needs a page
        grow = np.flatnonzero(full)
        if grow.size:
            # all or nothing: on AllocationError no sequence has changed
            new_ids = self._alloc.allocate(int(grow.size))
            for i, b in zip(grow.tolist(), new_ids):
                self.seqs[i].block_ids.append(b)
            # each new id goes at the end of its sequence's list
            self._indices = np.insert(self._indices, self._indptr[1:][grow],
                                      np.asarray(new_ids, np.int64))
            self._indptr[1:] += np.cumsum(full)
            self._nblk += full
        for s in self.seqs:
            s.num_tokens += 1
        kv += 1
        self.steps += 1
        pos = kv - 1
        page, off = np.divmod(pos, bs)
        slots = self._indices[self._indptr[:-1] + page] * bs + off
        n = kv.shape[0]
        ar = self._ar
        parts = {
            "query_lens": self._ones, "cu_query_lens": ar, "kv_lens": kv.copy(),
            "last_token_ix": ar[:n], "kv_indptr": self._indptr.copy(),
            "kv_indices": self._indices, "kv_last_page_len": off + 1,
            "batch_indices": ar[:n], "slot_mapping": slots,
        }
        fields = _upload(parts, pos, self.device, self.dtype_index)
        mirror = HostMirror(arrays={k: parts[k] for k in MIRRORED},
                            of=tuple(fields[k] for k in MIRRORED))
        return BatchMeta(**fields, page_size=bs, is_prefill=False, host=mirror)
