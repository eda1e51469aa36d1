"""
KVSwapSpace — GPU <-> pinned-host movement of preempted sequences' KV, for
the MI355X backend.

Same contract as the reference's swap space
(serving/scheduler/preemption.py:298-523): ``swap_out`` copies every block of
a live sequence, every layer, K and V, in LOGICAL order into host memory
shaped ``(num_layers, num_blocks, block_size, n_kv_heads, head_dim)`` per
tensor and leaves freeing to the caller; ``swap_in`` restores a handle into
freshly allocated (different) blocks; the same checks and messages
(``SwapSpaceFull``, "freed", "resume mismatch", "blocks allocated",
``TypeError`` "paged backend"); ``release`` is idempotent.

What is different, and why it is safe: the reference copies synchronously
because an asynchronous D2H followed by an immediate ``free()`` would let the
allocator hand the blocks to another sequence mid-copy
(preemption.py:355-360). Here one gather kernel packs the victim's blocks
into a device staging buffer on a side stream, the caller's stream is made to
wait for THAT (a ~0.1 ms HBM-bound kernel), and only the slow PCIe transfer
from staging to pinned host memory, on a transfer stream of its own, overlaps
with later compute and with the next victim's gather. So freeing right after
``swap_out`` returns is safe: any kernel that could overwrite those blocks is
ordered after the gather. Swap-in mirrors it: H2D into staging on the
transfer stream, then a scatter kernel on the side stream that also waits for
the caller's stream (earlier users of the new blocks), and the caller's
stream waits for the scatter.
"""

from __future__ import annotations

import time

import torch

from . import _native
from .paging import SequenceBlocks

__all__ = ["KVSwapSpace", "SwapHandle", "SwapSpaceFull"]


class SwapSpaceFull(RuntimeError):
    """Host swap budget exhausted; callers fall back to recompute."""


class SwapHandle:
    """One sequence's KV parked in pinned host memory."""

    def __init__(self, request_id, seq_id, num_tokens, num_blocks, host, nbytes,
                 block_size, n_kv_heads, head_dim, done_event, staging):
        self.request_id = request_id
        self.seq_id = seq_id
        self.num_tokens = num_tokens
        self.num_blocks = num_blocks
        self.nbytes = nbytes
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.released = False
        self._host = host          # (2, L, nb, bs, Hkv, d) pinned
        self._done = done_event    # D2H completion
        self._staging = staging    # device staging, kept alive until the D2H lands

    def _wait(self) -> None:
        if self._done is not None:
            self._done.synchronize()
            self._done = None
            self._staging = None

    @property
    def k(self) -> torch.Tensor:
        """(L, nb, bs, Hkv, d) host tensor; waits for the copy to land."""
        self._wait()
        return self._host[0]

    @property
    def v(self) -> torch.Tensor:
        self._wait()
        return self._host[1]

    @property
    def host_buffer(self) -> torch.Tensor:
        """The whole (2, L, nb, bs, Hkv, d) pinned buffer; waits for the copy."""
        self._wait()
        return self._host


class KVSwapSpace:
    """Swap space over an ``MI355XBackend``'s fused pool."""

    def __init__(self, backend, max_bytes: int | None = None):
        for attr in ("k_pool", "v_pool", "num_layers", "block_size", "n_kv_heads",
                     "head_dim", "_pool", "_lib"):
            if not hasattr(backend, attr):
                raise TypeError(
                    f"KVSwapSpace needs a paged backend exposing .{attr}; got "
                    f"{type(backend).__name__}. The swap path moves physical KV, so it "
                    "cannot run against a backend that does not own a pool."
                )
        self.backend = backend
        self.max_bytes = max_bytes
        self.bytes_in_use = 0
        self.peak_bytes = 0
        self.last_swap_out_seconds = 0.0
        self._live: dict[int, SwapHandle] = {}
        self.device = backend.device
        self.dtype = backend.dtype
        self.pinned = True
        # kernels (gather / scatter) on one side stream, host transfers on
        # another, so one sequence's transfer overlaps the next one's kernel
        self._side = torch.cuda.Stream(device=self.device)
        self._copy = torch.cuda.Stream(device=self.device)

    def bytes_for(self, num_blocks: int) -> int:
        return 2 * self.backend.num_layers * num_blocks * self.backend._block_bytes

    @property
    def num_swapped(self) -> int:
        return len(self._live)

    def _ids(self, block_ids) -> torch.Tensor:
        for b in block_ids:
            if not 0 <= b < self.backend.num_blocks:
                raise IndexError(f"block id {b} outside [0, {self.backend.num_blocks})")
        # from pinned memory, so the upload is queued on the caller's stream
        # instead of waiting for it (the side stream waits for that stream
        # before its kernel reads the ids)
        host = torch.tensor(list(block_ids), dtype=torch.int32).pin_memory()
        return host.to(self.device, non_blocking=True)

    def _shape(self, nb: int) -> tuple:
        b = self.backend
        return (2, b.num_layers, nb, b.block_size, b.n_kv_heads, b.head_dim)

    def swap_out(self, request_id: str, blocks: SequenceBlocks) -> SwapHandle:
        """Copy every block of ``blocks`` to host; the caller frees afterwards."""
        if blocks.is_freed:
            raise RuntimeError(
                f"swap_out on freed SequenceBlocks(seq_id={blocks.seq_id}); its blocks may "
                "already belong to another sequence"
            )
        nb = len(blocks.block_ids)
        want = self.bytes_for(nb)
        if self.max_bytes is not None and self.bytes_in_use + want > self.max_bytes:
            raise SwapSpaceFull(f"swapping {nb} blocks needs {want} B; {self.bytes_in_use} B "
                                f"of {self.max_bytes} B host swap space already in use")
        t0 = time.perf_counter()
        b = self.backend
        b._flush()  # a deferred append must land before the blocks are read
        host = torch.empty(self._shape(nb), dtype=self.dtype, pin_memory=True)
        done = staging = None
        if nb:
            main = torch.cuda.current_stream(self.device)
            ids = self._ids(blocks.block_ids)
            side = self._side
            side.wait_stream(main)
            with torch.cuda.stream(side):
                staging = torch.empty(self._shape(nb), dtype=self.dtype, device=self.device)
                rc = b._lib.pkv_gather_blocks(b._pool.data_ptr(), b.num_layers, b._plane_bytes,
                                              b._block_bytes, b.num_blocks, ids.data_ptr(), nb,
                                              staging.data_ptr(), b._status.data_ptr(),
                                              side.cuda_stream)
                _native.check(rc, "swap_out gather")
                ids.record_stream(side)
                packed = torch.cuda.Event()
                packed.record(side)
            # The blocks may be reused by the caller's stream once packed.
            main.wait_stream(side)
            copy = self._copy
            copy.wait_event(packed)
            with torch.cuda.stream(copy):
                host.copy_(staging, non_blocking=True)
                staging.record_stream(copy)
                done = torch.cuda.Event()
                done.record(copy)
        self.last_swap_out_seconds = time.perf_counter() - t0
        h = SwapHandle(request_id, blocks.seq_id, blocks.num_tokens, nb, host, want,
                       b.block_size, b.n_kv_heads, b.head_dim, done, staging)
        self._live[id(h)] = h
        self.bytes_in_use += want
        self.peak_bytes = max(self.peak_bytes, self.bytes_in_use)
        return h

    def swap_in(self, handle: SwapHandle, blocks: SequenceBlocks) -> None:
        """Restore ``handle`` into ``blocks`` (already grown to handle.num_tokens)."""
        if handle.released:
            raise RuntimeError(f"swap_in on a released handle for {handle.request_id!r}")
        if blocks.num_tokens != handle.num_tokens:
            raise RuntimeError(f"resume mismatch for {handle.request_id!r}: block table holds "
                               f"{blocks.num_tokens} tokens, handle holds {handle.num_tokens}")
        if len(blocks.block_ids) != handle.num_blocks:
            raise RuntimeError(
                f"resume mismatch for {handle.request_id!r}: {len(blocks.block_ids)} blocks "
                f"allocated, {handle.num_blocks} swapped out. Logical block order would shift."
            )
        if handle.block_size != self.backend.block_size:
            raise RuntimeError(f"handle block_size={handle.block_size} != backend "
                               f"{self.backend.block_size}")
        nb = handle.num_blocks
        if nb == 0:
            return
        if len(set(blocks.block_ids)) != nb:
            raise RuntimeError("swap_in target block ids must be distinct")
        b = self.backend
        b._flush()
        main = torch.cuda.current_stream(self.device)
        ids = self._ids(blocks.block_ids)
        side = self._side
        copy = self._copy
        if handle._done is not None:
            copy.wait_event(handle._done)
        with torch.cuda.stream(copy):
            staging = torch.empty(self._shape(nb), dtype=self.dtype, device=self.device)
            staging.copy_(handle._host, non_blocking=True)
            landed = torch.cuda.Event()
            landed.record(copy)
        side.wait_event(landed)
        side.wait_stream(main)  # earlier kernels may still read the new blocks
        with torch.cuda.stream(side):
            rc = b._lib.pkv_scatter_blocks(b._pool.data_ptr(), b.num_layers, b._plane_bytes,
                                           b._block_bytes, b.num_blocks, ids.data_ptr(), nb,
                                           staging.data_ptr(), b._status.data_ptr(),
                                           side.cuda_stream)
            _native.check(rc, "swap_in scatter")
            ids.record_stream(side)
            staging.record_stream(side)
        main.wait_stream(side)

    def release(self, handle: SwapHandle) -> None:
        """Drop a handle's host memory. Idempotent."""
        if handle.released:
            return
        handle.released = True
        self._live.pop(id(handle), None)
        self.bytes_in_use -= handle.nbytes
        handle._wait()
        handle._host = torch.empty(0)

    def synchronize(self) -> None:
        """Wait for every outstanding swap copy."""
        self._side.synchronize()
        self._copy.synchronize()
