"""
Block-id bookkeeping on the host: the refcounted page pool, the per-sequence
page list with its slot arithmetic, and the CSR flattening the kernels read.

Behaviour follows the reference:

* ``BlockAllocator``   serving/memory/allocator.py:53-259 (FIFO free list so
  a use-after-free reads obvious garbage; ``can_allocate`` honours the
  watermark, ``allocate`` does not; all-or-nothing; double free raises);
* ``SequenceBlocks``   serving/memory/block_table.py:37-181
  (``slot = block_ids[p // bs] * bs + p % bs``; ``last_page_len`` in
  ``[1, bs]``, an exact multiple reports ``bs``);
* ``build_csr``        serving/memory/block_table.py:184-208.

Pure Python integers: nothing here touches a device.
"""

from __future__ import annotations

from collections import deque
from collections.abc import Iterable, Sequence

__all__ = ["AllocationError", "BlockAllocator", "SequenceBlocks", "build_csr"]


class AllocationError(RuntimeError):
    """A request for blocks that cannot be met. Nothing is handed out."""


class BlockAllocator:
    """Fixed pool of ``num_blocks`` page ids with per-id reference counts."""

    def __init__(self, num_blocks: int, block_size: int = 16, watermark_blocks: int = 0):
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {num_blocks}")
        if block_size <= 0:
            raise ValueError(f"block_size must be positive, got {block_size}")
        if not 0 <= watermark_blocks < num_blocks:
            raise ValueError(
                f"watermark_blocks must lie in [0, {num_blocks}), got {watermark_blocks}"
            )
        self._n = num_blocks
        self._bs = block_size
        self._watermark = watermark_blocks
        self._free: deque[int] = deque(range(num_blocks))
        self._refcount: list[int] = [0] * num_blocks
        self.total_allocated = 0
        self.total_freed = 0
        self.peak_used = 0

    num_blocks = property(lambda self: self._n)
    block_size = property(lambda self: self._bs)
    watermark_blocks = property(lambda self: self._watermark)
    num_free = property(lambda self: len(self._free))
    num_used = property(lambda self: self._n - len(self._free))

    @property
    def utilization(self) -> float:
        return self.num_used / self._n

    def refcount(self, block_id: int) -> int:
        self._check_id(block_id)
        return self._refcount[block_id]

    def tokens_capacity(self) -> int:
        return self._n * self._bs

    def can_allocate(self, n_blocks: int) -> bool:
        """Admission test: would ``n_blocks`` still leave the watermark free?"""
        if n_blocks < 0:
            raise ValueError(f"n_blocks must be non-negative, got {n_blocks}")
        return len(self._free) - n_blocks >= self._watermark

    def allocate(self, n_blocks: int) -> list[int]:
        """Take ``n_blocks`` ids from the front of the free list (refcount 1 each)."""
        if n_blocks < 0:
            raise ValueError(f"n_blocks must be non-negative, got {n_blocks}")
        if n_blocks == 0:
            return []
        if n_blocks > len(self._free):
            raise AllocationError(
                f"Cannot allocate {n_blocks} blocks: only {len(self._free)} free of "
                f"{self._n} (watermark {self._watermark})."
            )
        got = [self._free.popleft() for _ in range(n_blocks)]
        for b in got:
            assert self._refcount[b] == 0, f"Block {b} on the free list has refcount {self._refcount[b]}"
            self._refcount[b] = 1
        self.total_allocated += n_blocks
        self.peak_used = max(self.peak_used, self.num_used)
        return got

    def incref(self, block_ids: Iterable[int]) -> None:
        for b in block_ids:
            self._check_id(b)
            if self._refcount[b] == 0:
                raise AllocationError(
                    f"Cannot incref block {b}: its refcount is 0, so it sits on the free list "
                    "and its contents belong to nobody")
            self._refcount[b] += 1

    def free(self, block_ids: Sequence[int]) -> None:
        """Drop one reference per id; an id returns to the BACK of the free list at 0."""
        for b in block_ids:
            self._check_id(b)
            if self._refcount[b] == 0:
                raise AllocationError(f"Double free of block {b}: refcount is already 0")
            self._refcount[b] -= 1
            if self._refcount[b] == 0:
                self._free.append(b)
                self.total_freed += 1

    def check_invariants(self) -> None:
        free_ids = list(self._free)
        free_set = set(free_ids)
        if len(free_set) != len(free_ids):
            seen, dup = set(), set()
            for b in free_ids:
                (dup if b in seen else seen).add(b)
            raise AssertionError(f"Free list contains duplicates: {sorted(dup)}")
        for b, rc in enumerate(self._refcount):
            if rc < 0:
                raise AssertionError(f"Block {b} has negative refcount {rc}")
            if rc == 0 and b not in free_set:
                raise AssertionError(
                    f"Block {b} has refcount 0 but is not on the free list: it leaked "
                    "(the pool silently lost capacity)")
            if rc > 0 and b in free_set:
                raise AssertionError(
                    f"Block {b} has refcount {rc} but IS on the free list: the next "
                    "allocation would hand a live block to a second owner")

    def reset(self) -> None:
        self._free = deque(range(self._n))
        self._refcount = [0] * self._n

    def _check_id(self, block_id: int) -> None:
        if not 0 <= block_id < self._n:
            raise ValueError(f"Block id {block_id} out of range [0, {self._n})")

    def __repr__(self) -> str:
        return (f"BlockAllocator(num_blocks={self._n}, block_size={self._bs}, "
                f"free={self.num_free}, used={self.num_used}, watermark={self._watermark})")


class SequenceBlocks:
    """One sequence's page list, in logical order, and its slot arithmetic."""

    def __init__(self, allocator: BlockAllocator, seq_id: int = 0):
        self._alloc = allocator
        self.seq_id = seq_id
        self.block_size = allocator.block_size
        self.block_ids: list[int] = []
        self.num_tokens = 0
        self._freed = False

    @property
    def num_blocks(self) -> int:
        return len(self.block_ids)

    @property
    def capacity(self) -> int:
        return len(self.block_ids) * self.block_size

    @property
    def is_freed(self) -> bool:
        return self._freed

    def _pages_for(self, n_tokens: int) -> int:
        return -(-n_tokens // self.block_size)

    def blocks_needed_for(self, n_new_tokens: int) -> int:
        if n_new_tokens < 0:
            raise ValueError(f"n_new_tokens must be non-negative, got {n_new_tokens}")
        return max(0, self._pages_for(self.num_tokens + n_new_tokens) - len(self.block_ids))

    def append(self, n_new_tokens: int) -> None:
        """Grow by ``n_new_tokens``, taking pages from the allocator as needed."""
        self._live()
        if n_new_tokens < 0:
            raise ValueError(f"n_new_tokens must be non-negative, got {n_new_tokens}")
        need = self.blocks_needed_for(n_new_tokens)
        if need:
            self.block_ids.extend(self._alloc.allocate(need))
        self.num_tokens += n_new_tokens

    def slot_for(self, position: int) -> int:
        self._live()
        if not 0 <= position < self.num_tokens:
            raise IndexError(f"position {position} outside sequence of length {self.num_tokens}")
        page, off = divmod(position, self.block_size)
        return self.block_ids[page] * self.block_size + off

    def slots_for_range(self, start: int, count: int) -> list[int]:
        return [self.slot_for(p) for p in range(start, start + count)]

    def slots_for_new_tokens(self, n_new_tokens: int) -> list[int]:
        return self.slots_for_range(self.num_tokens - n_new_tokens, n_new_tokens)

    def last_page_len(self) -> int:
        self._live()
        if self.num_tokens == 0:
            raise ValueError("last_page_len is undefined for an empty sequence")
        return self.num_tokens % self.block_size or self.block_size

    def free(self) -> None:
        """Release every page reference; calling it again is a no-op."""
        if self._freed:
            return
        if self.block_ids:
            self._alloc.free(self.block_ids)
        self.block_ids = []
        self.num_tokens = 0
        self._freed = True

    def _live(self) -> None:
        if self._freed:
            raise RuntimeError(
                f"SequenceBlocks(seq_id={self.seq_id}) was freed; its pages may belong "
                "to another sequence now"
            )

    def __len__(self) -> int:
        return self.num_tokens

    def __repr__(self) -> str:
        if self._freed:
            return f"SequenceBlocks(seq_id={self.seq_id}, freed)"
        lpl = self.last_page_len() if self.num_tokens else "-"
        return (f"SequenceBlocks(seq_id={self.seq_id}, {self.num_tokens} tokens, "
                f"blocks={self.block_ids}, last_page_len={lpl})")


def build_csr(seqs: Sequence[SequenceBlocks]) -> tuple[list[int], list[int], list[int]]:
    """(kv_indptr, kv_indices, kv_last_page_len) over ``seqs`` in order."""
    indptr, indices, last = [0], [], []
    for s in seqs:
        indices.extend(s.block_ids)
        indptr.append(len(indices))
        last.append(s.last_page_len())
    return indptr, indices, last
