"""
Host addressing: allocator, block table slot arithmetic, CSR.

Restates the behaviour pinned by the reference's tests/test_allocator.py
(FIFO order :394-425, slot arithmetic on scattered blocks :639-760,
last_page_len sweep and exact multiples :762-825, build_csr :937-1009).
"""

from __future__ import annotations

import random

import pytest

from llm_serving_layer_amd import AllocationError, BlockAllocator, SequenceBlocks, build_csr


def test_free_list_is_fifo():
    a = BlockAllocator(8, 16)
    got = a.allocate(8)
    assert got == list(range(8))
    a.free([5, 2, 7])
    assert a.allocate(3) == [5, 2, 7], "freed blocks must come back in free order"


def test_allocate_is_all_or_nothing_and_double_free_raises():
    a = BlockAllocator(4, 16)
    a.allocate(3)
    with pytest.raises(AllocationError):
        a.allocate(2)
    assert a.num_free == 1
    b = a.allocate(1)
    a.free(b)
    with pytest.raises(AllocationError, match="Double free"):
        a.free(b)
    a.check_invariants()


def test_watermark_applies_to_admission_only():
    a = BlockAllocator(10, 16, watermark_blocks=3)
    assert a.can_allocate(7) and not a.can_allocate(8)
    assert len(a.allocate(9)) == 9  # a running sequence may dip into the reserve


def test_incref_and_shared_free():
    a = BlockAllocator(4, 16)
    b = a.allocate(1)
    a.incref(b)
    a.free(b)
    assert a.refcount(b[0]) == 1 and a.num_free == 3
    a.free(b)
    assert a.num_free == 4
    with pytest.raises(AllocationError, match="refcount is 0"):
        a.incref(b)


def test_check_invariants_detects_corruption():
    """The reference's allocator tests corrupt the private state directly and
    match these fragments (tests/test_allocator.py:300-366)."""
    a = BlockAllocator(4, 16)
    a.allocate(2)
    a._refcount[0] = 0  # leaked: refcount 0 but not free
    with pytest.raises(AssertionError, match="leaked"):
        a.check_invariants()
    b = BlockAllocator(4, 16)
    (x,) = b.allocate(1)
    b._free.append(x)  # live AND free
    with pytest.raises(AssertionError, match="second owner"):
        b.check_invariants()
    c = BlockAllocator(4, 16)
    (y,) = c.allocate(1)
    c.free([y])
    with pytest.raises(AllocationError, match="refcount is 0"):
        c.incref([y])


def test_slot_for_scattered_blocks():
    a = BlockAllocator(32, 16)
    a.allocate(32)
    a.free([21, 4, 13])
    s = SequenceBlocks(a)
    s.append(40)
    assert s.block_ids == [21, 4, 13]
    for p in range(40):
        assert s.slot_for(p) == [21, 4, 13][p // 16] * 16 + p % 16
    with pytest.raises(IndexError):
        s.slot_for(40)


@pytest.mark.parametrize("n", range(1, 41))
def test_last_page_len_sweep(n):
    s = SequenceBlocks(BlockAllocator(8, 16))
    s.append(n)
    assert s.num_blocks == -(-n // 16)
    assert s.last_page_len() == (n % 16 or 16)
    assert 1 <= s.last_page_len() <= 16


def test_incremental_appends_match_bulk():
    a1, a2 = BlockAllocator(16, 16), BlockAllocator(16, 16)
    s1, s2 = SequenceBlocks(a1), SequenceBlocks(a2)
    s1.append(37)
    for _ in range(37):
        s2.append(1)
    assert s1.block_ids == s2.block_ids and s1.last_page_len() == s2.last_page_len()
    assert s2.slots_for_new_tokens(3) == [s2.slot_for(p) for p in (34, 35, 36)]


def test_freed_sequence_refuses_use():
    s = SequenceBlocks(BlockAllocator(4, 16))
    s.append(3)
    s.free()
    s.free()  # idempotent
    for op in (lambda: s.slot_for(0), lambda: s.append(1), s.last_page_len):
        with pytest.raises(RuntimeError, match="freed"):
            op()


def test_build_csr_round_trip():
    a = BlockAllocator(64, 16)
    seqs = []
    for i, n in enumerate([1, 16, 17, 40, 33]):
        s = SequenceBlocks(a, seq_id=i)
        s.append(n)
        seqs.append(s)
    indptr, indices, last = build_csr(seqs)
    assert indptr[0] == 0 and indptr[-1] == len(indices)
    for i, s in enumerate(seqs):
        assert indices[indptr[i]:indptr[i + 1]] == s.block_ids
        assert last[i] == s.last_page_len()
    assert len(set(indices)) == len(indices), "pages shared across sequences"


def test_randomised_lifecycle_preserves_invariants():
    rng = random.Random(7)
    a = BlockAllocator(64, 4)
    live: list[SequenceBlocks] = []
    for step in range(500):
        if live and rng.random() < 0.3:
            live.pop(rng.randrange(len(live))).free()
        else:
            s = live[rng.randrange(len(live))] if live and rng.random() < 0.5 else None
            if s is None:
                s = SequenceBlocks(a, seq_id=step)
                live.append(s)
            n = rng.randint(1, 9)
            if a.num_free >= s.blocks_needed_for(n):
                s.append(n)
        a.check_invariants()
    used = sum(s.num_blocks for s in live)
    assert a.num_used == used
