"""
DecodeStepper against the reference's per-step path, on the host: each
step grows every sequence by one token (scheduler.py:749, ``append(1)`` per
sequence) and assembles the batch (``build_batch_meta``, batch.py:190-318).
The stepper must leave the same block tables (the same page ids from the
same FIFO allocator) and produce the same BatchMeta, field for field, over
steps that cross page boundaries; its host mirror must describe its own
fields; and it must refuse what build_batch_meta refuses.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import (AllocationError, BlockAllocator, ScheduledSeq,
                                   SequenceBlocks, build_batch_meta)
from llm_serving_layer_amd.contract import MIRRORED
from llm_serving_layer_amd.stepping import DecodeStepper

FIELDS = ("query_lens", "cu_query_lens", "kv_lens", "positions", "kv_indptr", "kv_indices",
          "kv_last_page_len", "batch_indices", "slot_mapping", "last_token_ix")


def _twin_batches(lens, nb, seed, bs=16):
    """Two identical allocators and sequence sets (shuffled free lists)."""
    out = []
    for _ in range(2):
        a = BlockAllocator(nb, bs)
        a.allocate(nb)
        a.free(random.Random(seed).sample(range(nb), nb))
        seqs = []
        for i, n in enumerate(lens):
            s = SequenceBlocks(a, seq_id=i)
            s.append(n)
            seqs.append(s)
        out.append((a, seqs))
    return out


@pytest.mark.parametrize("bs", [16, 4, 1])
def test_stepper_equals_append_then_build_batch_meta(bs):
    rng = random.Random(bs)
    lens = [rng.randint(1, 90) for _ in range(37)] + [bs, 2 * bs, bs - 1 if bs > 1 else 1]
    nb = sum(-(-n // bs) for n in lens) + 40 * 60 // bs + 64
    (a_ref, ref), (a_new, new) = _twin_batches(lens, nb, 11, bs)
    stepper = DecodeStepper(new, "cpu", bs)
    for step in range(40):                          # every sequence crosses pages
        for s in ref:
            s.append(1)
        want = build_batch_meta([ScheduledSeq(s, [0]) for s in ref], "cpu", bs)
        got = stepper.step()
        for name in FIELDS:
            w, g = getattr(want, name), getattr(got, name)
            assert g.dtype == w.dtype and torch.equal(g, w), f"step {step} {name}"
        assert got.page_size == bs and got.is_prefill is False
        assert [s.block_ids for s in new] == [s.block_ids for s in ref], f"step {step}"
        assert [s.num_tokens for s in new] == [s.num_tokens for s in ref]
        mirror = got.host_arrays()
        assert mirror is not None
        for name in MIRRORED:
            assert np.array_equal(mirror[name], getattr(got, name).numpy()), name
        got.validate()
    assert a_new.num_free == a_ref.num_free
    a_new.check_invariants()


def test_stepper_allocation_failure_changes_nothing():
    """All or nothing, like the allocator: when the pages a step needs are
    not free, the step raises and no sequence has grown."""
    a = BlockAllocator(4, 16)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(2)]
    seqs[0].append(16)
    seqs[1].append(32)
    a.allocate(a.num_free - 1)                       # one page left, two needed
    st = DecodeStepper(seqs, "cpu", 16)
    with pytest.raises(AllocationError):
        st.step()
    assert [s.num_tokens for s in seqs] == [16, 32]
    assert [len(s.block_ids) for s in seqs] == [1, 2] and a.num_free == 1


def test_stepper_uses_spare_capacity_before_allocating():
    """A sequence whose table already holds a page past its tokens grows
    into it, as append(1) does (blocks_needed_for)."""
    a = BlockAllocator(8, 16)
    s = SequenceBlocks(a, seq_id=0)
    s.append(16)
    s.block_ids.extend(a.allocate(1))                 # a spare page
    st = DecodeStepper([s], "cpu", 16)
    free = a.num_free
    m = st.step()
    assert a.num_free == free and len(s.block_ids) == 2 and s.num_tokens == 17
    assert m.slot_mapping.tolist() == [s.block_ids[1] * 16]


def test_stepper_refuses_what_assembly_refuses():
    a = BlockAllocator(8, 16)
    other = BlockAllocator(8, 16)
    s = SequenceBlocks(a, seq_id=3)
    s.append(5)
    dead = SequenceBlocks(a, seq_id=4)
    dead.append(3)
    dead.free()
    with pytest.raises(ValueError, match="at least one"):
        DecodeStepper([], "cpu", 16)
    with pytest.raises(ValueError, match="has been freed"):
        DecodeStepper([s, dead], "cpu", 16)
    with pytest.raises(ValueError, match="page_size"):
        DecodeStepper([s], "cpu", 8)
    t = SequenceBlocks(other, seq_id=5)
    t.append(1)
    with pytest.raises(ValueError, match="one allocator"):
        DecodeStepper([s, t], "cpu", 16)
