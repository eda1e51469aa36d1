"""
Property tests of the host-side path (no GPU): the array-based
build_batch_meta agrees field by field with an independent per-sequence
construction (tests/_util.make_meta, the reference's own test-side assembly,
tests/test_paged_torch.py:66-103) on random ragged batches over fragmented
pools, and the decode planner covers every page exactly once, split or
packed, for any lengths and partition size.
"""

from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from llm_serving_layer_amd import (BlockAllocator, ScheduledSeq, SequenceBlocks, _native,
                                   build_batch_meta)

from ._util import make_meta, plan_decode

SETTINGS = settings(max_examples=60, deadline=None,
                    suppress_health_check=[HealthCheck.too_slow])


@st.composite
def batches(draw):
    block_size = draw(st.sampled_from([1, 4, 16, 32]))
    n = draw(st.integers(1, 24))
    hist = draw(st.lists(st.integers(0, 300), min_size=n, max_size=n))
    new = draw(st.lists(st.integers(1, 40), min_size=n, max_size=n))
    decode_only = draw(st.booleans())
    if decode_only:
        new = [1] * n
    seed = draw(st.integers(0, 2**16))
    return block_size, hist, new, seed


@SETTINGS
@given(batches())
def test_array_assembly_equals_per_sequence_assembly(batch):
    block_size, hist, new, seed = batch
    need = sum(-(-(h + q) // block_size) for h, q in zip(hist, new))
    nb = need + 8
    alloc = BlockAllocator(nb, block_size)
    rng = np.random.default_rng(seed)
    alloc.allocate(nb)
    alloc.free([int(b) for b in rng.permutation(nb)])   # scattered free list
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(hist))]
    for s, h in zip(seqs, hist):
        if h:
            s.append(h)
    for s, q in zip(seqs, new):
        s.append(q)
    got = build_batch_meta([ScheduledSeq(s, [0] * q) for s, q in zip(seqs, new)],
                           device="cpu", page_size=block_size)
    want = make_meta(seqs, new, block_size)
    for f in dataclasses.fields(want):
        if f.name == "host":   # only the assembler keeps host arrays
            continue
        a, b = getattr(got, f.name), getattr(want, f.name)
        if isinstance(b, torch.Tensor):
            assert a.dtype == b.dtype and torch.equal(a, b), f.name
        else:
            assert a == b, f.name
    mirror = got.host_arrays()
    assert want.host_arrays() is None and mirror is not None
    for name, arr in mirror.items():
        assert arr.tolist() == getattr(want, name).tolist(), name


@SETTINGS
@given(st.lists(st.integers(1, 3000), min_size=1, max_size=200), st.integers(1, 64),
       st.integers(1, 1024))
def test_decode_plan_covers_every_page_exactly_once(kv_lens, part_pages, workgroups):
    indptr, bins, n_work, n_slots = plan_decode(kv_lens, part_pages, workgroups)
    covered = np.zeros(int(indptr[-1]), np.int32)
    slots = []
    for items in bins:
        for it in items:
            seq, first = it["seq"], it["tok0"] // 16
            assert 1 <= it["np"] <= part_pages + 3 and it["kv"] == kv_lens[seq]
            ids = [pid for pid, _, _ in it["pages"]]
            assert ids == list(range(indptr[seq] + first, indptr[seq] + first + it["np"]))
            covered[indptr[seq] + first:indptr[seq] + first + it["np"]] += 1
            if it["nparts"] > 1:
                slots.append(it["slot"])
            else:
                assert it["slot"] == -1
    assert sorted(slots) == list(range(n_slots))
    assert (covered == 1).all()
    assert 1 <= n_work <= max(workgroups, 2)
