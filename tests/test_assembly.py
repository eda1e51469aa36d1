"""
Batch assembly and BatchMeta.validate().

Restates the exact-integer expectations of the reference's
tests/test_batch_assembly.py (:58-133 every field of single, multi and mixed
steps; :345-384 validate() rejections and their message fragments;
:512-548 dtypes), against this package's BatchMeta / build_batch_meta.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

from llm_serving_layer_amd import (BlockAllocator, ScheduledSeq, SequenceBlocks,
                                   build_batch_meta, build_token_tensor)

PAGE = 16
DEV = torch.device("cpu")


def ints(t):
    return [int(x) for x in t]


def grow(seq, n, first=0):
    seq.append(n)
    return ScheduledSeq(blocks=seq, new_token_ids=list(range(first, first + n)))


def test_single_decode_every_field():
    a = BlockAllocator(256, PAGE)
    s = SequenceBlocks(a)
    s.append(20)
    sc = grow(s, 1, first=777)
    meta = build_batch_meta([sc], DEV, PAGE)
    assert ints(build_token_tensor([sc], DEV)) == [777]
    assert meta.n_seqs == 1 and meta.n_tokens == 1
    assert ints(meta.query_lens) == [1]
    assert ints(meta.cu_query_lens) == [0, 1]
    assert ints(meta.kv_lens) == [21]
    assert ints(meta.positions) == [20]
    assert ints(meta.last_token_ix) == [0]
    assert ints(meta.batch_indices) == [0]
    assert ints(meta.kv_indptr) == [0, 2]
    assert ints(meta.kv_indices) == s.block_ids
    assert ints(meta.kv_last_page_len) == [5]
    assert ints(meta.slot_mapping) == [s.block_ids[1] * PAGE + 4]
    assert meta.page_size == PAGE and meta.is_prefill is False


def test_mixed_prefill_and_decode():
    a = BlockAllocator(256, PAGE)
    x, y, z = (SequenceBlocks(a, seq_id=i) for i in range(3))
    y.append(30)
    z.append(5)
    meta = build_batch_meta([grow(x, 8), grow(y, 1), grow(z, 1)], DEV, PAGE)
    assert ints(meta.query_lens) == [8, 1, 1]
    assert ints(meta.cu_query_lens) == [0, 8, 9, 10]
    assert ints(meta.last_token_ix) == [7, 8, 9]
    assert ints(meta.batch_indices) == [0] * 8 + [1, 2]
    assert ints(meta.kv_lens) == [8, 31, 6]
    assert ints(meta.positions) == list(range(8)) + [30, 5]
    assert meta.is_prefill is True and meta.n_tokens == 10


def test_chunked_prefill_positions_are_absolute():
    a = BlockAllocator(256, PAGE)
    s = SequenceBlocks(a)
    build_batch_meta([grow(s, 32)], DEV, PAGE)
    meta = build_batch_meta([grow(s, 8)], DEV, PAGE)
    assert ints(meta.positions) == list(range(32, 40))
    assert ints(meta.slot_mapping) == [s.slot_for(p) for p in range(32, 40)]


def test_fragmented_slots_follow_the_block_table():
    a = BlockAllocator(8, PAGE)
    a.allocate(8)
    a.free([6, 1, 4])
    s = SequenceBlocks(a)
    meta = build_batch_meta([grow(s, 40)], DEV, PAGE)
    want = [[6, 1, 4][p // PAGE] * PAGE + p % PAGE for p in range(40)]
    assert ints(meta.slot_mapping) == want
    assert ints(meta.kv_last_page_len) == [8]


def _one_seq_meta():
    a = BlockAllocator(256, PAGE)
    return build_batch_meta([grow(SequenceBlocks(a), 4)], DEV, PAGE)


def test_validate_rejects_zeroed_last_page_len():
    a = BlockAllocator(256, PAGE)
    meta = build_batch_meta([grow(SequenceBlocks(a), 32)], DEV, PAGE)
    assert ints(meta.kv_last_page_len) == [PAGE]
    bad = dataclasses.replace(meta, kv_last_page_len=torch.tensor([0], dtype=torch.int32))
    with pytest.raises(AssertionError, match="kv_last_page_len"):
        bad.validate()


def test_validate_rejects_bad_cu_query_lens():
    bad = dataclasses.replace(_one_seq_meta(),
                              cu_query_lens=torch.tensor([0, 99], dtype=torch.int32))
    with pytest.raises(AssertionError):
        bad.validate()


def test_validate_rejects_page_count_mismatch():
    bad = dataclasses.replace(_one_seq_meta(), kv_lens=torch.tensor([999], dtype=torch.int32))
    with pytest.raises(AssertionError, match="pages allocated"):
        bad.validate()


def test_validate_rejects_short_batch_indices():
    bad = dataclasses.replace(_one_seq_meta(),
                              batch_indices=torch.tensor([0], dtype=torch.int32))
    with pytest.raises(AssertionError, match="batch_indices"):
        bad.validate()


def test_assembly_rejections():
    a = BlockAllocator(256, PAGE)
    s = SequenceBlocks(a)
    s.append(2)
    with pytest.raises(ValueError, match="blocks.append"):
        build_batch_meta([ScheduledSeq(s, [1, 2, 3, 4, 5])], DEV, PAGE)
    with pytest.raises(ValueError, match="contributes 0 tokens"):
        build_batch_meta([ScheduledSeq(s, [])], DEV, PAGE)
    with pytest.raises(ValueError, match="empty"):
        build_batch_meta([], DEV, PAGE)
    small = SequenceBlocks(BlockAllocator(8, 8))
    with pytest.raises(ValueError, match="page_size"):
        build_batch_meta([grow(small, 4)], DEV, PAGE)
    s.free()
    with pytest.raises(ValueError, match="freed"):
        build_batch_meta([ScheduledSeq(s, [1])], DEV, PAGE)


def test_page_size_one():
    a = BlockAllocator(64, 1)
    s = SequenceBlocks(a)
    meta = build_batch_meta([grow(s, 5)], DEV, 1)
    assert ints(meta.kv_last_page_len) == [1]
    assert ints(meta.slot_mapping) == s.block_ids


def test_large_ragged_batch_validates():
    a = BlockAllocator(1024, PAGE)
    scheds = []
    for i in range(24):
        s = SequenceBlocks(a, seq_id=i)
        s.append(i * 3)
        scheds.append(grow(s, 1 if i % 3 else 7))
    meta = build_batch_meta(scheds, DEV, PAGE)
    cu = ints(meta.cu_query_lens)
    assert ints(meta.last_token_ix) == [cu[i + 1] - 1 for i in range(24)]
    assert cu[-1] == meta.n_tokens


def test_dtypes_match_the_contract():
    a = BlockAllocator(256, PAGE)
    meta = build_batch_meta([grow(SequenceBlocks(a, seq_id=i), 4 + i) for i in range(3)],
                            DEV, PAGE)
    for name in ("query_lens", "cu_query_lens", "kv_lens", "last_token_ix", "kv_indptr",
                 "kv_indices", "kv_last_page_len", "batch_indices", "slot_mapping"):
        assert getattr(meta, name).dtype == torch.int32, name
    assert meta.positions.dtype == torch.int64
    m64 = build_batch_meta([grow(SequenceBlocks(a), 4)], DEV, PAGE, dtype_index=torch.int64)
    assert m64.kv_indices.dtype == torch.int64 and m64.positions.dtype == torch.int64


def test_host_mirror_matches_the_fields_and_dies_with_a_replaced_field():
    """build_batch_meta keeps its host arrays on the meta (so a backend can
    plan without reading the device back); they equal the fields, and a meta
    rebuilt with dataclasses.replace no longer vouches for them."""
    a = BlockAllocator(64, 16)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(3)]
    for s, n in zip(seqs, [5, 17, 40]):
        s.append(n)
    meta = build_batch_meta([ScheduledSeq(s, [0] * q) for s, q in zip(seqs, [5, 1, 3])],
                            "cpu", 16)
    h = meta.host_arrays()
    assert h is not None
    for name in ("query_lens", "cu_query_lens", "kv_lens", "kv_indptr", "kv_indices",
                 "kv_last_page_len", "slot_mapping"):
        assert getattr(meta, name).tolist() == h[name].tolist(), name
    assert dataclasses.replace(meta, is_prefill=True).host_arrays() is h
    moved = dataclasses.replace(meta, slot_mapping=meta.slot_mapping.clone())
    assert moved.host_arrays() is None
    assert dataclasses.replace(meta, host=None).host_arrays() is None
