"""
The C-ABI boundary without a GPU: the library loads, exports exactly what
include/pagedkv.h declares, and its host-side planners (pure CPU code) cover
every page / query row exactly once and reject inconsistent metadata with the
reference's messages (serving/backends/paged_torch.py:379-392).
"""

from __future__ import annotations

import ctypes as C
import random
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import _native
from llm_serving_layer_amd.backend import MI355XBackend

HEADER = Path(__file__).resolve().parents[1] / "include" / "pagedkv.h"


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\*]+\s+\*?\s*(pkv_\w+)\s*\(", text, re.M))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    decl = declared_symbols()
    assert decl == set(_native.SIGNATURES), "binding table and header disagree"
    for name in decl:
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.pkv_abi_version() == _native.ABI_VERSION


def plan_decode(kv_lens, part_pages, ps=16):
    n = len(kv_lens)
    npages = [-(-k // ps) for k in kv_lens]
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    kvl = np.array(kv_lens, np.int32)
    last = np.array([k % ps or ps for k in kv_lens], np.int32)
    cap = 8 * (int(indptr[-1]) + n)
    buf = np.empty(cap, np.int32)
    nw, ns = C.c_int32(), C.c_int32()
    rc = _native.load().pkv_plan_decode(ptr(indptr), ptr(kvl), ptr(last), n, ps, part_pages,
                                        ptr(buf), cap, C.byref(nw), C.byref(ns))
    _native.check(rc, "plan")
    return indptr, npages, buf[:8 * nw.value].reshape(-1, 8), ns.value


@pytest.mark.parametrize("part_pages", [1, 3, 8, 16, 64])
def test_decode_plan_covers_every_page_once(part_pages):
    """Every page of every sequence is in exactly one partition."""
    rng = random.Random(part_pages)
    kv_lens = [rng.randint(1, 2048) for _ in range(300)] + [16, 64, 65, 1]
    indptr, npages, work, n_slots = plan_decode(kv_lens, part_pages)
    covered = [[0] * p for p in npages]
    slots = []
    for seq, pbase, n, slot, kv, tok0, nparts, slot0 in work:
        first = pbase - indptr[seq]
        assert 1 <= n <= part_pages and kv == kv_lens[seq] and tok0 == first * 16
        assert nparts == -(-npages[seq] // part_pages) and first + n <= npages[seq]
        for p in range(first, first + n):
            covered[seq][p] += 1
        if nparts == 1:
            assert slot == -1 and slot0 == -1
        else:
            assert slot - slot0 == first // part_pages
            slots.append(slot)
    assert all(all(c == 1 for c in row) for row in covered)
    assert sorted(slots) == list(range(n_slots)), "partial slots must be dense and unique"
    assert list(work[:, 2]) == sorted(work[:, 2], reverse=True), "longest partitions first"


@pytest.mark.parametrize("part_pages", [1, 4, 10, 64])
def test_decode_plan_packs_consecutive_sequences_when_none_is_split(part_pages):
    """No sequence longer than a partition: the plan has no partial slots and
    each entry is a maximal run of consecutive whole sequences (at most 16,
    at most part_pages pages unless a single sequence), longest first."""
    rng = random.Random(part_pages)
    kv_lens = [rng.randint(1, 16 * part_pages) for _ in range(500)] + [16 * part_pages, 1]
    indptr, npages, work, n_slots = plan_decode(kv_lens, part_pages)
    assert n_slots == 0
    seen = []
    for seq0, pbase, pages, slot, nseq, tok0, nparts, slot0 in work:
        assert (slot, tok0, nparts, slot0) == (-1, 0, 1, -1)
        assert 1 <= nseq <= 16 and pbase == indptr[seq0]
        assert pages == indptr[seq0 + nseq] - indptr[seq0]
        assert pages <= part_pages
        nxt = seq0 + nseq
        if nxt < len(kv_lens) and nseq < 16:
            assert pages + npages[nxt] > part_pages, "pack could have taken the next sequence"
        seen.extend(range(seq0, nxt))
    assert sorted(seen) == list(range(len(kv_lens))), "every sequence in exactly one pack"
    assert list(work[:, 2]) == sorted(work[:, 2], reverse=True), "longest packs first"


def test_decode_plan_rejects_partitions_beyond_one_wave():
    lib = _native.load()
    indptr = np.array([0, 1], np.int32)
    kvl, last = np.array([16], np.int32), np.array([16], np.int32)
    out = np.empty(16, np.int32)
    nw, ns = C.c_int32(), C.c_int32()
    for bad in (0, 65):
        rc = lib.pkv_plan_decode(ptr(indptr), ptr(kvl), ptr(last), 1, 16, bad, ptr(out), 16,
                                 C.byref(nw), C.byref(ns))
        with pytest.raises(ValueError, match="part_pages"):
            _native.check(rc, "plan")
    assert lib.pkv_decode_fast_path(32, 8, 64, 16, _native.DTYPE_F16, 64) == 1
    assert lib.pkv_decode_fast_path(32, 8, 64, 16, _native.DTYPE_F16, 65) == 0


def test_decode_plan_rejects_inconsistent_metadata():
    lib = _native.load()
    indptr = np.array([0, 1], np.int32)
    out = np.empty(16, np.int32)
    nw, ns = C.c_int32(), C.c_int32()
    kvl = np.array([16], np.int32)
    last = np.array([9], np.int32)
    rc = lib.pkv_plan_decode(ptr(indptr), ptr(kvl), ptr(last), 1, 16, 4, ptr(out), 16,
                             C.byref(nw), C.byref(ns))
    with pytest.raises(ValueError, match="kv_last_page_len"):
        _native.check(rc, "plan")
    kvl[0] = 999
    rc = lib.pkv_plan_decode(ptr(indptr), ptr(kvl), ptr(last), 1, 16, 4, ptr(out), 16,
                             C.byref(nw), C.byref(ns))
    with pytest.raises(ValueError, match="pages supplied"):
        _native.check(rc, "plan")


def test_prefill_plan_covers_every_query_row_once():
    lib = _native.load()
    ql = [512, 1, 1, 77, 130]
    kv = [2048, 300, 17, 77, 400]
    n = len(ql)
    cu = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    npages = [-(-k // 16) for k in kv]
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    kvl = np.array(kv, np.int32)
    last = np.array([k % 16 or 16 for k in kv], np.int32)
    cap = 4 * (int(cu[-1]) // 64 + n + 1)
    buf = np.empty(cap, np.int32)
    nt = C.c_int32()
    rc = lib.pkv_plan_prefill(ptr(cu), ptr(indptr), ptr(kvl), ptr(last), n, 16, 64, ptr(buf),
                              cap, C.byref(nt))
    _native.check(rc, "plan")
    tiles = buf[:4 * nt.value].reshape(-1, 4)
    seen = [[0] * q for q in ql]
    for seq, q0, qn, _ in tiles:
        assert 1 <= qn <= 64
        for j in range(q0, q0 + qn):
            seen[seq][j] += 1
    assert all(all(c == 1 for c in row) for row in seen)


def test_backend_validates_before_touching_the_library():
    with pytest.raises(ValueError, match="divisible"):
        MI355XBackend(1, 8, 16, 3, 4, 8)
    with pytest.raises(ValueError, match="num_blocks must be positive"):
        MI355XBackend(1, 0, 16, 2, 4, 8)
    with pytest.raises(ValueError, match="supports"):
        MI355XBackend(1, 8, 16, 2, 4, 8, dtype=torch.float64)
    with pytest.raises(ValueError, match="GPU device"):
        MI355XBackend(1, 8, 16, 2, 4, 8, device="cpu")
    with pytest.raises(ValueError, match="part_pages"):
        MI355XBackend(1, 8, 16, 2, 4, 8, part_pages=65)


def test_error_codes_map_to_reference_exception_types():
    lib = _native.load()
    rc = lib.pkv_copy_blocks(None, 0, 0, 0, 0, None, None, 1, None, None)
    with pytest.raises(ValueError):
        _native.check(rc, "copy")
    assert lib.pkv_last_error()


def _host_backend(part_pages=10):
    """The backend's host half (planning) over the real library, with CPU
    tensors standing in for device ones: exercises every host call the
    launch path makes, with the binding table's signatures."""
    bk = object.__new__(MI355XBackend)
    bk._lib = _native.load()
    bk.device = torch.device("cpu")
    bk.num_layers, bk.num_blocks, bk.block_size = 1, 64, 16
    bk.n_kv_heads, bk.n_heads, bk.head_dim = 8, 32, 64
    bk.part_pages = part_pages
    bk.q_tile = bk._prefill_tile = bk._lib.pkv_prefill_q_tile(32, 8, 64, 16, _native.DTYPE_F16)
    bk._split_mixed = True
    bk._upload = lambda a: torch.from_numpy(np.array(a))   # CPU tensors stand in
    bk._workspace = torch.zeros(0, dtype=torch.uint8)
    bk._planned, bk._slot_cache, bk._pending = None, None, None
    bk.n_plans = bk.n_runs = 0
    return bk


def test_backend_plans_decode_and_prefill_through_the_library():
    from llm_serving_layer_amd import BlockAllocator, SequenceBlocks

    from ._util import grow_and_assemble

    bk = _host_backend(part_pages=2)
    alloc = BlockAllocator(64, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(3)]
    pre = grow_and_assemble(seqs, [40, 100, 7], 16)
    p = bk._ensure_planned(pre)
    assert p.use_prefill and p.n_work > 0 and p.plan.numel() == 4 * p.n_work
    assert bk._ensure_planned(pre) is p and bk.n_plans == 1, "planned once per meta"
    dec = grow_and_assemble(seqs, [1, 1, 1], 16)
    p = bk._ensure_planned(dec)
    assert not p.use_prefill and p.fusable and p.n_slots > 0
    assert p.plan.numel() == 8 * p.n_work
    assert bk._workspace.numel() >= bk._lib.pkv_decode_workspace_bytes(
        3, p.n_slots, 32, 8, 64)


def test_mixed_batch_plans_its_decodes_for_the_decode_kernel():
    """Prefill chunks beside one-token decodes: the prefill tiles cover only
    the multi-token sequences, and the one-token sequences form a decode
    batch of their own (rows, CSR over their own pages, plan)."""
    from llm_serving_layer_amd import BlockAllocator, SequenceBlocks

    from ._util import grow_and_assemble

    bk = _host_backend(part_pages=2)
    alloc = BlockAllocator(64, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(4)]
    grow_and_assemble(seqs, [40, 100, 7, 20], 16)
    meta = grow_and_assemble(seqs, [1, 30, 1, 5], 16)
    p = bk._ensure_planned(meta)
    assert p.use_prefill and p.dec is not None
    tiles = p.plan.reshape(-1, 4).numpy()
    assert set(tiles[:, 0]) == {1, 3}, "prefill tiles must skip the one-token sequences"
    d = p.dec
    assert d.n == 2 and d.rows.tolist() == [0, 31]   # token rows of sequences 0 and 2
    assert d.kv_lens.tolist() == [41, 8]
    indptr, indices = meta.kv_indptr.tolist(), meta.kv_indices.tolist()
    want = indices[indptr[0]:indptr[1]] + indices[indptr[2]:indptr[3]]
    assert d.indices.tolist() == want and d.indptr.tolist() == [0, 3, 4]
    work = d.plan.reshape(-1, 8).numpy()
    assert d.n_slots > 0 and set(work[:, 0]) == {0, 1}, "decode plan over the sub-batch"
