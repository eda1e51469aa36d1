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

from ._util import expected_cut, plan_decode

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


def test_integration_stub_matches_the_binding_table():
    """The ctypes stub the integration guide gives a maintainer to copy binds
    the same functions with the same argument lists as the package, and
    checks the library's current ABI version."""
    text = (HEADER.parents[1] / "INTEGRATION.md").read_text()
    stub = text[text.index("SIG = {"):text.index("\n}", text.index("SIG = {"))]
    entries = re.findall(r'"(pkv_\w+)":\s*\(C\.(\w+),\s*\[([^\]]*)\]', stub)
    assert {name for name, _, _ in entries} == set(_native.SIGNATURES)
    kinds = {"P": C.c_void_p, "I32": C.c_int32, "I64": C.c_int64, "F32": C.c_float}
    for name, res, args in entries:
        assert getattr(C, res) is _native.SIGNATURES[name][0], name
        got = [kinds[a.strip()] for a in args.split(",") if a.strip()]
        assert got == list(_native.SIGNATURES[name][1]), name
    assert f"pkv_abi_version() == {_native.ABI_VERSION}" in text


def _role(it):
    """0: a cut sequence's piece before its last, 1: a whole sequence,
    2: a cut sequence's last piece (it merges)."""
    return 1 if it["slot"] < 0 else 2 if it["last"] else 0


@pytest.mark.parametrize("part_pages", [1, 3, 8, 10, 16, 64])
@pytest.mark.parametrize("workgroups", [1, 96, 512])
def test_decode_plan_covers_every_page_once(part_pages, workgroups):
    """Every page of every sequence is in exactly one piece of one bin, with
    its id and live row count; pieces of a sequence are consecutive, of
    part_pages pages with the remainder last (a remainder below 4 pages
    joins the piece before it); in a bin, pieces of cut
    sequences before their last come first and last pieces last; the partial
    slots of cut sequences are dense and unique, so no two pieces share one,
    and every (sequence, head) arrival counter index stays below
    n_seqs * n_kv_heads."""
    rng = random.Random(part_pages * 1000 + workgroups)
    kv_lens = [rng.randint(1, 2048) for _ in range(300)] + [16, 64, 65, 1]
    ids = np.array(rng.sample(range(100000), sum(-(-k // 16) for k in kv_lens)), np.int32)
    indptr, bins, n_work, n_slots = plan_decode(kv_lens, part_pages, workgroups,
                                                indices=ids, num_blocks=100000)
    n_items = sum(len(b) for b in bins)
    assert n_work == 2 * len(bins) and len(bins) == min(max(workgroups // 2, 1), n_items)
    npages = np.diff(indptr)
    covered = [np.zeros(k, int) for k in npages]
    by_seq = {}
    slots = []
    for items in bins:
        roles = [_role(it) for it in items]
        assert roles == sorted(roles), "cut pieces first, whole sequences, last pieces at the end"
        for it in items:
            seq, first = it["seq"], it["tok0"] // 16
            assert 0 <= seq < len(kv_lens) and it["kv"] == kv_lens[seq] and it["tok0"] % 16 == 0
            k = len(expected_cut(int(npages[seq]), part_pages))
            assert it["nparts"] == k and 1 <= it["np"] <= part_pages + 3
            assert it["last"] == (first + it["np"] == npages[seq])
            for t, (pid, live, bad) in enumerate(it["pages"]):
                pg = first + t
                assert not bad and pid == ids[indptr[seq] + pg]
                assert live == (kv_lens[seq] - 16 * pg if pg == npages[seq] - 1 else 16)
                covered[seq][pg] += 1
            by_seq.setdefault(seq, []).append((first, it["np"], it["slot"], it["slot0"]))
            if k == 1:
                assert it["slot"] == -1 and it["slot0"] == -1
            else:
                slots.append(it["slot"])
    assert all((c == 1).all() for c in covered)
    assert sorted(slots) == list(range(n_slots)), "partial slots must be dense and unique"
    for seq, ps_ in by_seq.items():
        ps_.sort()
        sz = [n for _, n, _, _ in ps_]
        assert sz == expected_cut(int(npages[seq]), part_pages), "the planner's cut"
        if len(ps_) > 1:  # slot = first slot + piece index, in page order
            assert [s - s0 for _, _, s, s0 in ps_] == list(range(len(ps_)))


@pytest.mark.parametrize("workgroups", [64, 512, 1024])
def test_decode_plan_balances_the_bins(workgroups):
    """LPT over the pieces' costs (pages, plus a merge for a cut sequence's
    last piece): no bin's cost exceeds the average by more than one piece."""
    rng = random.Random(workgroups)
    kv_lens = [max(1, min(2048, int(round(rng.lognormvariate(5.23, 0.8))))) for _ in range(256)]
    _, bins, _, _ = plan_decode(kv_lens, 10, workgroups)

    def cost(it):
        return 16 * it["np"] + 4 + (40 if _role(it) == 2 else 0)

    loads = [sum(cost(it) for it in items) for items in bins]
    assert max(loads) <= sum(loads) / len(loads) + 16 * 10 + 44


def test_decode_plan_cut_depends_only_on_the_sequence():
    """Batch invariance of the cut: a sequence's pieces (first page, size,
    piece index) are the same alone and inside any batch."""
    rng = random.Random(7)
    kv_lens = [rng.randint(1, 2048) for _ in range(64)]

    def cut_of(lens, seq):
        _, bins, _, _ = plan_decode(lens, 10, 96)
        return sorted((it["tok0"], it["np"], it["slot"] - it["slot0"] if it["slot"] >= 0 else -1)
                      for items in bins for it in items if it["seq"] == seq)

    for i in (0, 5, 63):
        assert cut_of(kv_lens, i) == cut_of([kv_lens[i]], 0)


def test_decode_plan_flags_out_of_range_pages():
    """An out-of-range kv_indices entry becomes page 0 with the bad bit set
    (the kernel reports it and never dereferences it)."""
    ids = np.array([3, -1, 7, 50], np.int32)
    _, bins, _, _ = plan_decode([64], 64, 2, indices=ids, num_blocks=10)
    pages = bins[0][0]["pages"]
    assert [(p, b) for p, _, b in pages] == [(3, False), (0, True), (7, False), (0, True)]


def test_decode_plan_rejections():
    lib = _native.load()
    indptr = np.array([0, 1], np.int32)
    ids = np.array([0], np.int32)
    out = np.empty(256, np.int32)
    nw, ns, st, need = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int64()

    def plan(kvl, last, part_pages=4, num_blocks=16, cap=256):
        rc = lib.pkv_plan_decode(ptr(indptr), ptr(ids), ptr(np.array([kvl], np.int32)),
                                 ptr(np.array([last], np.int32)), 1, 16, num_blocks, 8,
                                 part_pages, 512, ptr(out), cap, C.byref(need), C.byref(nw),
                                 C.byref(ns), C.byref(st))
        return rc

    for bad in (0, 65):
        with pytest.raises(ValueError, match="part_pages"):
            _native.check(plan(16, 16, part_pages=bad), "plan")
    with pytest.raises(ValueError, match="kv_last_page_len"):
        _native.check(plan(16, 9), "plan")
    with pytest.raises(ValueError, match="pages supplied"):
        _native.check(plan(999, 9), "plan")
    with pytest.raises(ValueError, match="num_blocks"):
        _native.check(plan(16, 16, num_blocks=(1 << 27) + 1), "plan")
    rc = plan(16, 16, cap=8)
    assert rc == _native.ERR_CAPACITY and need.value > 8
    assert plan(16, 16, cap=int(need.value)) == _native.OK
    assert lib.pkv_decode_fast_path(32, 8, 64, 16, _native.DTYPE_F16, 64) == 1
    assert lib.pkv_decode_fast_path(32, 8, 64, 16, _native.DTYPE_F16, 65) == 0


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
    bk._fast_decode = True
    bk._decode_wgs = 512     # what pkv_decode_workgroups gives on a 256-CU device
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
    bins = p.n_work // 2
    assert p.plan.numel() == bins * p.stride + 64
    assert sum(int(p.plan[b * p.stride + 1]) for b in range(bins)) == 3 + 7 + 1, "every page"
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
    seqs_planned = set()
    for b in range(d.n_work // 2):
        blk = d.plan[b * d.stride:(b + 1) * d.stride].numpy()
        seqs_planned |= {int(blk[d.stride - 8 * (i + 1)]) for i in range(int(blk[0]))}
    assert d.n_slots > 0 and seqs_planned == {0, 1}, "decode plan over the sub-batch"


def test_decode_plan_falls_back_to_larger_pieces_past_2gib_of_partials():
    """4096 sequences of 2048 tokens cut into 1-page pieces would need
    524 288 partial slots (4.4 GB, past the kernel's 32-bit buffer offsets):
    the backend re-plans that launch with pieces twice as large until the
    partials fit (4 pages: 131 072 slots, 1.1 GB)."""
    class _Reserved:   # a workspace already large enough: nothing is allocated
        def numel(self):
            return 1 << 40

        def __getitem__(self, _):
            return torch.zeros(0, dtype=torch.uint8)

    bk = _host_backend(part_pages=1)
    bk._workspace = _Reserved()
    bk._ws_zero = 0
    n, pages = 4096, 128
    indptr = np.arange(0, (n + 1) * pages, pages, dtype=np.int32)
    indices = np.arange(n * pages, dtype=np.int32) % 64
    kvl = np.full(n, pages * 16, np.int32)
    last = np.full(n, 16, np.int32)
    plan, n_work, n_slots, stride = bk._plan_decode(indptr, indices, kvl, last, n)
    assert n_slots == n * pages // 4
    need = bk._lib.pkv_decode_workspace_bytes(n, n_slots, 32, 8, 64)
    assert need < 2**31
    assert bk._lib.pkv_decode_workspace_bytes(n, n * pages // 2, 32, 8, 64) > 2**31


@pytest.mark.parametrize("n_pages, sizes", [
    (5, [5]), (17, [17]), (18, [18]), (20, [20]), (21, [17, 4]), (34, [17, 17]),
    (36, [17, 19]), (40, [17, 17, 6]), (86, [17, 17, 17, 17, 18])])
def test_decode_plan_cut_known_answers(n_pages, sizes):
    """The planner's pieces of one sequence at 17-page partitions, in page
    order: full pieces first, the remainder last, a remainder of 1..3
    pages joined to the piece before it (and at 2-page partitions, where
    half a piece is one page, no remainder is joined)."""
    _, bins, _, n_slots = plan_decode([16 * n_pages], 17, 512)
    got = sorted((it["tok0"] // 16, it["np"]) for b in bins for it in b)
    assert [n for _, n in got] == sizes == expected_cut(n_pages, 17)
    assert n_slots == (len(sizes) if len(sizes) > 1 else 0)
    _, bins, _, _ = plan_decode([16 * n_pages], 2, 512)
    got = sorted((it["tok0"] // 16, it["np"]) for b in bins for it in b)
    assert [n for _, n in got] == [2] * (n_pages // 2) + [1] * (n_pages % 2)
