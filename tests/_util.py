"""Shared test helpers: batch construction the way a scheduler does it."""

from __future__ import annotations

import numpy as np
import torch

from llm_serving_layer_amd import (BatchMeta, BlockAllocator, ScheduledSeq, SequenceBlocks,
                                   build_batch_meta, build_csr)


def make_meta(seqs: list[SequenceBlocks], query_lens: list[int], block_size: int,
              device="cpu") -> BatchMeta:
    """
    Hand-assemble a BatchMeta from grown block tables, independently of
    build_batch_meta (the reference's own tests do the same,
    tests/test_paged_torch.py:66-103), then validate it.
    """
    indptr, indices, last = build_csr(seqs)
    slots, positions, bidx = [], [], []
    for i, (s, ql) in enumerate(zip(seqs, query_lens)):
        slots.extend(s.slots_for_new_tokens(ql))
        positions.extend(range(s.num_tokens - ql, s.num_tokens))
        bidx.extend([i] * ql)
    cu = [0]
    for ql in query_lens:
        cu.append(cu[-1] + ql)

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    meta = BatchMeta(
        query_lens=i32(query_lens), cu_query_lens=i32(cu),
        kv_lens=i32([s.num_tokens for s in seqs]),
        positions=torch.tensor(positions, dtype=torch.int64, device=device),
        kv_indptr=i32(indptr), kv_indices=i32(indices), kv_last_page_len=i32(last),
        batch_indices=i32(bidx), slot_mapping=i32(slots),
        last_token_ix=i32([cu[i + 1] - 1 for i in range(len(seqs))]),
        page_size=block_size, is_prefill=any(q > 1 for q in query_lens),
    )
    meta.validate()
    return meta


def grow_and_assemble(blocks: list[SequenceBlocks], counts: list[int], block_size: int,
                      device="cpu") -> BatchMeta:
    """Grow each table by counts[i] (0 = not scheduled) and assemble for real."""
    scheds = []
    for b, n in zip(blocks, counts):
        if n == 0:
            continue
        b.append(n)
        scheds.append(ScheduledSeq(blocks=b, new_token_ids=[0] * n))
    return build_batch_meta(scheds, device=device, page_size=block_size)


def fragmented_allocator(num_blocks: int, block_size: int) -> tuple[BlockAllocator, list]:
    """
    Exhaust the pool, then free every other block: later allocations receive
    scattered, non-monotonic ids (the FIFO free list only hands out holes).
    """
    alloc = BlockAllocator(num_blocks=num_blocks, block_size=block_size)
    holders = [SequenceBlocks(alloc, seq_id=900 + i) for i in range(num_blocks)]
    for h in holders:
        h.append(block_size)
    assert alloc.num_free == 0
    for h in holders[::2]:
        h.free()
    return alloc, holders[1::2]


def lognormal_lengths(n: int, mean_len: int, sigma: float, max_seq: int, seed: int) -> list[int]:
    """The reference's length law (bench/capacity.py:196-242), lognormal branch."""
    import math
    import random

    rng = random.Random(seed)
    mu = math.log(mean_len) - sigma ** 2 / 2.0
    return [max(1, min(max_seq, int(round(rng.lognormvariate(mu, sigma))))) for _ in range(n)]


def assert_attention_close(got: torch.Tensor, want: torch.Tensor, atol=2e-3, rtol=1e-2,
                           label=""):
    """
    Parity bar for attention outputs against the fp32 reference computation:
    max |got - want| <= atol everywhere, and |got - want| / |want| <= rtol
    wherever |want| > atol / rtol (below that the absolute bound is the
    tighter one).
    """
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape, f"{label}: shape {tuple(g.shape)} != {tuple(w.shape)}"
    assert torch.isfinite(g).all(), f"{label}: non-finite output"
    d = (g - w).abs()
    max_abs = float(d.max()) if d.numel() else 0.0
    assert max_abs <= atol, f"{label}: max|delta|={max_abs:.3g} > atol {atol}"
    big = w.abs() > atol / rtol
    if bool(big.any()):
        max_rel = float((d[big] / w.abs()[big]).max())
        assert max_rel <= rtol, f"{label}: max relative error {max_rel:.3g} > rtol {rtol}"
    return max_abs


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------- decode plan

def plan_decode(kv_lens, part_pages, workgroups=512, n_kv_heads=8, ps=16, indices=None,
                num_blocks=None):
    """Run the library's host decode planner over sequences of ``kv_lens``
    (page ids default to 0, 1, 2, ... in order) and parse the plan into
    ``(indptr, bins, n_work, n_slots)``: ``bins`` a list of items in stream
    order, each a dict of its fields with ``pages``, a list of
    (id, live rows, bad) per page."""
    import ctypes as C

    from llm_serving_layer_amd import _native

    n = len(kv_lens)
    npages = [-(-k // ps) for k in kv_lens]
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    if indices is None:
        indices = np.arange(int(indptr[-1]), dtype=np.int32)
    indices = np.ascontiguousarray(indices, dtype=np.int32)
    if num_blocks is None:
        num_blocks = max(1, int(indptr[-1]))
    kvl = np.array(kv_lens, np.int32)
    last = np.array([k % ps or ps for k in kv_lens], np.int32)
    p = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    nw, ns, stride, need = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int64()
    lib = _native.load()
    cap = 64
    for _ in range(2):
        buf = np.zeros(cap, np.int32)
        rc = lib.pkv_plan_decode(p(indptr), p(indices), p(kvl), p(last), n, ps, num_blocks,
                                 n_kv_heads, part_pages, workgroups, p(buf), cap,
                                 C.byref(need), C.byref(nw), C.byref(ns), C.byref(stride))
        if rc == _native.ERR_CAPACITY and need.value > cap:
            cap = int(need.value)
            continue
        break
    _native.check(rc, "plan (decode)")
    S = stride.value
    heads_per_wg = 4 if n_kv_heads % 4 == 0 else 2 if n_kv_heads % 2 == 0 else 1
    n_bins = nw.value // (n_kv_heads // heads_per_wg)
    assert need.value == n_bins * S + 64 and not buf[n_bins * S:need.value].any()
    bins = []
    for b in range(n_bins):
        blk = buf[b * S:(b + 1) * S]
        n_items, n_pg = int(blk[0]), int(blk[1])
        words = blk[4:4 + n_pg].astype(np.int64) & 0xFFFFFFFF
        assert 4 + n_pg <= S - 8 * n_items, "words and items overlap"
        items, pos = [], 0
        for i in range(n_items):   # item i ends the block, 8 ints from its end per item
            seq, np_, tok0, kv, slot, nparts, slot0, flags = (int(x) for x in
                                                              blk[S - 8 * (i + 1):S - 8 * i])
            pages = [(int(w & ((1 << 27) - 1)), int((w >> 27) & 15) + 1, bool(w >> 31))
                     for w in words[pos:pos + np_]]
            pos += np_
            items.append(dict(seq=seq, np=np_, tok0=tok0, kv=kv, slot=slot, nparts=nparts,
                              slot0=slot0, last=bool(flags & 1), pages=pages))
        assert pos == n_pg
        bins.append(items)
    return indptr, bins, nw.value, ns.value


def meta_to_device(meta: BatchMeta, device, mirror: bool = True) -> BatchMeta:
    """
    ``meta`` with every tensor field moved to ``device``. With ``mirror``
    (the default) the result carries a host mirror of its index fields,
    built from ``meta``'s own values, exactly as ``build_batch_meta(...,
    device=...)`` leaves one: the backend then plans from the host arrays, as
    a serving loop does. With ``mirror=False`` it has none, and the backend
    reads the device tensors back to plan.
    """
    import dataclasses

    from llm_serving_layer_amd.contract import MIRRORED, HostMirror

    moved = {f.name: getattr(meta, f.name).to(device) for f in dataclasses.fields(meta)
             if isinstance(getattr(meta, f.name), torch.Tensor)}
    host = None
    if mirror:
        arrays = {k: (None if getattr(meta, k) is None
                      else getattr(meta, k).cpu().numpy().astype(np.int64)) for k in MIRRORED}
        host = HostMirror(arrays=arrays, of=tuple(moved.get(k) for k in MIRRORED))
    out = dataclasses.replace(meta, **moved, host=host)
    assert (out.host_arrays() is not None) == mirror
    return out


def expected_cut(n_pages: int, part_pages: int) -> list:
    """Piece sizes of a sequence of ``n_pages`` pages as the decode planner
    cuts it: pieces of ``part_pages`` pages, the remainder last, a remainder
    shorter than both 4 pages and half a piece joining the piece before it."""
    full, rem = divmod(n_pages, part_pages)
    if full == 0:
        return [rem]
    sizes = [part_pages] * full
    if 0 < rem < min(4, (part_pages + 1) // 2):
        sizes[-1] += rem
    elif rem:
        sizes.append(rem)
    return sizes
