"""
The no-allocation decode entry point (pkv_attend_decode_noalloc) against
the workspace entry point (pkv_attend_decode), through the C ABI: the same
kernels, so the outputs (and, with the append fused in, the pools) must be
bitwise equal. Two calls in a row, the second with a smaller batch, so the
shared device array is reused with the first call's contents still in it.
"""

from __future__ import annotations

import ctypes as C
import gc

import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, SequenceBlocks, _native
from llm_serving_layer_amd.backend import MI355XBackend, _current_stream

from ._util import grow_and_assemble, lognormal_lengths

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _batch(lens, nb, seed, fuse):
    """Two identical backends (pools, plans) over one decode batch."""
    pair = []
    for _ in range(2):
        bk = MI355XBackend(1, nb, 16, 8, 32, 64, device=DEV, fuse_append=False)
        g = torch.Generator(device=DEV).manual_seed(seed)
        bk._pool.copy_(torch.randn(bk._pool.shape, generator=g, device=DEV).half())
        pair.append(bk)
    a = BlockAllocator(nb, 16)
    a.allocate(nb)
    a.free(torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).tolist())
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(len(lens))]
    for s, n in zip(seqs, lens):
        s.append(n - 1)
    meta = grow_and_assemble(seqs, [1] * len(lens), 16, device=DEV)
    plans = [bk._ensure_planned(meta) for bk in pair]
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    n = len(lens)
    q = torch.randn(n, 32, 64, generator=g, device=DEV).half()
    k = torch.randn(n, 8, 64, generator=g, device=DEV).half() if fuse else None
    v = torch.randn(n, 8, 64, generator=g, device=DEV).half() if fuse else None
    return pair, plans, q, k, v


def _call(lib, fn_name, bk, p, q, out, k, v, with_workspace):
    args = [q.data_ptr(), out.data_ptr(), bk._k_pool[0].data_ptr(), bk._v_pool[0].data_ptr(),
            bk.num_blocks, p.indptr.data_ptr(), p.indices.data_ptr(), p.kv_lens.data_ptr(),
            p.n_seqs, 32, 8, 64, 16, 0.125, _native.DTYPE_F16, p.plan.data_ptr(), p.n_work,
            p.n_slots, p.stride, k.data_ptr() if k is not None else None,
            v.data_ptr() if v is not None else None,
            p.slots.data_ptr() if k is not None else None]
    if with_workspace:
        ws = bk._workspace
        args += [ws.data_ptr() if ws.numel() else None, ws.numel()]
    args += [bk._status.data_ptr(), _current_stream(bk.device)]
    return getattr(lib, fn_name)(*args)


@pytest.mark.parametrize("fuse", [False, True])
def test_noalloc_decode_equals_workspace_decode_twice(fuse):
    lib = _native.load()
    cases = [lognormal_lengths(256, 256, 0.8, 2048, 20260731),        # split sequences
             [1, 17, 300, 33, 1200, 64, 5, 161]]                      # a smaller second call
    for ci, lens in enumerate(cases):
        print(f"noalloc vs workspace decode, call {ci}, {len(lens)} seqs, fuse={fuse}",
              flush=True)
        nb = 2 * sum(-(-n // 16) for n in lens) + 16
        (ref_bk, new_bk), (p_ref, p_new), q, k, v = _batch(lens, nb, 11 + ci, fuse)
        assert p_ref.n_slots > 0, "the case must split sequences (use the workspace)"
        need = lib.pkv_decode_workspace_bytes(p_new.n_seqs, p_new.n_slots, 32, 8, 64)
        assert 0 < need <= _native.DECODE_SCRATCH_BYTES
        out_ref = torch.empty_like(q)
        out_new = torch.full_like(q, float("nan"))
        _native.check(_call(lib, "pkv_attend_decode", ref_bk, p_ref, q, out_ref, k, v, True),
                      "pkv_attend_decode")
        _native.check(_call(lib, "pkv_attend_decode_noalloc", new_bk, p_new, q, out_new, k, v,
                            False), "pkv_attend_decode_noalloc")
        torch.cuda.synchronize()
        ref_bk.check_device_errors()
        new_bk.check_device_errors()
        assert torch.equal(out_new, out_ref), f"call {ci}: outputs differ"
        assert torch.equal(new_bk._pool, ref_bk._pool), f"call {ci}: pools differ"


def test_noalloc_rejects_a_plan_beyond_its_array():
    """A split-K plan needing more than PKV_DECODE_SCRATCH_BYTES is refused on
    the host, before any launch."""
    print("noalloc capacity limit", flush=True)
    lib = _native.load()
    n_slots = 100_000
    need = lib.pkv_decode_workspace_bytes(1, n_slots, 32, 8, 64)
    assert need > _native.DECODE_SCRATCH_BYTES
    dummy = torch.zeros(64, dtype=torch.int32, device=DEV)
    rc = lib.pkv_attend_decode_noalloc(
        dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 1,
        dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), 1, 32, 8, 64, 16, 0.125,
        _native.DTYPE_F16, dummy.data_ptr(), 2, n_slots, 4, None, None, None,
        dummy.data_ptr(), _current_stream(torch.device(DEV)))
    assert rc == _native.ERR_CAPACITY
    assert b"at most" in lib.pkv_last_error()
    torch.cuda.synchronize()
    assert int(dummy.abs().sum()) == 0, "nothing may have run"


def test_noalloc_allocates_nothing_and_replays_from_a_graph():
    """What the entry point is for: after a first call on the device (which
    looks up the array's address), a call changes neither torch's allocated
    bytes nor the device's free memory, and the call captured into a HIP
    graph replays (three times, with eager work between) to the bits of an
    eager call."""
    print("noalloc: no allocation, graph capture and replay", flush=True)
    lib = _native.load()
    lens = lognormal_lengths(256, 256, 0.8, 2048, 20260731)
    nb = 2 * sum(-(-n // 16) for n in lens) + 16
    (_, bk), (_, p), q, k, v = _batch(lens, nb, 21, True)
    assert p.n_slots > 0
    eager = torch.empty_like(q)
    _native.check(_call(lib, "pkv_attend_decode_noalloc", bk, p, q, eager, k, v, False),
                  "pkv_attend_decode_noalloc")          # warm-up: the address lookup
    torch.cuda.synchronize()
    again = torch.full_like(q, float("nan"))
    # Torch's allocator counts every allocation it makes (cumulatively), and
    # an allocation outside it (hipMalloc) would take device memory: neither
    # may move. (Frees of earlier tensors whose release the allocator
    # deferred may still land inside the window and only raise free memory.)
    gc.collect()
    gc.disable()
    try:
        torch.cuda.synchronize()
        made0 = torch.cuda.memory_stats(DEV)["allocation.all.allocated"]
        free0, _ = torch.cuda.mem_get_info(DEV)
        _native.check(_call(lib, "pkv_attend_decode_noalloc", bk, p, q, again, k, v, False),
                      "pkv_attend_decode_noalloc")
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info(DEV)
        made1 = torch.cuda.memory_stats(DEV)["allocation.all.allocated"]
    finally:
        gc.enable()
    assert made1 == made0, f"torch made {made1 - made0} allocations during the call"
    assert free1 >= free0, f"device free memory fell by {free0 - free1} bytes"
    assert torch.equal(again, eager)
    replayed = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _native.check(_call(lib, "pkv_attend_decode_noalloc", bk, p, q, replayed, k, v, False),
                      "pkv_attend_decode_noalloc (captured)")
    for rep in range(3):
        replayed.fill_(float("nan"))
        torch.randn(1 << 20, device=DEV).sum().item()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        bk.check_device_errors()
        assert torch.equal(replayed, eager), f"replay {rep} differs from the eager call"
