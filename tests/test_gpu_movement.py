"""
GPU parity of the pure data movement (bit-exact bar): KV append, batched
copy-on-write block copies, and the preemption swap round trip.

Oracles: the numpy closed forms in oracle/naive.py and the reference tests'
known answers (tests/test_paged_torch.py:183-234, tests/test_copy_block.py:
39-82, tests/test_preemption.py:337-463).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, SequenceBlocks
from llm_serving_layer_amd.backend import MI355XBackend
from llm_serving_layer_amd.swap import KVSwapSpace, SwapSpaceFull
from oracle import (append_closed_form, copy_blocks_closed_form, gather_closed_form,
                    scatter_closed_form)

from ._util import make_meta

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def backend(num_layers=2, num_blocks=64, block_size=16, n_kv=8, n_heads=32, head_dim=64,
            dtype=torch.float16):
    return MI355XBackend(num_layers, num_blocks, block_size, n_kv, n_heads, head_dim,
                         device=DEV, dtype=dtype)


def poison(bk, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    bk._pool.copy_(torch.randn(bk._pool.shape, generator=g, device=DEV).to(bk.dtype))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("geom", [(8, 64, 16), (2, 8, 16), (2, 128, 4), (1, 4, 1)])
def test_append_bit_exact(dtype, geom):
    n_kv, d, bs = geom
    print(f"append dtype={dtype} n_kv={n_kv} d={d} bs={bs}", flush=True)
    bk = backend(num_layers=2, num_blocks=40, block_size=bs, n_kv=n_kv, n_heads=n_kv * 2,
                 head_dim=d, dtype=dtype)
    poison(bk, 1)
    a = BlockAllocator(40, bs)
    a.allocate(40)
    a.free([31, 2, 17, 9, 24, 5, 38, 11])
    seqs = []
    for i, n in enumerate([3, bs + 1, 2 * bs]):
        s = SequenceBlocks(a, seq_id=i)
        s.append(n)
        seqs.append(s)
    meta = make_meta(seqs, [3, bs + 1, 2 * bs], bs, device=DEV)
    T = meta.n_tokens
    k = torch.randn(T, n_kv, d, device=DEV).to(dtype)
    v = torch.randn(T, n_kv, d, device=DEV).to(dtype)
    before = [bk.k_pool[1].clone(), bk.v_pool[1].clone()]
    want_k = append_closed_form(bk.k_pool[0].float().cpu().numpy(), k.float().cpu().numpy(),
                                meta.slot_mapping.tolist())
    want_v = append_closed_form(bk.v_pool[0].float().cpu().numpy(), v.float().cpu().numpy(),
                                meta.slot_mapping.tolist())
    bk.append_kv(0, k, v, meta)
    torch.cuda.synchronize()
    assert np.array_equal(bk.k_pool[0].float().cpu().numpy(), want_k)
    assert np.array_equal(bk.v_pool[0].float().cpu().numpy(), want_v)
    assert torch.equal(bk.k_pool[1], before[0]) and torch.equal(bk.v_pool[1], before[1])
    snap = bk._pool.clone()
    bk.append_kv(0, k, v, meta)  # idempotent
    assert torch.equal(bk._pool, snap)
    bk.check_device_errors()


def test_append_bad_slot_is_skipped_and_reported():
    print("append with an out-of-range slot (host-forced, kernel bounds check)", flush=True)
    bk = backend(num_layers=1, num_blocks=4)
    s = SequenceBlocks(BlockAllocator(4, 16))
    s.append(2)
    meta = make_meta([s], [2], 16, device=DEV)
    import dataclasses

    bad = dataclasses.replace(meta, slot_mapping=torch.tensor([1, 4 * 16 + 5], dtype=torch.int32,
                                                              device=DEV))
    snap = bk._pool.clone()
    bk.append_kv(0, torch.ones(2, 8, 64, device=DEV, dtype=torch.float16),
                 torch.ones(2, 8, 64, device=DEV, dtype=torch.float16), bad)
    with pytest.raises(IndexError, match="slot_mapping"):
        bk.check_device_errors()
    snap.view(1, 2, -1, 8, 64)[0, :, 1] = 1.0
    assert torch.equal(bk._pool, snap), "only the valid slot may be written"


def fill_blocks(bk):
    for layer in range(bk.num_layers):
        for b in range(bk.num_blocks):
            bk.k_pool[layer][b] = float(b + layer * 100 % 997) / 8
            bk.v_pool[layer][b] = -float(b + layer * 100 % 997) / 8 - 1


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_copy_blocks_every_layer_bit_exact(dtype):
    print(f"copy_blocks dtype={dtype}", flush=True)
    bk = backend(num_layers=4, num_blocks=48, dtype=dtype)
    poison(bk, 3)
    pairs = [(1, 2), (5, 40), (7, 8), (30, 31), (1, 47)]  # a shared source, as COW does
    want_k, want_v = copy_blocks_closed_form([p.float().cpu().numpy() for p in bk.k_pool],
                                             [p.float().cpu().numpy() for p in bk.v_pool], pairs)
    bk.copy_blocks([s for s, _ in pairs], [d for _, d in pairs])
    torch.cuda.synchronize()
    for layer in range(4):
        assert np.array_equal(bk.k_pool[layer].float().cpu().numpy(), want_k[layer])
        assert np.array_equal(bk.v_pool[layer].float().cpu().numpy(), want_v[layer])
    bk.check_device_errors()


@pytest.mark.parametrize("seed", range(8))
def test_copy_blocks_random_bit_exact(seed):
    """Seeded random pools (KV heads, head_dim, block size, layers, dtype)
    and random copy-on-write batches: distinct destinations, sources drawn
    with repeats (a shared prefix copied to several sequences), against the
    closed form."""
    import random
    r = random.Random(seed)
    n_kv, d = r.choice([(8, 64), (2, 128), (1, 8), (4, 32)])
    bs, layers = r.choice([1, 4, 16]), r.randint(1, 5)
    nb = r.randint(8, 96)
    dtype = r.choice([torch.float16, torch.bfloat16, torch.float32])
    print(f"copy_blocks random seed={seed} kv={n_kv} d={d} bs={bs} L={layers} nb={nb} {dtype}",
          flush=True)
    bk = backend(num_layers=layers, num_blocks=nb, block_size=bs, n_kv=n_kv,
                 n_heads=n_kv, head_dim=d, dtype=dtype)
    poison(bk, 100 + seed)
    n = r.randint(1, nb // 2)
    dsts = r.sample(range(nb), n)
    pool = [b for b in range(nb) if b not in dsts]
    shared = r.sample(pool, max(1, len(pool) // 8))
    srcs = [r.choice(shared) if r.random() < 0.27 else r.choice(pool) for _ in range(n)]
    pairs = list(zip(srcs, dsts))
    want_k, want_v = copy_blocks_closed_form([p.float().cpu().numpy() for p in bk.k_pool],
                                             [p.float().cpu().numpy() for p in bk.v_pool], pairs)
    bk.copy_blocks(srcs, dsts)
    torch.cuda.synchronize()
    for layer in range(layers):
        assert np.array_equal(bk.k_pool[layer].float().cpu().numpy(), want_k[layer])
        assert np.array_equal(bk.v_pool[layer].float().cpu().numpy(), want_v[layer])
    bk.check_device_errors()


def test_copy_block_contract():
    print("copy_block single pair / errors", flush=True)
    bk = backend(num_layers=3, num_blocks=8, block_size=4, n_kv=2, n_heads=4, head_dim=8,
                 dtype=torch.float32)
    fill_blocks(bk)
    bk.copy_block(1, 2)
    for layer in range(3):
        assert torch.equal(bk.k_pool[layer][2], bk.k_pool[layer][1])
        assert torch.equal(bk.v_pool[layer][2], bk.v_pool[layer][1])
    before = bk.k_pool[2][1].clone()
    bk.k_pool[2][2] += 99.0
    assert torch.equal(bk.k_pool[2][1], before), "destination aliases the source"
    snap = bk._pool.clone()
    bk.copy_block(3, 3)
    assert torch.equal(bk._pool, snap)
    for s, d in [(-1, 0), (0, -1), (999, 0), (0, 8)]:
        with pytest.raises(IndexError):
            bk.copy_block(s, d)
    with pytest.raises(ValueError):
        bk.copy_blocks([1, 2], [2, 3])  # a destination is also a source


# -------------------------------------------------------------------- swap

def _fill_seq(bk, blocks, base):
    for layer in range(bk.num_layers):
        for i, b in enumerate(blocks.block_ids):
            bk.k_pool[layer][b] = base + layer * 100 + i
            bk.v_pool[layer][b] = -(base + layer * 100 + i)


def _snap(bk, blocks):
    return [(bk.k_pool[l][b].clone(), bk.v_pool[l][b].clone())
            for l in range(bk.num_layers) for b in blocks.block_ids]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_swap_round_trip_into_different_blocks(dtype):
    print(f"swap round trip dtype={dtype}", flush=True)
    bk = backend(num_layers=3, num_blocks=16, block_size=4, n_kv=2, n_heads=4, head_dim=8,
                 dtype=dtype)
    a = BlockAllocator(16, 4)
    swap = KVSwapSpace(bk)
    src = SequenceBlocks(a, seq_id=1)
    src.append(10)
    _fill_seq(bk, src, 7.0)
    before = _snap(bk, src)
    orig = list(src.block_ids)
    h = swap.swap_out("r", src)
    src.free()
    decoy = SequenceBlocks(a, seq_id=2)
    decoy.append(10)
    _fill_seq(bk, decoy, -99.0)  # overwrites freed blocks while the D2H may be in flight
    dst = SequenceBlocks(a, seq_id=3)
    dst.append(h.num_tokens)
    assert set(dst.block_ids).isdisjoint(orig)
    for layer in range(3):
        for i in range(3):
            assert torch.all(h.k[layer, i] == 7.0 + layer * 100 + i)
    swap.swap_in(h, dst)
    for i, (got, want) in enumerate(zip(_snap(bk, dst), before)):
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), i
    swap.release(h)
    swap.release(h)
    assert swap.bytes_in_use == 0 and swap.num_swapped == 0
    bk.check_device_errors()


def test_swap_checks_and_budget():
    print("swap error paths", flush=True)
    bk = backend(num_layers=2, num_blocks=32, block_size=4, n_kv=2, n_heads=4, head_dim=8,
                 dtype=torch.float32)
    a = BlockAllocator(32, 4)
    one = KVSwapSpace(bk).bytes_for(1)
    swap = KVSwapSpace(bk, max_bytes=2 * one)
    s = SequenceBlocks(a, seq_id=1)
    s.append(8)
    h = swap.swap_out("a", s)
    assert swap.bytes_in_use == 2 * one
    t = SequenceBlocks(a, seq_id=2)
    t.append(4)
    with pytest.raises(SwapSpaceFull):
        swap.swap_out("b", t)
    s.free()
    wrong = SequenceBlocks(a, seq_id=3)
    wrong.append(5)
    with pytest.raises(RuntimeError, match="resume mismatch"):
        swap.swap_in(h, wrong)
    same = SequenceBlocks(a, seq_id=4)
    same.append(8)
    same.block_ids.pop()
    with pytest.raises(RuntimeError, match="blocks allocated"):
        swap.swap_in(h, same)
    dead = SequenceBlocks(a, seq_id=5)
    dead.append(4)
    dead.free()
    with pytest.raises(RuntimeError, match="freed"):
        swap.swap_out("c", dead)
    with pytest.raises(TypeError, match="paged backend"):
        KVSwapSpace(object())
    swap.release(h)


def test_swap_bulk_bit_exact():
    """64 sequences x 16 blocks at full geometry, scattered ids, bit-exact:
    the host buffers against the oracle's gather (logical block order), the
    pool after swap-in against its scatter into the new blocks."""
    print("swap bulk 64x16 blocks, 16 layers", flush=True)
    bk = backend(num_layers=16, num_blocks=2200, dtype=torch.float16)
    poison(bk, 9)
    perm = torch.randperm(2200, generator=torch.Generator().manual_seed(4)).tolist()
    out_ids, in_ids = perm[:1024], perm[1024:2048]
    a = BlockAllocator(2200, 16)
    a.allocate(2200)
    a.free(out_ids)
    src = SequenceBlocks(a, seq_id=0)
    src.append(1024 * 16)
    assert src.block_ids == out_ids
    pools = bk._pool.cpu().numpy()                       # (L, 2, NB, bs, Hkv, d)
    want_k = gather_closed_form([pools[l, 0] for l in range(16)], out_ids)
    want_v = gather_closed_form([pools[l, 1] for l in range(16)], out_ids)
    swap = KVSwapSpace(bk)
    h = swap.swap_out("big", src)
    a.free(in_ids)
    src.free()
    dst = SequenceBlocks(a, seq_id=1)
    dst.append(1024 * 16)
    assert dst.block_ids == in_ids
    swap.synchronize()
    assert np.array_equal(h.k.numpy(), want_k) and np.array_equal(h.v.numpy(), want_v)
    swap.swap_in(h, dst)
    torch.cuda.synchronize()
    after = bk._pool.cpu().numpy()
    exp_k = scatter_closed_form([pools[l, 0] for l in range(16)], want_k, in_ids)
    exp_v = scatter_closed_form([pools[l, 1] for l in range(16)], want_v, in_ids)
    for l in range(16):
        assert np.array_equal(after[l, 0], exp_k[l]) and np.array_equal(after[l, 1], exp_v[l]), l
    swap.release(h)


def test_swap_64_victims_lifo_one_handle_each():
    """The preemption workload the way the reference's scheduler swaps
    (serving/scheduler/preemption.py:399-472; LIFO victims, :130-194): 64
    running sequences of 256 tokens (16 blocks each) on a shuffled 16-layer
    pool are swapped out one handle per victim, the most recently admitted
    first. Each victim's blocks are freed as soon as its swap_out returns
    and overwritten at once on the caller's stream (another owner taking
    them), while that victim's and earlier victims' transfers are still in
    flight. Then every victim is swapped back into new blocks. Each handle's
    host bytes must equal the logical-order gather of the pool as it was
    before the swaps, and the pool after all swap-ins the scatter of every
    handle into its new blocks over the overwritten pool."""
    print("swap 64 victims x 16 blocks, LIFO, one handle each", flush=True)
    L, n_vict, per = 16, 64, 16
    nb = 2 * n_vict * per + 256
    bk = backend(num_layers=L, num_blocks=nb, dtype=torch.float16)
    poison(bk, 13)
    a = BlockAllocator(nb, 16)
    a.allocate(nb)
    a.free(torch.randperm(nb, generator=torch.Generator().manual_seed(14)).tolist())
    victims = [SequenceBlocks(a, seq_id=i) for i in range(n_vict)]
    for s in victims:
        s.append(per * 16)
    torch.cuda.synchronize()
    before = bk._pool.cpu().numpy()                      # (L, 2, NB, bs, Hkv, d)
    swap = KVSwapSpace(bk)
    handles = []
    for s in reversed(victims):                          # LIFO: last admitted first
        old = list(s.block_ids)
        h = swap.swap_out(f"req-{s.seq_id}", s)
        s.free()
        # the freed blocks are rewritten right away on the caller's stream
        ids = torch.tensor(old, dtype=torch.int64, device=DEV)
        bk._pool.index_fill_(2, ids, float(s.seq_id % 7) - 3.0)
        handles.append((s.seq_id, h, old))
    assert swap.num_swapped == n_vict
    for sid, h, old in handles:                          # each waits for its own copy only
        want_k = gather_closed_form([before[l, 0] for l in range(L)], old)
        want_v = gather_closed_form([before[l, 1] for l in range(L)], old)
        assert np.array_equal(h.k.numpy(), want_k), f"victim {sid} K"
        assert np.array_equal(h.v.numpy(), want_v), f"victim {sid} V"
    torch.cuda.synchronize()
    mid = bk._pool.cpu().numpy()
    exp_k = [mid[l, 0] for l in range(L)]
    exp_v = [mid[l, 1] for l in range(L)]
    for sid, h, old in reversed(handles):                # resume in admission order
        new = SequenceBlocks(a, seq_id=1000 + sid)
        new.append(per * 16)
        assert new.block_ids != old
        swap.swap_in(h, new)
        exp_k = scatter_closed_form(exp_k, h.k.numpy(), new.block_ids)
        exp_v = scatter_closed_form(exp_v, h.v.numpy(), new.block_ids)
        swap.release(h)
    torch.cuda.synchronize()
    after = bk._pool.cpu().numpy()
    for l in range(L):
        assert np.array_equal(after[l, 0], exp_k[l]) and np.array_equal(after[l, 1], exp_v[l]), l
    assert swap.num_swapped == 0 and swap.bytes_in_use == 0
    bk.check_device_errors()
