"""
Pinning the oracle (oracle/paged_torch_cpu.py, the CPU restatement of the
reference's PagedTorchBackend) before anything is checked against it.

Every check is independent of the restatement's own formula:
* the textbook float64 attention (oracle/naive.py, after the reference's
  tests/test_paged_torch.py:106-149);
* the reference tests' known answers (tests/test_paged_torch.py:183-649):
  slots written and only those, idempotence, layer independence, kv_len==1
  => out==V per KV head, orthogonal keys => key map, per-sequence constant V
  => isolation, block straddle over a 1e3-poisoned pool, scattered and
  descending pages == contiguous bitwise, batched == solo bitwise, future-key
  poison => causality, decode sees itself, 512 KiB/block accounting;
* planted mistakes (a repeat instead of repeat_interleave GQA map, a top-left
  causal mask, a dropped scale, reading past kv_len): each must FAIL one of
  the checks above, so the checks demonstrably have teeth;
* the committed golden fixture (tests/golden/config1.npz) for the
  Llama-3.2-1B-geometry plumbing case.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, SequenceBlocks
from oracle import (PagedTorchOracle, append_closed_form, copy_blocks_closed_form,
                    gather_closed_form, naive_attention, scatter_closed_form)

from ._util import make_meta

DT = torch.float32
TOL = dict(atol=1e-5, rtol=1e-5)
GOLDEN = Path(__file__).resolve().parent / "golden" / "config1.npz"


def make(num_layers=1, num_blocks=32, block_size=16, n_kv=2, n_heads=4, head_dim=8, cls=None):
    return (cls or PagedTorchOracle)(num_layers, num_blocks, block_size, n_kv, n_heads,
                                     head_dim, device="cpu", dtype=DT)


def write_history(bk, alloc, lengths, seed=0, layer=0):
    g = torch.Generator().manual_seed(seed)
    seqs, ks, vs = [], [], []
    for i, n in enumerate(lengths):
        s = SequenceBlocks(alloc, seq_id=i)
        s.append(n)
        seqs.append(s)
        ks.append(torch.randn(n, bk.n_kv_heads, bk.head_dim, generator=g, dtype=DT))
        vs.append(torch.randn(n, bk.n_kv_heads, bk.head_dim, generator=g, dtype=DT))
    bk.append_kv(layer, torch.cat(ks), torch.cat(vs), make_meta(seqs, lengths, alloc.block_size))
    return seqs, ks, vs


def naive(q, k, v, scale, n_kv):
    return torch.from_numpy(naive_attention(q.numpy(), k.numpy(), v.numpy(), scale, n_kv)).float()


def check_vs_naive(bk, lengths, seed):
    alloc = BlockAllocator(32, 16)
    seqs, ks, vs = write_history(bk, alloc, lengths, seed=seed)
    meta = make_meta(seqs, lengths, 16)
    scale = 1.0 / bk.head_dim ** 0.5
    q = torch.randn(sum(lengths), bk.n_heads, bk.head_dim, generator=torch.Generator().manual_seed(seed + 1))
    got = bk.attend(q, 0, scale, meta)
    cu = meta.cu_query_lens.tolist()
    for i in range(len(lengths)):
        torch.testing.assert_close(got[cu[i]:cu[i + 1]],
                                   naive(q[cu[i]:cu[i + 1]], ks[i], vs[i], scale, bk.n_kv_heads),
                                   **TOL)


def check_chunked_vs_naive(bk, hist, chunks, seed):
    """History written first, then a chunk of queries per sequence: q_len < kv_len."""
    alloc = BlockAllocator(32, 16)
    seqs, ks, vs = write_history(bk, alloc, hist, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    nk, nv = [], []
    for i, (s, n) in enumerate(zip(seqs, chunks)):
        s.append(n)
        k1 = torch.randn(n, bk.n_kv_heads, bk.head_dim, generator=g)
        v1 = torch.randn(n, bk.n_kv_heads, bk.head_dim, generator=g)
        nk.append(k1)
        nv.append(v1)
        ks[i], vs[i] = torch.cat([ks[i], k1]), torch.cat([vs[i], v1])
    meta = make_meta(seqs, chunks, 16)
    bk.append_kv(0, torch.cat(nk), torch.cat(nv), meta)
    q = torch.randn(sum(chunks), bk.n_heads, bk.head_dim, generator=g)
    got = bk.attend(q, 0, 0.35, meta)
    cu = meta.cu_query_lens.tolist()
    for i in range(len(chunks)):
        torch.testing.assert_close(got[cu[i]:cu[i + 1]],
                                   naive(q[cu[i]:cu[i + 1]], ks[i], vs[i], 0.35, bk.n_kv_heads),
                                   **TOL)


# ---------------------------------------------------------------- write path

def test_append_lands_in_named_slots_only():
    bk = make()
    a = BlockAllocator(32, 16)
    s = SequenceBlocks(a)
    s.append(20)
    meta = make_meta([s], [20], 16)
    k, v = torch.randn(20, 2, 8), torch.randn(20, 2, 8)
    bk.append_kv(0, k, v, meta)
    kf = bk.k_pool[0].view(-1, 2, 8)
    vf = bk.v_pool[0].view(-1, 2, 8)
    slots = meta.slot_mapping.tolist()
    for t, sl in enumerate(slots):
        assert torch.equal(kf[sl], k[t]) and torch.equal(vf[sl], v[t])
    nz = {int(i) for i in (kf.abs().sum(dim=(1, 2)) != 0).nonzero().flatten()}
    assert nz == set(slots)
    before = bk.k_pool[0].clone()
    bk.append_kv(0, k, v, meta)
    assert torch.equal(bk.k_pool[0], before), "append must be idempotent"


def test_layers_independent_and_copy_block_all_layers():
    bk = make(num_layers=3, num_blocks=8, block_size=4)
    for layer in range(3):
        for b in range(8):
            bk.k_pool[layer][b] = b + layer * 100
            bk.v_pool[layer][b] = b + layer * 100 + 50
    want_k, want_v = copy_blocks_closed_form([p.numpy() for p in bk.k_pool],
                                             [p.numpy() for p in bk.v_pool], [(1, 2)])
    bk.copy_block(1, 2)
    for layer in range(3):
        assert np.array_equal(bk.k_pool[layer].numpy(), want_k[layer])
        assert np.array_equal(bk.v_pool[layer].numpy(), want_v[layer])
    with pytest.raises(IndexError):
        bk.copy_block(0, 8)


def _encoded_pools(n_layers=3, nb=10, bs=4, hkv=2, d=3, offset=0.0):
    """Every element of block b of layer l holds 1000 l + b + offset, so a
    wrong layer, a wrong block or a transposed index shows in the values."""
    return [np.broadcast_to((1000.0 * l + np.arange(nb) + offset)[:, None, None, None],
                            (nb, bs, hkv, d)).copy() for l in range(n_layers)]


def test_swap_gather_closed_form_known_answer():
    """The swap-out copy (serving/scheduler/preemption.py:490-509) keeps a
    victim's blocks in LOGICAL order: host[l, i] is block ids[i] of layer l,
    shaped (L, n, bs, Hkv, d) (preemption.py:303-332)."""
    pools = _encoded_pools()
    ids = [7, 2, 9, 2, 0]          # scattered, descending runs, a repeat
    host = gather_closed_form(pools, ids)
    assert host.shape == (3, 5, 4, 2, 3)
    for l in range(3):
        for i, b in enumerate(ids):
            assert np.all(host[l, i] == 1000.0 * l + b), (l, i)
    assert gather_closed_form(pools, []).shape[1] == 0


def test_swap_scatter_closed_form_known_answer_and_round_trip():
    """The swap-in copy (preemption.py:511-523): block ids[i] of layer l
    receives host[l, i]; no other block changes. A gather from one set of
    blocks scattered into another set reproduces the victim's KV there."""
    pools = _encoded_pools()
    host = np.stack([np.broadcast_to((-1.0 - 100.0 * l - np.arange(3))[:, None, None, None],
                                     (3, 4, 2, 3)) for l in range(3)])
    ids = [8, 1, 5]
    out = scatter_closed_form(pools, host, ids)
    for l in range(3):
        for b in range(10):
            if b in ids:
                assert np.all(out[l][b] == -1.0 - 100.0 * l - ids.index(b))
            else:
                assert np.all(out[l][b] == pools[l][b]), (l, b)
        assert np.all(pools[l] == _encoded_pools()[l]), "scatter must not modify its input"
    src, dst = [4, 0, 6], [9, 3, 2]
    moved = scatter_closed_form(pools, gather_closed_form(pools, src), dst)
    for l in range(3):
        for s_, d_ in zip(src, dst):
            assert np.array_equal(moved[l][d_], pools[l][s_])


def test_planted_swap_mistakes_fail_the_known_answers():
    pools = _encoded_pools()
    ids = [7, 2, 9]
    want = gather_closed_form(pools, ids)
    wrong_order = np.stack([p[np.sort(ids)] for p in pools])        # physical, not logical
    wrong_layer = np.stack([pools[0][ids] for _ in pools])          # layer index dropped
    assert not np.array_equal(want, wrong_order)
    assert not np.array_equal(want, wrong_layer)


def test_append_and_copy_closed_forms_known_answers():
    """append: flat slot s = block * bs + row receives token t's row
    (paged_torch.py:270-276); copy: every layer, K and V, dst = src, pair by
    pair, src == dst a no-op (paged_torch.py:181-207)."""
    pool = _encoded_pools(n_layers=1)[0]
    x = -np.arange(2 * 2 * 3, dtype=np.float64).reshape(2, 2, 3) - 1
    got = append_closed_form(pool, x, [4 * 6 + 1, 4 * 9 + 3])
    assert np.array_equal(got[6, 1], x[0]) and np.array_equal(got[9, 3], x[1])
    mask = np.ones(got.shape[:2], bool)
    mask[6, 1] = mask[9, 3] = False
    assert np.array_equal(got[mask], pool[mask])
    ks, vs = _encoded_pools(), _encoded_pools(offset=0.5)
    ck, cv = copy_blocks_closed_form(ks, vs, [(1, 4), (3, 3), (4, 8)])
    for l in range(3):
        assert np.all(ck[l][4] == 1000.0 * l + 1) and np.all(cv[l][4] == 1000.0 * l + 1.5)
        assert np.all(ck[l][8] == 1000.0 * l + 1), "pairs apply in order: 4 was already 1"
        assert np.all(ck[l][3] == 1000.0 * l + 3)


# ----------------------------------------------------------- vs textbook

def test_prefill_matches_textbook():
    check_vs_naive(make(), [5, 17, 32], seed=1)


def test_chunked_prefill_matches_textbook():
    check_chunked_vs_naive(make(), [6, 18, 16], [4, 3, 17], seed=5)


def test_decode_matches_textbook():
    bk = make()
    a = BlockAllocator(32, 16)
    seqs, ks, vs = write_history(bk, a, [7, 16, 33], seed=2)
    nk, nv = [], []
    for i, s in enumerate(seqs):
        s.append(1)
        k1, v1 = torch.randn(1, 2, 8), torch.randn(1, 2, 8)
        nk.append(k1)
        nv.append(v1)
        ks[i], vs[i] = torch.cat([ks[i], k1]), torch.cat([vs[i], v1])
    meta = make_meta(seqs, [1, 1, 1], 16)
    bk.append_kv(0, torch.cat(nk), torch.cat(nv), meta)
    q = torch.randn(3, 4, 8)
    got = bk.attend(q, 0, 0.35, meta)
    for i in range(3):
        torch.testing.assert_close(got[i:i + 1], naive(q[i:i + 1], ks[i], vs[i], 0.35, 2), **TOL)


@pytest.mark.parametrize("n", [1, 15, 16, 17, 31, 32, 33])
def test_block_straddle_over_poisoned_pool(n):
    bk = make()
    bk.k_pool[0].fill_(1e3)
    bk.v_pool[0].fill_(1e3)
    a = BlockAllocator(32, 16)
    seqs, ks, vs = write_history(bk, a, [n], seed=n)
    meta = make_meta(seqs, [n], 16)
    q = torch.randn(n, 4, 8)
    torch.testing.assert_close(bk.attend(q, 0, 0.35, meta), naive(q, ks[0], vs[0], 0.35, 2), **TOL)


def test_scattered_and_descending_pages_equal_contiguous():
    k, v = torch.randn(40, 2, 8), torch.randn(40, 2, 8)
    q = torch.randn(40, 4, 8)
    outs = []
    for free_order in (None, [21, 4, 13], [13, 4, 2]):
        bk = make()
        a = BlockAllocator(32, 16)
        if free_order:
            a.allocate(32)
            a.free(free_order)
        s = SequenceBlocks(a)
        s.append(40)
        if free_order:
            assert s.block_ids == free_order
        meta = make_meta([s], [40], 16)
        bk.append_kv(0, k, v, meta)
        outs.append(bk.attend(q, 0, 0.35, meta))
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    torch.testing.assert_close(outs[0], naive(q, k, v, 0.35, 2), **TOL)


# -------------------------------------------------------- known answers

def test_gqa_value_map_is_floor_divide():
    bk = make(n_kv=2, n_heads=6)
    a = BlockAllocator(8, 16)
    s = SequenceBlocks(a)
    s.append(1)
    meta = make_meta([s], [1], 16)
    v = torch.zeros(1, 2, 8)
    v[0, 0], v[0, 1] = 1.0, 2.0
    bk.append_kv(0, torch.zeros(1, 2, 8), v, meta)
    out = bk.attend(torch.randn(1, 6, 8), 0, 1.0, meta)
    for h in range(6):
        assert torch.allclose(out[0, h], torch.full((8,), float(h // 3 + 1)))


def test_gqa_key_map_is_floor_divide():
    bk = make(n_kv=2, n_heads=4)
    a = BlockAllocator(8, 16)
    s = SequenceBlocks(a)
    s.append(2)
    meta = make_meta([s], [2], 16)
    k, v = torch.zeros(2, 2, 8), torch.zeros(2, 2, 8)
    for j in range(2):
        k[0, j, j] = 50.0
        k[1, j, 2 + j] = 50.0
        v[0, j], v[1, j] = 1.0, -1.0
    bk.append_kv(0, k, v, meta)
    q = torch.zeros(2, 4, 8)
    for h in range(4):
        q[:, h, h // 2] = 1.0
    out = bk.attend(q, 0, 1.0, meta)
    assert (out[1, :, 0] > 0.99).all()


def test_sequences_isolated():
    bk = make()
    a = BlockAllocator(32, 16)
    lens = [3, 1, 20]
    seqs = []
    for i, n in enumerate(lens):
        s = SequenceBlocks(a, seq_id=i)
        s.append(n)
        seqs.append(s)
    meta = make_meta(seqs, lens, 16)
    vs = torch.cat([torch.full((n, 2, 8), float(i + 1)) for i, n in enumerate(lens)])
    bk.append_kv(0, torch.zeros(sum(lens), 2, 8), vs, meta)
    out = bk.attend(torch.randn(sum(lens), 4, 8), 0, 1.0, meta)
    cu = meta.cu_query_lens.tolist()
    for i in range(3):
        assert torch.allclose(out[cu[i]:cu[i + 1]], torch.full_like(out[cu[i]:cu[i + 1]], i + 1.0))


def test_mixed_batch_equals_solo_bitwise():
    bk = make()
    a = BlockAllocator(32, 16)
    seqs, ks, vs = write_history(bk, a, [6, 18, 16], seed=11)
    ql = [4, 1, 1]
    nk = []
    for s, n in zip(seqs, ql):
        s.append(n)
        nk.append(torch.randn(n, 2, 8))
    meta = make_meta(seqs, ql, 16)
    bk.append_kv(0, torch.cat(nk), torch.cat(nk), meta)
    q = torch.randn(6, 4, 8)
    batched = bk.attend(q, 0, 0.35, meta)
    cu = meta.cu_query_lens.tolist()
    for i, n in enumerate(ql):
        solo = bk.attend(q[cu[i]:cu[i + 1]], 0, 0.35, make_meta([seqs[i]], [n], 16))
        assert torch.equal(batched[cu[i]:cu[i + 1]], solo)


def test_causality_and_decode_sees_itself():
    bk = make()
    a = BlockAllocator(32, 16)
    seqs, _, _ = write_history(bk, a, [6], seed=21)
    meta = make_meta(seqs, [6], 16)
    q = torch.randn(6, 4, 8)
    base = bk.attend(q, 0, 0.35, meta)
    slot = seqs[0].slot_for(5)
    bk.k_pool[0].view(-1, 2, 8)[slot] = 100.0
    bk.v_pool[0].view(-1, 2, 8)[slot] = -999.0
    pois = bk.attend(q, 0, 0.35, meta)
    assert torch.equal(base[:5], pois[:5])
    assert not torch.allclose(base[5], pois[5])

    bk2 = make()
    s = SequenceBlocks(BlockAllocator(8, 16))
    s.append(1)
    m1 = make_meta([s], [1], 16)
    bk2.append_kv(0, torch.zeros(1, 2, 8), torch.full((1, 2, 8), 7.0), m1)
    assert torch.allclose(bk2.attend(torch.randn(1, 4, 8), 0, 1.0, m1), torch.full((1, 4, 8), 7.0))


def test_accounting_512_kib_per_block():
    bk = PagedTorchOracle(16, 100, 16, 8, 32, 64, dtype=torch.float16)
    assert bk.block_bytes() == 512 * 1024
    assert bk.pool_bytes() == 100 * 512 * 1024
    assert bk.tokens_capacity() == 1600


def test_constructor_validation():
    with pytest.raises(ValueError, match="divisible"):
        make(n_kv=3, n_heads=4)
    with pytest.raises(ValueError, match="positive"):
        make(num_blocks=0)


# ------------------------------------------- planted mistakes must be caught

class _WrongGqa(PagedTorchOracle):
    def _attend_one(self, q, k, v, scale, q_len, kv_len):
        k = k.repeat(1, self.groups, 1)  # h % n_kv_heads: the plausible wrong map
        v = v.repeat(1, self.groups, 1)
        s = torch.matmul(q.transpose(0, 1).float(), k.transpose(0, 1).float().transpose(1, 2)) * scale
        if q_len > 1:
            s = s + torch.triu(torch.full((q_len, kv_len), float("-inf")), diagonal=kv_len - q_len + 1)
        return torch.matmul(torch.softmax(s, -1).to(self.dtype), v.transpose(0, 1)).transpose(0, 1)


class _TopLeftMask(PagedTorchOracle):
    def _attend_one(self, q, k, v, scale, q_len, kv_len):
        k = torch.repeat_interleave(k, self.groups, dim=1)
        v = torch.repeat_interleave(v, self.groups, dim=1)
        s = torch.matmul(q.transpose(0, 1).float(), k.transpose(0, 1).float().transpose(1, 2)) * scale
        if q_len > 1:
            s = s + torch.triu(torch.full((q_len, kv_len), float("-inf")), diagonal=1)  # wrong
        return torch.matmul(torch.softmax(s, -1).to(self.dtype), v.transpose(0, 1)).transpose(0, 1)


class _NoScale(PagedTorchOracle):
    def _attend_one(self, q, k, v, scale, q_len, kv_len):
        return super()._attend_one(q, k, v, 1.0, q_len, kv_len)


class _ReadsPastKvLen(PagedTorchOracle):
    def _gather(self, layer_idx, pages, kv_len, last_page_len):
        k = self.k_pool[layer_idx][pages].reshape(-1, self.n_kv_heads, self.head_dim)
        v = self.v_pool[layer_idx][pages].reshape(-1, self.n_kv_heads, self.head_dim)
        return k, v  # forgot the [:kv_len] truncation


@pytest.mark.parametrize("cls", [_WrongGqa, _TopLeftMask, _NoScale])
def test_planted_arithmetic_mistakes_fail_textbook_check(cls):
    with pytest.raises(AssertionError):
        check_vs_naive(make(cls=cls), [5, 17, 32], seed=1)
        check_chunked_vs_naive(make(cls=cls), [6, 18, 16], [4, 3, 17], seed=5)


def test_planted_overread_fails_straddle_check():
    bk = make(cls=_ReadsPastKvLen)
    bk.k_pool[0].fill_(1e3)
    bk.v_pool[0].fill_(1e3)
    with pytest.raises(Exception):
        seqs, ks, vs = write_history(bk, BlockAllocator(32, 16), [17], seed=3)
        meta = make_meta(seqs, [17], 16)
        q = torch.randn(17, 4, 8)
        torch.testing.assert_close(bk.attend(q, 0, 0.35, meta), naive(q, ks[0], vs[0], 0.35, 2), **TOL)


# ------------------------------------------------------------ golden fixture

def test_golden_config1_against_oracle():
    from .golden.make_config1 import build_inputs, input_digest

    fx = np.load(GOLDEN, allow_pickle=False)
    inp = build_inputs()
    assert input_digest(inp) == str(fx["input_sha256"]), "input generator drifted"
    bk = PagedTorchOracle(1, inp["num_blocks"], 16, 8, 32, 64, dtype=torch.float32)
    meta = inp["meta"]
    # history, then the one appended token, then one decode step
    bk.append_kv(0, torch.from_numpy(inp["k_hist"]), torch.from_numpy(inp["v_hist"]), inp["hist_meta"])
    bk.append_kv(0, torch.from_numpy(inp["k_new"]), torch.from_numpy(inp["v_new"]), meta)
    out = bk.attend(torch.from_numpy(inp["q"]), 0, 0.125, meta)
    np.testing.assert_allclose(out.numpy(), fx["out_f64"], atol=1e-5, rtol=1e-5)
    digest = hashlib.sha256(bk.k_pool[0].numpy().tobytes() + bk.v_pool[0].numpy().tobytes()).hexdigest()
    assert digest == str(fx["pool_sha256"]), "pool bytes after append differ from the fixture"
