"""
GPU parity at the benchmark workloads' full sizes, through the C ABI.

The reference's differential harness runs its workloads as stated
(tests/test_flashinfer_differential.py:450-517); these tests do the same for
the benchmark configurations, each against the oracle on the same inputs:

* radix copy-on-write: 4096 block pairs, 16 layers, 27% of sources from a
  shared-prefix set -- bit-exact against the numpy closed form;
* chunked prefill: 8 sequences x 512-token chunks over one shared
  1536-token paged prefix -- fp16 within 2e-3 / 1e-2 of the fp32 oracle;
* capacity decode: 4096 sequences of 16..64 tokens, and 512 sequences of
  lognormal mean 2048 clipped to 2048 -- one layer each, same bar;
* the headline decode step exactly as benchmarked: batch 256, lognormal mean
  258, the backend's default partitions, KV append fused into the attention
  launch, captured in a HIP graph and replayed, every replay checked.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, SequenceBlocks
from llm_serving_layer_amd.backend import DEFAULT_PART_PAGES, MI355XBackend
from oracle import PagedTorchOracle, append_closed_form, copy_blocks_closed_form

from ._util import assert_attention_close, grow_and_assemble, lognormal_lengths, meta_to_device

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SEED = 20260731


def _to_dev(meta, mirror=True):
    """On the device, with the host mirror a serving loop's meta carries
    (the backend plans from it), unless ``mirror=False``."""
    return meta_to_device(meta, DEV, mirror)


def _shuffled(nb, seed):
    a = BlockAllocator(nb, 16)
    a.allocate(nb)
    a.free(torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).tolist())
    return a


def _half(shape, g, scale=0.5):
    """fp16 values ~ N(0, 1) * scale, drawn on the device (fast at these sizes)."""
    return (torch.randn(shape, generator=g, device=DEV) * scale).half()


class _Decode:
    """A one-layer fp16 GPU backend and the fp32 oracle over the same pages,
    with each sequence's history written through both appends."""

    def __init__(self, lens, seed, part_pages=DEFAULT_PART_PAGES, slack=1.25, **backend_kw):
        pages = sum(-(-(n + 1) // 16) for n in lens)
        nb = int(pages * slack) + 8
        self.gpu = MI355XBackend(1, nb, 16, 8, 32, 64, device=DEV, part_pages=part_pages,
                                 **backend_kw)
        self.ref = PagedTorchOracle(1, nb, 16, 8, 32, 64, device="cpu", dtype=torch.float32)
        alloc = _shuffled(nb, seed)
        self.seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(lens))]
        hist = grow_and_assemble(self.seqs, lens, 16)
        self.g = torch.Generator(device=DEV).manual_seed(seed + 1)
        T = hist.n_tokens
        k, v = _half((T, 8, 64), self.g), _half((T, 8, 64), self.g)
        self.gpu.append_kv(0, k, v, _to_dev(hist))
        self.ref.append_kv(0, k.float().cpu(), v.float().cpu(), hist)

    def step(self, label):
        meta = grow_and_assemble(self.seqs, [1] * len(self.seqs), 16)
        n = meta.n_tokens
        k, v, q = _half((n, 8, 64), self.g), _half((n, 8, 64), self.g), _half((n, 32, 64), self.g)
        dm = _to_dev(meta)   # one meta for both calls: the append is fused into the attend
        self.gpu.append_kv(0, k, v, dm)
        out = self.gpu.attend(q, 0, 0.125, dm)
        self.gpu.check_device_errors()
        self.ref.append_kv(0, k.float().cpu(), v.float().cpu(), meta)
        want = self.ref.attend(q.float().cpu(), 0, 0.125, meta)
        assert_attention_close(out, want, label=label)
        # pool bytes after the fused append, compared on the device
        assert torch.equal(self.gpu.k_pool[0].float(), self.ref.k_pool[0].to(DEV)), label
        assert torch.equal(self.gpu.v_pool[0].float(), self.ref.v_pool[0].to(DEV)), label
        return meta


def test_copy_on_write_4096_pairs_16_layers():
    """4096 (src, dst) pairs per step over 16 layers, K and V; 27% of the
    sources drawn from a 64-block shared prefix (repeats), the rest unique;
    destinations distinct free blocks."""
    print("cow 4096 pairs x 16 layers", flush=True)
    pairs, nb, shared = 4096, 8320, 64
    bk = MI355XBackend(16, nb, 16, 8, 32, 64, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(SEED)
    bk._pool.copy_(torch.randn(bk._pool.shape, generator=g, device=DEV).half())
    rng = random.Random(SEED)
    perm = list(range(nb))
    rng.shuffle(perm)
    prefix, uniq, dsts = perm[:shared], perm[shared:shared + pairs], perm[-pairs:]
    srcs = [rng.choice(prefix) if rng.random() < 0.27 else uniq[i] for i in range(pairs)]
    assert not set(dsts) & set(srcs) and len(set(dsts)) == pairs
    frac = sum(s in set(prefix) for s in srcs) / pairs
    assert 0.24 < frac < 0.30, frac
    before = bk._pool.clone()
    layers = (0, 7, 15)   # the numpy closed form on three layers, the device check on all
    want_k, want_v = copy_blocks_closed_form(
        [before[l, 0].cpu().numpy() for l in layers],
        [before[l, 1].cpu().numpy() for l in layers], list(zip(srcs, dsts)))
    bk.copy_blocks(srcs, dsts)
    torch.cuda.synchronize()
    bk.check_device_errors()
    for i, l in enumerate(layers):
        assert np.array_equal(bk._pool[l, 0].cpu().numpy(), want_k[i]), l
        assert np.array_equal(bk._pool[l, 1].cpu().numpy(), want_v[i]), l
    s_ix = torch.tensor(srcs, device=DEV)
    d_ix = torch.tensor(dsts, device=DEV)
    assert torch.equal(bk._pool[:, :, d_ix], before[:, :, s_ix])
    keep = torch.ones(nb, dtype=torch.bool, device=DEV)
    keep[d_ix] = False
    assert torch.equal(bk._pool[:, :, keep], before[:, :, keep]), "a non-destination changed"


def test_chunked_prefill_8x512_over_shared_1536_prefix():
    """8 sequences share a radix-cached 1536-token prefix (96 blocks, one
    common table prefix) and each appends a 512-token chunk: causal within
    the chunk, full attention to the prefix; one layer against the oracle."""
    print("prefill 8 x 512 over a shared 1536 prefix", flush=True)
    n_seq, prefix, chunk = 8, 1536, 512
    nb = 2 * (prefix // 16 + n_seq * chunk // 16)
    bk = MI355XBackend(1, nb, 16, 8, 32, 64, device=DEV)
    ref = PagedTorchOracle(1, nb, 16, 8, 32, 64, device="cpu", dtype=torch.float32)
    alloc = _shuffled(nb, SEED)
    pre = SequenceBlocks(alloc, seq_id=1000)
    pre_meta = grow_and_assemble([pre], [prefix], 16)
    g = torch.Generator(device=DEV).manual_seed(SEED + 2)
    kp, vp = _half((prefix, 8, 64), g), _half((prefix, 8, 64), g)
    bk.append_kv(0, kp, vp, _to_dev(pre_meta))
    ref.append_kv(0, kp.float().cpu(), vp.float().cpu(), pre_meta)
    seqs = []
    for i in range(n_seq):
        s = SequenceBlocks(alloc, seq_id=i)
        alloc.incref(pre.block_ids)
        s.block_ids = list(pre.block_ids)
        s.num_tokens = prefix
        seqs.append(s)
    meta = grow_and_assemble(seqs, [chunk] * n_seq, 16)
    assert all(meta.kv_indices[int(meta.kv_indptr[i]):int(meta.kv_indptr[i]) + 96].tolist()
               == pre.block_ids for i in range(n_seq)), "tables must share the prefix blocks"
    T = meta.n_tokens
    k, v, q = _half((T, 8, 64), g), _half((T, 8, 64), g), _half((T, 32, 64), g)
    dm = _to_dev(meta)
    bk.append_kv(0, k, v, dm)
    out = bk.attend(q, 0, 0.125, dm)
    bk.check_device_errors()
    assert bk.q_tile == bk._prefill_tile > 0, "the matrix-core prefill must serve this batch"
    ref.append_kv(0, k.float().cpu(), v.float().cpu(), meta)
    want = ref.attend(q.float().cpu(), 0, 0.125, meta)
    assert_attention_close(out, want, label="prefill 8x512 over 1536")
    assert torch.equal(bk.k_pool[0].float().cpu(), ref.k_pool[0])


def test_capacity_phase_a_4096_short_sequences():
    """4096 concurrent sequences of 16..64 tokens (no sequence split: packs)."""
    print("capacity phase A: 4096 x U[16,64]", flush=True)
    rng = random.Random(SEED)
    lens = [rng.randint(16, 64) for _ in range(4096)]
    d = _Decode([n - 1 for n in lens], SEED + 10)
    d.step("capacity phase A")


def test_capacity_phase_b_512_long_sequences():
    """512 sequences of lognormal mean 2048 clipped to 2048 (every one split)."""
    print("capacity phase B: 512 x lognormal 2048", flush=True)
    lens = lognormal_lengths(512, 2048, 0.8, 2048, SEED)
    d = _Decode([n - 1 for n in lens], SEED + 20)
    d.step("capacity phase B")


@pytest.mark.parametrize("part_pages", [4, DEFAULT_PART_PAGES])
def test_headline_batch256_decode_vs_oracle(part_pages):
    """The headline batch (256 sequences, lognormal mean 258, seed 20260731),
    one layer, at the backend's default partitions and at 4 pages."""
    print(f"headline batch 256, part_pages={part_pages}", flush=True)
    lens = lognormal_lengths(256, 256, 0.8, 2048, SEED)
    d = _Decode([n - 1 for n in lens], 5, part_pages=part_pages, slack=2.0)
    d.step(f"batch 256 part_pages={part_pages}")
    d.step(f"batch 256 part_pages={part_pages}, second step")


def test_workspace_reserved_by_the_sizing_bound_is_never_regrown():
    """A backend given the sizing bound's workspace up front (as a pool sized
    by plan_kv_pool is) runs the headline batch without allocating: the
    workspace keeps its size and address, and the outputs match the oracle."""
    from llm_serving_layer_amd.sizing import decode_workspace_bound

    print("headline batch 256 on a reserved workspace", flush=True)
    lens = lognormal_lengths(256, 256, 0.8, 2048, SEED)
    nb = int(sum(-(-n // 16) for n in lens) * 2.0) + 8
    reserve = decode_workspace_bound(nb, 256, 32, 8, 64, DEFAULT_PART_PAGES)
    d = _Decode([n - 1 for n in lens], 7, slack=2.0, decode_workspace_bytes=reserve)
    addr = d.gpu._workspace.data_ptr()
    assert d.gpu.workspace_bytes() == reserve
    d.step("batch 256 on the reserved workspace")
    assert d.gpu._planned.n_slots > 0
    assert d.gpu.workspace_bytes() == reserve and d.gpu._workspace.data_ptr() == addr


def test_headline_step_graph_replayed_vs_oracle():
    """The benchmarked configuration exactly: default partitions, the append
    deferred into the attention launch, two layers captured in one HIP graph
    and replayed three times with other work between replays; every replay's
    outputs against the oracle, and the pools against the append's closed
    form."""
    print("headline step, graph replay", flush=True)
    lens = lognormal_lengths(256, 256, 0.8, 2048, SEED)
    pages = sum(-(-n // 16) for n in lens)
    nb = 2 * pages
    L = 2
    bk = MI355XBackend(L, nb, 16, 8, 32, 64, device=DEV)
    assert bk.part_pages == DEFAULT_PART_PAGES and bk._fuse_append
    g = torch.Generator(device=DEV).manual_seed(SEED)
    bk._pool.copy_((torch.randn(bk._pool.shape, generator=g, device=DEV) * 0.5).half())
    alloc = _shuffled(nb, SEED)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(256)]
    for s, n in zip(seqs, lens):
        s.append(n - 1)
    meta_cpu = grow_and_assemble(seqs, [1] * 256, 16)
    meta = _to_dev(meta_cpu)
    k, v, q = _half((L, 256, 8, 64), g), _half((L, 256, 8, 64), g), _half((L, 256, 32, 64), g)
    pool0 = bk._pool.cpu()
    outs = [None] * L

    def step():
        for l in range(L):
            bk.append_kv(l, k[l], v[l], meta)
            outs[l] = bk.attend(q[l], l, 0.125, meta)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()                                   # plan + workspace outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert bk._planned.n_slots > 0, "the headline batch splits its long sequences"
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    slots = meta_cpu.slot_mapping.tolist()
    refs = []
    for l in range(L):
        ref = PagedTorchOracle(1, nb, 16, 8, 32, 64, device="cpu", dtype=torch.float32)
        ref.k_pool[0].copy_(pool0[l, 0].float())
        ref.v_pool[0].copy_(pool0[l, 1].float())
        ref.append_kv(0, k[l].float().cpu(), v[l].float().cpu(), meta_cpu)
        refs.append((ref.attend(q[l].float().cpu(), 0, 0.125, meta_cpu),
                     append_closed_form(pool0[l, 0].float().numpy(), k[l].float().cpu().numpy(),
                                        slots),
                     append_closed_form(pool0[l, 1].float().numpy(), v[l].float().cpu().numpy(),
                                        slots)))
    for rep in range(3):
        torch.randn(1 << 20, device=DEV).sum().item()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for l in range(L):
            assert_attention_close(outs[l], refs[l][0], label=f"replay {rep} layer {l}")
            assert np.array_equal(bk._pool[l, 0].float().cpu().numpy(), refs[l][1])
            assert np.array_equal(bk._pool[l, 1].float().cpu().numpy(), refs[l][2])
    bk.check_device_errors()
