"""
GPU parity of paged attention against the oracle.

Bar: fp16/bf16 output within max-abs 2e-3 / max-rel 1e-2
of the oracle's fp32 computation on the same (fp16-rounded) inputs; fp32
pools within 1e-5 of the float64 textbook. Structural known answers from the
reference's tests/test_paged_torch.py (:303-649) and the differential harness
of tests/test_flashinfer_differential.py (:381-600: pure decode, mixed,
page-boundary sweep, fragmented + poisoned pools, isolation, GQA 8->{1,2,4,8},
plan once per step) are restated against this backend.
"""

from __future__ import annotations

import dataclasses
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, SequenceBlocks
from llm_serving_layer_amd.backend import DEFAULT_PART_PAGES, MI355XBackend
from oracle import PagedTorchOracle

from ._util import (assert_attention_close, fragmented_allocator, grow_and_assemble,
                    lognormal_lengths, make_meta, meta_to_device)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class Pair:
    """The GPU backend and the CPU fp32 oracle fed identical (dtype-rounded) inputs."""

    def __init__(self, num_layers, num_blocks, block_size, n_kv, n_heads, head_dim,
                 dtype=torch.float16, part_pages=4, q_tile=None, decode_workgroups=None):
        self.gpu = MI355XBackend(num_layers, num_blocks, block_size, n_kv, n_heads, head_dim,
                                 device=DEV, dtype=dtype, part_pages=part_pages, q_tile=q_tile,
                                 decode_workgroups=decode_workgroups)
        self.ref = PagedTorchOracle(num_layers, num_blocks, block_size, n_kv, n_heads, head_dim,
                                    device="cpu", dtype=torch.float32)
        self.dtype = dtype

    def poison(self, seed):
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(self.gpu._pool.shape, generator=g).to(self.dtype)
        self.gpu._pool.copy_(x.to(DEV))
        for l in range(self.gpu.num_layers):
            self.ref.k_pool[l].copy_(x[l, 0].float())
            self.ref.v_pool[l].copy_(x[l, 1].float())

    def rand(self, shape, g, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(self.dtype)

    def step(self, meta_cpu, seed, scale=0.125, layers=None, kv_scale=1.0, mirror=True):
        """append + attend for each layer; returns [(layer, gpu_out, ref_out)]."""
        g = torch.Generator().manual_seed(seed)
        meta_gpu = _to_dev(meta_cpu, mirror)
        T = meta_cpu.n_tokens
        res = []
        for layer in (layers if layers is not None else range(self.gpu.num_layers)):
            k = self.rand((T, self.gpu.n_kv_heads, self.gpu.head_dim), g, kv_scale)
            v = self.rand((T, self.gpu.n_kv_heads, self.gpu.head_dim), g, kv_scale)
            q = self.rand((T, self.gpu.n_heads, self.gpu.head_dim), g)
            self.gpu.append_kv(layer, k.to(DEV), v.to(DEV), meta_gpu)
            out = self.gpu.attend(q.to(DEV), layer, scale, meta_gpu)
            self.ref.append_kv(layer, k.float(), v.float(), meta_cpu)
            want = self.ref.attend(q.float(), layer, scale, meta_cpu)
            res.append((layer, out, want))
        self.gpu.check_device_errors()
        return res


def _to_dev(meta, mirror=True):
    """On the device, with the host mirror a serving loop's meta carries
    (the backend plans from it), unless ``mirror=False``."""
    return meta_to_device(meta, DEV, mirror)


def check(res, label, atol=2e-3, rtol=1e-2):
    for layer, got, want in res:
        assert got.dtype == (got.dtype) and got.shape == want.shape
        assert_attention_close(got, want, atol=atol, rtol=rtol, label=f"{label} layer {layer}")


# ------------------------------------------------ the differential harness

GEOMS = [
    # (n_kv, n_heads, head_dim): bench geometry, the reference differential's, odd shapes
    (8, 32, 64), (2, 8, 128), (8, 8, 64), (4, 8, 64), (1, 8, 64), (2, 4, 8),
]


@pytest.mark.parametrize("geom", GEOMS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_then_decode_across_page_boundaries(geom, dtype):
    n_kv, n_heads, d = geom
    print(f"differential geom={geom} dtype={dtype}", flush=True)
    p = Pair(2, 256, 16, n_kv, n_heads, d, dtype=dtype)
    p.poison(1)
    alloc, _keep = fragmented_allocator(256, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(5)]
    tol = 2e-3 if dtype == torch.float16 else 1.6e-2  # bf16 rounds p to 8 bits
    rtol = 1e-2 if dtype == torch.float16 else 8e-2
    check(p.step(grow_and_assemble(seqs, [15, 16, 17, 1, 40], 16), 10), "prefill", tol, rtol)
    for it in range(20):  # each sequence crosses at least one page boundary
        check(p.step(grow_and_assemble(seqs, [1, 1, 1, 1, 1], 16), 100 + it), f"decode {it}",
              tol, rtol)
    check(p.step(grow_and_assemble(seqs, [1, 5, 0, 1, 9], 16), 7), "mixed", tol, rtol)


@pytest.mark.parametrize("part_pages", [1, 3, 8, 16, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_long_sequences_split_k(part_pages, dtype):
    """Sequences far longer than one partition: the split-K merge path."""
    print(f"split-K decode part_pages={part_pages} dtype={dtype}", flush=True)
    p = Pair(1, 512, 16, 8, 32, 64, dtype=dtype, part_pages=part_pages)
    p.poison(2)
    alloc, _keep = fragmented_allocator(512, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(6)]
    for s, n in zip(seqs, [1, 63, 64, 65, 700, 1200]):
        s.append(n)
    meta = grow_and_assemble(seqs, [1] * 6, 16)
    tol, rtol = (2e-3, 1e-2) if dtype == torch.float16 else (1.6e-2, 8e-2)
    check(p.step(meta, 3), "split-K", tol, rtol)


@pytest.mark.parametrize("geom", [(8, 8, 64), (4, 8, 64), (1, 8, 64), (2, 32, 64),
                                  (2, 8, 128), (4, 32, 128), (2, 32, 128)])
def test_split_k_and_packed_items_other_geometries(geom):
    """Cut sequences and many items per bin at every group size and head_dim
    the decode kernel instantiates (1 to 16 query heads per KV head, 64 and
    128 dims): pieces of 3 pages (up to 59 of one sequence), their merges
    (by the last arriver, or by the last piece with its own partial in
    registers), and a bin's item slots refilled in batches, with the fused
    append, over two decode steps against the oracle."""
    n_kv, n_heads, d = geom
    print(f"split-K + packed items geom={geom}", flush=True)
    p = Pair(1, 512, 16, n_kv, n_heads, d, part_pages=3, decode_workgroups=8)
    p.poison(4)
    alloc, _keep = fragmented_allocator(512, 16)
    rng = np.random.default_rng(d * 100 + n_heads)
    lens = [1, 40, 100, 333, 940] + [int(x) for x in rng.integers(1, 60, 24)]
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(lens))]
    for s, n in zip(seqs, lens):
        s.append(n)
    for step in range(2):
        meta = grow_and_assemble(seqs, [1] * len(lens), 16)
        check(p.step(meta, 20 + step), f"decode step {step}")
        plan = p.gpu._planned
        assert plan.n_slots > 0, "expected cut sequences"
        assert plan.n_work // (n_kv // min(n_kv, 4)) < len(lens), "expected several items per bin"


@pytest.mark.parametrize("geom", [(8, 32, 64), (1, 8, 64), (2, 32, 128)])
def test_merge_bits_do_not_depend_on_which_wave_merges(geom):
    """With one bin, every piece of a cut sequence runs before its last piece
    in the same wave, so the last piece always merges with its own partial
    from registers; with many bins whichever piece arrives last merges from
    stored partials. The outputs must be the same bits."""
    n_kv, n_heads, d = geom
    print(f"merge paths geom={geom}", flush=True)
    groups = n_kv // min(n_kv, 4)
    outs = []
    for wgs in (groups, 64 * groups):
        p = Pair(1, 512, 16, n_kv, n_heads, d, part_pages=2, decode_workgroups=wgs)
        p.poison(6)
        alloc, _keep = fragmented_allocator(512, 16)
        seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(6)]
        for s, n in zip(seqs, [1, 17, 63, 200, 333, 700]):
            s.append(n)
        res = p.step(grow_and_assemble(seqs, [1] * 6, 16), 30)
        check(res, f"workgroups {wgs}")
        outs.append(res[0][1].cpu())
    assert torch.equal(outs[0], outs[1])


def _shared_prefix_batch(alloc, n_seqs, prefix_tokens):
    """Radix-style sharing: n_seqs tables start with the same prefix blocks
    (refcounted); each then grows its own blocks."""
    pre = SequenceBlocks(alloc, seq_id=100)
    pre.append(prefix_tokens)
    seqs = []
    for i in range(n_seqs):
        s = SequenceBlocks(alloc, seq_id=i)
        alloc.incref(pre.block_ids)
        s.block_ids = list(pre.block_ids)
        s.num_tokens = prefix_tokens
        seqs.append(s)
    return pre, seqs


@pytest.mark.parametrize("geom", [(8, 32, 64), (2, 8, 128), (8, 8, 64), (1, 16, 64),
                                  (4, 8, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_chunked_prefill_over_shared_prefix(geom, dtype):
    """The chunked-prefill workload at reduced size: a prefix written once,
    shared by every table, then each sequence appends its own query chunk
    (causal within the chunk, full attention to the prefix)."""
    n_kv, n_heads, d = geom
    print(f"shared-prefix prefill geom={geom} dtype={dtype}", flush=True)
    p = Pair(2, 256, 16, n_kv, n_heads, d, dtype=dtype)
    assert p.gpu.q_tile == 128 // (n_heads // n_kv), "matrix-core prefill expected"
    alloc, _keep = fragmented_allocator(256, 16)
    # a whole number of pages, as a radix cache shares them (a partial last
    # page would be copied on write before a sequence appends into it)
    pre, seqs = _shared_prefix_batch(alloc, 3, 192)
    tol, rtol = (2e-3, 1e-2) if dtype == torch.float16 else (1.6e-2, 8e-2)
    check(p.step(make_meta([pre], [192], 16), 5, kv_scale=0.5), "prefix", tol, rtol)
    meta = grow_and_assemble(seqs, [150, 77, 1], 16)
    check(p.step(meta, 6, kv_scale=0.5), "chunk over shared prefix", tol, rtol)


@pytest.mark.parametrize("lens,hist", [([int(x) for x in np.random.default_rng(5).integers(1, 64, 300)], 0),
                                       ([300, 517, 64, 1000], 700)])
def test_prefill_bits_do_not_change_between_runs(lens, hist):
    """The prefill kernel's K/V tile ring (direct-to-LDS loads, one barrier
    a tile) gives the same bits on every run: a tile read before its loads
    have landed, or a buffer refilled while still read, shows up as
    run-to-run differences. Short sequences (one or two tiles each, many
    workgroups ending early) and chunks over a long history."""
    print(f"prefill determinism: {len(lens)} sequences, history {hist}", flush=True)
    bk = MI355XBackend(1, 2048, 16, 8, 32, 64, device=DEV)
    alloc = BlockAllocator(2048, 16)
    alloc.allocate(2048)
    alloc.free(torch.randperm(2048, generator=torch.Generator().manual_seed(3)).tolist())
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(lens))]
    g = torch.Generator(device=DEV).manual_seed(4)
    if hist:
        h = _to_dev(grow_and_assemble(seqs, [hist] * len(lens), 16))
        kv = [(torch.randn(h.n_tokens, 8, 64, generator=g, device=DEV) * 0.5).half()
              for _ in range(2)]
        bk.append_kv(0, kv[0], kv[1], h)
    meta = _to_dev(grow_and_assemble(seqs, lens, 16))
    T = meta.n_tokens
    k, v = [(torch.randn(T, 8, 64, generator=g, device=DEV) * 0.5).half() for _ in range(2)]
    q = (torch.randn(T, 32, 64, generator=g, device=DEV) * 0.5).half()
    bk.append_kv(0, k, v, meta)
    first = bk.attend(q, 0, 0.125, meta)
    for i in range(10):
        again = bk.attend(q, 0, 0.125, meta)
        assert torch.equal(first, again), f"run {i + 1} differs from the first"
    bk.check_device_errors()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_matrix_core_prefill_matches_generic_kernel(dtype):
    """Same batch through the MFMA prefill (default tile) and the generic
    kernel (a tile the MFMA kernel does not take): both within the bar of
    the oracle, and of each other."""
    print(f"mfma vs generic prefill dtype={dtype}", flush=True)
    outs = []
    for q_tile in (None, 17):
        p = Pair(1, 256, 16, 8, 32, 64, dtype=dtype, q_tile=q_tile)
        p.poison(3)
        alloc, _keep = fragmented_allocator(256, 16)
        seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(4)]
        for s, n in zip(seqs, [5, 40, 0, 130]):
            s.append(n)
        res = p.step(grow_and_assemble(seqs, [300, 33, 64, 1], 16), 9)
        tol, rtol = (2e-3, 1e-2) if dtype == torch.float16 else (1.6e-2, 8e-2)
        check(res, f"q_tile={q_tile}", tol, rtol)
        outs.append(res[0][1].float())
    diff = (outs[0] - outs[1]).abs().max().item()
    assert diff <= (4e-3 if dtype == torch.float16 else 3.2e-2), diff


@pytest.mark.parametrize("profile", ["rising", "falling", "alternating"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_running_reference_under_score_profiles(profile, dtype):
    """The matrix-core prefill keeps each row's softmax reference until some
    lane's sum of its probabilities passes 2^12 (then every probability it
    holds is at most 2^12), and only then takes the row max and rescales.
    Scores built to move the reference on every 32-key tile (rising by
    about 11 in log2 units a tile), never after the first (falling), or on
    every other tile (alternating), over a 600-token history and a
    300-token chunk, against the oracle."""
    print(f"prefill running reference: {profile} scores, {dtype}", flush=True)
    n_kv, n_heads, d = 8, 32, 64
    p = Pair(1, 256, 16, n_kv, n_heads, d, dtype=dtype)
    assert p.gpu.q_tile == 128 // (n_heads // n_kv), "matrix-core prefill expected"
    alloc, _keep = fragmented_allocator(256, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(2)]
    g = torch.Generator().manual_seed(31)
    u = torch.ones(d) / d ** 0.5

    def kv_rows(first, n):
        t = torch.arange(first, first + n, dtype=torch.float32)
        if profile == "rising":
            f = t / 32.0
        elif profile == "falling":
            f = (1000.0 - t) / 32.0
        else:
            f = torch.where((t // 32) % 2 == 0, t / 32.0, torch.zeros_like(t))
        # every KV head's key row along u, scaled by f(position), plus noise
        k = f[:, None, None] * u + 0.05 * torch.randn(n, n_kv, d, generator=g)
        v = torch.randn(n, n_kv, d, generator=g)
        return k.to(dtype), v.to(dtype)

    tol, rtol = (2e-3, 1e-2) if dtype == torch.float16 else (1.6e-2, 8e-2)
    for counts, first in (([600, 40], 0), ([300, 1], 600)):
        meta = grow_and_assemble(seqs, counts, 16)
        meta_gpu = _to_dev(meta)
        T = meta.n_tokens
        ks, vs = [], []
        for i, n in enumerate(counts):
            k, v = kv_rows(first if i == 0 else first // 15, n)
            ks.append(k)
            vs.append(v)
        k, v = torch.cat(ks), torch.cat(vs)
        # query rows along u: scores 64 * f(key) / 8, in log2 units x 0.18
        q = (64.0 * u + 0.05 * torch.randn(T, n_heads, d, generator=g)).to(dtype)
        p.gpu.append_kv(0, k.to(DEV), v.to(DEV), meta_gpu)
        out = p.gpu.attend(q.to(DEV), 0, 0.125, meta_gpu)
        p.ref.append_kv(0, k.float(), v.float(), meta)
        want = p.ref.attend(q.float(), 0, 0.125, meta)
        check([(0, out, want)], f"{profile} first={first}", tol, rtol)
    p.gpu.check_device_errors()


def test_prefill_with_a_negative_scale_matches_the_oracle():
    """The matrix-core prefill takes the row max before scaling, so it
    declines a non-positive scale; the generic kernel then serves the same
    plan. Either way the result is the oracle's."""
    print("prefill, negative scale", flush=True)
    p = Pair(1, 64, 16, 8, 32, 64)
    alloc = BlockAllocator(64, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(2)]
    res = p.step(grow_and_assemble(seqs, [70, 33], 16), 21, scale=-0.125)
    check(res, "negative scale")


def test_config1_fp16_fast_path_and_fp32_fixture():
    """The CPU plumbing case on the GPU: fp32 pools vs the golden float64
    outputs, fp16 pools (fast decode kernel) vs the fp32 oracle."""
    from .golden.make_config1 import build_inputs

    print("config1 fp32 + fp16", flush=True)
    fx = np.load(Path(__file__).resolve().parent / "golden" / "config1.npz", allow_pickle=False)
    inp = build_inputs()
    for dtype in (torch.float32, torch.float16):
        bk = MI355XBackend(1, inp["num_blocks"], 16, 8, 32, 64, device=DEV, dtype=dtype)
        hist, meta = _to_dev(inp["hist_meta"]), _to_dev(inp["meta"])
        cast = lambda a: torch.from_numpy(a).to(DEV, dtype)  # noqa: E731
        bk.append_kv(0, cast(inp["k_hist"]), cast(inp["v_hist"]), hist)
        bk.append_kv(0, cast(inp["k_new"]), cast(inp["v_new"]), meta)
        out = bk.attend(cast(inp["q"]), 0, 0.125, meta)
        bk.check_device_errors()
        if dtype == torch.float32:
            np.testing.assert_allclose(out.cpu().numpy(), fx["out_f64"], atol=1e-5, rtol=1e-5)
        else:
            ref = PagedTorchOracle(1, inp["num_blocks"], 16, 8, 32, 64)
            r = lambda a: torch.from_numpy(a).half().float()  # noqa: E731
            ref.append_kv(0, r(inp["k_hist"]), r(inp["v_hist"]), inp["hist_meta"])
            ref.append_kv(0, r(inp["k_new"]), r(inp["v_new"]), inp["meta"])
            want = ref.attend(r(inp["q"]), 0, 0.125, inp["meta"])
            assert_attention_close(out, want, label="config1 fp16")


@pytest.mark.parametrize("part_pages, mirror", [(4, True), (DEFAULT_PART_PAGES, True),
                                                (DEFAULT_PART_PAGES, False)])
def test_config2_batch256_one_layer_vs_oracle(part_pages, mirror):
    """Full decode-bench batch (256 sequences, lognormal mean 258), fused
    append then attend on two layers, at 4-page partitions and at the
    backend's default (the headline's setting); planned from the host
    mirror a serving loop's meta carries, and (``mirror=False``) from the
    device tensors read back."""
    print(f"config2 batch 256 parity part_pages={part_pages} mirror={mirror}", flush=True)
    lens = lognormal_lengths(256, 256, 0.8, 2048, 20260731)
    pages = sum(-(-(n + 1) // 16) for n in lens)
    nb = 2 * pages
    p = Pair(2, nb, 16, 8, 32, 64, part_pages=part_pages)
    g = torch.Generator().manual_seed(5)
    perm = torch.randperm(nb, generator=g).tolist()
    a = BlockAllocator(nb, 16)
    a.allocate(nb)
    a.free(perm)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(256)]
    hist = grow_and_assemble(seqs, lens, 16)
    gk = torch.Generator().manual_seed(6)
    T = hist.n_tokens
    for layer in range(2):
        k = (torch.randn(T, 8, 64, generator=gk) * 0.5).half()
        v = (torch.randn(T, 8, 64, generator=gk) * 0.5).half()
        p.gpu.append_kv(layer, k.to(DEV), v.to(DEV), _to_dev(hist))
        p.ref.append_kv(layer, k.float(), v.float(), hist)
    meta = grow_and_assemble(seqs, [1] * 256, 16)
    check(p.step(meta, 8, kv_scale=0.5, mirror=mirror), "config2")


# ------------------------------------------------------ known answers

def small(dtype=torch.float16, n_kv=2, n_heads=4, d=64, bs=16, nb=32):
    return MI355XBackend(1, nb, bs, n_kv, n_heads, d, device=DEV, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gqa_value_map_and_decode_sees_itself(dtype):
    print(f"gqa value map dtype={dtype}", flush=True)
    for n_kv, n_heads in ((2, 8), (8, 32), (1, 4)):
        bk = small(dtype, n_kv, n_heads)
        s = SequenceBlocks(BlockAllocator(32, 16))
        s.append(1)
        meta = make_meta([s], [1], 16, device=DEV)
        v = torch.zeros(1, n_kv, 64, device=DEV, dtype=dtype)
        for j in range(n_kv):
            v[0, j] = j + 1.0
        bk.append_kv(0, torch.zeros_like(v), v, meta)
        out = bk.attend(torch.randn(1, n_heads, 64, device=DEV, dtype=dtype), 0, 1.0, meta)
        groups = n_heads // n_kv
        for h in range(n_heads):
            assert torch.all(out[0, h] == h // groups + 1.0), (n_kv, n_heads, h)


def test_gqa_key_map():
    print("gqa key map", flush=True)
    bk = small(torch.float16, 2, 8)
    s = SequenceBlocks(BlockAllocator(32, 16))
    s.append(2)
    meta = make_meta([s], [2], 16, device=DEV)
    k = torch.zeros(2, 2, 64, device=DEV, dtype=torch.float16)
    v = torch.zeros_like(k)
    for j in range(2):
        k[0, j, j] = 50.0
        k[1, j, 2 + j] = 50.0
        v[0, j], v[1, j] = 1.0, -1.0
    bk.append_kv(0, k, v, meta)
    q = torch.zeros(2, 8, 64, device=DEV, dtype=torch.float16)
    for h in range(8):
        q[:, h, h // 4] = 1.0
    out = bk.attend(q, 0, 1.0, meta)
    assert (out[1, :, 0].float() > 0.99).all()


@pytest.mark.parametrize("n", [1, 15, 16, 17, 31, 32, 33])
def test_block_straddle_poisoned_decode(n):
    """The unwritten tail of the last page holds 1e3; reading it would be loud."""
    print(f"straddle n={n}", flush=True)
    p = Pair(1, 32, 16, 8, 32, 64)
    p.gpu._pool.fill_(1e3)
    for t in p.ref.k_pool + p.ref.v_pool:
        t.fill_(1e3)
    seqs = [SequenceBlocks(BlockAllocator(32, 16))]
    if n > 1:  # history as one prefill chunk, then the decode step reaching kv_len n
        check(p.step(grow_and_assemble(seqs, [n - 1], 16), 1), f"straddle prefill {n - 1}")
    check(p.step(grow_and_assemble(seqs, [1], 16), 2), f"straddle decode {n}")


def test_scattered_pages_equal_contiguous_and_batched_equals_solo():
    print("bitwise page-order / batch invariance", flush=True)
    g = torch.Generator().manual_seed(0)
    k = torch.randn(300, 8, 64, generator=g).half().to(DEV)
    v = torch.randn(300, 8, 64, generator=g).half().to(DEV)
    q = torch.randn(3, 32, 64, generator=g).half().to(DEV)
    outs = []
    for frag in (False, True):
        bk = MI355XBackend(1, 128, 16, 8, 32, 64, device=DEV)
        a = BlockAllocator(128, 16)
        if frag:
            a.allocate(128)
            a.free(list(range(127, 0, -3)))
        seqs = [SequenceBlocks(a, seq_id=i) for i in range(3)]
        lens = [100, 1, 199]
        meta = make_meta_grow(seqs, lens, device=DEV)
        bk.append_kv(0, k, v, meta)
        dmeta = make_meta_grow(seqs, [1, 1, 1], device=DEV)
        bk.append_kv(0, k[:3], v[:3], dmeta)
        batched = bk.attend(q, 0, 0.125, dmeta)
        outs.append(batched)
        for i in range(3):
            solo = bk.attend(q[i:i + 1], 0, 0.125, make_meta([seqs[i]], [1], 16, device=DEV))
            assert torch.equal(solo, batched[i:i + 1]), f"seq {i} changed when batched"
    assert torch.equal(outs[0], outs[1]), "physical page order changed the answer"


def make_meta_grow(seqs, counts, device):
    for s, n in zip(seqs, counts):
        s.append(n)
    return make_meta(seqs, counts, 16, device=device)


def test_isolation_and_causality_prefill():
    print("isolation + causality", flush=True)
    bk = small(torch.float16, 2, 8, nb=64)
    a = BlockAllocator(64, 16)
    lens = [3, 1, 20]
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(3)]
    meta = make_meta_grow(seqs, lens, device=DEV)
    vs = torch.cat([torch.full((n, 2, 64), i + 1.0) for i, n in enumerate(lens)]).half().to(DEV)
    bk.append_kv(0, torch.zeros_like(vs), vs, meta)
    out = bk.attend(torch.randn(24, 8, 64, device=DEV).half(), 0, 1.0, meta)
    cu = meta.cu_query_lens.tolist()
    for i in range(3):
        assert torch.all(out[cu[i]:cu[i + 1]] == i + 1.0)
    # causality: poisoning the last key changes only the last query's output
    s = [SequenceBlocks(a, seq_id=9)]
    m = make_meta_grow(s, [6], device=DEV)
    g = torch.Generator().manual_seed(3)
    bk.append_kv(0, torch.randn(6, 2, 64, generator=g).half().to(DEV),
                  torch.randn(6, 2, 64, generator=g).half().to(DEV), m)
    q = torch.randn(6, 8, 64, generator=g).half().to(DEV)
    base = bk.attend(q, 0, 0.125, m)
    slot = s[0].slot_for(5)
    bk.k_pool[0].view(-1, 2, 64)[slot] = 100.0
    bk.v_pool[0].view(-1, 2, 64)[slot] = -999.0
    pois = bk.attend(q, 0, 0.125, m)
    assert torch.equal(base[:5], pois[:5])
    assert not torch.allclose(base[5], pois[5])


def test_plan_once_per_step_and_prefill_hint_checked():
    print("plan caching + is_prefill cross-check", flush=True)
    p = Pair(4, 64, 16, 8, 32, 64)
    seqs = [SequenceBlocks(BlockAllocator(64, 16), seq_id=0)]
    p.step(grow_and_assemble(seqs, [20], 16), 1)
    assert p.gpu.n_plans == 1 and p.gpu.n_runs == 4
    p.step(grow_and_assemble(seqs, [1], 16), 2)
    assert p.gpu.n_plans == 2 and p.gpu.n_runs == 8
    meta = _to_dev(grow_and_assemble(seqs, [1], 16))
    bad = dataclasses.replace(meta, is_prefill=True)
    with pytest.raises(ValueError, match="is_prefill"):
        p.gpu.attend(torch.zeros(1, 32, 64, device=DEV, dtype=torch.float16), 0, 0.125, bad)


def test_plan_from_the_host_mirror_reads_nothing_back(monkeypatch):
    """A meta from build_batch_meta carries its host arrays: planning it, the
    fused append and the decode launch make no device-to-host copy. A meta
    without the mirror falls back to one read-back (caught the same way)."""
    print("sync-free planning", flush=True)
    from llm_serving_layer_amd import ScheduledSeq, build_batch_meta

    bk = MI355XBackend(2, 256, 16, 8, 32, 64, device=DEV)
    a = BlockAllocator(256, 16)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(5)]
    for s, n in zip(seqs, [3, 40, 170, 700, 16]):
        s.append(n)
    meta = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], DEV, 16)
    q = torch.randn(5, 32, 64, device=DEV).half()
    k = torch.randn(5, 8, 64, device=DEV).half()

    def no_readback(self, *args, **kwargs):
        raise AssertionError("device-to-host copy during planning")

    with monkeypatch.context() as m:
        m.setattr(torch.Tensor, "cpu", no_readback)
        for layer in range(2):
            bk.append_kv(layer, k, k, meta)
            out = bk.attend(q, layer, 0.125, meta)
        bare = dataclasses.replace(meta, host=None)
        with pytest.raises(AssertionError, match="device-to-host"):
            bk.attend(q, 0, 0.125, bare)
    assert bk.n_plans == 1
    bk.invalidate_plan()
    again = bk.attend(q, 1, 0.125, dataclasses.replace(meta, host=None))
    assert torch.equal(again, out), "mirror and read-back plans must agree"


def test_protocol_and_accounting():
    from llm_serving_layer_amd import AttentionBackend

    bk = MI355XBackend(16, 100, 16, 8, 32, 64, device=DEV)
    assert isinstance(bk, AttentionBackend)
    assert bk.block_bytes() == 512 * 1024
    assert bk.pool_bytes() == 100 * 512 * 1024 == MI355XBackend.estimate_pool_bytes(16, 100, 16, 8, 64)
    assert bk.tokens_capacity() == 1600
    assert tuple(bk.zeros_like_pool().shape) == (100, 16, 8, 64)
    for l in range(16):
        assert bk.k_pool[l].is_contiguous() and bk.v_pool[l].is_contiguous()
        assert tuple(bk.k_pool[l].shape) == (100, 16, 8, 64)


# ------------------------------------------- one launch per layer (fused append)

def _decode_batch(nb, lens, seed):
    a = BlockAllocator(nb, 16)
    a.allocate(nb)
    a.free(torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).tolist())
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(len(lens))]
    return seqs, grow_and_assemble(seqs, lens, 16)


@pytest.mark.parametrize("part_pages", [1, 3, 8, 16])
def test_fused_append_equals_separate_launches(part_pages):
    """Deferred append fused into attend == append kernel then attend, bitwise."""
    print(f"fused vs separate part_pages={part_pages}", flush=True)
    lens = [1, 15, 16, 17, 63, 64, 65, 200, 700, 1300]
    outs, pools = [], []
    for fuse in (True, False):
        bk = MI355XBackend(2, 512, 16, 8, 32, 64, device=DEV, part_pages=part_pages,
                           fuse_append=fuse)
        seqs, hist = _decode_batch(512, lens, 3)
        g = torch.Generator().manual_seed(4)
        hist = _to_dev(hist)
        T = hist.n_tokens
        for l in range(2):
            bk.append_kv(l, torch.randn(T, 8, 64, generator=g).half().to(DEV),
                         torch.randn(T, 8, 64, generator=g).half().to(DEV), hist)
        res = []
        for step in range(3):
            meta = _to_dev(grow_and_assemble(seqs, [1] * len(lens), 16))
            for l in range(2):
                k = torch.randn(len(lens), 8, 64, generator=g).half().to(DEV)
                v = torch.randn(len(lens), 8, 64, generator=g).half().to(DEV)
                q = torch.randn(len(lens), 32, 64, generator=g).half().to(DEV)
                bk.append_kv(l, k, v, meta)
                res.append(bk.attend(q, l, 0.125, meta))
        bk.check_device_errors()
        outs.append(torch.stack(res))
        pools.append(bk._pool.clone())
    assert torch.equal(outs[0], outs[1]), "fused append changed the attention output"
    assert torch.equal(pools[0], pools[1]), "fused append wrote different pool bytes"


def test_deferred_append_visible_through_pool_reads():
    print("deferred append flushed by a pool read", flush=True)
    bk = MI355XBackend(1, 64, 16, 8, 32, 64, device=DEV)
    seqs, hist = _decode_batch(64, [20, 5], 1)
    meta = _to_dev(grow_and_assemble(seqs, [1, 1], 16))
    k = torch.randn(2, 8, 64, device=DEV).half()
    v = torch.randn(2, 8, 64, device=DEV).half()
    bk.append_kv(0, k, v, meta)
    assert bk._pending is not None, "decode-shaped append on the fast path should defer"
    kf = bk.k_pool[0].view(-1, 8, 64)  # the property read lands the rows
    vf = bk.v_pool[0].view(-1, 8, 64)
    for t, s in enumerate(meta.slot_mapping.tolist()):
        assert torch.equal(kf[s], k[t]) and torch.equal(vf[s], v[t])


def test_inplace_modification_before_fused_launch_raises():
    print("in-place modification detection", flush=True)
    bk = MI355XBackend(1, 64, 16, 8, 32, 64, device=DEV)
    seqs, _ = _decode_batch(64, [20], 1)
    meta = _to_dev(grow_and_assemble(seqs, [1], 16))
    k = torch.randn(1, 8, 64, device=DEV).half()
    bk.append_kv(0, k, k.clone(), meta)
    k.add_(1.0)
    with pytest.raises(RuntimeError, match="modified in place"):
        bk.attend(torch.randn(1, 32, 64, device=DEV).half(), 0, 0.125, meta)


def test_fused_append_with_slot_mapping_off_the_page_table():
    """slot_mapping naming a slot other than the page table's last position:
    the row lands in slot_mapping's slot and attention reads the table's slot,
    exactly as append-then-attend does in the oracle."""
    print("fused append, slot_mapping disagreeing with the page table", flush=True)
    p = Pair(1, 64, 16, 8, 32, 64)
    p.poison(7)
    seqs, hist = _decode_batch(64, [30, 40], 2)
    check(p.step(hist, 1), "history")
    meta = grow_and_assemble(seqs, [1, 1], 16)
    free_page = next(b for b in range(64) if b not in meta.kv_indices.tolist())
    odd = dataclasses.replace(meta, slot_mapping=torch.tensor(
        [free_page * 16 + 3, int(meta.slot_mapping[1])], dtype=torch.int32))
    res = p.step(odd, 2)
    check(res, "off-table slot")
    assert torch.equal(p.gpu.k_pool[0].float().cpu(), p.ref.k_pool[0]), "pool bytes differ"


# ------------------------------------- packs of short sequences (no split)

@pytest.mark.parametrize("part_pages,workgroups", [(5, 16), (10, 64), (64, 512), (10, 2)])
def test_packed_short_sequences_vs_oracle(part_pages, workgroups):
    """A batch of short sequences (the 4096-sequence capacity batch is of this
    kind): a bin of the plan streams many whole sequences one after another
    with the fused append; every decode matches the oracle across the
    sequence switches inside a bin."""
    print(f"packed short sequences part_pages={part_pages} workgroups={workgroups}", flush=True)
    rng = np.random.default_rng(part_pages)
    lens = [int(x) for x in rng.integers(1, 64, 300)] + [16, 17, 1, 64]
    p = Pair(1, 1024, 16, 8, 32, 64, part_pages=part_pages, decode_workgroups=workgroups)
    alloc = BlockAllocator(1024, 16)
    alloc.allocate(1024)
    alloc.free(torch.randperm(1024, generator=torch.Generator().manual_seed(2)).tolist())
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(lens))]
    check(p.step(grow_and_assemble(seqs, lens, 16), 1), "packed history")
    for step in range(2):
        meta = grow_and_assemble(seqs, [1] * len(lens), 16)
        check(p.step(meta, 10 + step), f"packed decode step {step}")
        plan = p.gpu._planned
        assert plan.n_work // 2 < len(lens), "expected several sequences per bin"


def test_packed_sequence_equals_solo_bitwise():
    """A sequence decoded inside a pack gives the same bits as decoded alone,
    and as inside a batch whose other sequences are split."""
    print("packed vs solo vs split-batch bitwise", flush=True)
    g = torch.Generator().manual_seed(9)
    lens = [5, 40, 100, 17, 63]
    bk = MI355XBackend(1, 256, 16, 8, 32, 64, device=DEV, part_pages=64, decode_workgroups=2)
    a = BlockAllocator(256, 16)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(len(lens) + 1)]
    hist = make_meta_grow(seqs[:-1], lens, device=DEV)
    T = sum(lens)
    bk.append_kv(0, torch.randn(T, 8, 64, generator=g).half().to(DEV),
                 torch.randn(T, 8, 64, generator=g).half().to(DEV), hist)
    long_hist = make_meta_grow(seqs[-1:], [1100], device=DEV)   # 69 pages: split
    bk.append_kv(0, torch.randn(1100, 8, 64, generator=g).half().to(DEV),
                 torch.randn(1100, 8, 64, generator=g).half().to(DEV), long_hist)
    q = torch.randn(len(seqs), 32, 64, generator=g).half().to(DEV)
    for s in seqs:
        s.append(1)
    packed = bk.attend(q[:-1], 0, 0.125, make_meta(seqs[:-1], [1] * len(lens), 16, device=DEV))
    assert bk._planned.n_slots == 0 and bk._planned.n_work == 2, "expected one bin"
    mixed = bk.attend(q, 0, 0.125, make_meta(seqs, [1] * len(seqs), 16, device=DEV))
    assert bk._planned.n_slots > 0, "expected the long sequence to be split"
    for i in range(len(lens)):
        solo = bk.attend(q[i:i + 1], 0, 0.125, make_meta([seqs[i]], [1], 16, device=DEV))
        assert torch.equal(solo, packed[i:i + 1]), f"seq {i}: pack changed the bits"
        assert torch.equal(solo, mixed[i:i + 1]), f"seq {i}: split batch changed the bits"


def test_mixed_batch_equals_solo_bitwise():
    """Prefill chunks and one-token decodes in one batch: each decode token's
    output has the same bits as the same decode run alone (the decodes of a
    mixed batch take the decode kernel), each prefill chunk the same bits as
    that chunk run alone, and the whole batch matches the oracle."""
    print("mixed prefill + decode batch", flush=True)
    p = Pair(1, 256, 16, 8, 32, 64, part_pages=4)
    a = BlockAllocator(256, 16)
    seqs = [SequenceBlocks(a, seq_id=i) for i in range(5)]
    check(p.step(grow_and_assemble(seqs, [40, 300, 7, 90, 500], 16), 1), "mixed history")
    meta = grow_and_assemble(seqs, [1, 24, 1, 70, 1], 16)
    res = p.step(meta, 2)
    check(res, "mixed step")
    assert p.gpu._planned.dec is not None and p.gpu._planned.dec.n == 3
    mixed = res[0][1]
    cu = meta.cu_query_lens.tolist()
    g = torch.Generator().manual_seed(2)   # the q the step drew (after k, v)
    T = meta.n_tokens
    p.rand((T, 8, 64), g), p.rand((T, 8, 64), g)
    q = p.rand((T, 32, 64), g).to(DEV)
    for i in (0, 2, 4):
        solo = p.gpu.attend(q[cu[i]:cu[i] + 1], 0, 0.125,
                            make_meta([seqs[i]], [1], 16, device=DEV))
        assert torch.equal(solo, mixed[cu[i]:cu[i] + 1]), f"decode {i} changed beside prefills"
    # and every prefill chunk of the mixed batch equals its solo run, bitwise
    # (the reference's batched == solo, tests/test_paged_torch.py:541-587)
    for i, ql in ((1, 24), (3, 70)):
        solo = p.gpu.attend(q[cu[i]:cu[i] + ql], 0, 0.125,
                            make_meta([seqs[i]], [ql], 16, device=DEV))
        assert torch.equal(solo, mixed[cu[i]:cu[i] + ql]), f"prefill {i} changed when batched"


@pytest.mark.parametrize("geom", [(8, 32, 128), (2, 32, 64), (8, 8, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_packed_decode_other_geometries(geom, dtype):
    """Packs at head_dim 128, 16 query heads per KV head and MHA, fp16 and
    bf16: a decode batch of short sequences (no split) against the oracle."""
    n_kv, n_heads, d = geom
    print(f"packed decode geom={geom} dtype={dtype}", flush=True)
    tol, rtol = (2e-3, 1e-2) if dtype == torch.float16 else (1.6e-2, 8e-2)
    p = Pair(1, 512, 16, n_kv, n_heads, d, dtype=dtype, part_pages=8, decode_workgroups=16)
    alloc = BlockAllocator(512, 16)
    rng = np.random.default_rng(d + n_heads)
    lens = [int(x) for x in rng.integers(1, 110, 60)]
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(lens))]
    check(p.step(grow_and_assemble(seqs, lens, 16), 1), "history", tol, rtol)
    check(p.step(grow_and_assemble(seqs, [1] * len(lens), 16), 2), "packed step", tol, rtol)
    assert p.gpu._planned.n_work < len(lens), "several sequences per bin"
