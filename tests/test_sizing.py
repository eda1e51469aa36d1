"""
Pool sizing (llm_serving_layer_amd/sizing.py) against the reference's own
sizing tests (tests/test_sizing.py:46-200, 371-438), restated, plus the
MI355X-side additions: a measured budget and the decode workspace charged to
the same budget.
"""

from __future__ import annotations

import ctypes as C
import json
import random

import numpy as np
import pytest

from llm_serving_layer_amd import _native

from ._util import plan_decode
from llm_serving_layer_amd.sizing import (DEFAULT_PART_PAGES, LLAMA_3_2_1B, MI355X_HBM_BYTES,
                                          SizingError, block_bytes, decode_workspace_bound,
                                          decode_workspace_slots, kv_bytes_per_token,
                                          plan_kv_pool)

KIB, MIB, GIB = 1024, 1024**2, 1024**3


def test_kv_bytes_per_token_llama_3_2_1b_is_exactly_32_kib():
    # 2 (K, V) x 16 layers x 8 KV heads (not 32 query heads) x 64 x 2 bytes
    assert kv_bytes_per_token(16, 8, 64, 2) == 32768
    assert kv_bytes_per_token() == 32768
    assert LLAMA_3_2_1B.bytes_per_token() == 32 * KIB


def test_kv_bytes_per_token_scales_linearly_in_every_term():
    base = kv_bytes_per_token(16, 8, 64, 2)
    assert kv_bytes_per_token(32, 8, 64, 2) == 2 * base
    assert kv_bytes_per_token(16, 16, 64, 2) == 2 * base
    assert kv_bytes_per_token(16, 8, 128, 2) == 2 * base
    assert kv_bytes_per_token(16, 8, 64, 4) == 2 * base
    assert kv_bytes_per_token(16, 8, 64, 1) == base // 2


@pytest.mark.parametrize("kwargs", [{"n_layers": 0}, {"n_kv_heads": 0}, {"head_dim": -64},
                                    {"dtype_bytes": 0}])
def test_kv_bytes_per_token_rejects_nonpositive_shape(kwargs):
    with pytest.raises(SizingError):
        kv_bytes_per_token(**kwargs)


def test_block_bytes_at_block_size_16_is_512_kib():
    assert block_bytes(16) == 524288 == 512 * KIB
    for bs in (1, 8, 16, 32, 64, 128):
        assert block_bytes(bs) == bs * 32768
    with pytest.raises(SizingError):
        block_bytes(0)


def test_block_bytes_is_the_backend_pool_stride():
    """One block of the single pool allocation, over every layer, K and V."""
    from llm_serving_layer_amd.backend import MI355XBackend

    assert MI355XBackend.estimate_pool_bytes(16, 1, 16, 8, 64) == block_bytes(16)


def test_without_workspace_the_plan_is_the_reference_floor_division():
    """max_batch_seqs=0 reserves nothing: num_blocks = floor(available / block)."""
    plan = plan_kv_pool(total_vram_bytes=40 * GIB, max_batch_seqs=0)
    assert plan.available_bytes == 40 * GIB - int(2357.1 * MIB) - 2 * GIB
    assert plan.num_blocks == plan.available_bytes // plan.bytes_per_block
    assert 0 <= plan.bytes_leftover < plan.bytes_per_block
    # the reference's A100 band (tests/test_sizing.py:158-171)
    assert 65_000 <= plan.num_blocks <= 75_000
    assert 1_000_000 <= plan.tokens_capacity <= 1_250_000


def test_mi355x_plan_by_hand():
    """288 GiB - 2357.1 MiB weights - 2 GiB headroom = 304,618,563,175 B; at
    512 KiB a block that is 581,013 blocks before the workspace, and the
    worst-case decode workspace of a 4096-sequence batch costs under 2000."""
    bare = plan_kv_pool(max_batch_seqs=0)
    assert bare.total_vram_bytes == MI355X_HBM_BYTES == 309_237_645_312
    assert bare.available_bytes == 304_618_563_175
    assert bare.num_blocks == 581_013
    plan = plan_kv_pool()
    assert 0 < bare.num_blocks - plan.num_blocks < 2000
    assert plan.workspace_bytes == decode_workspace_bound(plan.num_blocks, 4096, 32, 8, 64,
                                                          DEFAULT_PART_PAGES)
    # ~200 GB capacity pool of the capacity workload fits with room to spare
    assert plan.num_blocks > 381_469


def test_plan_is_self_consistent_one_more_block_would_not_fit():
    plan = plan_kv_pool()
    ws_next = decode_workspace_bound(plan.num_blocks + 1, 4096, 32, 8, 64,
                                     DEFAULT_PART_PAGES)
    assert plan.num_blocks * plan.bytes_per_block + plan.workspace_bytes <= plan.available_bytes
    assert (plan.num_blocks + 1) * plan.bytes_per_block + ws_next > plan.available_bytes
    assert plan.is_self_consistent()
    assert plan.bytes_used == plan.num_blocks * plan.bytes_per_block
    assert plan.bytes_leftover == plan.available_bytes - plan.bytes_used - plan.workspace_bytes
    assert plan.tokens_capacity == plan.num_blocks * plan.block_size


@pytest.mark.parametrize("block_size", [1, 8, 16, 32, 64, 256])
@pytest.mark.parametrize("headroom_gib", [0, 1, 2, 8])
@pytest.mark.parametrize("max_seqs", [0, 256, 4096])
def test_plan_self_consistent_across_configurations(block_size, headroom_gib, max_seqs):
    plan = plan_kv_pool(activation_headroom_bytes=headroom_gib * GIB, block_size=block_size,
                        max_batch_seqs=max_seqs)
    assert plan.is_self_consistent()


def _plan_slots(kv_lens, part_pages, ps=16):
    """(pages, n_slots) of the library's decode plan for these lengths."""
    indptr, _, _, n_slots = plan_decode(kv_lens, part_pages, 512, ps=ps)
    return int(indptr[-1]), n_slots


@pytest.mark.parametrize("part_pages", [1, 3, 10, 64])
def test_workspace_bound_covers_every_batch_the_pool_can_hold(part_pages):
    """Batches that fill a 2000-block pool in many shapes, including the
    worst case for the bound (every sequence one page over a partition):
    the workspace the library asks for never exceeds the reserved bound."""
    num_blocks, ps = 2000, 16
    rng = random.Random(part_pages)
    fill = []
    while sum(-(-k // ps) for k in fill) + 256 <= num_blocks:
        fill.append(rng.randint(1, 4096))
    shapes = [[part_pages * ps + 1] * (num_blocks // (part_pages + 1)), fill,
              [num_blocks * ps]]
    for lens in shapes:
        pages, slots = _plan_slots(lens, part_pages)
        assert pages <= num_blocks
        need = _native.load().pkv_decode_workspace_bytes(len(lens), max(slots, 1), 32, 8, 64)
        for shared in (False, True):  # distinct blocks: both bounds hold
            assert need <= decode_workspace_bound(num_blocks, max(len(lens), 1), 32, 8, 64,
                                                  part_pages, max_seq_len=max(lens),
                                                  shared_blocks=shared)


@pytest.mark.parametrize("part_pages", [3, 10, 64])
def test_workspace_bound_holds_under_radix_prefix_sharing(part_pages):
    """64 sequences share one 120-page prefix (refcounted blocks, as the radix
    cache shares them) and own one page each: the batch references 7744
    pages of a 200-block pool. The slots the library's plan really takes
    exceed the distinct-block bound floor(2 N / part_pages), and stay within
    the bound reserved for shared blocks."""
    num_blocks, n = 200, 64
    lens = [120 * 16 + 1 + i % 16 for i in range(n)]      # 121 pages, <= 2048 tokens
    pages, slots = _plan_slots(lens, part_pages)
    assert pages == n * 121 > num_blocks
    need = _native.load().pkv_decode_workspace_bytes(n, slots, 32, 8, 64)
    distinct = decode_workspace_bound(num_blocks, n, 32, 8, 64, part_pages,
                                      shared_blocks=False)
    shared = decode_workspace_bound(num_blocks, n, 32, 8, 64, part_pages)
    assert need > distinct, "the distinct-block bound must not be used with sharing"
    assert need <= shared
    assert decode_workspace_slots(num_blocks, n, part_pages) >= slots


def test_derivation_is_printable_and_shows_the_arithmetic():
    plan = plan_kv_pool()
    text = plan.explain()
    for token in (f"{plan.bytes_per_token:,}", f"{plan.bytes_per_block:,}",
                  f"{plan.available_bytes:,}", f"{plan.num_blocks:,}",
                  f"{plan.tokens_capacity:,}", f"{plan.workspace_bytes:,}"):
        assert token in text, f"derivation omits {token}"
    assert len(plan.derivation()) >= 8
    json.dumps(plan.as_dict())


def test_sequences_at_length_rounds_up_to_whole_blocks():
    plan = plan_kv_pool()
    assert plan.sequences_at_length(16) == plan.num_blocks
    assert plan.sequences_at_length(17) == plan.num_blocks // 2
    with pytest.raises(SizingError):
        plan.sequences_at_length(0)


def test_weights_larger_than_vram_raises_and_names_the_problem():
    with pytest.raises(SizingError, match="exceed total VRAM"):
        plan_kv_pool(total_vram_bytes=2 * GIB, model_weight_bytes=8 * GIB)


def test_headroom_consuming_all_remaining_vram_raises():
    with pytest.raises(SizingError, match="No VRAM left"):
        plan_kv_pool(total_vram_bytes=8 * GIB, model_weight_bytes=4 * GIB,
                     activation_headroom_bytes=4 * GIB)


def test_available_memory_smaller_than_one_block_raises_not_zero_blocks():
    with pytest.raises(SizingError, match="smaller than one block"):
        plan_kv_pool(total_vram_bytes=4 * GIB, model_weight_bytes=4 * GIB - 100_000,
                     activation_headroom_bytes=0, block_size=16)


@pytest.mark.parametrize("bad", [0, -1])
def test_nonpositive_vram_raises(bad):
    with pytest.raises(SizingError):
        plan_kv_pool(total_vram_bytes=bad)


def test_negative_headroom_raises():
    with pytest.raises(SizingError):
        plan_kv_pool(activation_headroom_bytes=-1)


def test_no_sizing_path_ever_returns_a_nonpositive_block_count():
    for weights_gib in range(0, 289, 24):
        for headroom_gib in (0, 2, 16, 287):
            try:
                plan = plan_kv_pool(model_weight_bytes=weights_gib * GIB,
                                    activation_headroom_bytes=headroom_gib * GIB)
            except SizingError:
                continue
            assert plan.num_blocks >= 1 and plan.is_self_consistent()


def test_measured_budget_needs_a_gpu():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; the measured plan is covered by the GPU test")
    with pytest.raises(SizingError, match="GPU"):
        plan_kv_pool(total_vram_bytes=None)
    with pytest.raises(SizingError, match="GPU device"):
        plan_kv_pool(total_vram_bytes=None, device="cpu")


@pytest.mark.gpu
def test_measured_plan_fits_the_free_memory_of_the_device():
    """A plan on the device's measured free HBM: the pool and its workspace
    fit in what the runtime reports free, and a backend built from a plan of
    a small slice of it allocates exactly the planned pool."""
    import torch

    free, total = torch.cuda.mem_get_info(0)
    plan = plan_kv_pool(total_vram_bytes=None, model_weight_bytes=0,
                        activation_headroom_bytes=4 * GIB, device="cuda:0")
    assert plan.measured and plan.total_vram_bytes <= total
    assert plan.bytes_used + plan.workspace_bytes <= free
    assert plan.is_self_consistent()
    small = plan_kv_pool(total_vram_bytes=256 * MIB, model_weight_bytes=0,
                         activation_headroom_bytes=0, max_batch_seqs=64)
    bk = small.backend(device="cuda:0")
    assert bk.num_blocks == small.num_blocks and bk.pool_bytes() == small.bytes_used
    assert bk.block_bytes() == small.bytes_per_block
    # the plan's decode workspace is allocated up front, for its partition size
    assert small.workspace_bytes > 0
    assert bk.workspace_bytes() == small.workspace_bytes
    assert bk.part_pages == small.part_pages


def test_plan_backend_forwards_its_workspace_and_partition_size(monkeypatch):
    """KVPoolPlan.backend() builds the backend with the decode workspace the
    plan reserved and the partition size it was reserved for (so a batch
    within the plan's limits never allocates during a step); explicit
    keyword arguments still win."""
    import llm_serving_layer_amd.backend as backend_mod

    seen = {}

    class Recorder:
        def __init__(self, *args, **kwargs):
            seen.clear()
            seen.update(kwargs)
            seen["args"] = args

    monkeypatch.setattr(backend_mod, "MI355XBackend", Recorder)
    plan = plan_kv_pool(total_vram_bytes=256 * MIB, model_weight_bytes=0,
                        activation_headroom_bytes=0, max_batch_seqs=64, part_pages=12)
    plan.backend(device="cpu")
    assert seen["decode_workspace_bytes"] == plan.workspace_bytes > 0
    assert seen["part_pages"] == 12
    assert seen["args"][:2] == (plan.shape.n_layers, plan.num_blocks)
    plan.backend(device="cpu", part_pages=20, decode_workspace_bytes=0)
    assert seen["part_pages"] == 20 and seen["decode_workspace_bytes"] == 0
