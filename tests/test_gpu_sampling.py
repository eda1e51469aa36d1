"""
Greedy sampling on the GPU (pkv_argmax_rows through ``sampling.greedy``)
against the reference's call, torch.argmax(logits, dim=-1)
(serving/scheduler/scheduler.py:752-757), bit for bit on the index, and
against the oracle's scan on small rows: f16, bf16 and f32 logits, vocab
sizes from 1 to past Llama-3's 128 256, batches of 1 to 300 rows, rows
that tie, hold NaN or are all -inf, and rows that are strided or not
16-byte aligned.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import greedy_ids

from llm_serving_layer_amd import _native
from llm_serving_layer_amd.sampling import StepTimer, greedy

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(1, 1), (3, 7), (5, 97), (256, 1000), (17, 32000),
                                        (256, 128256), (2, 151939)])
def test_greedy_equals_torch_argmax(dtype, rows, vocab):
    print(f"greedy {dtype} rows={rows} vocab={vocab}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * 131 + vocab)
    x = (torch.randn(rows, vocab, generator=g, device=DEV) * 4).to(dtype)
    got = greedy(x)
    assert got.dtype == torch.int64 and got.shape == (rows,)
    assert torch.equal(got, torch.argmax(x, dim=-1))
    if vocab <= 1000:
        assert got.tolist() == greedy_ids(x.float().cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_greedy_ties_nan_and_infinities(dtype):
    print(f"greedy special rows {dtype}", flush=True)
    vocab = 5000
    x = torch.randn(8, vocab, device=DEV).to(dtype)
    x[0, 17] = x[0, 4000] = 100          # tie of the max: the first
    x[1, :] = 3                          # all equal: index 0
    x[2, 2500] = math.nan                # NaN beats everything
    x[3, 10] = math.nan                  # two NaNs: the first
    x[3, 9] = math.nan
    x[4, :] = -math.inf                  # all -inf: index 0
    x[5, 4999] = math.inf                # +inf at the very end
    x[6, 0] = 50                         # max at index 0
    x[7, 4999] = 50                      # max at the last index
    got = greedy(x)
    assert got.tolist() == greedy_ids(x.float().cpu().numpy())
    assert torch.equal(got, torch.argmax(x, dim=-1))
    assert got.tolist()[:6] == [17, 0, 2500, 9, 0, 4999]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_greedy_single_max_or_nan_at_every_position(dtype):
    """One row per position p of the first 80 (every element of several
    16-byte chunks): the row's only maximum at p, a runner-up 40 further on;
    then the same rows with a NaN at p instead, and a NaN at p after a
    larger NaN-free maximum. Rows are 16-byte aligned (vocab 4096)."""
    print(f"greedy every position {dtype}", flush=True)
    vocab, n = 4096, 80
    x = torch.zeros(n, vocab, device=DEV, dtype=dtype)
    idx = torch.arange(n, device=DEV)
    x[idx, idx] = 5
    x[idx, idx + 40] = 3
    assert greedy(x).tolist() == list(range(n))
    y = torch.zeros(n, vocab, device=DEV, dtype=dtype)
    y[idx, idx] = math.nan
    y[idx, (idx + 7) % n] = 9
    assert greedy(y).tolist() == list(range(n))
    assert torch.equal(greedy(y), torch.argmax(y, dim=-1))


def test_greedy_strided_and_unaligned_rows():
    """Rows taken from a wider tensor (row stride > vocab) and starting at
    an odd element (no 16-byte alignment)."""
    print("greedy strided / unaligned rows", flush=True)
    wide = torch.randn(33, 4101, device=DEV).half()
    for view in (wide[:, :4000], wide[:, 1:4001], wide[:, 3:]):
        assert torch.equal(greedy(view), torch.argmax(view, dim=-1))


def test_greedy_overlapping_and_transposed_rows():
    """Views whose rows overlap in memory (an expanded row: row stride 0; an
    as_strided view with a row stride below vocab) or whose elements are
    strided are read through a contiguous copy, never past the allocation."""
    print("greedy overlapping / transposed rows", flush=True)
    row = torch.randn(1, 5000, device=DEV).half()
    flat = torch.randn(6000, device=DEV).half()
    sq = torch.randn(300, 300, device=DEV)
    for view in (row.expand(64, 5000), flat.as_strided((8, 5000), (100, 1)), sq.t(),
                 row.expand(1, 5000)):
        assert torch.equal(greedy(view), torch.argmax(view, dim=-1))


def test_argmax_rows_rejects_bad_arguments():
    lib = _native.load()
    out = torch.empty(2, dtype=torch.int64, device=DEV)
    x = torch.zeros(2, 10, device=DEV)
    for args in ((x.data_ptr(), 2, 0, 10), (x.data_ptr(), 2, 10, 9), (x.data_ptr(), -1, 10, 10)):
        rc = lib.pkv_argmax_rows(*args, _native.DTYPE_F32, out.data_ptr(), None)
        with pytest.raises(ValueError):
            _native.check(rc, "argmax")
    assert lib.pkv_argmax_rows(x.data_ptr(), 0, 10, 10, _native.DTYPE_F32, out.data_ptr(),
                               None) == 0


def test_step_timer_times_the_stream():
    """Events bracket work on torch's current stream; the elapsed time is
    read at the declared synchronisation point and kept in history."""
    print("step timer", flush=True)
    t = StepTimer(DEV)
    x = torch.randn(256, 128256, device=DEV).half()
    t.start()
    for _ in range(20):
        ids = greedy(x)
    t.stop()
    ms = t.elapsed_ms()
    assert ms > 0 and t.history == [ms]
    assert torch.equal(ids, torch.argmax(x, dim=-1))
    with pytest.raises(RuntimeError):
        t.stop()
