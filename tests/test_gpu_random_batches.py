"""
Seeded random batches against the fp32 oracle: random geometry (GQA group
sizes 1..16, head_dim 64 and 128), partition size, decode grid size,
sequence count and lengths, on a fragmented pool, with fp16 and bf16
pools. Each case prefills a ragged chunk beside one-token decodes (a mixed
batch), then runs decode steps with the append fused into attention, two
layers each, every step compared with the oracle (paged_torch.py:280-485
restated in oracle/paged_torch_cpu.py) at the tolerance of its dtype.
"""

from __future__ import annotations

import random

import pytest
import torch

from llm_serving_layer_amd import SequenceBlocks

from ._util import fragmented_allocator, grow_and_assemble
from .test_gpu_attention import Pair, check

pytestmark = pytest.mark.gpu

GEOMS = [(8, 32, 64), (2, 8, 128), (4, 8, 64), (1, 8, 64), (8, 8, 64), (2, 32, 128),
         (4, 16, 64)]


def _case(seed: int) -> dict:
    r = random.Random(seed)
    n_kv, n_heads, d = r.choice(GEOMS)
    n = r.randint(1, 40)
    return dict(
        geom=(n_kv, n_heads, d), n=n,
        part_pages=r.choice([1, 2, 5, 13, 20, 40]),
        groups=r.choice([None, 1, 2, 8]),
        hist=[int(r.lognormvariate(4.5, 1.0)) % 400 + 1 for _ in range(n)],
        chunk=[r.choice([1, 1, r.randint(2, 40)]) for _ in range(n)],
        decode_steps=r.randint(2, 4),
    )


@pytest.mark.parametrize("seed", range(48))
def test_random_batch_vs_oracle(seed):
    _run(seed, torch.float16, 2e-3, 1e-2)


@pytest.mark.parametrize("seed", range(100, 116))
def test_random_batch_bf16_vs_oracle(seed):
    _run(seed, torch.bfloat16, 1.6e-2, 8e-2)   # bf16 rounds p to 8 bits


def _run(seed, dtype, atol, rtol):
    c = _case(seed)
    print(f"random batch seed={seed} {dtype} {c['geom']} n={c['n']} "
          f"part_pages={c['part_pages']} groups={c['groups']}", flush=True)
    n_kv, n_heads, d = c["geom"]
    pages = sum(-(-(h + x + c["decode_steps"]) // 16) for h, x in zip(c["hist"], c["chunk"]))
    nb = max(64, 2 * pages + 16)
    hgw = 4 if n_kv % 4 == 0 else 2 if n_kv % 2 == 0 else 1
    wgs = None if c["groups"] is None else c["groups"] * (n_kv // hgw)
    p = Pair(2, nb, 16, n_kv, n_heads, d, dtype=dtype, part_pages=c["part_pages"],
             decode_workgroups=wgs)
    p.poison(seed)
    alloc, _keep = fragmented_allocator(nb, 16)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(c["n"])]
    # history (one prefill of each sequence's first tokens), then the mixed step
    check(p.step(grow_and_assemble(seqs, c["hist"], 16), 1000 + seed), f"seed {seed} history",
          atol, rtol)
    check(p.step(grow_and_assemble(seqs, c["chunk"], 16), 2000 + seed), f"seed {seed} mixed",
          atol, rtol)
    for i in range(c["decode_steps"]):
        check(p.step(grow_and_assemble(seqs, [1] * c["n"], 16), 3000 + 10 * seed + i),
              f"seed {seed} decode {i}", atol, rtol)
