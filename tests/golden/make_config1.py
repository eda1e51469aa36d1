"""
Golden fixture for the CPU plumbing case (one layer, fp32, Llama-3.2-1B
attention geometry: 32 query heads, 8 KV heads, head_dim 64, block_size 16,
pool of 1024 blocks; four sequences with histories {17, 64, 130, 255}; each
block table a consecutive slice of a seeded permutation of the pool; Q/K/V
~ N(0, 1); append one token per sequence, then one decode step at scale 1/8).

The inputs are regenerated from the seed (numpy PCG64) by ``build_inputs``;
the fixture stores what must not depend on the code under test:

* ``out_f64``      — textbook float64 attention on the dense histories
                     (oracle/naive.py), shape (4, 32, 64);
* ``pool_sha256``  — digest of the fp32 K then V pool after both appends,
                     computed with the numpy closed form of the scatter;
* ``input_sha256`` — digest of the generated inputs, to detect generator drift.

Run ``python -m tests.golden.make_config1`` from the repo root to rewrite it.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import torch

SEED = 20260731
HQ, HKV, D, BS, NB = 32, 8, 64, 16, 1024
HIST = [17, 64, 130, 255]
OUT = Path(__file__).resolve().parent / "config1.npz"


def meta_from_tables(tables, kv_lens, q_lens, page_size, device="cpu"):
    """A validated BatchMeta from explicit page lists (post-append kv_lens)."""
    from llm_serving_layer_amd import BatchMeta

    n = len(tables)
    indptr, indices, last, slots, pos, bidx, cu = [0], [], [], [], [], [], [0]
    for i, (tab, kv, ql) in enumerate(zip(tables, kv_lens, q_lens)):
        np_ = -(-kv // page_size)
        indices.extend(tab[:np_])
        indptr.append(len(indices))
        last.append(kv % page_size or page_size)
        for p in range(kv - ql, kv):
            slots.append(tab[p // page_size] * page_size + p % page_size)
            pos.append(p)
            bidx.append(i)
        cu.append(cu[-1] + ql)

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    meta = BatchMeta(query_lens=i32(q_lens), cu_query_lens=i32(cu), kv_lens=i32(kv_lens),
                     positions=torch.tensor(pos, dtype=torch.int64, device=device),
                     kv_indptr=i32(indptr), kv_indices=i32(indices), kv_last_page_len=i32(last),
                     batch_indices=i32(bidx), slot_mapping=i32(slots),
                     last_token_ix=i32([cu[i + 1] - 1 for i in range(n)]),
                     page_size=page_size, is_prefill=any(q > 1 for q in q_lens))
    meta.validate()
    return meta


def build_inputs() -> dict:
    rng = np.random.default_rng(SEED)
    perm = rng.permutation(NB)
    final = [h + 1 for h in HIST]
    tables, off = [], 0
    for kv in final:
        np_ = -(-kv // BS)
        tables.append([int(x) for x in perm[off:off + np_]])
        off += np_
    k_hist = rng.standard_normal((sum(HIST), HKV, D), dtype=np.float32)
    v_hist = rng.standard_normal((sum(HIST), HKV, D), dtype=np.float32)
    k_new = rng.standard_normal((4, HKV, D), dtype=np.float32)
    v_new = rng.standard_normal((4, HKV, D), dtype=np.float32)
    q = rng.standard_normal((4, HQ, D), dtype=np.float32)
    return {
        "num_blocks": NB, "tables": tables, "k_hist": k_hist, "v_hist": v_hist,
        "k_new": k_new, "v_new": v_new, "q": q,
        "hist_meta": meta_from_tables(tables, HIST, HIST, BS),
        "meta": meta_from_tables(tables, final, [1] * 4, BS),
    }


def input_digest(inp: dict) -> str:
    h = hashlib.sha256()
    for key in ("k_hist", "v_hist", "k_new", "v_new", "q"):
        h.update(inp[key].tobytes())
    h.update(repr(inp["tables"]).encode())
    return h.hexdigest()


def expected(inp: dict) -> tuple[np.ndarray, str]:
    import sys

    sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
    from oracle.naive import append_closed_form, naive_attention

    out = np.zeros((4, HQ, D), dtype=np.float64)
    offs = np.concatenate([[0], np.cumsum(HIST)])
    for i in range(4):
        k = np.concatenate([inp["k_hist"][offs[i]:offs[i + 1]], inp["k_new"][i:i + 1]])
        v = np.concatenate([inp["v_hist"][offs[i]:offs[i + 1]], inp["v_new"][i:i + 1]])
        out[i] = naive_attention(inp["q"][i:i + 1], k, v, 0.125, HKV)[0]
    pool = np.zeros((NB, BS, HKV, D), dtype=np.float32)
    kp = append_closed_form(pool, inp["k_hist"], inp["hist_meta"].slot_mapping.tolist())
    kp = append_closed_form(kp, inp["k_new"], inp["meta"].slot_mapping.tolist())
    vp = append_closed_form(pool, inp["v_hist"], inp["hist_meta"].slot_mapping.tolist())
    vp = append_closed_form(vp, inp["v_new"], inp["meta"].slot_mapping.tolist())
    return out, hashlib.sha256(kp.tobytes() + vp.tobytes()).hexdigest()


def main() -> None:
    inp = build_inputs()
    out, pool_digest = expected(inp)
    np.savez(OUT, out_f64=out, pool_sha256=np.array(pool_digest),
             input_sha256=np.array(input_digest(inp)))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
