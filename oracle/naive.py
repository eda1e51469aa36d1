"""
ORACLE — test infrastructure, not product code (see oracle/paged_torch_cpu.py
for who may import it).

Independent reference computations, written in a style that shares nothing with the kernels
or with the op-for-op restatement:

* ``naive_attention`` — textbook causal GQA attention on DENSE, unpaged K/V,
  explicit loops over heads and queries, float64, masking by not summing the
  disallowed keys. Follows the reference's own independent naive attention,
  tests/test_paged_torch.py:106-149 (query j may see keys
  [0, kv_len - q_len + j]; query head h reads KV head h // groups).
* numpy closed forms for the pure data movement the reference performs with
  torch indexing:
  - ``append_closed_form``: ``pool_flat[slot_mapping[t]] = x[t]``
    (serving/backends/paged_torch.py:270-276);
  - ``copy_blocks_closed_form``: every layer, K and V, ``pool[dst] = pool[src]``
    (serving/backends/paged_torch.py:199-207), applied pair by pair;
  - ``gather_closed_form`` / ``scatter_closed_form``: the swap copies
    ``host[l] = pool[l][ids]`` and ``pool[l][ids] = host[l]``
    (serving/scheduler/preemption.py:490-523).
* ``greedy_ids``: the scheduler's greedy pick, ``torch.argmax(logits,
  dim=-1)`` (serving/scheduler/scheduler.py:752-757), as an explicit scan.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = ["naive_attention", "append_closed_form", "copy_blocks_closed_form",
           "gather_closed_form", "scatter_closed_form", "greedy_ids"]


def naive_attention(q: np.ndarray, k_full: np.ndarray, v_full: np.ndarray,
                    scale: float, n_kv_heads: int) -> np.ndarray:
    """q (q_len, H, d); k/v_full (kv_len, Hkv, d) -> (q_len, H, d) float64."""
    q = np.asarray(q, dtype=np.float64)
    k_full = np.asarray(k_full, dtype=np.float64)
    v_full = np.asarray(v_full, dtype=np.float64)
    q_len, n_heads, d = q.shape
    kv_len = k_full.shape[0]
    groups = n_heads // n_kv_heads
    out = np.zeros((q_len, n_heads, d), dtype=np.float64)
    for h in range(n_heads):
        kvh = h // groups
        for j in range(q_len):
            last = kv_len - q_len + j
            s = [float(np.dot(q[j, h], k_full[t, kvh])) * scale for t in range(last + 1)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            tot = sum(w)
            acc = np.zeros(d, dtype=np.float64)
            for t in range(last + 1):
                acc += (w[t] / tot) * v_full[t, kvh]
            out[j, h] = acc
    return out


def append_closed_form(pool: np.ndarray, x: np.ndarray, slots) -> np.ndarray:
    """pool (NB, bs, Hkv, d); x (T, Hkv, d). Returns the updated copy."""
    out = pool.copy()
    flat = out.reshape(-1, *pool.shape[2:])
    for t, s in enumerate(slots):
        flat[int(s)] = x[t]
    return out


def copy_blocks_closed_form(k_pools: list, v_pools: list, pairs) -> tuple[list, list]:
    """Lists of per-layer (NB, ...) arrays; sequential pair-by-pair semantics."""
    ks = [p.copy() for p in k_pools]
    vs = [p.copy() for p in v_pools]
    for src, dst in pairs:
        if src == dst:
            continue
        for layer in range(len(ks)):
            ks[layer][dst] = ks[layer][src]
            vs[layer][dst] = vs[layer][src]
    return ks, vs


def gather_closed_form(pools: list, ids) -> np.ndarray:
    """(L, len(ids), bs, Hkv, d): host[l, i] = pool[l][ids[i]]."""
    return np.stack([p[np.asarray(ids, dtype=np.int64)] for p in pools])


def scatter_closed_form(pools: list, host: np.ndarray, ids) -> list:
    out = [p.copy() for p in pools]
    for layer, p in enumerate(out):
        for i, b in enumerate(ids):
            p[int(b)] = host[layer, i]
    return out



def greedy_ids(logits) -> list[int]:
    """
    The greedy token of every row of ``logits`` (n_rows, vocab), the order
    torch.argmax(logits, dim=-1) uses (serving/scheduler/scheduler.py:
    752-757): a NaN beats every number (torch's max reductions propagate
    NaN), a larger value beats a smaller one, and of equal values the first
    wins. An explicit scan over each row, in float64.
    """
    out = []
    for row in np.asarray(logits, dtype=np.float64):
        best, bi = None, -1
        for i, v in enumerate(row.tolist()):
            if bi < 0:
                best, bi = v, i
            elif math.isnan(best):
                continue
            elif math.isnan(v) or v > best:
                best, bi = v, i
        out.append(bi)
    return out

