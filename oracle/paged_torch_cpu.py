"""
ORACLE — test infrastructure, not product code.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this module, and only to check results against (or, for the
baseline, as the timed CPU restatement). The product path never calls it.

A CPU restatement of the reference's pure-PyTorch paged backend,
serving/backends/paged_torch.py, op for op and at the same precisions:

* constructor validation and messages ............ paged_torch.py:95-109
* per-layer K and V pools [NB, bs, Hkv, d] ....... paged_torch.py:127-137
* accounting (pool/block bytes, capacity) ........ paged_torch.py:148-177
* copy_block (every layer, K and V) .............. paged_torch.py:181-207
* append_kv: flat-slot scatter via slot_mapping .. paged_torch.py:209-276
* attend: host-side loop over sequences .......... paged_torch.py:280-346
* _gather: CSR page gather, truncate to kv_len ... paged_torch.py:348-398
* _attend_one: repeat_interleave GQA, fp32 scores, bottom-right triu mask
  when q_len > 1, fp32 softmax, cast to pool dtype, PV matmul in pool
  dtype ....................................... paged_torch.py:400-485

How the restatement is pinned (tests/test_oracle.py): against an independent
float64 textbook attention (oracle/naive.py) and the reference tests' known
answers (kv_len==1 => out==V, GQA value/key maps, isolation, causality
poison, block straddle over a poisoned pool, non-contiguous == contiguous
bitwise, batched == solo bitwise), and against the committed golden fixture
under tests/golden/.
"""

from __future__ import annotations

import torch

__all__ = ["PagedTorchOracle"]


class PagedTorchOracle:
    """Same constructor, pool layout and methods as the reference's backend."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int,
                 n_kv_heads: int, n_heads: int, head_dim: int,
                 device="cpu", dtype: torch.dtype = torch.float32):
        if n_heads % n_kv_heads != 0:
            raise ValueError(
                f"n_heads={n_heads} must be divisible by n_kv_heads={n_kv_heads}; "
                "GQA maps query head h to KV head h // (n_heads // n_kv_heads)."
            )
        for name, val in (("num_layers", num_layers), ("num_blocks", num_blocks),
                          ("block_size", block_size), ("n_kv_heads", n_kv_heads),
                          ("n_heads", n_heads), ("head_dim", head_dim)):
            if val <= 0:
                raise ValueError(f"{name} must be positive, got {val}")
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.n_kv_heads, self.n_heads, self.head_dim = n_kv_heads, n_heads, head_dim
        self.device = torch.device(device)
        self.dtype = dtype
        self.groups = n_heads // n_kv_heads
        shape = (num_blocks, block_size, n_kv_heads, head_dim)
        self.k_pool = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(num_layers)]
        self.v_pool = [torch.zeros(shape, dtype=dtype, device=self.device) for _ in range(num_layers)]

    # accounting (paged_torch.py:148-177)
    def pool_bytes(self) -> int:
        return self.num_layers * 2 * self.k_pool[0].numel() * self.k_pool[0].element_size()

    def block_bytes(self) -> int:
        return self.pool_bytes() // self.num_blocks

    def tokens_capacity(self) -> int:
        return self.num_blocks * self.block_size

    # write path (paged_torch.py:181-276)
    def copy_block(self, src: int, dst: int) -> None:
        if not (0 <= src < self.num_blocks and 0 <= dst < self.num_blocks):
            raise IndexError(f"copy_block({src} -> {dst}) outside [0, {self.num_blocks})")
        if src == dst:
            return
        for layer in range(self.num_layers):
            self.k_pool[layer][dst].copy_(self.k_pool[layer][src])
            self.v_pool[layer][dst].copy_(self.v_pool[layer][src])

    def append_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, meta) -> None:
        self._check_layer(layer_idx)
        if meta.slot_mapping is None:
            raise ValueError("append_kv requires meta.slot_mapping")
        tokens = k.shape[0]
        if tuple(k.shape) != (tokens, self.n_kv_heads, self.head_dim):
            raise ValueError(f"k has shape {tuple(k.shape)}, expected "
                             f"({tokens}, {self.n_kv_heads}, {self.head_dim})")
        if v.shape != k.shape:
            raise ValueError(f"v shape {tuple(v.shape)} != k shape {tuple(k.shape)}")
        if meta.slot_mapping.shape[0] != tokens:
            raise ValueError(f"slot_mapping has {meta.slot_mapping.shape[0]} entries but "
                             f"{tokens} tokens were supplied")
        slots = meta.slot_mapping.to(device=self.device, dtype=torch.long)
        kf = self.k_pool[layer_idx].view(-1, self.n_kv_heads, self.head_dim)
        vf = self.v_pool[layer_idx].view(-1, self.n_kv_heads, self.head_dim)
        kf[slots] = k.to(device=self.device, dtype=self.dtype)
        vf[slots] = v.to(device=self.device, dtype=self.dtype)

    # read path (paged_torch.py:280-485)
    def attend(self, q: torch.Tensor, layer_idx: int, scale: float, meta) -> torch.Tensor:
        self._check_layer(layer_idx)
        tokens = q.shape[0]
        if tuple(q.shape) != (tokens, self.n_heads, self.head_dim):
            raise ValueError(f"q has shape {tuple(q.shape)}, expected "
                             f"({tokens}, {self.n_heads}, {self.head_dim})")
        q = q.to(self.device)
        out = torch.empty_like(q)
        cu_q = meta.cu_query_lens.tolist()
        q_lens = meta.query_lens.tolist()
        kv_lens = meta.kv_lens.tolist()
        indptr = meta.kv_indptr.tolist()
        indices = meta.kv_indices.to(device=self.device, dtype=torch.long)
        last = meta.kv_last_page_len.tolist()
        for i in range(len(q_lens)):
            a, b = cu_q[i], cu_q[i + 1]
            if q_lens[i] == 0:
                continue
            pages = indices[indptr[i]:indptr[i + 1]]
            ks, vs = self._gather(layer_idx, pages, kv_lens[i], last[i])
            out[a:b] = self._attend_one(q[a:b], ks, vs, scale, q_lens[i], kv_lens[i])
        return out

    def _gather(self, layer_idx: int, pages: torch.Tensor, kv_len: int, last_page_len: int):
        n_pages = pages.shape[0]
        need = (kv_len + self.block_size - 1) // self.block_size
        if n_pages != need:
            raise ValueError(f"{n_pages} pages supplied but kv_len={kv_len} with "
                             f"block_size={self.block_size} needs {need}")
        tail = kv_len - (n_pages - 1) * self.block_size
        if last_page_len != tail:
            raise ValueError(f"kv_last_page_len={last_page_len} but kv_len={kv_len} over "
                             f"{n_pages} pages implies {tail}")
        k = self.k_pool[layer_idx][pages].reshape(-1, self.n_kv_heads, self.head_dim)
        v = self.v_pool[layer_idx][pages].reshape(-1, self.n_kv_heads, self.head_dim)
        return k[:kv_len], v[:kv_len]

    def _attend_one(self, q, k, v, scale, q_len, kv_len):
        k = torch.repeat_interleave(k, self.groups, dim=1)
        v = torch.repeat_interleave(v, self.groups, dim=1)
        qh, kh, vh = q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)
        scores = torch.matmul(qh.float(), kh.float().transpose(1, 2)) * scale
        if q_len > 1:
            mask = torch.triu(torch.full((q_len, kv_len), float("-inf"), device=scores.device),
                              diagonal=kv_len - q_len + 1)
            scores = scores + mask.unsqueeze(0)
        probs = torch.softmax(scores, dim=-1).to(self.dtype)
        return torch.matmul(probs, vh).transpose(0, 1)

    def _check_layer(self, layer_idx) -> None:
        if layer_idx is None or not 0 <= layer_idx < self.num_layers:
            raise ValueError(f"layer_idx {layer_idx} out of range [0, {self.num_layers})")

    def reset(self) -> None:
        for t in self.k_pool + self.v_pool:
            t.zero_()
