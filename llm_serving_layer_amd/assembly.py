"""
Scheduler state -> ``BatchMeta``.

Follows serving/engine_iface/batch.py:77-318 in behaviour: each sequence's
block table must already be grown to include this step's tokens, positions
are absolute (``kv_len - q .. kv_len - 1``), the CSR triple comes from
``build_csr``, and the same rejections with the same message fragments
(``has been freed``, ``contributes 0 tokens``, ``blocks.append``,
``page_size``).

Different from the reference in two respects that matter on MI355X: all ten
index arrays (the int64 positions included) are packed into ONE pinned host
buffer and uploaded with ONE non-blocking copy, then exposed as views (ten separate ``torch.tensor(...,
device=...)`` calls are ten synchronous H2D round trips per step); and the
host arrays stay attached to the meta (``BatchMeta.host``), so a backend
plans the step from them instead of copying the device tensors back.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from itertools import chain
from operator import attrgetter

import numpy as np
import torch

from .contract import MIRRORED, BatchMeta, HostMirror, validate_host
from .paging import SequenceBlocks
from .upload import uploader

_BLOCKS = attrgetter("blocks")
_NEW_IDS = attrgetter("new_token_ids")
_NUM_TOKENS = attrgetter("num_tokens")
_BLOCK_IDS = attrgetter("block_ids")
_BLOCK_SIZE = attrgetter("block_size")
_IS_FREED = attrgetter("is_freed")

__all__ = ["ScheduledSeq", "build_batch_meta", "build_token_tensor"]


@dataclass
class ScheduledSeq:
    """One sequence's contribution to one step; ``blocks`` is already grown."""

    blocks: SequenceBlocks
    new_token_ids: list[int] = field(default_factory=list)
    wants_logits: bool = True

    @property
    def query_len(self) -> int:
        return len(self.new_token_ids)

    @property
    def kv_len(self) -> int:
        return self.blocks.num_tokens

    @property
    def start_position(self) -> int:
        return self.kv_len - self.query_len

    def positions(self) -> list[int]:
        return list(range(self.start_position, self.kv_len))


def _check_seq(i: int, s: ScheduledSeq) -> None:
    sid = s.blocks.seq_id
    if s.blocks.is_freed:
        raise ValueError(f"seq {i} (seq_id={sid}) has been freed; its pages may belong "
                         "to another sequence")
    q, k = s.query_len, s.kv_len
    if q <= 0:
        raise ValueError(f"seq {i} (seq_id={sid}) contributes {q} tokens; a sequence "
                         "with nothing to run must not be in the batch")
    if q > k:
        raise ValueError(f"seq {i} (seq_id={sid}) contributes {q} tokens but its block "
                         f"table holds only {k}: blocks.append() must run before assembly")
    if k > s.blocks.capacity:
        raise ValueError(f"seq {i} (seq_id={sid}) claims kv_len={k} but its "
                         f"{s.blocks.num_blocks} blocks hold {s.blocks.capacity} tokens")


def build_token_tensor(seqs: list[ScheduledSeq], device) -> torch.Tensor:
    flat: list[int] = []
    for i, s in enumerate(seqs):
        _check_seq(i, s)
        flat.extend(s.new_token_ids)
    return torch.tensor(flat, dtype=torch.int64, device=device)


def build_batch_meta(seqs: list[ScheduledSeq], device, page_size: int,
                     dtype_index: torch.dtype = torch.int32,
                     validate: bool = True) -> BatchMeta:
    if not seqs:
        raise ValueError("build_batch_meta() called with an empty sequence list")
    if page_size <= 0:
        raise ValueError(f"page_size must be positive, got {page_size}")

    # Per-sequence scalars in one pass each; the index arrays below are built
    # with array operations from them and the concatenated page lists.
    # (map over attribute getters: the per-sequence work stays in C)
    n = len(seqs)
    blocks = list(map(_BLOCKS, seqs))
    qlens = np.fromiter(map(len, map(_NEW_IDS, seqs)), np.int64, n)
    kvlens = np.fromiter(map(_NUM_TOKENS, blocks), np.int64, n)
    id_lists = list(map(_BLOCK_IDS, blocks))
    nblk = np.fromiter(map(len, id_lists), np.int64, n)
    bsz = np.fromiter(map(_BLOCK_SIZE, blocks), np.int64, n)
    freed = np.fromiter(map(_IS_FREED, blocks), bool, n)
    bad = freed | (qlens <= 0) | (qlens > kvlens) | (kvlens > nblk * bsz) | (bsz != page_size)
    if bad.any():  # the first offender raises the per-sequence message
        i = int(np.argmax(bad))
        _check_seq(i, seqs[i])
        raise ValueError(f"seq {i} (seq_id={blocks[i].seq_id}) has block_size="
                         f"{blocks[i].block_size} but the batch declares "
                         f"page_size={page_size}")

    cu = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(qlens, out=cu[1:])
    T = int(cu[-1])
    batch_idx = np.repeat(np.arange(n), qlens)
    # absolute positions kv_len - q .. kv_len - 1 of each sequence's tokens
    positions = np.arange(T, dtype=np.int64) + (kvlens - qlens - cu[:-1])[batch_idx]
    indptr = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(nblk, out=indptr[1:])
    indices = np.fromiter(chain.from_iterable(id_lists), np.int64, int(indptr[-1]))
    last = kvlens % page_size
    last[last == 0] = page_size
    # slot = block_ids[p // page_size] * page_size + p % page_size
    slots = (indices[indptr[:-1][batch_idx] + positions // page_size] * page_size
             + positions % page_size)

    parts = {
        "query_lens": qlens, "cu_query_lens": cu, "kv_lens": kvlens,
        "last_token_ix": cu[1:] - 1, "kv_indptr": indptr,
        "kv_indices": indices, "kv_last_page_len": last,
        "batch_indices": batch_idx, "slot_mapping": slots,
    }
    if validate:  # on the host arrays, before anything reaches the device
        validate_host(n, page_size, qlens, cu, kvlens, indptr, last, cu[1:] - 1, positions,
                      batch_idx, n_slots=T, n_pages=int(indices.shape[0]))
    fields = _upload(parts, positions, device, dtype_index)
    # the host arrays travel with the meta, so planning needs no read-back
    mirror = HostMirror(arrays={k: parts[k] for k in MIRRORED},
                        of=tuple(fields[k] for k in MIRRORED))
    return BatchMeta(**fields, page_size=page_size, is_prefill=bool((qlens > 1).any()),
                     host=mirror)


def _upload(parts: dict, positions: np.ndarray, device, dtype_index: torch.dtype) -> dict:
    """Pack every index array and the int64 positions into one pinned host
    buffer, move it with one upload (upload.py), and expose typed views of
    the device copy."""
    device = torch.device(device)
    idx_np = {torch.int32: np.int32, torch.int64: np.int64}[dtype_index]
    isz = np.dtype(idx_np).itemsize
    names = list(parts)
    sizes = [parts[k].shape[0] for k in names]
    total = sum(sizes)
    pos_off = -(-total * isz // 8) * 8            # positions start 8-byte aligned
    nbytes = pos_off + 8 * positions.shape[0]
    up = uploader(device) if device.type == "cuda" else None
    host = up.buffer(nbytes) if up is not None else torch.empty(nbytes, dtype=torch.uint8)
    hb = host.numpy()
    hv = hb[:total * isz].view(idx_np)
    off = 0
    for k, sz in zip(names, sizes):
        hv[off:off + sz] = parts[k]
        off += sz
    hb[pos_off:].view(np.int64)[:] = positions
    dev = up.send(host) if up is not None else host
    idx = dev[:total * isz].view(dtype_index)
    out, off = {}, 0
    for k, sz in zip(names, sizes):
        out[k] = idx[off:off + sz]
        off += sz
    out["positions"] = dev[pos_off:].view(torch.int64)
    return out
