"""
The per-step batch description and the attention-backend protocol.

The reference imports both types from its engine submodule
(``engine.attention_backend``, imported at serving/backends/paged_torch.py:66
and serving/engine_iface/batch.py:62), which is not vendored. They are
restated here from their documented contract:

* fields and dtypes: docs/ARCHITECTURE.md:92-117;
* protocol and per-layer call order: docs/ARCHITECTURE.md:152-174;
* ``validate()`` behaviour, including the message fragments callers match
  (``kv_last_page_len``, ``pages allocated``, ``batch_indices``):
  tests/test_batch_assembly.py:345-384;
* ``n_seqs`` / ``n_tokens``: tests/test_batch_assembly.py:67-69,132.

``BatchMeta`` is frozen: one object describes one forward pass and is passed,
unchanged, to every layer's ``append_kv`` and ``attend``. Backends rely on
that to cache a launch plan by object identity.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional, Protocol, runtime_checkable

import numpy as np
import torch

__all__ = ["BatchMeta", "HostMirror", "AttentionBackend", "validate_host"]

#: The index fields a host mirror may carry, in this order.
MIRRORED = ("query_lens", "cu_query_lens", "kv_lens", "kv_indptr", "kv_indices",
            "kv_last_page_len", "slot_mapping")


@dataclass(frozen=True, eq=False)
class HostMirror:
    """
    Host (int64 numpy) copies of a BatchMeta's index fields, kept by the
    assembler that built them, so a backend can plan a step without reading
    the device tensors back. ``of`` holds the device tensors the arrays
    describe; the mirror speaks for a BatchMeta only while its fields are
    those very tensors (``BatchMeta.host_arrays``), so a meta rebuilt with
    ``dataclasses.replace`` never plans from stale arrays.
    """

    arrays: dict
    of: tuple


@dataclass(frozen=True)
class BatchMeta:
    """
    One forward pass over a ragged batch.

    Tokens of all sequences are packed along axis 0 in sequence order;
    sequence ``i`` owns ``[cu_query_lens[i], cu_query_lens[i + 1])``.

    query_lens        (n,)    int32  new tokens of each sequence this step
    cu_query_lens     (n+1,)  int32  exclusive prefix sum of query_lens
    kv_lens           (n,)    int32  KV length AFTER this step's append
    positions         (T,)    int64  absolute position of each new token
    kv_indptr         (n+1,)  int32  CSR row pointer into kv_indices
    kv_indices        (P,)    int32  physical page ids, sequence after sequence
    kv_last_page_len  (n,)    int32  tokens on each sequence's last page, 1..page_size
    batch_indices     (T,)    int32  owning sequence of each new token
    slot_mapping      (T,)    int32  flat pool slot of each new token (or None)
    last_token_ix     (n,)    int32  packed index of each sequence's last token
    page_size         tokens per page
    is_prefill        hint: True iff some sequence contributes > 1 token
    """

    query_lens: torch.Tensor
    cu_query_lens: torch.Tensor
    kv_lens: torch.Tensor
    positions: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    batch_indices: torch.Tensor
    slot_mapping: Optional[torch.Tensor]
    last_token_ix: torch.Tensor
    page_size: int = 16
    is_prefill: bool = False
    host: Optional[HostMirror] = field(default=None, compare=False, repr=False)

    def host_arrays(self) -> Optional[dict]:
        """The host mirror's arrays if it still describes this meta's fields
        (same tensor objects), else None: the caller then reads the device."""
        h = self.host
        if h is None or len(h.of) != len(MIRRORED):
            return None
        for name, t in zip(MIRRORED, h.of):
            if getattr(self, name) is not t:
                return None
        return h.arrays

    @property
    def n_seqs(self) -> int:
        return int(self.query_lens.shape[0])

    @property
    def n_tokens(self) -> int:
        # Shape-derived on purpose: backends compare it once per layer and a
        # value read (cu_query_lens[-1]) would cost a device sync each time.
        return int(self.positions.shape[0])

    def validate(self) -> None:
        """
        Assert every structural invariant whose violation would otherwise be
        silent (wrong pages read, a page dropped, a token routed to another
        sequence). Raises ``AssertionError``. Pulls the fields to the host
        in one transfer; it is meant for batch assembly, not for the
        per-layer path.
        """
        names = ("query_lens", "cu_query_lens", "kv_lens", "kv_indptr", "kv_last_page_len",
                 "last_token_ix", "positions", "batch_indices")
        ts = [getattr(self, k).detach().reshape(-1) for k in names]
        flat = torch.cat([t.to(torch.int64) for t in ts]).to("cpu").numpy()
        parts, off = [], 0
        for t in ts:
            parts.append(flat[off:off + t.shape[0]])
            off += t.shape[0]
        n_slots = None if self.slot_mapping is None else int(self.slot_mapping.shape[0])
        validate_host(self.n_seqs, int(self.page_size), *parts, n_slots=n_slots,
                      n_pages=int(self.kv_indices.shape[0]))


def validate_host(n: int, ps: int, ql, cu, kv, indptr, last, ltok, pos, bidx, *,
                  n_slots: Optional[int], n_pages: int) -> None:
    """
    BatchMeta's invariants over host int64 arrays. The common case (all
    hold) is checked with array operations; on any violation the
    sequence-by-sequence walk below reports the first one, in a fixed order.
    """
    ql, cu, kv, indptr, last, ltok, pos, bidx = (
        np.asarray(x, dtype=np.int64) for x in (ql, cu, kv, indptr, last, ltok, pos, bidx))
    ok = (ps > 0 and n > 0 and kv.shape[0] == n and last.shape[0] == n and ltok.shape[0] == n
          and ql.shape[0] == n and cu.shape[0] == n + 1 and indptr.shape[0] == n + 1)
    if ok:
        tokens = int(cu[-1])
        ok = (cu[0] == 0 and bool((np.diff(cu) == ql).all()) and pos.shape[0] == tokens
              and bidx.shape[0] == tokens and (n_slots is None or n_slots == tokens)
              and indptr[0] == 0 and indptr[-1] == n_pages)
    if ok:
        pages = np.diff(indptr)
        ok = bool(((last >= 1) & (last <= ps) & (ql >= 1) & (ql <= kv)
                   & (pages == (kv + ps - 1) // ps) & (kv - (pages - 1) * ps == last)
                   & (ltok == cu[1:] - 1)).all())
    if ok:
        owner = np.repeat(np.arange(n, dtype=np.int64), ql)
        ok = bool((bidx == owner).all()
                  and (pos == np.arange(tokens, dtype=np.int64) + (kv - ql - cu[:-1])[owner]).all())
    if not ok:
        _walk(n, ps, [int(x) for x in ql], [int(x) for x in cu], [int(x) for x in kv],
              [int(x) for x in indptr], [int(x) for x in last], [int(x) for x in ltok],
              [int(x) for x in pos], [int(x) for x in bidx], n_slots, n_pages)


def _walk(n, ps, ql, cu, kv, indptr, last, ltok, pos, bidx, n_slots, n_pages) -> None:
    assert ps > 0, f"page_size must be positive, got {ps}"
    assert n > 0, "BatchMeta describes no sequences"
    for name, vals in (("kv_lens", kv), ("kv_last_page_len", last),
                       ("last_token_ix", ltok), ("query_lens", ql)):
        assert len(vals) == n, f"{name} has {len(vals)} entries for {n} sequences"
    assert len(cu) == n + 1, f"cu_query_lens has {len(cu)} entries, expected {n + 1}"
    assert len(indptr) == n + 1, f"kv_indptr has {len(indptr)} entries, expected {n + 1}"

    assert cu[0] == 0, f"cu_query_lens must start at 0, got {cu[0]}"
    for i in range(n):
        assert cu[i + 1] - cu[i] == ql[i], (
            f"cu_query_lens {cu[i]}..{cu[i + 1]} disagrees with query_lens[{i}]={ql[i]}"
        )
    tokens = cu[-1]
    assert len(pos) == tokens, f"positions has {len(pos)} entries for {tokens} tokens"
    assert len(bidx) == tokens, (
        f"batch_indices has {len(bidx)} entries for {tokens} tokens"
    )
    if n_slots is not None:
        assert n_slots == tokens, f"slot_mapping has {n_slots} entries for {tokens} tokens"

    assert indptr[0] == 0, f"kv_indptr must start at 0, got {indptr[0]}"
    assert indptr[-1] == n_pages, (
        f"kv_indptr ends at {indptr[-1]} but kv_indices holds {n_pages} pages"
    )

    for i in range(n):
        assert 1 <= last[i] <= ps, (
            f"seq {i}: kv_last_page_len={last[i]} outside [1, {ps}]; an exact "
            f"multiple of page_size reports {ps}, never 0"
        )
        assert 1 <= ql[i] <= kv[i], (
            f"seq {i}: query_len={ql[i]} must lie in [1, kv_len={kv[i]}]"
        )
        pages = indptr[i + 1] - indptr[i]
        need = (kv[i] + ps - 1) // ps
        assert pages == need, (
            f"seq {i}: kv_len={kv[i]} needs {need} pages but {pages} pages allocated"
        )
        assert kv[i] - (pages - 1) * ps == last[i], (
            f"seq {i}: kv_last_page_len={last[i]} but kv_len={kv[i]} over "
            f"{pages} pages implies {kv[i] - (pages - 1) * ps}"
        )
        assert ltok[i] == cu[i + 1] - 1, (
            f"seq {i}: last_token_ix={ltok[i]}, expected {cu[i + 1] - 1}"
        )
        for j in range(ql[i]):
            t = cu[i] + j
            assert bidx[t] == i, f"batch_indices[{t}]={bidx[t]}, expected {i}"
            want = kv[i] - ql[i] + j
            assert pos[t] == want, (
                f"positions[{t}]={pos[t]}, expected absolute position {want}"
            )
    # is_prefill is a hint, not an invariant: backends that dispatch on it
    # cross-check it against query_lens themselves and raise ValueError.
    raise AssertionError("BatchMeta invariants disagree between checks")  # unreachable


@runtime_checkable
class AttentionBackend(Protocol):
    """
    What a model's forward pass calls, per layer, in this order
    (docs/ARCHITECTURE.md:166-174): ``append_kv`` then ``attend``, so a
    decoding token attends to the K/V it just wrote.
    """

    def append_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
                  meta: BatchMeta) -> None:
        """Write this step's ``(tokens, n_kv_heads, head_dim)`` K/V into the pool."""

    def attend(self, q: torch.Tensor, layer_idx: int, scale: float,
               meta: BatchMeta) -> torch.Tensor:
        """Causal (bottom-right) GQA attention; returns a new tensor shaped like q."""
