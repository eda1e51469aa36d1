"""
MI355XBackend — a third implementation of the attention-backend contract,
next to the reference's PagedTorchBackend (serving/backends/paged_torch.py)
and FlashInferBackend (serving/backends/flashinfer_backend.py), running on
hand-written gfx950 kernels through the C ABI in include/pagedkv.h.

Drop-in surface (same as both reference backends):

* constructor ``(num_layers, num_blocks, block_size, n_kv_heads, n_heads,
  head_dim, device="cuda:0", dtype=torch.float16, *, ...)`` with the same
  validation and messages (paged_torch.py:95-109), checked BEFORE the native
  library is touched so errors do not depend on the machine
  (flashinfer_backend.py:271-300);
* ``k_pool[l]`` / ``v_pool[l]``: per-layer contiguous
  ``[num_blocks, block_size, n_kv_heads, head_dim]`` tensors
  (paged_torch.py:127-137). Here they are views of ONE allocation laid out
  ``[num_layers, 2, num_blocks, block_size, n_kv_heads, head_dim]`` so that a
  whole-block copy across every layer, or a swap, is one kernel launch;
* ``append_kv`` / ``attend`` / ``copy_block`` and the accounting methods
  (paged_torch.py:139-207), plus ``workspace_bytes()``, ``invalidate_plan()``
  and the ``n_plans`` / ``n_runs`` counters (flashinfer_backend.py:354-394,
  678-688);
* plan once per ``BatchMeta`` identity, run once per layer
  (flashinfer_backend.py:566-676), including the ``is_prefill`` cross-check.

One launch per layer on decode steps: for a decode-shaped batch on the fast
geometry, ``append_kv`` records its rows and the following ``attend`` of the
same layer performs the append inside the attention kernel (the result is
exactly append-then-attend). Anything else that could observe the pool --
reading ``k_pool`` / ``v_pool``, another append or attend, ``copy_block(s)``,
``reset``, swapping, ``check_device_errors`` -- first launches the recorded
append on its own. A caller must not modify ``k`` / ``v`` in place between
``append_kv`` and the next backend call; that is detected (tensor version
counters) and raises.

Everything runs on torch's current stream of the backend's device. Not
thread-safe and not re-entrant, like the reference backends.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _native
from .contract import BatchMeta
from .upload import uploader
from .sizing import DEFAULT_PART_PAGES  # split-K pieces: 17 pages = 272 tokens

__all__ = ["MI355XBackend", "is_available", "unavailable_reason"]

_DTYPES = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16,
           torch.float32: _native.DTYPE_F32}

MAX_PART_PAGES = 64      # a partition's page ids are read by one wavefront
DEFAULT_Q_TILE = 64      # prefill tile when the geometry has no matrix-core kernel


def is_available() -> bool:
    """True if the gfx950 library loads in this process (says nothing of a GPU)."""
    return _native.available()


def unavailable_reason() -> str | None:
    return _native.reason()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(device: torch.device) -> int:
    """Handle of torch's current stream on ``device`` (the raw-handle query
    skips building a Stream object on every launch)."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


class _Plan:
    """Device-side metadata and launch plan for one BatchMeta (one step)."""

    __slots__ = ("meta", "use_prefill", "slots", "indptr", "indices", "kv_lens", "cu_q",
                 "bidx", "plan", "n_work", "n_slots", "stride", "n_tokens", "n_seqs", "fusable",
                 "dec", "ptrs")


def _decode_ptrs(indptr, indices, kv_lens, plan, slots) -> tuple:
    """Device addresses a decode launch passes, taken once per plan."""
    return (indptr.data_ptr(), indices.data_ptr(), kv_lens.data_ptr(), plan.data_ptr(),
            slots.data_ptr() if slots is not None else None)


class _DecodeRows:
    """The one-token sequences of a mixed batch, run through the decode kernel:
    their token rows in q/out, and their paging metadata and decode plan as a
    batch of their own."""

    __slots__ = ("rows", "indptr", "indices", "kv_lens", "plan", "n", "n_work", "n_slots",
                 "stride")


class _Pending:
    """An append_kv whose rows will be written by the next launch."""

    __slots__ = ("layer", "k", "v", "meta", "slots", "stream", "kver", "vver")


class MI355XBackend:
    """Paged KV storage plus attention on gfx950 kernels."""

    def __init__(self, num_layers: int, num_blocks: int, block_size: int, n_kv_heads: int,
                 n_heads: int, head_dim: int, device: str | torch.device = "cuda:0",
                 dtype: torch.dtype = torch.float16, *,
                 part_pages: int = DEFAULT_PART_PAGES, q_tile: int | None = None,
                 fuse_append: bool = True, decode_workgroups_per_cu: int = 2,
                 decode_workgroups: int | None = None, decode_workspace_bytes: int = 0):
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
        if dtype not in _DTYPES:
            raise ValueError(f"MI355XBackend supports float16, bfloat16 and float32 pools, "
                             f"got {dtype}")
        if head_dim > 256:
            raise ValueError(f"head_dim={head_dim} > 256 is not supported")
        if q_tile is not None and q_tile < 1:
            raise ValueError(f"q_tile={q_tile} must be positive")
        if not 1 <= part_pages <= MAX_PART_PAGES:
            raise ValueError(f"part_pages={part_pages} must be in [1, {MAX_PART_PAGES}]")
        if decode_workgroups_per_cu < 1:
            raise ValueError(f"decode_workgroups_per_cu={decode_workgroups_per_cu} must be "
                             "positive")
        if decode_workgroups is not None and decode_workgroups < 1:
            raise ValueError(f"decode_workgroups={decode_workgroups} must be positive")
        if decode_workspace_bytes < 0:
            raise ValueError(f"decode_workspace_bytes={decode_workspace_bytes} must be >= 0")
        try:
            self._lib = _native.load()
        except RuntimeError as exc:
            raise RuntimeError(
                f"MI355XBackend requires the gfx950 paged-KV library: {exc}\n"
                "Use PagedTorchBackend (the correctness oracle) instead, or build the "
                "library. Check availability without raising via "
                "llm_serving_layer_amd.backend.is_available()."
            ) from exc
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"MI355XBackend requires a GPU device, got {self.device}. "
                             "PagedTorchBackend is the CPU path.")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())

        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.n_kv_heads, self.n_heads, self.head_dim = n_kv_heads, n_heads, head_dim
        self.dtype = dtype
        self.groups = n_heads // n_kv_heads
        self.part_pages = part_pages
        # The matrix-core prefill kernel owns 128 query rows (tokens x heads)
        # of one KV head; other geometries run the generic kernel.
        self._prefill_tile = int(self._lib.pkv_prefill_q_tile(
            n_heads, n_kv_heads, head_dim, block_size, _DTYPES[dtype]))
        self.q_tile = q_tile or self._prefill_tile or DEFAULT_Q_TILE
        self._code = _DTYPES[dtype]
        self._fast_decode = bool(self._lib.pkv_decode_fast_path(
            n_heads, n_kv_heads, head_dim, block_size, self._code, part_pages))
        self._fuse_append = fuse_append and self._fast_decode
        # The decode grid: every bin of the plan a resident workgroup (per
        # group of KV heads), so none waits for a slot. ``decode_workgroups``
        # overrides the count (tests force many sequences into a bin with it).
        self._decode_wgs = 0
        if self._fast_decode:
            with torch.cuda.device(self.device):
                self._decode_wgs = int(self._lib.pkv_decode_workgroups(
                    n_heads, n_kv_heads, head_dim, self._code, decode_workgroups_per_cu))
            if self._decode_wgs <= 0:
                raise RuntimeError("pkv_decode_workgroups found no resident decode workgroup "
                                   "on this device")
            if decode_workgroups is not None:
                self._decode_wgs = decode_workgroups
        # A mixed batch (prefill chunks beside one-token decodes) runs its
        # decodes through the decode kernel, so a decode step's bits do not
        # depend on whether prefills share its batch.
        self._split_mixed = self._fast_decode and self.q_tile == self._prefill_tile > 0

        self._pool = torch.zeros((num_layers, 2, num_blocks, block_size, n_kv_heads, head_dim),
                                 dtype=dtype, device=self.device)
        self._k_pool = [self._pool[l, 0] for l in range(num_layers)]
        self._v_pool = [self._pool[l, 1] for l in range(num_layers)]
        # the pools never move: their addresses are taken once
        self._k_ptr = [t.data_ptr() for t in self._k_pool]
        self._v_ptr = [t.data_ptr() for t in self._v_pool]
        self._block_bytes = block_size * n_kv_heads * head_dim * self._pool.element_size()
        self._plane_bytes = num_blocks * self._block_bytes
        self._status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._status_ptr = self._status.data_ptr()
        # The split-K workspace. A pool sized by sizing.plan_kv_pool passes its
        # workspace_bytes here, so no batch within that plan's limits ever
        # allocates at run time; a plan that needs more grows it.
        self._set_workspace(torch.zeros(decode_workspace_bytes, dtype=torch.uint8,
                                        device=self.device))
        self._planned: _Plan | None = None
        self._slot_cache: tuple[BatchMeta, torch.Tensor] | None = None
        self._pending: _Pending | None = None
        self.n_plans = 0
        self.n_runs = 0

    # -- the pools (reading them first lands any deferred append) ---------------

    @property
    def k_pool(self) -> list[torch.Tensor]:
        self._flush()
        return self._k_pool

    @property
    def v_pool(self) -> list[torch.Tensor]:
        self._flush()
        return self._v_pool

    # -- pool construction / accounting ---------------------------------------

    def zeros_like_pool(self) -> torch.Tensor:
        return torch.zeros_like(self._k_pool[0])

    def pool_bytes(self) -> int:
        return self.num_layers * 2 * self._plane_bytes

    def block_bytes(self) -> int:
        return self.pool_bytes() // self.num_blocks

    def workspace_bytes(self) -> int:
        """Split-K partials and arrival counters; grows with the largest batch
        planned, not with the pool."""
        return self._workspace.numel()

    def tokens_capacity(self) -> int:
        return self.num_blocks * self.block_size

    @staticmethod
    def estimate_pool_bytes(num_layers: int, num_blocks: int, block_size: int,
                            n_kv_heads: int, head_dim: int,
                            dtype: torch.dtype = torch.float16) -> int:
        elem = torch.empty((), dtype=dtype).element_size()
        return num_layers * 2 * num_blocks * block_size * n_kv_heads * head_dim * elem

    # -- helpers -----------------------------------------------------------------

    def _check_layer(self, layer_idx) -> None:
        if layer_idx is None or not 0 <= layer_idx < self.num_layers:
            raise ValueError(f"layer_idx {layer_idx} out of range [0, {self.num_layers})")

    def _dev_i32(self, t: torch.Tensor) -> torch.Tensor:
        return t.to(device=self.device, dtype=torch.int32).contiguous()

    def _as_pool(self, x: torch.Tensor) -> torch.Tensor:
        # (a tensor already in the pool dtype, contiguous and on this device is
        # used as it is, without a conversion call per launch)
        if x.dtype is self.dtype and x.get_device() == self.device.index and x.is_contiguous():
            return x
        return x.to(device=self.device, dtype=self.dtype).contiguous()

    def _set_workspace(self, ws: torch.Tensor) -> None:
        self._workspace = ws
        self._ws_ptr = ws.data_ptr() if ws.numel() else None
        self._ws_bytes = ws.numel()
        # leading bytes known to be zero between launches (a new workspace
        # is zero-filled)
        self._ws_zero = ws.numel()

    def check_device_errors(self) -> None:
        """
        Declared check point: synchronise and raise if any kernel since the
        last check skipped an out-of-range slot, page or block id.
        """
        self._flush()
        bits = int(self._status.item())
        if bits:
            self._status.zero_()
            what = []
            if bits & _native.STATUS_BAD_SLOT:
                what.append("slot_mapping entry outside the pool")
            if bits & _native.STATUS_BAD_PAGE:
                what.append("kv_indices entry outside [0, num_blocks)")
            if bits & _native.STATUS_BAD_BLOCK:
                what.append("block id outside [0, num_blocks)")
            raise IndexError("device kernels skipped invalid ids: " + "; ".join(what))

    # -- write path -----------------------------------------------------------------

    def copy_block(self, src: int, dst: int) -> None:
        """Duplicate one block's KV in every layer (copy-on-write)."""
        if not (0 <= src < self.num_blocks and 0 <= dst < self.num_blocks):
            raise IndexError(f"copy_block({src} -> {dst}) outside [0, {self.num_blocks})")
        if src == dst:
            return
        self.copy_blocks([src], [dst])

    def copy_blocks(self, src, dst) -> None:
        """
        Batched ``copy_block``: one launch for every (src, dst) pair, every
        layer, K and V. Destinations must be distinct and must not appear among
        the sources (so the result cannot depend on the order of the pairs).
        """
        src = [int(s) for s in src]
        dst = [int(d) for d in dst]
        if len(src) != len(dst):
            raise ValueError(f"{len(src)} sources but {len(dst)} destinations")
        for s, d in zip(src, dst):
            if not (0 <= s < self.num_blocks and 0 <= d < self.num_blocks):
                raise IndexError(f"copy_block({s} -> {d}) outside [0, {self.num_blocks})")
        pairs = [(s, d) for s, d in zip(src, dst) if s != d]
        if not pairs:
            return
        ds = [d for _, d in pairs]
        if len(set(ds)) != len(ds) or set(ds) & {s for s, _ in pairs}:
            raise ValueError("copy_blocks needs distinct destinations that are not also sources")
        self._flush()
        # pinned, so the upload queues on the stream without a host wait
        ids = torch.tensor([s for s, _ in pairs] + ds, dtype=torch.int32).pin_memory()
        ids = ids.to(self.device, non_blocking=True)
        n = len(pairs)
        rc = self._lib.pkv_copy_blocks(self._pool.data_ptr(), self.num_layers,
                                       self._plane_bytes, self._block_bytes, self.num_blocks,
                                       ids.data_ptr(), ids.data_ptr() + 4 * n, n,
                                       self._status.data_ptr(), _current_stream(self.device))
        _native.check(rc, "copy_blocks")

    def append_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
                  meta: BatchMeta) -> None:
        """Scatter this step's K/V into the pool through ``meta.slot_mapping``."""
        # (checks and conversions inlined: this runs once per layer per step)
        if layer_idx is None or not 0 <= layer_idx < self.num_layers:
            self._check_layer(layer_idx)
        if meta.slot_mapping is None:
            raise ValueError("MI355XBackend.append_kv requires meta.slot_mapping")
        ks = k.shape
        tokens = ks[0]
        if ks != (tokens, self.n_kv_heads, self.head_dim):
            raise ValueError(f"k has shape {tuple(ks)}, expected "
                             f"({tokens}, {self.n_kv_heads}, {self.head_dim})")
        if v.shape != ks:
            raise ValueError(f"v shape {tuple(v.shape)} != k shape {tuple(ks)}")
        if meta.slot_mapping.shape[0] != tokens:
            raise ValueError(f"slot_mapping has {meta.slot_mapping.shape[0]} entries but "
                             f"{tokens} tokens were supplied")
        if self._pending is not None:
            self._flush()
        dt, di = self.dtype, self.device.index
        if not (k.dtype is dt and k.get_device() == di and k.is_contiguous()):
            k = self._as_pool(k)
        if not (v.dtype is dt and v.get_device() == di and v.is_contiguous()):
            v = self._as_pool(v)
        stream = _raw_stream(di) if _raw_stream is not None else _current_stream(self.device)
        if self._fuse_append:
            try:
                p = self._ensure_planned(meta)
            except ValueError:
                p = None  # inconsistent paging metadata: append now, attend will raise
            if p is not None and p.fusable:
                pend = _Pending()
                pend.layer, pend.k, pend.v, pend.meta = layer_idx, k, v, meta
                pend.slots, pend.stream = p.slots, stream
                pend.kver, pend.vver = k._version, v._version
                self._pending = pend
                return
        self._launch_append(layer_idx, k, v, self._slots_for(meta), stream)

    def _slots_for(self, meta: BatchMeta) -> torch.Tensor:
        p = self._planned
        if p is not None and p.meta is meta:
            return p.slots
        sc = self._slot_cache
        if sc is not None and sc[0] is meta:
            return sc[1]
        slots = self._dev_i32(meta.slot_mapping)
        self._slot_cache = (meta, slots)
        return slots

    def _launch_append(self, layer, k, v, slots, stream) -> None:
        rc = self._lib.pkv_append_kv(
            self._k_ptr[layer], self._v_ptr[layer],
            self.num_blocks * self.block_size, k.data_ptr(), v.data_ptr(), slots.data_ptr(),
            k.shape[0], self.n_kv_heads, self.head_dim, self._code, self._status_ptr,
            stream)
        _native.check(rc, "append_kv")

    def _check_pending_intact(self, pend: _Pending) -> None:
        if pend.k._version != pend.kver or pend.v._version != pend.vver:
            self._pending = None
            raise RuntimeError(
                "k/v passed to append_kv were modified in place before the rows were "
                "written; pass tensors that stay unchanged until the next backend call"
            )

    def _flush(self) -> None:
        """Launch a deferred append on its own (on the stream it was issued on)."""
        pend = self._pending
        if pend is None:
            return
        self._check_pending_intact(pend)
        self._pending = None
        self._launch_append(pend.layer, pend.k, pend.v, pend.slots, pend.stream)
        cur = _current_stream(self.device)
        if cur != pend.stream:  # later work on this stream must see the rows
            ev = torch.cuda.Event()
            ev.record(torch.cuda.ExternalStream(pend.stream, device=self.device))
            torch.cuda.current_stream(self.device).wait_event(ev)

    # -- read path ------------------------------------------------------------------

    def attend(self, q: torch.Tensor, layer_idx: int, scale: float,
               meta: BatchMeta) -> torch.Tensor:
        """Causal GQA attention over each sequence's full paged history."""
        if layer_idx is None or not 0 <= layer_idx < self.num_layers:
            self._check_layer(layer_idx)
        qs = q.shape
        tokens = qs[0]
        if qs != (tokens, self.n_heads, self.head_dim):
            raise ValueError(f"q has shape {tuple(qs)}, expected "
                             f"({tokens}, {self.n_heads}, {self.head_dim})")
        if meta.n_tokens != tokens:
            raise ValueError(f"meta describes {meta.n_tokens} tokens but q has {tokens}")
        p = self._planned
        if p is None or p.meta is not meta:
            p = self._ensure_planned(meta)
        di = self.device.index
        stream = _raw_stream(di) if _raw_stream is not None else _current_stream(self.device)
        pend = self._pending
        fused = (pend is not None and pend.layer == layer_idx and pend.meta is meta
                 and pend.stream == stream and p.fusable)
        if fused:
            self._check_pending_intact(pend)
            self._pending = None
        elif pend is not None:
            self._flush()
        if not (q.dtype is self.dtype and q.get_device() == di and q.is_contiguous()):
            q = self._as_pool(q)
        out = torch.empty_like(q)
        kp = self._k_ptr[layer_idx]
        vp = self._v_ptr[layer_idx]
        self.n_runs += 1
        if not p.use_prefill:
            self._launch_decode(q, out, kp, vp, p.ptrs, p.n_seqs, p.n_work, p.n_slots,
                                p.stride, scale, stream, pend if fused else None)
        else:
            rc = self._lib.pkv_attend_prefill(
                q.data_ptr(), out.data_ptr(), kp, vp, self.num_blocks, p.cu_q.data_ptr(),
                p.indptr.data_ptr(), p.indices.data_ptr(), p.kv_lens.data_ptr(),
                p.bidx.data_ptr(), p.n_seqs, p.n_tokens, self.n_heads, self.n_kv_heads,
                self.head_dim, self.block_size, float(scale), self._code, p.plan.data_ptr(),
                p.n_work, self.q_tile, self._status.data_ptr(), stream)
            _native.check(rc, "attend (prefill)")
            d = p.dec
            if d is not None:
                qd = q.index_select(0, d.rows)
                od = torch.empty_like(qd)
                self._launch_decode(qd, od, kp, vp, _decode_ptrs(d.indptr, d.indices,
                                                                 d.kv_lens, d.plan, None),
                                    d.n, d.n_work, d.n_slots, d.stride, scale, stream, None)
                out.index_copy_(0, d.rows, od)
        return out

    def _launch_decode(self, q, out, kp, vp, ptrs, n_seqs, n_work, n_slots, stride, scale,
                       stream, pend) -> None:
        """``ptrs``: device addresses of (indptr, indices, kv_lens, plan, slots)."""
        indptr, indices, kv_lens, plan, slots = ptrs
        rc = self._lib.pkv_attend_decode(
            q.data_ptr(), out.data_ptr(), kp, vp, self.num_blocks, indptr, indices, kv_lens,
            n_seqs, self.n_heads, self.n_kv_heads, self.head_dim, self.block_size,
            float(scale), self._code, plan, n_work, n_slots, stride,
            pend.k.data_ptr() if pend else None, pend.v.data_ptr() if pend else None,
            slots if pend else None, self._ws_ptr, self._ws_bytes, self._status_ptr, stream)
        _native.check(rc, "attend (decode)")

    # -- planning ---------------------------------------------------------------

    def _ensure_planned(self, meta: BatchMeta) -> _Plan:
        """
        Build the launch plan for ``meta`` at most once per forward pass.
        Keyed on the object identity of the (frozen) BatchMeta, with a strong
        reference held so the identity cannot be recycled. The softmax scale
        is a launch argument, not part of the plan.
        """
        pl = self._planned
        if pl is not None and pl.meta is meta:
            return pl
        n = meta.n_seqs
        with_slots = (meta.slot_mapping is not None and meta.slot_mapping.shape[0] == n
                      and meta.kv_indices.shape[0] > 0 and meta.kv_indptr.shape[0] == n + 1)
        mirror = meta.host_arrays()
        n_pages = int(meta.kv_indices.shape[0])
        if mirror is not None:
            # the assembler's own host arrays: no device read-back
            ql, cu = mirror["query_lens"], mirror["cu_query_lens"]
            kvl, indptr = mirror["kv_lens"], mirror["kv_indptr"]
            last, indices = mirror["kv_last_page_len"], mirror["kv_indices"]
            if with_slots:
                new_slot = mirror["slot_mapping"]
        else:
            parts = [meta.query_lens, meta.cu_query_lens, meta.kv_lens, meta.kv_indptr,
                     meta.kv_last_page_len, meta.kv_indices]
            if with_slots:
                parts.append(meta.slot_mapping)
            # ONE device->host transfer for everything the host plan reads.
            host = torch.cat([t.reshape(-1).to(torch.int64) for t in parts]).cpu().numpy()
            ql, cu = host[:n], host[n:2 * n + 1]
            kvl, indptr = host[2 * n + 1:3 * n + 1], host[3 * n + 1:4 * n + 2]
            last = host[4 * n + 2:5 * n + 2]
            indices = host[5 * n + 2:5 * n + 2 + n_pages]
            if with_slots:
                new_slot = host[5 * n + 2 + n_pages:6 * n + 2 + n_pages]
        if with_slots:  # for the fused append: each sequence's last page id
            last_page = indices[np.clip(indptr[1:] - 1, 0, n_pages - 1)]
        use_prefill = bool((ql > 1).any())
        if bool(meta.is_prefill) != use_prefill:
            raise ValueError(
                f"BatchMeta.is_prefill={meta.is_prefill} disagrees with query_lens "
                f"(max={int(ql.max())}). is_prefill must be True iff some sequence "
                "contributes more than one token."
            )
        p = _Plan()
        p.meta, p.use_prefill = meta, use_prefill
        # Fusing the append into attention is exact only if every sequence's
        # new row lands at the last slot of its own page list (then no other
        # sequence of the launch reads that slot).
        p.fusable = False
        if with_slots and not use_prefill:
            p.fusable = bool((new_slot == last_page * self.block_size + last - 1).all())
        p.n_seqs, p.n_tokens = n, int(cu[-1])
        if p.n_tokens != meta.n_tokens:
            raise ValueError(f"cu_query_lens ends at {p.n_tokens} but meta has "
                             f"{meta.n_tokens} positions")
        if int(indptr[0]) != 0 or int(indptr[-1]) != int(meta.kv_indices.shape[0]):
            raise ValueError(f"kv_indptr spans [{int(indptr[0])}, {int(indptr[-1])}) but "
                             f"kv_indices holds {int(meta.kv_indices.shape[0])} pages")
        if int(meta.batch_indices.shape[0]) != p.n_tokens:
            raise ValueError(f"batch_indices has {int(meta.batch_indices.shape[0])} entries "
                             f"for {p.n_tokens} tokens")
        i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32)  # noqa: E731
        kvl32, indptr32, last32, cu32 = i32(kvl), i32(indptr), i32(last), i32(cu)
        ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
        decodes = None
        p.stride = 0
        if not use_prefill:
            plan, p.n_work, p.n_slots, p.stride = self._plan_decode(indptr32, i32(indices),
                                                                    kvl32, last32, n)
        else:
            n_work = C.c_int32()
            cap = 4 * (int(cu[-1]) // self.q_tile + n + 1)
            buf = np.empty(cap, dtype=np.int32)
            rc = self._lib.pkv_plan_prefill(ptr(cu32), ptr(indptr32), ptr(kvl32), ptr(last32),
                                            n, self.block_size, self.q_tile, ptr(buf), cap,
                                            C.byref(n_work))
            _native.check(rc, "plan (prefill)")
            tiles = buf[:4 * n_work.value].reshape(-1, 4)
            if self._split_mixed and bool((ql == 1).any()):
                decodes = np.flatnonzero(ql == 1)
                tiles = tiles[ql[tiles[:, 0]] > 1]  # the decode kernel takes the rest
            plan, p.n_work, p.n_slots = tiles.reshape(-1).copy(), tiles.shape[0], 0
        p.plan = self._upload(plan)
        p.indptr = self._dev_i32(meta.kv_indptr)
        p.indices = self._dev_i32(meta.kv_indices)
        p.kv_lens = self._dev_i32(meta.kv_lens)
        p.dec = None
        if decodes is not None:
            p.dec = self._decode_rows(decodes, cu, indptr, kvl, last, indices, p.indices)
        p.cu_q = self._dev_i32(meta.cu_query_lens)
        p.bidx = self._dev_i32(meta.batch_indices)
        p.slots = (self._dev_i32(meta.slot_mapping) if meta.slot_mapping is not None
                   else None)
        p.ptrs = _decode_ptrs(p.indptr, p.indices, p.kv_lens, p.plan, p.slots)
        self._planned = p
        self.n_plans += 1
        return p

    def _plan_decode(self, indptr32, indices32, kvl32, last32, n):
        """Host decode plan (pkv_plan_decode) plus a workspace large enough for it.
        Returns (plan, n_work, n_slots, stride)."""
        if not self._fast_decode:  # the generic kernel reads the CSR, not a plan
            return np.zeros(4, dtype=np.int32), 1, 0, 4
        ptr = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
        n_work, n_slots, stride = C.c_int32(), C.c_int32(), C.c_int32()
        needed = C.c_int64()
        cap = 6 * self._decode_wgs + 2 * int(indptr32[-1]) + 24 * n + 128
        counter_bytes = (4 * n * self.n_kv_heads + 255) // 256 * 256
        part_pages = self.part_pages
        while True:
            for _ in range(2):
                buf = np.empty(cap, dtype=np.int32)
                rc = self._lib.pkv_plan_decode(
                    ptr(indptr32), ptr(indices32), ptr(kvl32), ptr(last32), n,
                    self.block_size, self.num_blocks, self.n_kv_heads, part_pages,
                    self._decode_wgs, ptr(buf), cap, C.byref(needed), C.byref(n_work),
                    C.byref(n_slots), C.byref(stride))
                if rc == _native.ERR_CAPACITY and needed.value > cap:
                    cap = int(needed.value)
                    continue
                break
            _native.check(rc, "plan (decode)")
            need = self._lib.pkv_decode_workspace_bytes(n, n_slots.value, self.n_heads,
                                                        self.n_kv_heads, self.head_dim)
            # The kernel addresses the partials with 32-bit buffer offsets
            # (at most 2 GiB). A batch whose partials would not fit is cut
            # into larger pieces for this launch only (its bits then differ
            # from a solo run's, which is cut at part_pages).
            if need - counter_bytes < 2**31 - 1 or part_pages >= MAX_PART_PAGES:
                break
            part_pages = min(2 * part_pages, MAX_PART_PAGES)
        if need > self._workspace.numel():
            # zero-filled (the arrival counters at the front start at zero),
            # with room to spare: a running batch's plans grow step by step
            # as its sequences do, and each regrowth is an allocation
            grown = max(need, self._workspace.numel() * 5 // 4)
            self._set_workspace(torch.zeros(grown, dtype=torch.uint8, device=self.device))
        elif counter_bytes > self._ws_zero:
            # the counters now reach over bytes an earlier layout used for
            # partials: clear what is new (every counter is zero after a launch)
            self._workspace[self._ws_zero:counter_bytes].zero_()
        # after this plan's launch the bytes past its counters hold partials
        self._ws_zero = counter_bytes
        return (buf[:int(needed.value)].copy(), n_work.value, n_slots.value, stride.value)

    def _decode_rows(self, dec, cu, indptr, kvl, last, indices, indices_dev) -> _DecodeRows:
        """The decode-kernel batch of a mixed batch's one-token sequences
        ``dec``: their own CSR over a gathered copy of their page ids."""
        npg = indptr[dec + 1] - indptr[dec]
        sub_ptr = np.concatenate([[0], np.cumsum(npg)])
        # position in the batch's kv_indices of every page of the sub-batch
        page_ix = np.repeat(indptr[dec] - sub_ptr[:-1], npg) + np.arange(int(sub_ptr[-1]))
        i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32)  # noqa: E731
        d = _DecodeRows()
        d.n = int(dec.shape[0])
        plan, d.n_work, d.n_slots, d.stride = self._plan_decode(
            i32(sub_ptr), i32(indices[page_ix]), i32(kvl[dec]), i32(last[dec]), d.n)
        d.plan = self._upload(plan)
        d.rows = self._upload(cu[dec].astype(np.int64))
        d.indptr = self._upload(i32(sub_ptr))
        d.kv_lens = self._upload(i32(kvl[dec]))
        d.indices = indices_dev.index_select(0, self._upload(page_ix.astype(np.int64)))
        return d

    def _upload(self, a: np.ndarray) -> torch.Tensor:
        """Host array to the device through a pinned ring buffer, uploaded by a
        kernel on the current stream without a host wait (upload.py)."""
        return uploader(self.device).array(a)

    def invalidate_plan(self) -> None:
        """Force the next ``attend`` to re-plan (and drop the cached meta)."""
        self._flush()
        self._planned = None
        self._slot_cache = None

    # -- misc -------------------------------------------------------------------------

    def reset(self) -> None:
        """Zero every pool and drop the plan. Tests only."""
        self._pending = None
        self._pool.zero_()
        self.invalidate_plan()

    def __repr__(self) -> str:
        mib = self.pool_bytes() / (1024 * 1024)
        return (f"MI355XBackend(layers={self.num_layers}, blocks={self.num_blocks}, "
                f"block_size={self.block_size}, kv_heads={self.n_kv_heads}, "
                f"heads={self.n_heads}, head_dim={self.head_dim}, dtype={self.dtype}, "
                f"device={self.device}, pool={mib:.1f} MiB)")
