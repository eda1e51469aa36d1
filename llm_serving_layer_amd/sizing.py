"""
KV pool sizing for one MI355X: the reference's ``plan_kv_pool``
(serving/memory/sizing.py:333-410, formulas at :166-222) with the two inputs
that change on this device.

* **The budget is measured.** With ``total_vram_bytes=None`` the plan reads
  the device's free HBM (``torch.cuda.mem_get_info``) instead of a nominal
  figure; the nominal 288 GiB of an MI355X is ``MI355X_HBM_BYTES``. The
  reference's default is a nominal 40 GiB A100, which it flags as an estimate
  (sizing.py:98-101).
* **The decode workspace is charged to the pool budget.** The split-K decode
  keeps partial outputs for every partition of a split sequence, so its
  workspace grows with the batch: at most ``max_batch_seqs`` sequences of at
  most ``max_seq_len`` tokens each (shared prefix blocks count once per
  sequence that reads them). The plan reserves that worst case with the
  library's own ``pkv_decode_workspace_bytes`` and picks the largest
  ``num_blocks`` for which pool + workspace fit: one block more would not.

The pool itself is one allocation ``[num_layers, 2, num_blocks, block_size,
n_kv_heads, head_dim]`` (``MI355XBackend``), so ``bytes_per_block`` is also
the stride of one block across every layer, K and V.

Errors are ``SizingError`` (a ``ValueError``), raised instead of returning a
zero or negative block count, with the messages of the reference
(sizing.py:346-387).
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from dataclasses import dataclass, field

__all__ = ["SizingError", "ModelKVShape", "LLAMA_3_2_1B", "KVPoolPlan", "kv_bytes_per_token",
           "block_bytes", "decode_workspace_bound", "decode_workspace_slots", "measure_free_hbm", "plan_kv_pool",
           "MI355X_HBM_BYTES", "LLAMA_3_2_1B_FP16_WEIGHT_BYTES",
           "DEFAULT_ACTIVATION_HEADROOM_BYTES", "DEFAULT_BLOCK_SIZE"]

GIB = 1024**3
MIB = 1024**2

#: Nominal HBM3E capacity of one MI355X. A plan made on the device measures
#: the free memory instead (``total_vram_bytes=None``).
MI355X_HBM_BYTES = 288 * GIB
#: Llama 3.2 1B fp16 weights as the reference records them (sizing.py:103-105).
LLAMA_3_2_1B_FP16_WEIGHT_BYTES = int(2357.1 * MIB)
#: Activations, allocator slack and the runtime context (sizing.py:107-112):
#: a parameter because it is the least certain input.
DEFAULT_ACTIVATION_HEADROOM_BYTES = 2 * GIB
DEFAULT_BLOCK_SIZE = 16
#: Largest batch the decode workspace is reserved for by default: the
#: 4096-sequence capacity workload.
DEFAULT_MAX_BATCH_SEQS = 4096
# Split-K piece size of the decode kernel, in pages (272 tokens): the
# backend's default, so the workspace reserved here is the one it uses.
DEFAULT_PART_PAGES = 17
#: Longest sequence the decode workspace is reserved for by default (the
#: reference's max_seq, bench/capacity.py:196-242).
DEFAULT_MAX_SEQ_LEN = 2048


class SizingError(ValueError):
    """A sizing request that cannot be satisfied (sizing.py:113-123)."""


@dataclass(frozen=True)
class ModelKVShape:
    """The numbers that fix KV size (sizing.py:126-147)."""

    n_layers: int
    n_kv_heads: int
    head_dim: int
    dtype_bytes: int = 2
    name: str = "unnamed"

    def bytes_per_token(self) -> int:
        return kv_bytes_per_token(self.n_layers, self.n_kv_heads, self.head_dim,
                                  self.dtype_bytes)

    def as_dict(self) -> dict:
        return {"name": self.name, "n_layers": self.n_layers, "n_kv_heads": self.n_kv_heads,
                "head_dim": self.head_dim, "dtype_bytes": self.dtype_bytes}


LLAMA_3_2_1B = ModelKVShape(16, 8, 64, 2, "Llama 3.2 1B (fp16)")


def kv_bytes_per_token(n_layers: int = 16, n_kv_heads: int = 8, head_dim: int = 64,
                       dtype_bytes: int = 2) -> int:
    """K and V of one token over all layers: 2 * L * Hkv * d * elem
    (sizing.py:166-199). Query heads do not enter: the cache holds KV heads."""
    for label, value in (("n_layers", n_layers), ("n_kv_heads", n_kv_heads),
                         ("head_dim", head_dim), ("dtype_bytes", dtype_bytes)):
        if value <= 0:
            raise SizingError(f"{label} must be positive, got {value}")
    return 2 * n_layers * n_kv_heads * head_dim * dtype_bytes


def block_bytes(block_size: int = DEFAULT_BLOCK_SIZE, n_layers: int = 16, n_kv_heads: int = 8,
                head_dim: int = 64, dtype_bytes: int = 2) -> int:
    """One physical block over all layers, K and V (sizing.py:202-222)."""
    if block_size <= 0:
        raise SizingError(f"block_size must be positive, got {block_size}")
    return block_size * kv_bytes_per_token(n_layers, n_kv_heads, head_dim, dtype_bytes)


def decode_workspace_slots(num_blocks: int, max_batch_seqs: int, part_pages: int,
                           max_seq_len: int = DEFAULT_MAX_SEQ_LEN,
                           block_size: int = DEFAULT_BLOCK_SIZE,
                           shared_blocks: bool = True) -> int:
    """
    Most split-K partial slots one decode batch can need.

    A sequence of p pages is cut into ceil(p / part_pages) partitions and
    takes one partial slot per partition only when p > part_pages, so a
    sequence of at most ``max_seq_len`` tokens takes at most
    ceil(ceil(max_seq_len / block_size) / part_pages) slots, and a batch of
    ``max_batch_seqs`` sequences that many times over. This holds whatever
    the pages are: a radix prefix cache lets every sequence of a batch share
    the same prefix blocks (serving/cache/radix.py:423-451), so the pages a
    batch references are not bounded by the pool.

    Only when no block is shared (``shared_blocks=False``) is the pool a
    second bound: the pages of the batch are then distinct blocks, a split
    sequence needs ceil(p / part_pages) <= 2 p / part_pages slots, and the
    batch at most floor(2 num_blocks / part_pages); the smaller bound holds.
    """
    if part_pages <= 0:
        raise SizingError(f"part_pages must be positive, got {part_pages}")
    if max_batch_seqs <= 0:
        raise SizingError(f"max_batch_seqs must be positive, got {max_batch_seqs}")
    if max_seq_len <= 0 or block_size <= 0:
        raise SizingError(f"max_seq_len ({max_seq_len}) and block_size ({block_size}) must "
                          "be positive")
    pages = -(-max_seq_len // block_size)
    per_seq = -(-pages // part_pages) if pages > part_pages else 0
    slots = max_batch_seqs * per_seq
    if not shared_blocks:
        slots = min(slots, (2 * num_blocks) // part_pages)
    return slots


def decode_workspace_bound(num_blocks: int, max_batch_seqs: int, n_heads: int,
                           n_kv_heads: int, head_dim: int, part_pages: int,
                           max_seq_len: int = DEFAULT_MAX_SEQ_LEN,
                           block_size: int = DEFAULT_BLOCK_SIZE,
                           shared_blocks: bool = True) -> int:
    """
    Largest decode workspace any batch of at most ``max_batch_seqs``
    sequences of at most ``max_seq_len`` tokens can need
    (``decode_workspace_slots`` slots). The byte count is the library's
    (``pkv_decode_workspace_bytes``), so it cannot drift from what the
    backend allocates.
    """
    from . import _native

    if n_heads <= 0 or n_kv_heads <= 0 or n_heads % n_kv_heads:
        raise SizingError(f"n_heads ({n_heads}) must be a positive multiple of n_kv_heads "
                          f"({n_kv_heads})")
    slots = decode_workspace_slots(num_blocks, max_batch_seqs, part_pages, max_seq_len,
                                   block_size, shared_blocks)
    if slots <= 0:
        return 0
    return int(_native.load().pkv_decode_workspace_bytes(max_batch_seqs, slots, n_heads,
                                                         n_kv_heads, head_dim))


def measure_free_hbm(device="cuda:0") -> tuple[int, int]:
    """(free, total) bytes of the device's memory as the runtime reports them."""
    import torch

    dev = torch.device(device)
    if dev.type != "cuda":
        raise SizingError(f"measuring HBM needs a GPU device, got {dev}")
    if not torch.cuda.is_available():
        raise SizingError("no GPU is visible: pass total_vram_bytes explicitly")
    free, total = torch.cuda.mem_get_info(dev)
    return int(free), int(total)


@dataclass(frozen=True)
class KVPoolPlan:
    """
    A sized pool plus the arithmetic that produced it (sizing.py:225-330),
    with the decode workspace reserved out of the same budget.
    """

    shape: ModelKVShape
    total_vram_bytes: int
    model_weight_bytes: int
    activation_headroom_bytes: int
    block_size: int
    available_bytes: int
    bytes_per_token: int
    bytes_per_block: int
    num_blocks: int
    tokens_capacity: int
    bytes_used: int
    bytes_leftover: int
    workspace_bytes: int = 0
    n_heads: int = 0
    max_batch_seqs: int = 0
    part_pages: int = 0
    max_seq_len: int = DEFAULT_MAX_SEQ_LEN
    shared_blocks: bool = True
    measured: bool = False
    notes: list[str] = field(default_factory=list)

    def _workspace_for(self, num_blocks: int) -> int:
        if not self.max_batch_seqs:
            return 0
        return decode_workspace_bound(num_blocks, self.max_batch_seqs, self.n_heads,
                                      self.shape.n_kv_heads, self.shape.head_dim,
                                      self.part_pages, self.max_seq_len, self.block_size,
                                      self.shared_blocks)

    def is_self_consistent(self) -> bool:
        """``num_blocks`` blocks and their workspace fit; one block more would not."""
        fits = self.num_blocks * self.bytes_per_block + self.workspace_bytes
        more = (self.num_blocks + 1) * self.bytes_per_block + self._workspace_for(
            self.num_blocks + 1)
        return fits <= self.available_bytes < more

    @property
    def utilization_of_available(self) -> float:
        return self.bytes_used / self.available_bytes

    def sequences_at_length(self, seq_len: int) -> int:
        """Concurrent sequences of exactly ``seq_len`` tokens (whole blocks each)."""
        if seq_len <= 0:
            raise SizingError(f"seq_len must be positive, got {seq_len}")
        return self.num_blocks // math.ceil(seq_len / self.block_size)

    def derivation(self) -> list[str]:
        s = self.shape
        src = "measured free HBM" if self.measured else "total HBM"
        lines = [
            f"model                 {s.name}: {s.n_layers} layers, {s.n_kv_heads} kv heads, "
            f"head_dim {s.head_dim}, {s.dtype_bytes} bytes/element",
            f"bytes per token       2 (K,V) x {s.n_layers} x {s.n_kv_heads} x {s.head_dim} x "
            f"{s.dtype_bytes} = {self.bytes_per_token:,} B",
            f"bytes per block       {self.block_size} tokens x {self.bytes_per_token:,} B = "
            f"{self.bytes_per_block:,} B ({self.bytes_per_block / 1024:.0f} KiB)",
            f"{src:<21s} {self.total_vram_bytes:,} B ({self.total_vram_bytes / GIB:.2f} GiB)",
            f"- model weights       {self.model_weight_bytes:,} B",
            f"- activation headroom {self.activation_headroom_bytes:,} B",
            f"= available for KV    {self.available_bytes:,} B "
            f"({self.available_bytes / GIB:.2f} GiB)",
        ]
        if self.max_batch_seqs:
            slots = decode_workspace_slots(self.num_blocks, self.max_batch_seqs,
                                           self.part_pages, self.max_seq_len, self.block_size,
                                           self.shared_blocks)
            lines.append(
                f"- decode workspace    {self.workspace_bytes:,} B (batches of <= "
                f"{self.max_batch_seqs} seqs of <= {self.max_seq_len} tokens, "
                f"{self.part_pages}-page partitions, <= {slots:,} partial slots"
                f"{'' if self.shared_blocks else ', no shared blocks'})")
        lines += [
            f"num_blocks            largest n with n x {self.bytes_per_block:,} + workspace(n) "
            f"<= {self.available_bytes:,}: {self.num_blocks:,}",
            f"tokens capacity       {self.num_blocks:,} x {self.block_size} = "
            f"{self.tokens_capacity:,} tokens",
            f"bytes used            {self.bytes_used:,} B ({self.bytes_used / GIB:.2f} GiB)",
            f"bytes left unused     {self.bytes_leftover:,} B (less than one more block and "
            "its workspace)",
        ]
        return lines

    def explain(self) -> str:
        lines = ["KV pool sizing", "=" * 72] + self.derivation()
        if self.notes:
            lines += ["", "notes:"] + [f"  - {n}" for n in self.notes]
        return "\n".join(lines)

    def as_dict(self) -> dict:
        return {"shape": self.shape.as_dict(), "total_vram_bytes": self.total_vram_bytes,
                "model_weight_bytes": self.model_weight_bytes,
                "activation_headroom_bytes": self.activation_headroom_bytes,
                "block_size": self.block_size, "available_bytes": self.available_bytes,
                "bytes_per_token": self.bytes_per_token, "bytes_per_block": self.bytes_per_block,
                "num_blocks": self.num_blocks, "tokens_capacity": self.tokens_capacity,
                "bytes_used": self.bytes_used, "bytes_leftover": self.bytes_leftover,
                "workspace_bytes": self.workspace_bytes, "measured": self.measured,
                "derivation": self.derivation(), "notes": list(self.notes)}

    def backend(self, n_heads: int | None = None, device="cuda:0", dtype=None, **kwargs):
        """An ``MI355XBackend`` with this plan's pool (one allocation)."""
        import torch

        from .backend import MI355XBackend

        if dtype is None:
            dtype = {2: torch.float16, 4: torch.float32}[self.shape.dtype_bytes]
        # the decode workspace this plan reserved, and the partition size it
        # was reserved for: a batch within the plan's limits then never
        # allocates while a step runs
        kwargs.setdefault("decode_workspace_bytes", self.workspace_bytes)
        kwargs.setdefault("part_pages", self.part_pages)
        return MI355XBackend(self.shape.n_layers, self.num_blocks, self.block_size,
                             self.shape.n_kv_heads, n_heads or self.n_heads, self.shape.head_dim,
                             device=device, dtype=dtype, **kwargs)


def plan_kv_pool(total_vram_bytes: int | None = MI355X_HBM_BYTES,
                 model_weight_bytes: int = LLAMA_3_2_1B_FP16_WEIGHT_BYTES,
                 activation_headroom_bytes: int = DEFAULT_ACTIVATION_HEADROOM_BYTES,
                 block_size: int = DEFAULT_BLOCK_SIZE, shape: ModelKVShape = LLAMA_3_2_1B,
                 notes: Sequence[str] | None = None, *, n_heads: int = 32,
                 max_batch_seqs: int = DEFAULT_MAX_BATCH_SEQS,
                 part_pages: int = DEFAULT_PART_PAGES,
                 max_seq_len: int = DEFAULT_MAX_SEQ_LEN, shared_blocks: bool = True,
                 device="cuda:0") -> KVPoolPlan:
    """
    Size the pool from an HBM budget:

        available  = budget - model_weights - activation_headroom
        num_blocks = largest n with n * block_bytes + workspace(n) <= available

    ``total_vram_bytes=None`` measures the budget on ``device`` (free bytes
    now, so weights already resident should be passed as 0).
    ``max_batch_seqs=0`` reserves no decode workspace, which gives the
    reference's floor(available / block_bytes) exactly. The workspace is
    reserved for batches of up to ``max_batch_seqs`` sequences of up to
    ``max_seq_len`` tokens whose prefix blocks may be shared; pass
    ``shared_blocks=False`` only for a deployment without a prefix cache.
    """
    notes = list(notes or [])
    measured = total_vram_bytes is None
    if measured:
        free, total = measure_free_hbm(device)
        total_vram_bytes = free
        notes.append(f"budget measured on {device}: {free:,} B free of {total:,} B")
    if total_vram_bytes <= 0:
        raise SizingError(f"total_vram_bytes must be positive, got {total_vram_bytes}")
    if model_weight_bytes < 0:
        raise SizingError(f"model_weight_bytes must be non-negative, got {model_weight_bytes}")
    if activation_headroom_bytes < 0:
        raise SizingError(
            f"activation_headroom_bytes must be non-negative, got {activation_headroom_bytes}")
    if model_weight_bytes > total_vram_bytes:
        raise SizingError(
            f"Model weights ({model_weight_bytes:,} B, {model_weight_bytes / GIB:.2f} GiB) "
            f"exceed total VRAM ({total_vram_bytes:,} B, {total_vram_bytes / GIB:.2f} GiB). "
            "Nothing is left over for KV blocks once the weights are loaded.")
    available = total_vram_bytes - model_weight_bytes - activation_headroom_bytes
    if available <= 0:
        raise SizingError(
            f"No VRAM left for KV: total {total_vram_bytes:,} B - weights "
            f"{model_weight_bytes:,} B - headroom {activation_headroom_bytes:,} B = "
            f"{available:,} B. Reduce the activation headroom or use a smaller model.")
    per_block = block_bytes(block_size, shape.n_layers, shape.n_kv_heads, shape.head_dim,
                            shape.dtype_bytes)

    def workspace(n: int) -> int:
        if not max_batch_seqs:
            return 0
        return decode_workspace_bound(n, max_batch_seqs, n_heads, shape.n_kv_heads,
                                      shape.head_dim, part_pages, max_seq_len, block_size,
                                      shared_blocks)

    # n * per_block + workspace(n) grows with n: binary search for the largest fit
    lo, hi = 0, available // per_block
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if mid * per_block + workspace(mid) <= available:
            lo = mid
        else:
            hi = mid - 1
    n = lo
    if n < 1:
        raise SizingError(
            f"Available KV memory ({available:,} B) is smaller than one block "
            f"({per_block:,} B at block_size={block_size}) plus its decode workspace. "
            "The pool would hold no block at all, so not even one token could be cached.")
    ws = workspace(n)
    used = n * per_block
    return KVPoolPlan(shape=shape, total_vram_bytes=int(total_vram_bytes),
                      model_weight_bytes=int(model_weight_bytes),
                      activation_headroom_bytes=int(activation_headroom_bytes),
                      block_size=int(block_size), available_bytes=int(available),
                      bytes_per_token=shape.bytes_per_token(), bytes_per_block=int(per_block),
                      num_blocks=int(n), tokens_capacity=int(n * block_size),
                      bytes_used=int(used), bytes_leftover=int(available - used - ws),
                      workspace_bytes=int(ws), n_heads=int(n_heads),
                      max_batch_seqs=int(max_batch_seqs), part_pages=int(part_pages),
                      max_seq_len=int(max_seq_len), shared_blocks=bool(shared_blocks),
                      measured=measured, notes=notes)
