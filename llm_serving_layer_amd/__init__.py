"""
MI355X-native paged-KV attention backend for the llm_serving_layer contract.

Host mirror of the reference interface (Python) over a C-ABI library of
hand-written gfx950 kernels (include/pagedkv.h, csrc/):

* ``contract``  — BatchMeta and the AttentionBackend protocol;
* ``paging``    — BlockAllocator, SequenceBlocks, build_csr;
* ``assembly``  — ScheduledSeq, build_batch_meta, build_token_tensor;
* ``backend``   — MI355XBackend (append_kv / attend / copy_block[s]);
* ``swap``      — KVSwapSpace / SwapHandle (preemption swap);
* ``sizing``    — plan_kv_pool / KVPoolPlan (pool sizing for one MI355X).
* ``sampling``  — greedy (argmax on the device), StepTimer, greedy_step (the
  scheduler step's forward-and-sample part, timed with HIP events).
"""

from .assembly import ScheduledSeq, build_batch_meta, build_token_tensor
from .contract import AttentionBackend, BatchMeta
from .paging import AllocationError, BlockAllocator, SequenceBlocks, build_csr

__all__ = ["AttentionBackend", "BatchMeta", "AllocationError", "BlockAllocator",
           "SequenceBlocks", "build_csr", "ScheduledSeq", "build_batch_meta",
           "build_token_tensor", "MI355XBackend", "KVSwapSpace", "SwapHandle",
           "SwapSpaceFull", "is_available", "unavailable_reason"]


def __getattr__(name):
    # The GPU-facing classes import lazily so the host-only modules stay
    # importable (and testable) without touching the native library.
    if name in ("MI355XBackend", "is_available", "unavailable_reason"):
        from . import backend
        return getattr(backend, name)
    if name in ("KVSwapSpace", "SwapHandle", "SwapSpaceFull"):
        from . import swap
        return getattr(swap, name)
    raise AttributeError(name)
