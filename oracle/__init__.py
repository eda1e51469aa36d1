"""
ORACLE — test infrastructure. CPU restatements of the reference's paged-KV
path, used only to check results in tests/ and ``__graft_entry__.smoke()``
and as the timed CPU baseline in bench.py. Nothing in llm_serving_layer_amd/ imports it.
"""

from .naive import (append_closed_form, copy_blocks_closed_form, gather_closed_form,
                    greedy_ids, naive_attention, scatter_closed_form)
from .paged_torch_cpu import PagedTorchOracle

__all__ = ["PagedTorchOracle", "naive_attention", "append_closed_form",
           "copy_blocks_closed_form", "gather_closed_form", "scatter_closed_form",
           "greedy_ids"]
