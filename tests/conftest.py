"""
Two tiers, as in the reference (tests/test_flashinfer_differential.py:130-167):
CPU tests run everywhere; tests marked ``gpu`` need an MI355X. With
REQUIRE_GPU=1 a missing GPU or an unbuilt library is a hard failure instead
of a skip, so a GPU run can never pass by skipping everything.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def gpu_reason() -> str | None:
    import torch

    if not torch.cuda.is_available():
        return "no GPU visible (torch.cuda.is_available() is False)"
    from llm_serving_layer_amd import backend

    if not backend.is_available():
        return f"native library unavailable: {backend.unavailable_reason()}"
    return None


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    reason = gpu_reason()
    if reason is None:
        return
    if os.environ.get("REQUIRE_GPU") == "1":
        raise pytest.UsageError(f"REQUIRE_GPU=1 but {reason}")
    skip = pytest.mark.skip(reason=reason)
    for it in gpu_items:
        it.add_marker(skip)
