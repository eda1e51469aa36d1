"""
bench.py's contract, without a GPU: the headline workload is the one the
reference's capacity law draws (bench/capacity.py:196-242, lognormal branch,
seed 20260731: 256 sequences, 65 980 tokens, 4247 pages), its algorithmic
bytes are the published per-layer count (138.29 MB, 2.213 GB per 16-layer
step), the JSON line carries every field the contract names, and more than
one GPU is refused with a message.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_headline_lengths_follow_the_reference_law():
    lens = bench.lognormal_lengths(256, 256)
    assert len(lens) == 256 and sum(lens) == 65_980
    assert sum(-(-n // 16) for n in lens) == 4247
    assert min(lens) >= 1 and max(lens) == 1371


def test_algorithmic_bytes_per_layer():
    """Restated term by term: K and V once per KV head (2 KiB per token at
    8 heads x 64 dims x fp16), Q read and O written (4 KiB each per token),
    the appended K/V rows read and written plus their slots, and the
    metadata the kernel reads."""
    lens = bench.lognormal_lengths(256, 256)
    pages = 4247
    kv = 65_980 * 2048
    q_and_o = 256 * 4096 * 2
    append = 256 * 1024 * 2 * 2 + 4 * 256
    meta = 4 * (pages + 2 * 256 + 1)
    assert bench.decode_bytes(lens, pages) == kv + q_and_o + append + meta == 138_292_832
    assert 16 * bench.decode_bytes(lens, pages) == 2_212_685_312


def test_json_line_has_the_contract_fields():
    args = SimpleNamespace(steps=30, warmup=5)
    line = bench.base_line(args, "m", 1.0, "GB/s", 0.5, "fp16", "w", batch=256)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["vs_baseline"] is None
    assert line["config"]["workload"] == "w" and "model" not in line["config"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2 and "one GPU" in r.stderr
