"""
Build the gfx950 paged-KV library in-tree: every csrc/*.hip is compiled by
hipcc for gfx950 only (in parallel) and linked into
llm_serving_layer_amd/_native/libpagedkv.so, which the package loads with
ctypes. Run ``python -m llm_serving_layer_amd.build``.

``--timeline`` builds the same sources with -DPKV_TIMELINE into
_native/libpagedkv_timeline.so instead: the decode kernel then records a
per-wave timeline (``bench.py --timeline`` loads that build through
PKV_LIBRARY and summarises it). The product library is never built with it.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT_DIR = PKG / "_native"
LIB = OUT_DIR / "libpagedkv.so"
TIMELINE_LIB = OUT_DIR / "libpagedkv_timeline.so"
OBJ_DIR = PKG.parent / "_build"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # No packed-fp32 VALU ops: some of their forms have given silently wrong
    # results on MI355X, so the kernels are built without them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the decode kernel's online softmax
    # rescales them every page, and the AGPR form would copy them back and forth.
    "-mllvm", "-amdgpu-mfma-vgpr-form=true",
    # The first 16 dwords of kernel arguments arrive in SGPRs at wave launch
    # instead of through a scalar load: one round trip less before a decode
    # wave can read its plan (0.5% of the batch-256 decode step).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return exe


def _compile(src: Path, obj_dir: Path, defines: tuple) -> Path:
    obj = obj_dir / (src.stem + ".o")
    cmd = [_hipcc(), *FLAGS, *defines, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, timeline: bool = False) -> Path:
    """Compile and link; always rebuilds. Returns the path of the library."""
    obj_dir = OBJ_DIR / "timeline" if timeline else OBJ_DIR
    lib = TIMELINE_LIB if timeline else LIB
    defines = ("-DPKV_TIMELINE",) if timeline else ()
    obj_dir.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(SRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), sources))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} from {len(sources)} sources")
    return lib


if __name__ == "__main__":
    build(verbose=True, timeline="--timeline" in sys.argv[1:])
    sys.exit(0)
