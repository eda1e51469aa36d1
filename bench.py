#!/usr/bin/env python3
"""
Decode-step benchmark of the MI355X paged-KV backend.

Workload (one "step"): Llama-3.2-1B attention geometry (32 query heads,
8 KV heads, head_dim 64), block_size 16, fp16, batch 256 with per-sequence
context lengths drawn lognormal (mean 256, sigma 0.8, clipped to [1, 2048],
seed 20260731 -> realized mean 257.7, p90 498, max 1371, 65 980 tokens,
4247 pages), block tables shuffled over a pool of 2x the pages needed,
K/V cache and Q ~ N(0,1)*0.5. A step is, for each of the 16 layers, one KV
append of the new token of every sequence followed by one paged decode
attention over every sequence's whole history, through the backend's public
``append_kv`` / ``attend``. All 16 layers are cycled so a layer's KV
(~135 MB) cannot stay resident in the 256 MB last-level cache.

Prints ONE JSON line. ``value`` is the algorithmic HBM bytes of the step
(KV read once per KV head, Q read, O written, append read+write, metadata)
divided by the measured step time. ``roofline`` is the decode kernel alone,
timed with HIP events on the stream it is launched on.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HQ, HKV, D, BS, LAYERS, BATCH = 32, 8, 64, 16, 16, 256
SEED = 20260731
PEAK_HBM_GBPS = 8000.0
METRIC = ("paged decode attn+append HBM GB/s (% peak); decode tok/s @ batch 256, 1 GPU")


def lengths():
    import math
    import random

    rng = random.Random(SEED)
    mu = math.log(256) - 0.8 ** 2 / 2.0
    return [max(1, min(2048, int(round(rng.lognormvariate(mu, 0.8))))) for _ in range(BATCH)]


def algorithmic_bytes(kv_lens, pages, T):
    """Per layer: (decode kernel bytes, append kernel bytes)."""
    kv = sum(kv_lens) * HKV * D * 2 * 2          # K and V rows, each KV head once
    qo = T * HQ * D * 2 * 2                      # Q read + O written
    meta = 4 * (pages + 2 * len(kv_lens) + 1)    # kv_indices, kv_lens, kv_indptr
    append = T * HKV * D * 2 * 2 * 2             # K,V rows read + written
    return kv + qo + meta, append + 4 * T


def build(device, lens, part_pages):
    import torch

    from llm_serving_layer_amd import BlockAllocator, ScheduledSeq, SequenceBlocks, build_batch_meta
    from llm_serving_layer_amd.backend import MI355XBackend

    pages = sum(-(-n // BS) for n in lens)
    nb = 2 * pages
    bk = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device=device, dtype=torch.float16,
                       part_pages=part_pages)
    g = torch.Generator(device=device).manual_seed(SEED)
    for l in range(LAYERS):  # the whole pool, so every page read holds real data
        bk._pool[l].copy_(torch.randn(bk._pool[l].shape, generator=g, device=device) * 0.5)
    alloc = BlockAllocator(nb, BS)
    alloc.allocate(nb)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(SEED)).tolist()
    alloc.free(perm)
    seqs = []
    for i, n in enumerate(lens):
        s = SequenceBlocks(alloc, seq_id=i)
        s.append(n - 1)          # history; the step appends the n-th token
        seqs.append(s)
    t0 = time.perf_counter()
    for s in seqs:
        s.append(1)
    meta = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], device, BS)
    torch.cuda.synchronize()
    meta_ms = (time.perf_counter() - t0) * 1e3
    k = (torch.randn(LAYERS, BATCH, HKV, D, generator=g, device=device) * 0.5).half()
    v = (torch.randn(LAYERS, BATCH, HKV, D, generator=g, device=device) * 0.5).half()
    q = (torch.randn(LAYERS, BATCH, HQ, D, generator=g, device=device) * 0.5).half()
    return bk, meta, k, v, q, pages, meta_ms


def cpu_baseline(lens, budget_s=12.0):
    """
    The oracle (CPU restatement of the reference's PagedTorchBackend, fp32)
    on the same workload: all 256 sequences, append + attend per layer.
    Bounded sample: as many single-layer passes as fit in ~budget_s, scaled
    to the 16-layer step.
    """
    import torch

    from llm_serving_layer_amd import BlockAllocator, ScheduledSeq, SequenceBlocks, build_batch_meta
    from oracle import PagedTorchOracle

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    pages = sum(-(-n // BS) for n in lens)
    ref = PagedTorchOracle(1, pages, BS, HKV, HQ, D, device="cpu", dtype=torch.float32)
    g = torch.Generator().manual_seed(SEED)
    ref.k_pool[0].copy_(torch.randn(ref.k_pool[0].shape, generator=g) * 0.5)
    ref.v_pool[0].copy_(torch.randn(ref.v_pool[0].shape, generator=g) * 0.5)
    alloc = BlockAllocator(pages, BS)
    seqs = []
    for i, n in enumerate(lens):
        s = SequenceBlocks(alloc, seq_id=i)
        s.append(n)
        seqs.append(s)
    meta = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], "cpu", BS)
    k = torch.randn(BATCH, HKV, D, generator=g) * 0.5
    q = torch.randn(BATCH, HQ, D, generator=g) * 0.5
    ref.append_kv(0, k, k, meta)
    ref.attend(q, 0, 0.125, meta)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        ref.append_kv(0, k, k, meta)
        ref.attend(q, 0, 0.125, meta)
        times.append(time.perf_counter() - t0)
    times.sort()
    layer_s = times[len(times) // 2]
    step_s = layer_s * LAYERS
    return {"value": round(BATCH / step_s, 2), "unit": "decode tok/s", "cores": cores,
            "kind": "port",
            "sample": (f"{len(times)} single-layer append+attend passes over all {BATCH} "
                       f"sequences (fp32, CPU restatement of PagedTorchBackend), median "
                       f"{layer_s * 1e3:.1f} ms/layer x {LAYERS} layers")}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--part-pages", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--graph", action="store_true",
                    help="also time the step captured in a HIP graph and replayed")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no cross-GPU exchange (each GPU "
              f"serves its own sequences); --gpus {args.gpus} is not supported.", file=sys.stderr)
        return 2

    import torch

    device = "cuda:0"
    lens = lengths()
    print(f"[bench] building workload: batch {BATCH}, {sum(lens)} tokens", file=sys.stderr, flush=True)
    bk, meta, k, v, q, pages, meta_ms = build(device, lens, args.part_pages)
    dec_bytes, app_bytes = algorithmic_bytes(lens, pages, BATCH)
    step_bytes = LAYERS * (dec_bytes + app_bytes)
    scale = 1.0 / 8.0

    def step(events=None):
        for l in range(LAYERS):
            bk.append_kv(l, k[l], v[l], meta)
            if events is not None:
                events[l][0].record()
            bk.attend(q[l], l, scale, meta)
            if events is not None:
                events[l][1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    bk.check_device_errors()

    # Timed region: K steps through the public API, bracketed by syncs.
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(LAYERS)] for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for s in range(args.steps):
        step(ev[s])
    stop.record()
    enqueue_s = time.perf_counter() - t0   # host time to issue every call (no sync yet)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = max(gpu_ms, wall * 1e3) / args.steps
    attend_ms = [ev[s][l][0].elapsed_time(ev[s][l][1]) for s in range(args.steps)
                 for l in range(LAYERS)]
    attend_avg_ms = sum(attend_ms) / len(attend_ms)
    bk.check_device_errors()

    graph = None
    if args.graph:
        # The same step captured once into a HIP graph and replayed: removes the
        # host's per-call cost; the kernels and their order are unchanged.
        print("[bench] graph capture", file=sys.stderr, flush=True)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        gs, ge = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        gs.record()
        for _ in range(args.steps):
            g.replay()
        ge.record()
        torch.cuda.synchronize()
        g_ms = gs.elapsed_time(ge) / args.steps
        graph = {"ms_per_step": round(g_ms, 4),
                 "GB/s": round(step_bytes / (g_ms * 1e-3) / 1e9, 1),
                 "decode_tok_s": round(BATCH / (g_ms * 1e-3), 1)}
        bk.check_device_errors()

    gbps = step_bytes / (ms_per_step * 1e-3) / 1e9
    dec_gbps = dec_bytes / (attend_avg_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (oracle)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(lens, args.cpu_budget)
    traffic = None
    tfile = ROOT / "profiles" / "decode_kernel_traffic_config2.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": ("paged decode step: 16 layers x (KV append + paged decode attention), "
                         "batch 256, Llama-3.2-1B attention geometry 32q/8kv/d64, block 16, "
                         "lognormal context lengths mean 258 (seed 20260731)"),
            "batch": BATCH, "layers": LAYERS, "context_tokens": sum(lens), "pages": pages,
            "pool_blocks": 2 * pages, "part_pages": args.part_pages,
        },
        "pct_peak_hbm": round(100 * gbps / PEAK_HBM_GBPS, 2),
        "decode_tok_s": round(BATCH / (ms_per_step * 1e-3), 1),
        "algorithmic_bytes_per_step": step_bytes,
        "metadata_build_upload_ms": round(meta_ms, 3),
        "timing": {"gpu_ms_per_step": round(gpu_ms / args.steps, 4),
                   "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "host_enqueue_ms_per_step": round(enqueue_s * 1e3 / args.steps, 4)},
        "roofline": {
            "kernel": "decode_kernel (+ merge_kernel for split sequences), per layer",
            "bound": "hbm",
            "achieved": round(dec_gbps, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(dec_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": dec_bytes,
            "avg_launch_ms": round(attend_avg_ms, 5),
        },
        "cpu_baseline": cpu,
        "graph_replay": graph,
    }
    if cpu:
        line["gpu_over_cpu"] = round(line["decode_tok_s"] / cpu["value"], 1)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
