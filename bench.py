#!/usr/bin/env python3
"""
Benchmarks of the MI355X paged-KV backend. Prints ONE JSON line.

Default workload (``--workload decode``), the headline: Llama-3.2-1B
attention geometry (32 query heads, 8 KV heads, head_dim 64), block_size 16,
fp16, batch 256 with per-sequence context lengths drawn lognormal (mean 256,
sigma 0.8, clipped to [1, 2048], seed 20260731 -> realized mean 257.7, p90
498, max 1371, 65 980 tokens, 4247 pages), block tables shuffled over a pool
of 2x the pages needed, K/V cache and Q ~ N(0,1)*0.5. A step is, for each of
the 16 layers, one KV append of every sequence's new token followed by one
paged decode attention over every sequence's whole history, through the
backend's public ``append_kv`` / ``attend`` (which run as one fused launch
per layer). All 16 layers are cycled so a layer's KV (~135 MB) cannot stay
resident in the 256 MB last-level cache.

``value`` = algorithmic HBM bytes of the step (KV read once per KV head, Q
read, O written, append read + write, metadata) / measured step time. The
step is issued eagerly, call by call on one stream, as the serving engine
issues its layers (host enqueue stays well below the GPU time); the same
step captured once in a HIP graph and replayed is reported under
``graph_replay`` (on this ROCm it adds ~0.4 us between launches).
``roofline`` is the per-layer decode launch.

Other workloads (one JSON line each, same fields):
  prefill   8 sequences share a 1536-token paged prefix and each appends a
            512-token chunk (causal in the chunk), 16 layers; TFLOP/s of the
            masked attention on matrix cores.
  copy      4096 copy-on-write block pairs per step (27% of sources from a
            shared-prefix set), every layer, K and V; GB/s.
  swap      64 sequences x 256 tokens out to pinned host memory and back into
            different blocks; GB/s per direction over the host link.
  capacity  decode at 4096 sequences of 16..64 tokens, then 512 sequences of
            lognormal mean 2048 (clipped to 2048), pool of ~200 GB; GB/s.
  calib     a 1 GiB device copy, the known-size reference for HBM counters.
  argmax    greedy sampling of a decode step's logits on the device: 256 rows
            of Llama-3's 128 256-entry vocabulary, fp16; GB/s of the read.
  timeline  the headline decode launch under the instrumented build
            (``python -m llm_serving_layer_amd.build --timeline``, loaded with
            PKV_LIBRARY=llm_serving_layer_amd/_native/libpagedkv_timeline.so):
            per-wave start / first page / last page / end times, summarised
            as ramp, steady stream and tail. Not a throughput line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import random
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HQ, HKV, D, BS, LAYERS = 32, 8, 64, 16, 16
SEED = 20260731
PEAK_HBM_GBPS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0
METRIC = ("paged decode attn+append HBM GB/s (% peak); decode tok/s @ batch 256, 1 GPU")
GEOM = "Llama-3.2-1B attention geometry 32q/8kv/d64, block 16, fp16"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def lognormal_lengths(n, mean_len, sigma=0.8, max_seq=2048, seed=SEED):
    """The reference's length law (bench/capacity.py:196-242), lognormal branch."""
    rng = random.Random(seed)
    mu = math.log(mean_len) - sigma ** 2 / 2.0
    return [max(1, min(max_seq, int(round(rng.lognormvariate(mu, sigma))))) for _ in range(n)]


def decode_bytes(kv_lens, pages):
    """Algorithmic HBM bytes of one layer's append + decode attention."""
    T = len(kv_lens)
    kv = sum(kv_lens) * HKV * D * 2 * 2          # K and V rows, each KV head once
    qo = T * HQ * D * 2 * 2                      # Q read + O written
    meta = 4 * (pages + 2 * T + 1)               # kv_indices, kv_lens, kv_indptr
    append = T * HKV * D * 2 * 2 * 2 + 4 * T     # new K,V rows read + written, slots
    return kv + qo + meta + append


# ----------------------------------------------------------------- helpers ---

def fill_pool(bk, seed):
    import torch
    g = torch.Generator(device=bk.device).manual_seed(seed)
    for l in range(bk.num_layers):  # every page read holds real data
        for kv in range(2):
            x = bk._pool[l, kv]
            x.copy_(torch.randn(x.shape, generator=g, device=bk.device, dtype=torch.float32)
                    .mul_(0.5))


def shuffled_allocator(nb, seed=SEED):
    import torch
    from llm_serving_layer_amd import BlockAllocator
    alloc = BlockAllocator(nb, BS)
    alloc.allocate(nb)
    alloc.free(torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).tolist())
    return alloc


def time_eager(step, steps, warmup, per_launch):
    """K steps through the public API between synchronizations, timed with
    events around the whole run only; then K more steps with HIP events
    around every launch (on the current stream, where the backend launches)
    for the per-launch average, which the extra events slow down."""
    import torch
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step(None)
    stop.record()
    enqueue = time.perf_counter() - t0
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(per_launch)] for _ in range(steps)]
    for s in range(steps):
        step(ev[s])
    torch.cuda.synchronize()
    launch = [a.elapsed_time(b) for row in ev for a, b in row]
    return {"ms_per_step": max(gpu_ms, wall * 1e3) / steps,
            "gpu_ms_per_step": gpu_ms / steps, "wall_ms_per_step": wall * 1e3 / steps,
            "host_enqueue_ms_per_step": enqueue * 1e3 / steps,
            "launch_ms": sum(launch) / len(launch)}


def time_graph(step, steps, warmup):
    """The same step captured once in a HIP graph and replayed K times,
    bracketed by events on the replay stream."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(None)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(None)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    gs, ge = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    gs.record()
    for _ in range(steps):
        g.replay()
    ge.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {"ms_per_step": max(gs.elapsed_time(ge), wall * 1e3) / steps,
            "gpu_ms_per_step": gs.elapsed_time(ge) / steps}, g


def traffic_for(name):
    f = ROOT / "profiles" / f"{name}_traffic.json"
    if f.exists():
        return json.loads(f.read_text()).get("hbm_bytes_per_launch")
    return None


def base_line(args, metric, value, unit, ms, dtype, workload, **cfg):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": dtype, "data": "synthetic", "config": {"workload": workload, **cfg}}


# ------------------------------------------------------------------ decode ---

def decode_setup(device, lens, nb, part_pages):
    import torch
    from llm_serving_layer_amd import ScheduledSeq, SequenceBlocks, build_batch_meta
    from llm_serving_layer_amd.backend import MI355XBackend

    bk = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device=device, dtype=torch.float16,
                       part_pages=part_pages)
    fill_pool(bk, SEED)
    alloc = shuffled_allocator(nb)
    seqs = []
    for i, n in enumerate(lens):
        s = SequenceBlocks(alloc, seq_id=i)
        s.append(n - 1)          # history; the step appends the n-th token
        seqs.append(s)
    for s in seqs:
        s.append(1)
    # steady-state host cost of one step's metadata: build + upload, the
    # median of several builds after a first (warm-up) one
    times = []
    for _ in range(8):
        t0 = time.perf_counter()
        meta = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], device, BS)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    meta_ms = float(np.median(times[1:]))
    T = len(lens)
    g = torch.Generator(device=device).manual_seed(SEED + 1)
    k = (torch.randn(LAYERS, T, HKV, D, generator=g, device=device) * 0.5).half()
    v = (torch.randn(LAYERS, T, HKV, D, generator=g, device=device) * 0.5).half()
    q = (torch.randn(LAYERS, T, HQ, D, generator=g, device=device) * 0.5).half()
    outs = [None] * LAYERS   # the last step's attention outputs, per layer
    # each layer's q, k, v as a tensor of its own (as a model's projections
    # hand them over), not sliced inside the timed loop
    qs, ks, vs = list(q.unbind(0)), list(k.unbind(0)), list(v.unbind(0))

    def step(events, m=None):
        m = meta if m is None else m
        for l in range(LAYERS):
            bk.append_kv(l, ks[l], vs[l], m)
            if events is not None:
                events[l][0].record()
            outs[l] = bk.attend(qs[l], l, 0.125, m)
            if events is not None:
                events[l][1].record()

    ctx = {"bk": bk, "meta": meta, "seqs": seqs, "q": q, "k": k, "v": v, "outs": outs}
    return bk, meta, step, meta_ms, ctx


def check_layers_vs_oracle(ctx, layers=(0, LAYERS - 1)):
    """
    Outside the timed region: the outputs the last (graph-replayed) step left
    for ``layers`` against the oracle (CPU fp32 restatement of the reference's
    PagedTorchBackend) on the same inputs, at the parity bar (max-abs 2e-3,
    max-rel 1e-2). The step's appends are idempotent, so the pool as it is
    now is the pool every replay attended over. Raises on a mismatch.
    """
    import torch
    from llm_serving_layer_amd import ScheduledSeq, build_batch_meta
    from oracle import PagedTorchOracle

    bk, seqs = ctx["bk"], ctx["seqs"]
    torch.cuda.synchronize()
    meta = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], "cpu", BS)
    worst = 0.0
    for l in layers:
        ref = PagedTorchOracle(1, bk.num_blocks, BS, HKV, HQ, D, device="cpu",
                               dtype=torch.float32)
        ref.k_pool[0].copy_(bk.k_pool[l].float().cpu())
        ref.v_pool[0].copy_(bk.v_pool[l].float().cpu())
        ref.append_kv(0, ctx["k"][l].float().cpu(), ctx["v"][l].float().cpu(), meta)
        want = ref.attend(ctx["q"][l].float().cpu(), 0, 0.125, meta)
        got = ctx["outs"][l].float().cpu()
        d = (got - want).abs()
        big = want.abs() > 0.2
        rel = float((d[big] / want.abs()[big]).max()) if bool(big.any()) else 0.0
        if not (float(d.max()) <= 2e-3 and rel <= 1e-2 and bool(torch.isfinite(got).all())):
            raise RuntimeError(f"layer {l}: graph-replayed decode differs from the oracle "
                               f"(max abs {float(d.max()):.3g}, max rel {rel:.3g})")
        worst = max(worst, float(d.max()))
    return {"layers": list(layers), "max_abs_vs_oracle": round(worst, 6),
            "bar": "max-abs 2e-3, max-rel 1e-2 vs fp32 oracle"}


def time_e2e(ctx, step, steps, warmup):
    """
    Serving-loop step, as the reference's scheduler runs one
    (serving/scheduler/scheduler.py:743-757): grow every sequence by the
    token it is about to write and describe the batch (DecodeStepper: one
    allocate call for the sequences whose last page is full, the CSR and
    the other index arrays updated in place, one pinned upload), plan the
    step, and enqueue its 16 layers (append_kv + attend each), with no host
    wait inside the loop, so step n+1's host work overlaps the GPU running
    step n. After `warmup` free-running steps, `steps` steps are timed with
    HIP events on the launch stream (the host's own time for them is
    reported beside it: below the GPU's, the loop is GPU-bound).

    Each step holds one more token per sequence than the one before, so the
    loop is compared with the GPU time of the same work: the step issued
    eagerly with fixed metadata (no host work but the enqueue), timed at
    the lengths the loop starts from and at those it ends at, and
    interpolated (the work is linear in the tokens) to the timed steps'
    mean length.
    Returns (ms per loop step, that GPU ms per step, host ms of each part of
    a loop step, measured in separate loops).
    """
    import torch
    from llm_serving_layer_amd import ScheduledSeq, build_batch_meta
    from llm_serving_layer_amd.stepping import DecodeStepper

    bk, seqs = ctx["bk"], ctx["seqs"]
    stepper = DecodeStepper(seqs, "cuda:0", BS)

    def one():
        step(None, stepper.step())

    def gpu_step_here():
        m = build_batch_meta([ScheduledSeq(s, [0]) for s in seqs], "cuda:0", BS)
        return time_eager(lambda ev: step(ev, m), steps, warmup, LAYERS)["gpu_ms_per_step"]

    gpu_start = gpu_step_here()
    # steady state: the loop runs free (no host wait); the timed steps are
    # bracketed by HIP events on the launch stream, so the figure is the GPU
    # timeline of those steps, including any time the GPU waits for the host
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(warmup):
        one()
    start.record()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    stop.record()
    host_ms = (time.perf_counter() - t0) * 1e3 / steps
    torch.cuda.synchronize()
    e2e_ms = start.elapsed_time(stop) / steps
    gpu_end = gpu_step_here()
    # the parts, each over `steps` repetitions (host time only)
    parts = {}
    t0 = time.perf_counter()
    metas = [stepper.step() for _ in range(steps)]
    parts["grow_and_describe"] = (time.perf_counter() - t0) * 1e3 / steps
    t0 = time.perf_counter()
    for m in metas:
        bk._ensure_planned(m)
    parts["plan"] = (time.perf_counter() - t0) * 1e3 / steps
    torch.cuda.synchronize()
    m = metas[-1]
    t0 = time.perf_counter()
    for _ in range(steps):
        step(None, m)
    parts["enqueue_16_layers"] = (time.perf_counter() - t0) * 1e3 / steps
    torch.cuda.synchronize()
    parts["loop_host_ms_per_step"] = host_ms
    # the GPU step at the timed steps' mean length (warmup + steps / 2 tokens
    # past the start; gpu_end is warmup + steps past it)
    gpu_ref = gpu_start + (gpu_end - gpu_start) * (warmup + steps / 2) / (warmup + steps)
    return (e2e_ms, gpu_ref,
            {k: round(v, 4) for k, v in parts.items()})


def run_decode_like(args, lens, nb, label, check=False, e2e=False):
    import torch
    pages = sum(-(-n // BS) for n in lens)
    log(f"{label}: {len(lens)} sequences, {sum(lens)} tokens, {pages} pages, pool {nb} blocks")
    bk, meta, step, meta_ms, ctx = decode_setup("cuda:0", lens, nb, args.part_pages)
    layer_bytes = decode_bytes(lens, pages)
    step_bytes = LAYERS * layer_bytes
    graph = graph_parity = None
    if not args.eager:
        log("graph capture + replay")
        graph, _g = time_graph(step, args.steps, args.warmup)
        bk.check_device_errors()
        if check:   # the outputs the last replay left
            graph_parity = check_layers_vs_oracle(ctx)
        del _g
    log("eager timing")
    eager = time_eager(step, args.steps, args.warmup, LAYERS)
    bk.check_device_errors()
    # planning (one device-to-host copy + the host plan + its upload), median
    # of several: dropping the plan forces a re-plan on the next attend
    qz = torch.zeros(len(lens), HQ, D, dtype=torch.float16, device="cuda:0")
    times = []
    for _ in range(6):
        bk.invalidate_plan()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        bk.attend(qz, 0, 0.125, meta)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    plan_ms = float(np.median(times[1:]))
    # the outputs the last eager step left (the plan was re-made above, so
    # run one more step on it first)
    if check:
        step(None)
        parity = check_layers_vs_oracle(ctx)
        if graph_parity is not None:
            parity["graph_replay_max_abs_vs_oracle"] = graph_parity["max_abs_vs_oracle"]
    else:
        parity = None
    e2e_ms, e2e_gpu, e2e_parts = (time_e2e(ctx, step, args.steps, args.warmup) if e2e
                                  else (None, None, None))
    ms = eager["ms_per_step"]
    # per launch: the GPU time of a step over its 16 launches (gaps between
    # launches included)
    launch_ms = eager["gpu_ms_per_step"] / LAYERS
    gbps = step_bytes / (ms * 1e-3) / 1e9
    kern_gbps = layer_bytes / (launch_ms * 1e-3) / 1e9
    return {
        "gbps": gbps, "ms": ms, "tok_s": len(lens) / (ms * 1e-3), "pages": pages,
        "step_bytes": step_bytes, "layer_bytes": layer_bytes, "launch_ms": launch_ms,
        "kern_gbps": kern_gbps, "eager": eager, "graph": graph, "meta_ms": meta_ms,
        "plan_ms": plan_ms, "parity": parity, "e2e_ms": e2e_ms, "e2e_parts": e2e_parts,
        "e2e_gpu_ms": e2e_gpu,
    }


def bench_decode(args):
    lens = lognormal_lengths(256, 256)
    r = run_decode_like(args, lens, 2 * sum(-(-n // BS) for n in lens), "decode",
                        check=True, e2e=not args.no_e2e)
    e = r["eager"]
    line = base_line(
        args, METRIC, round(r["gbps"], 1), "GB/s", r["ms"], "fp16",
        ("paged decode step: 16 layers x (KV append + paged decode attention), batch 256, "
         f"{GEOM}, lognormal context lengths mean 258 (seed {SEED})"),
        batch=256, layers=LAYERS, context_tokens=sum(lens), pages=r["pages"],
        pool_blocks=2 * r["pages"], part_pages=args.part_pages,
        execution=("eager: 16 x (append_kv + attend) issued call by call on one stream, "
                   "as the serving engine issues a decode step"))
    line.update({
        "pct_peak_hbm": round(100 * r["gbps"] / PEAK_HBM_GBPS, 2),
        "decode_tok_s": round(r["tok_s"], 1),
        "algorithmic_bytes_per_step": r["step_bytes"],
        "eager": {"ms_per_step": round(e["ms_per_step"], 4),
                  "gpu_ms_per_step": round(e["gpu_ms_per_step"], 4),
                  "host_enqueue_ms_per_step": round(e["host_enqueue_ms_per_step"], 4),
                  "attend_event_avg_ms": round(e["launch_ms"], 5)},
        "graph_replay": None if not r["graph"] else {
            "ms_per_step": round(r["graph"]["ms_per_step"], 4),
            "GB/s": round(r["step_bytes"] / (r["graph"]["ms_per_step"] * 1e-3) / 1e9, 1),
            "decode_tok_s": round(256 / (r["graph"]["ms_per_step"] * 1e-3), 1),
            "what": "the same step captured once in a HIP graph and replayed"},
        "host_side_ms": {"batch_meta_build_upload": round(r["meta_ms"], 3),
                         "plan": round(r["plan_ms"], 3)},
        "e2e": None if r["e2e_ms"] is None else {
            "ms_per_step": round(r["e2e_ms"], 4),
            "decode_tok_s": round(256 / (r["e2e_ms"] * 1e-3), 1),
            "gpu_ms_per_step_same_lengths": round(r["e2e_gpu_ms"], 4),
            "ratio_to_gpu_step": round(r["e2e_ms"] / r["e2e_gpu_ms"], 3),
            "host_ms_per_step": r["e2e_parts"],
            "what": ("per step: every sequence grown by one token and the batch described "
                     "(DecodeStepper), planned, 16 x (append_kv + attend) enqueued call by "
                     "call; no host wait inside the loop")},
        "parity": r["parity"],
        "roofline": {
            "kernel": "pkv::decode_kernel<_Float16,64,4> (LPT bins of (sequence, piece) items, split-K merge by the last arriver, KV append fused), one launch per layer",
            "bound": "hbm", "achieved": round(r["kern_gbps"], 1), "peak": PEAK_HBM_GBPS,
            "unit": "GB/s", "frac": round(r["kern_gbps"] / PEAK_HBM_GBPS, 4),
            "traffic": traffic_for("decode_kernel_batch256"),
            "algorithmic_bytes_per_launch": r["layer_bytes"],
            "avg_launch_ms": round(r["launch_ms"], 5),
            "timing": ("GPU time of an eagerly issued step (HIP events on the launch stream "
                       "around K steps) / 16 launches, gaps between launches included"),
        },
    })
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle)")
        cpu = cpu_baseline(lens, args.cpu_budget)
    line["cpu_baseline"] = cpu
    if cpu:
        line["gpu_over_cpu"] = round(line["decode_tok_s"] / cpu["value"], 1)
    return line


def cpu_baseline(lens, budget_s=10.0):
    """
    The oracle (CPU restatement of the reference's PagedTorchBackend, fp32)
    on the same workload: all 256 sequences, append + attend per layer.
    Bounded sample: as many single-layer passes as fit in ~budget_s, scaled
    to the 16-layer step; once on every core of this process's affinity
    mask, once on one thread.
    """
    import torch

    from llm_serving_layer_amd import BlockAllocator, ScheduledSeq, SequenceBlocks, build_batch_meta
    from oracle import PagedTorchOracle

    T = len(lens)
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
    k = torch.randn(T, HKV, D, generator=g) * 0.5
    q = torch.randn(T, HQ, D, generator=g) * 0.5

    def run(threads):
        torch.set_num_threads(threads)
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
        return times[len(times) // 2], len(times)

    prev = torch.get_num_threads()
    cores = len(os.sched_getaffinity(0))
    layer_s, n = run(cores)
    one_s, n1 = run(1)
    torch.set_num_threads(prev)
    return {"value": round(T / (layer_s * LAYERS), 2), "unit": "decode tok/s", "cores": cores,
            "kind": "port",
            "sample": (f"{n} single-layer append+attend passes over all {T} sequences (fp32, "
                       f"CPU restatement of PagedTorchBackend), median {layer_s * 1e3:.1f} "
                       f"ms/layer x {LAYERS} layers, torch.set_num_threads({cores}) = every core "
                       "of the affinity mask"),
            "single_thread": {"value": round(T / (one_s * LAYERS), 2), "cores": 1,
                              "sample": f"{n1} passes, median {one_s * 1e3:.1f} ms/layer"}}


# ------------------------------------------------------------------ argmax ---

def bench_argmax(args):
    """pkv_argmax_rows over (256, 128256) fp16 logits, the greedy pick of a
    batch-256 decode step (torch.argmax(logits, dim=-1) in the reference's
    scheduler), checked against torch.argmax outside the timed region."""
    import torch
    from llm_serving_layer_amd.sampling import greedy

    rows, vocab = 256, 128256
    g = torch.Generator(device="cuda:0").manual_seed(SEED)
    x = (torch.randn(rows, vocab, generator=g, device="cuda:0") * 4).half()
    if not torch.equal(greedy(x), torch.argmax(x, dim=-1)):
        raise RuntimeError("greedy ids differ from torch.argmax")
    for _ in range(args.warmup):
        greedy(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        greedy(x)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    nbytes = rows * vocab * 2 + rows * 8
    gbps = nbytes / (ms * 1e-3) / 1e9
    line = base_line(args, "greedy argmax HBM GB/s, 1 GPU", round(gbps, 1), "GB/s", ms, "fp16",
                     f"greedy sampling: argmax of {rows} rows x {vocab} fp16 logits",
                     rows=rows, vocab=vocab)
    line.update({"roofline": {"kernel": "pkv::argmax_kernel<_Float16>", "bound": "hbm",
                              "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                              "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None,
                              "algorithmic_bytes_per_launch": nbytes,
                              "avg_launch_ms": round(ms, 5),
                              "timing": "HIP events around K launches on the current stream"}})
    return line


# ---------------------------------------------------------------- timeline ---

def bench_timeline(args):
    """
    Ramp / steady / tail of one decode launch (the headline step, or with
    --timeline-of capacity-a the capacity workload's phase A), from the per-wave
    records of the instrumented build (100 MHz s_memrealtime ticks): each wave
    (one KV head of one bin) records its start, the end of its first and last
    page, its end (after any merge), its page and item counts, and its merges
    with the time they took. Every layer's launch runs the same plan, so the
    records the last launch leaves describe the launch.
    """
    import ctypes as C
    import torch
    from llm_serving_layer_amd import _native

    lib = _native.load()
    if not hasattr(lib, "pkv_timeline_read"):
        raise RuntimeError("the timeline workload needs the instrumented build: run "
                           "`python -m llm_serving_layer_amd.build --timeline` and set "
                           "PKV_LIBRARY=llm_serving_layer_amd/_native/libpagedkv_timeline.so")
    lib.pkv_timeline_read.restype = C.c_int
    lib.pkv_timeline_read.argtypes = [C.c_void_p, C.c_int64]
    if args.timeline_of == "capacity-a":
        # the capacity workload's phase A: 4096 sequences of uniform[16, 64]
        # tokens (the same lengths as bench_capacity), on a pool twice their pages
        rng = random.Random(SEED)
        lens = [rng.randint(16, 64) for _ in range(4096)]
        what = "capacity phase A (4096 sequences, uniform[16,64] tokens)"
    else:
        lens = lognormal_lengths(256, 256)
        what = "batch-256 headline step (lognormal mean 258)"
    pages = sum(-(-n // BS) for n in lens)
    bk, meta, step, _, ctx = decode_setup("cuda:0", lens, 2 * pages, args.part_pages)
    log("graph replay (instrumented build)")
    graph, _g = time_graph(step, args.steps, args.warmup)
    bk.check_device_errors()
    buf = np.zeros(16384 * 8, dtype=np.uint64)
    if lib.pkv_timeline_read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("pkv_timeline_read failed")
    t = buf.reshape(-1, 8).astype(np.int64)
    wid = np.nonzero(t[:, 0] > 0)[0]   # waves of bins with no item record nothing
    t = t[wid]
    t0 = t[:, 0].min()
    start, first, last, end = [(t[:, i] - t0) / 100.0 for i in range(4)]
    npg, nit, nmg = t[:, 4], t[:, 5], t[:, 6]
    merge_us = t[:, 7] / 100.0

    def pct(v):
        return {k: round(float(np.percentile(v, q)), 2)
                for k, q in (("p10", 10), ("p50", 50), ("p90", 90), ("max", 100))}

    page_bytes = 2 * BS * D * 2       # one KV head's K and V slice of a page
    rate = (npg - 1) / np.maximum(last - first, 1e-3)   # pages per us, per wave
    span = float(end.max())
    layer_bytes = decode_bytes(lens, pages)
    # waves still running, every half microsecond of the launch
    grid = np.arange(0.0, span + 0.5, 0.5)
    active = [int(((start <= x) & (end > x)).sum()) for x in grid]
    line = base_line(
        args, "decode launch timeline (per-wave, instrumented build)", round(span, 2), "us",
        graph["ms_per_step"], "fp16",
        f"one paged decode launch of the {what}, {GEOM}",
        batch=len(lens), pages=pages, part_pages=args.part_pages)
    # record w: wave w % waves of workgroup w // waves = bin * groups + KV
    # head group, its dispatch index (round-robin over the 8 XCDs)
    hgw = 4 if HKV % 4 == 0 else 2 if HKV % 2 == 0 else 1
    head = (wid // hgw % (HKV // hgw)) * hgw + wid % hgw
    xcd = (wid // hgw) % 8

    def by(key, n):
        return [{"pages_per_us_p50": round(float(np.median(rate[key == i])), 3),
                 "last_page_done_p90": round(float(np.percentile(last[key == i], 90)), 2)}
                for i in range(n)]

    line.update({
        "higher_is_better": False,
        "launch_us_graph_replay": round(graph["ms_per_step"] * 1e3 / LAYERS, 2),
        "by_kv_head": by(head, HKV), "by_xcd": by(xcd, 8),
        "waves": int(len(t)),
        "ramp_us": {"start": pct(start), "first_page_done": pct(first)},
        "steady": {"pages_per_wave": pct(npg), "items_per_wave": pct(nit),
                   "pages_per_us_per_wave": pct(rate),
                   "stream_GBps_all_waves": round(float(rate.sum()) * page_bytes / 1e3, 1),
                   "page_bytes_per_wave": page_bytes},
        "tail_us": {"last_page_done": pct(last), "end": pct(end),
                    "end_minus_last_page": pct(end - last)},
        "merges": {"count": int(nmg.sum()), "waves_merging": int((nmg > 0).sum()),
                   "us_per_merge": round(float(merge_us.sum() / max(int(nmg.sum()), 1)), 2)},
        "span_us": round(span, 2),
        "span_GBps": round(layer_bytes / (span * 1e-6) / 1e9, 1),
        "active_waves_every_0p5us": active,
    })
    return line


# ---------------------------------------------------------------- capacity ---

def bench_capacity(args):
    import torch
    # ~200 GB pool: 381 469 blocks of 512 KiB (16 layers x K,V x 16 KiB)
    nb = int(200e9 // (LAYERS * 2 * BS * HKV * D * 2))
    rng = random.Random(SEED)
    phase_a = [rng.randint(16, 64) for _ in range(4096)]
    phase_b = lognormal_lengths(512, 2048)
    out = {}
    for name, lens in (("A", phase_a), ("B", phase_b)):
        r = run_decode_like(args, lens, nb, f"capacity phase {name}",
                            e2e=name == "A" and not args.no_e2e)
        out[name] = {"sequences": len(lens), "mean_len": round(sum(lens) / len(lens), 1),
                     "tokens": sum(lens), "pages": r["pages"], "ms_per_step": round(r["ms"], 4),
                     "GB/s": round(r["gbps"], 1),
                     "pct_peak_hbm": round(100 * r["gbps"] / PEAK_HBM_GBPS, 2),
                     "decode_tok_s": round(r["tok_s"], 1),
                     "launch_ms": round(r["launch_ms"], 5),
                     "graph_replay_ms_per_step": (round(r["graph"]["ms_per_step"], 4)
                                                  if r["graph"] else None)}
        if r["e2e_ms"] is not None:
            out[name]["e2e"] = {"ms_per_step": round(r["e2e_ms"], 4),
                                "gpu_ms_per_step_same_lengths": round(r["e2e_gpu_ms"], 4),
                                "ratio_to_gpu_step": round(r["e2e_ms"] / r["e2e_gpu_ms"], 3),
                                "host_ms_per_step": r["e2e_parts"]}
        del r
        torch.cuda.empty_cache()
    total_bytes = sum(LAYERS * decode_bytes(l, sum(-(-n // BS) for n in l))
                      for l in (phase_a, phase_b))
    total_ms = out["A"]["ms_per_step"] + out["B"]["ms_per_step"]
    gbps = total_bytes / (total_ms * 1e-3) / 1e9
    line = base_line(
        args, "capacity decode attn+append HBM GB/s (% peak), 1 GPU", round(gbps, 1), "GB/s",
        total_ms, "fp16",
        (f"capacity decode: phase A 4096 seqs uniform[16,64], phase B 512 seqs lognormal "
         f"mean 2048 clipped 2048; {GEOM}; pool {nb} blocks (~200 GB), shuffled tables"),
        layers=LAYERS, pool_blocks=nb, part_pages=args.part_pages)
    line.update({"pct_peak_hbm": round(100 * gbps / PEAK_HBM_GBPS, 2), "phases": out,
                 "roofline": {"bound": "hbm", "achieved": round(gbps, 1),
                              "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                              "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None}})
    return line


# ----------------------------------------------------------------- prefill ---

def bench_prefill(args):
    import torch
    from llm_serving_layer_amd import ScheduledSeq, SequenceBlocks, build_batch_meta
    from llm_serving_layer_amd.backend import MI355XBackend

    n_seq, prefix, chunk = 8, 1536, 512
    nb = 2 * (prefix // BS + n_seq * chunk // BS)
    device = "cuda:0"
    bk = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device=device, dtype=torch.float16)
    fill_pool(bk, SEED)
    alloc = shuffled_allocator(nb)
    pre = SequenceBlocks(alloc, seq_id=1000)
    pre.append(prefix)                      # the radix-cached prefix, 96 full blocks
    seqs = []
    for i in range(n_seq):
        s = SequenceBlocks(alloc, seq_id=i)
        alloc.incref(pre.block_ids)
        s.block_ids = list(pre.block_ids)
        s.num_tokens = prefix
        s.append(chunk)
        seqs.append(s)
    meta = build_batch_meta([ScheduledSeq(s, [0] * chunk) for s in seqs], device, BS)
    T = n_seq * chunk
    g = torch.Generator(device=device).manual_seed(SEED + 2)
    k = (torch.randn(LAYERS, T, HKV, D, generator=g, device=device) * 0.5).half()
    v = (torch.randn(LAYERS, T, HKV, D, generator=g, device=device) * 0.5).half()
    q = (torch.randn(LAYERS, T, HQ, D, generator=g, device=device) * 0.5).half()

    def step(events):
        for l in range(LAYERS):
            bk.append_kv(l, k[l], v[l], meta)
            if events is not None:
                events[l][0].record()
            bk.attend(q[l], l, 0.125, meta)
            if events is not None:
                events[l][1].record()

    log(f"prefill: {n_seq} x ({prefix} shared + {chunk}) tokens, q_tile {bk.q_tile}")
    eager = time_eager(step, args.steps, args.warmup, LAYERS)
    bk.check_device_errors()
    # masked-exact flops: 4 d per visible (query, key) pair and query head
    pairs = sum(prefix + j + 1 for j in range(chunk))
    layer_flops = 4 * D * pairs * HQ * n_seq
    attend_ms = eager["launch_ms"]
    tflops = layer_flops / (attend_ms * 1e-3) / 1e12
    ms = eager["ms_per_step"]
    step_tflops = LAYERS * layer_flops / (ms * 1e-3) / 1e12
    line = base_line(
        args, "chunked-prefill attention TFLOP/s over a shared paged prefix, 1 GPU",
        round(step_tflops, 2), "TFLOP/s", ms, "fp16",
        (f"chunked prefill: 8 seqs share a 1536-token paged prefix, each appends a 512-token "
         f"chunk (causal in the chunk), 16 layers x (KV append + attention); {GEOM}"),
        layers=LAYERS, q_tile=bk.q_tile)
    line.update({
        "flops_per_layer": layer_flops,
        "roofline": {"kernel": "pkv::prefill_kernel<_Float16,64,4>", "bound": "mfma",
                     "achieved": round(tflops, 2), "peak": PEAK_MFMA_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
                     "traffic": traffic_for("prefill_kernel_8x512"),
                     "avg_launch_ms": round(attend_ms, 5),
                     "timing": "HIP events around each attend launch"},
        "eager": {k2: round(v2, 4) for k2, v2 in eager.items()},
    })
    return line


# -------------------------------------------------------------------- copy ---

def bench_copy(args):
    import torch
    from llm_serving_layer_amd import _native
    from llm_serving_layer_amd.backend import MI355XBackend

    pairs, nb, shared = 4096, 16384, 64
    device = "cuda:0"
    bk = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device=device, dtype=torch.float16)
    fill_pool(bk, SEED)
    rng = random.Random(SEED)
    perm = list(range(nb))
    rng.shuffle(perm)
    prefix_set = perm[:shared]                    # shared-prefix blocks, sources repeat
    uniq = perm[shared:shared + pairs]
    dsts = perm[shared + pairs:shared + 2 * pairs]
    srcs = [rng.choice(prefix_set) if rng.random() < 0.27 else uniq[i] for i in range(pairs)]
    n_shared = sum(1 for s in srcs if s in set(prefix_set))
    ids = torch.tensor(srcs + dsts, dtype=torch.int32, device=device)
    lib = bk._lib

    def launch(events):
        if events is not None:
            events[0][0].record()
        rc = lib.pkv_copy_blocks(bk._pool.data_ptr(), LAYERS, bk._plane_bytes, bk._block_bytes,
                                 nb, ids.data_ptr(), ids.data_ptr() + 4 * pairs, pairs,
                                 bk._status.data_ptr(),
                                 torch.cuda.current_stream().cuda_stream)
        _native.check(rc, "copy_blocks")
        if events is not None:
            events[0][1].record()

    log(f"copy: {pairs} pairs ({n_shared} from {shared} shared-prefix blocks)")
    eager = time_eager(launch, args.steps, args.warmup, 1)
    bk.check_device_errors()
    # the public API (host validation + id upload) for comparison
    t0 = time.perf_counter()
    for _ in range(3):
        bk.copy_blocks(srcs, dsts)
    torch.cuda.synchronize()
    api_ms = (time.perf_counter() - t0) * 1e3 / 3
    step_bytes = 2 * pairs * LAYERS * 2 * bk._block_bytes + 8 * pairs
    ms = eager["launch_ms"]
    gbps = step_bytes / (ms * 1e-3) / 1e9
    line = base_line(
        args, "copy-on-write block copy HBM GB/s (% peak), 1 GPU", round(gbps, 1), "GB/s",
        eager["ms_per_step"], "fp16",
        (f"radix copy-on-write: {pairs} block pairs per step, 27% of sources from a "
         f"{shared}-block shared prefix, 16 layers x K,V x 16 KiB per block"),
        pairs=pairs, pool_blocks=nb, shared_sources=n_shared)
    line.update({
        "pct_peak_hbm": round(100 * gbps / PEAK_HBM_GBPS, 2),
        "copies_per_s": round(pairs / (ms * 1e-3), 1),
        "public_api_ms_per_step": round(api_ms, 3),
        "roofline": {"kernel": "pkv::block_kernel (copy)", "bound": "hbm",
                     "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_HBM_GBPS, 4),
                     "traffic": traffic_for("block_copy_4096_pairs"),
                     "avg_launch_ms": round(ms, 5)},
    })
    return line


# -------------------------------------------------------------------- swap ---

def bench_swap(args):
    import torch
    from llm_serving_layer_amd import SequenceBlocks
    from llm_serving_layer_amd.backend import MI355XBackend
    from llm_serving_layer_amd.swap import KVSwapSpace

    n_seq, toks = 64, 256
    nb = 4 * n_seq * toks // BS
    device = "cuda:0"
    bk = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device=device, dtype=torch.float16)
    fill_pool(bk, SEED)
    alloc = shuffled_allocator(nb)
    space = KVSwapSpace(bk)
    seqs = []
    for i in range(n_seq):
        s = SequenceBlocks(alloc, seq_id=i)
        s.append(toks)
        seqs.append(s)
    nbytes = space.bytes_for(n_seq * toks // BS)

    # the host link itself: one pinned copy of the same size each way
    dev = torch.empty(nbytes, dtype=torch.uint8, device=device)
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    for _ in range(2):
        host.copy_(dev, non_blocking=True)
        dev.copy_(host, non_blocking=True)
    torch.cuda.synchronize()
    link = {}
    for name, (dst, src) in (("d2h", (host, dev)), ("h2d", (dev, host))):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(3):
            dst.copy_(src, non_blocking=True)
        b.record()
        torch.cuda.synchronize()
        link[name] = nbytes * 3 / (a.elapsed_time(b) * 1e-3) / 1e9
    del dev, host

    log(f"swap: {n_seq} x {toks} tokens, {nbytes / 2**20:.0f} MiB each way")
    outs, ins = [], []
    n_iter = args.warmup + args.steps
    for it in range(n_iter):
        if it == n_iter - 1:
            # outside the timed region: every victim's bytes before the last
            # round trip, (2, L, blocks, bs, Hkv, d) in logical block order
            torch.cuda.synchronize()
            before = [bk._pool[:, :, torch.tensor(s.block_ids, device=device)]
                      .transpose(0, 1).cpu() for s in seqs]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        handles = [space.swap_out(f"r{i}", s) for i, s in enumerate(seqs)]
        space.synchronize()
        t1 = time.perf_counter()
        fresh = []
        for s in seqs:
            s.free()
        for i in range(n_seq):
            s = SequenceBlocks(alloc, seq_id=i)
            s.append(toks)
            fresh.append(s)
        t2 = time.perf_counter()
        for h, s in zip(handles, fresh):
            space.swap_in(h, s)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        if it == n_iter - 1:
            # outside the timed region: the host copies equal the victims'
            # blocks as they were, and the blocks they were restored into
            # hold the same bytes (raises on a mismatch)
            for i, (h, s) in enumerate(zip(handles, fresh)):
                back = bk._pool[:, :, torch.tensor(s.block_ids, device=device)]
                if not (torch.equal(h.host_buffer, before[i])
                        and torch.equal(back.transpose(0, 1).cpu(), before[i])):
                    raise RuntimeError(f"swap round trip of sequence {i} is not bit-exact")
        for h in handles:
            space.release(h)
        seqs = fresh
        if it >= args.warmup:
            outs.append(t1 - t0)
            ins.append(t3 - t2)
    bk.check_device_errors()
    out_s, in_s = sorted(outs)[len(outs) // 2], sorted(ins)[len(ins) // 2]
    out_gbps, in_gbps = nbytes / out_s / 1e9, nbytes / in_s / 1e9
    both = 2 * nbytes / (out_s + in_s) / 1e9
    line = base_line(
        args, "preemption swap GB/s per direction over the host link, 1 GPU", round(both, 2),
        "GB/s", (out_s + in_s) * 1e3, "fp16",
        (f"preemption swap: {n_seq} sequences x {toks} tokens (1024 blocks, 512 MiB) out to "
         f"pinned host memory and back into different blocks; {GEOM}"),
        sequences=n_seq, tokens_each=toks)
    line.update({
        "swap_out_GB/s": round(out_gbps, 2), "swap_in_GB/s": round(in_gbps, 2),
        "roofline": {"bound": "host link", "achieved": round(both, 2),
                     "peak": round(min(link.values()), 2), "unit": "GB/s",
                     "frac": round(both / min(link.values()), 4), "traffic": None,
                     "peak_source": "pinned copy of the same size in this run",
                     "link_d2h_GB/s": round(link["d2h"], 2),
                     "link_h2d_GB/s": round(link["h2d"], 2)},
        "parity": "last round trip bit-exact: every handle's host bytes and every restored "
                  "block equal the victim's blocks before swap-out",
    })
    return line


# ------------------------------------------------------------- calibration ---

def bench_calib(args):
    """A plain device-to-device copy of 1 GiB: the known-size reference that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    n = 1 << 30
    x = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    y = torch.empty_like(x)
    x.fill_(1)
    for _ in range(args.warmup):
        y.copy_(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    gbps = 2 * n / (ms * 1e-3) / 1e9
    line = base_line(args, "device copy HBM GB/s (calibration)", round(gbps, 1), "GB/s", ms,
                     "u8", "1 GiB device-to-device copy (reads 1 GiB, writes 1 GiB)", bytes=n)
    line["roofline"] = {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                        "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4), "traffic": None}
    return line


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "prefill", "copy", "swap", "capacity", "calib",
                             "timeline", "argmax"])
    ap.add_argument("--timeline-of", default="headline", choices=["headline", "capacity-a"],
                    help="timeline: the launch to record (the headline step or capacity phase A)")
    ap.add_argument("--part-pages", type=int, default=None,
                    help="split-K partition size in pages (default: the backend's)")
    ap.add_argument("--eager", action="store_true",
                    help="decode: report the call-by-call step, no graph replay")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the serving loop (its steps grow the sequences; profiles of "
                         "the headline step leave it out)")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU work per CPU-baseline thread setting")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no cross-GPU exchange (each GPU "
              f"serves its own sequences); --gpus {args.gpus} is not supported.", file=sys.stderr)
        return 2
    if args.part_pages is None:
        from llm_serving_layer_amd.backend import DEFAULT_PART_PAGES
        args.part_pages = DEFAULT_PART_PAGES
    fn = {"decode": bench_decode, "prefill": bench_prefill, "copy": bench_copy,
          "swap": bench_swap, "capacity": bench_capacity, "calib": bench_calib,
          "timeline": bench_timeline, "argmax": bench_argmax}[args.workload]
    print(json.dumps(fn(args)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
