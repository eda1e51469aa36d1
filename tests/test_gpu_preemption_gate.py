"""
Greedy tokens under forced preemption are bit-identical to an unpreempted
run (the reference's phase-3 gate, tests/test_preemption_gpu.py:209-231),
driven through this backend's whole path: chunked prefill of the prompts,
decode steps with the fused KV append, then two running sequences preempted
and their blocks freed, reused and overwritten by another owner, and resumed:
- swap policy: their KV goes to pinned host memory and is swapped back into
  different block ids;
- recompute policy: their KV is dropped and rebuilt by prefilling the whole
  history again. Prefill and decode then produce the same KV only if the
  two paths round alike, so, as the reference suggests for this gate
  (fp16 prefill and decode kernels round differently), it runs with fp32
  pools, where both go through the same generic kernel.

The reference's gate needs Llama weights; here a small random model stands
in. Everything except attention runs per token row in float64 on the host,
so a row's result cannot depend on what it is batched with; attention runs
on the GPU. Equal tokens then require exactly what the gate tests on this
path: the swapped bytes come back bit for bit, and a sequence's decode
result does not depend on the batch it runs in or the block ids it holds.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llm_serving_layer_amd import BlockAllocator, ScheduledSeq, SequenceBlocks, build_batch_meta

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN, HQ, HKV, D, LAYERS, BS = 97, 64, 32, 8, 64, 2, 16
PROMPTS = [[(7 * i + 3 * j) % VOCAB for j in range(n)] for i, n in
           enumerate((20, 45, 70, 33, 90, 17))]
NEW_TOKENS = 12
SWAP_AT, RESUME_AT, VICTIMS = 3, 7, (1, 4)


class ToyModel:
    """Embedding, per layer q/k/v/o projections around paged attention with a
    residual, and an output head; all host math is per row in float64."""

    def __init__(self, seed=11):
        rng = np.random.default_rng(seed)
        self.emb = rng.standard_normal((VOCAB, HIDDEN))
        s = 1.0 / np.sqrt(HIDDEN)
        self.wq = [rng.standard_normal((HIDDEN, HQ * D)) * s for _ in range(LAYERS)]
        self.wk = [rng.standard_normal((HIDDEN, HKV * D)) * s for _ in range(LAYERS)]
        self.wv = [rng.standard_normal((HIDDEN, HKV * D)) * s for _ in range(LAYERS)]
        self.wo = [rng.standard_normal((HQ * D, HIDDEN)) / np.sqrt(HQ * D) for _ in range(LAYERS)]
        self.head = rng.standard_normal((HIDDEN, VOCAB)) * s

    @staticmethod
    def rows(x, w):
        return np.stack([r @ w for r in x])

    def forward(self, backend, scheduled):
        """Next greedy token of every scheduled sequence."""
        meta = build_batch_meta(scheduled, device=backend.device, page_size=BS)
        ids = [t for s in scheduled for t in s.new_token_ids]
        h = self.emb[ids]
        dev = backend.device
        for layer in range(LAYERS):
            def half(a, heads):
                return torch.from_numpy(a.reshape(len(ids), heads, D)).to(dev, backend.dtype)
            q = half(self.rows(h, self.wq[layer]), HQ)
            k = half(self.rows(h, self.wk[layer]), HKV)
            v = half(self.rows(h, self.wv[layer]), HKV)
            backend.append_kv(layer, k, v, meta)
            o = backend.attend(q, layer, D ** -0.5, meta)
            o = o.float().cpu().numpy().astype(np.float64).reshape(len(ids), HQ * D)
            h = h + self.rows(o, self.wo[layer])
        last = np.cumsum([s.query_len for s in scheduled]) - 1
        return [int(np.argmax(h[i] @ self.head)) for i in last]


class DeviceToyModel(ToyModel):
    """The same model on the GPU, driven the way the reference's scheduler
    drives its model (serving/scheduler/scheduler.py:743-757): ``forward``
    is ``greedy_step`` (metadata, token ids, ``forward_varlen`` returning
    device logits, greedy ids picked on the device, one copy of the ids to
    the host), timed with HIP events. Every projection runs one token row at
    a time in float32 with the same matrix shapes whatever the batch, so a
    row's logits cannot depend on what it is batched with."""

    def __init__(self, seed=11, device="cuda:0"):
        super().__init__(seed)
        dev = torch.device(device)
        f = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dev)  # noqa: E731
        self.d_emb, self.d_head = f(self.emb), f(self.head)
        self.d_w = [[f(w[l]) for l in range(LAYERS)] for w in (self.wq, self.wk, self.wv, self.wo)]
        from llm_serving_layer_amd.sampling import StepTimer
        self.timer = StepTimer(dev)
        self.step_ms = []

    @staticmethod
    def drows(x, w):
        return torch.cat([x[i:i + 1] @ w for i in range(x.shape[0])])

    def forward_varlen(self, tokens, meta, backend):
        h = self.d_emb[tokens]
        n = tokens.shape[0]
        wq, wk, wv, wo = self.d_w
        for layer in range(LAYERS):
            q = self.drows(h, wq[layer]).reshape(n, HQ, D).to(backend.dtype)
            k = self.drows(h, wk[layer]).reshape(n, HKV, D).to(backend.dtype)
            v = self.drows(h, wv[layer]).reshape(n, HKV, D).to(backend.dtype)
            backend.append_kv(layer, k, v, meta)
            o = backend.attend(q, layer, D ** -0.5, meta).float().reshape(n, HQ * D)
            h = h + self.drows(o, wo[layer])
        last = meta.cu_query_lens[1:].long() - 1
        return self.drows(h[last], self.d_head)

    def forward(self, backend, scheduled):
        from llm_serving_layer_amd.sampling import greedy_step
        ids = greedy_step(self, scheduled, backend, BS, self.timer)
        self.step_ms.append(self.timer.elapsed_ms())
        return ids


def generate(model, preempt: bool, policy: str = "swap", dtype=torch.float16):
    """Run every prompt to NEW_TOKENS tokens. With ``preempt`` the victims are
    swapped out at decode step SWAP_AT and their blocks freed; those blocks
    are then taken by other owners and overwritten, and the victims are
    swapped back in, into newly allocated blocks, at RESUME_AT."""
    from llm_serving_layer_amd.backend import MI355XBackend
    from llm_serving_layer_amd.swap import KVSwapSpace

    nb, reserve = 96, 8
    backend = MI355XBackend(LAYERS, nb, BS, HKV, HQ, D, device="cuda:0", dtype=dtype)
    alloc = BlockAllocator(nb, BS)
    seqs = [SequenceBlocks(alloc, seq_id=i) for i in range(len(PROMPTS))]
    out = [[] for _ in PROMPTS]
    for s, p in zip(seqs, PROMPTS):
        s.append(len(p))
    first = model.forward(backend, [ScheduledSeq(s, list(p)) for s, p in zip(seqs, PROMPTS)])
    for o, t in zip(out, first):
        o.append(t)
    swap = KVSwapSpace(backend)
    handles, moved, fill, resumed = {}, {}, [], {}
    step = 0
    while any(len(o) < NEW_TOKENS for o in out):
        step += 1
        if preempt and step == SWAP_AT:
            for i in VICTIMS:
                moved[i] = list(seqs[i].block_ids)
                if policy == "swap":
                    handles[i] = swap.swap_out(f"req{i}", seqs[i])
                seqs[i].free()
                seqs[i] = None
            old = sorted({b for v in moved.values() for b in v})
            # every free block, the victims' included, goes to another owner,
            # but for a reserve the running sequences grow into
            fill = alloc.allocate(alloc.num_free)
            spare = [b for b in fill if b not in old][:reserve]
            alloc.free(spare)
            fill = [b for b in fill if b not in spare]
            ids = torch.tensor(old, device=backend.device)
            g = torch.Generator(device=backend.device).manual_seed(5)
            for layer in range(LAYERS):
                for pool in (backend.k_pool[layer], backend.v_pool[layer]):
                    pool.index_copy_(0, ids, torch.randn(pool[ids].shape, generator=g,
                                                         device=backend.device).to(dtype))
        just_resumed = set()
        if preempt and step == RESUME_AT:
            alloc.free(fill)
            redo = []
            for i in VICTIMS:
                s = SequenceBlocks(alloc, seq_id=100 + i)
                if policy == "swap":
                    h = handles.pop(i)
                    s.append(h.num_tokens)
                    swap.swap_in(h, s)
                    swap.release(h)
                else:   # rebuild the KV of the prompt and every generated token
                    hist = PROMPTS[i] + out[i]
                    s.append(len(hist))
                    redo.append((i, ScheduledSeq(s, list(hist))))
                seqs[i] = s
                resumed[i] = list(s.block_ids)
            if redo:
                for (i, _), t in zip(redo, model.forward(backend, [r for _, r in redo])):
                    out[i].append(t)
                    just_resumed.add(i)
        live = [i for i, o in enumerate(out)
                if len(o) < NEW_TOKENS and seqs[i] is not None and i not in just_resumed]
        sched = []
        for i in live:
            seqs[i].append(1)
            sched.append(ScheduledSeq(seqs[i], [out[i][-1]]))
        for i, t in zip(live, model.forward(backend, sched)):
            out[i].append(t)
    backend.check_device_errors()
    return out, {"moved": moved, "resumed": resumed, "steps": step}


@pytest.mark.parametrize("policy,dtype", [("swap", torch.float16), ("swap", torch.float32),
                                          ("recompute", torch.float32)])
def test_greedy_tokens_are_bit_identical_under_preemption(policy, dtype):
    print(f"preemption gate policy={policy} dtype={dtype}", flush=True)
    model = ToyModel()
    ref, _ = generate(model, preempt=False, dtype=dtype)
    got, info = generate(model, preempt=True, policy=policy, dtype=dtype)
    # the rig really preempted: both victims were out for several steps and
    # came back into a different block list
    assert set(info["moved"]) == set(VICTIMS) and info["steps"] > RESUME_AT
    assert all(info["resumed"][i] != info["moved"][i] for i in VICTIMS)
    assert all(len(o) == NEW_TOKENS for o in got)
    for i, (a, b) in enumerate(zip(ref, got)):
        assert a == b, f"request {i}: {a} unpreempted vs {b} under preemption"
    assert len({t for o in ref for t in o}) > 3, "tokens should not be trivially constant"


@pytest.mark.parametrize("policy", ["swap", "recompute"])
def test_greedy_step_on_device_is_bit_identical_under_preemption(policy):
    """The gate through the scheduler's step structure on the device: greedy
    ids picked by the library's argmax kernel from device logits, each step
    timed with HIP events; swap and recompute (fp32 pools) both give the
    unpreempted tokens."""
    print(f"device greedy-step gate policy={policy}", flush=True)
    dtype = torch.float16 if policy == "swap" else torch.float32
    model = DeviceToyModel()
    ref, _ = generate(model, preempt=False, dtype=dtype)
    got, info = generate(model, preempt=True, policy=policy, dtype=dtype)
    assert set(info["moved"]) == set(VICTIMS) and info["steps"] > RESUME_AT
    for i, (a, b) in enumerate(zip(ref, got)):
        assert a == b, f"request {i}: {a} unpreempted vs {b} under preemption"
    assert len({t for o in ref for t in o}) > 3, "tokens should not be trivially constant"
    assert len(model.step_ms) > 2 * NEW_TOKENS and all(ms > 0 for ms in model.step_ms)

