"""The HIP engine beats the reference's PyTorch gather-and-attend path on the same GPU.

Both run the decode-throughput shape (GPT-2 124M fp32, 256 sequences, contexts
U[256,1024], block size 16) from the same state: the HIP path through
``Engine.step`` (graph-replayed decode), the reference path as the oracle's
restatement of tokquay's paged forward (write + gather + masked softmax,
tokquay/kv_cache.py:228-242, tokquay/model.py:94-96) on torch-ROCm, fed the
tokens the HIP engine picked so both see the same inputs at every step. Their
greedy ids must agree under the margin rule of tests/golden_ids.py: a
difference is allowed only where the gather path's own pick had a top-1 /
top-2 logit gap below MARGIN_BOUND. The measured rates are printed.
"""

from __future__ import annotations

import json
import random
import time

import pytest
import torch

from oracle.gpt2_ref import RefConfig, build_ref_model
from oracle.paged_ref import RefPagedBatch
from tests.golden_ids import MARGIN_BOUND
from tokquay_amd.engine import Engine
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.scheduler import SchedulerConfig
from tokquay_amd.sequence import SamplingParams
from tokquay_amd.weights import random_state_dict

pytestmark = pytest.mark.gpu

N, STEPS = 256, 6


def test_hip_engine_beats_the_reference_gather_path():
    cfg = GPT2Config()
    sd = random_state_dict(cfg, seed=0)
    model = GPT2(cfg)
    model.load_state_dict(sd)
    model = model.cuda().eval()
    alloc = BlockAllocator(cfg, 12288, 16, device="cuda")
    engine = Engine(model, alloc, SchedulerConfig(max_num_seqs=N, max_num_batched_tokens=32768))
    rng = random.Random(7)
    for _ in range(N):
        ctx = rng.randint(256, 1024 - 4 * STEPS)
        engine.add_request([rng.randrange(50256) for _ in range(ctx)], SamplingParams(max_tokens=4 * STEPS, ignore_eos=True))
    while engine.scheduler.waiting:
        engine.step()
    for _ in range(2):
        engine.step()  # graph capture + warm-up
    engine.drain()  # the step launched ahead: afterwards every token is on the host
    seqs = list(engine.scheduler.running)
    assert len(seqs) == N
    state = [(list(s.block_table), s.num_cached_tokens, list(s.token_ids)) for s in seqs]
    pool_copy = alloc.pool.clone()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hip_ids = []
    for _ in range(STEPS):
        hip_ids.append([e.token_id for e in engine.step()])
    torch.cuda.synchronize()
    hip_s = (time.perf_counter() - t0) / STEPS

    ref = build_ref_model(RefConfig(), sd, device="cuda")
    tables = [t for t, _, _ in state]
    cached = [c for _, c, _ in state]
    tokens = [t for _, _, t in state]
    ref_ids, margins, times = [], [], []
    for step in range(STEPS):
        for i in range(N):  # grow tables exactly as the allocator did for the HIP run
            if cached[i] + 1 > len(tables[i]) * 16:
                tables[i] = tables[i] + [seqs[i].block_table[len(tables[i])]]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            batch = RefPagedBatch(pool_copy, 16, tables, cached, [1] * N)
            ids = torch.tensor([[t[c]] for t, c in zip(tokens, cached)], device="cuda")
            logits = ref(ids, batch, last_only=True)[:, 0]
            nxt = logits.argmax(-1).tolist()
        times.append(time.perf_counter() - t0)
        top2 = logits.topk(2, dim=-1).values
        margins.append((top2[:, 0] - top2[:, 1]).tolist())
        ref_ids.append(nxt)
        for i in range(N):  # the HIP engine's pick is the next input of both runs
            tokens[i].append(hip_ids[step][i])
            cached[i] += 1
    ref_s = sorted(times)[len(times) // 2]
    same = sum(a == b for s1, s2 in zip(hip_ids, ref_ids) for a, b in zip(s1, s2))
    differ = [(st, i, m[i]) for st, (h, r, m) in enumerate(zip(hip_ids, ref_ids, margins))
              for i in range(N) if h[i] != r[i]]  # fmt: skip
    print("\n" + json.dumps({"hip_engine_tok_s": round(N / hip_s, 1), "reference_gather_path_tok_s": round(N / ref_s, 1),
                             "speedup": round(ref_s / hip_s, 2), "greedy_ids_identical": f"{same}/{N * STEPS}",
                             "differences (step, row, gather-path margin)": differ}))  # fmt: skip
    assert all(m < MARGIN_BOUND for _, _, m in differ), differ
    assert hip_s < ref_s
