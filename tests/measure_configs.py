"""Side-by-side measurements for the workload configurations (not collected by pytest).

Run on a GPU box: ``python tests/measure_configs.py``. Prints one JSON object
per configuration comparing the HIP path with the reference's gather-and-attend
path (the oracle's restatement of tokquay/kv_cache.py:228-242 and
tokquay/model.py:94-96) on the same GPU and on this host's CPU cores.

* config 1: GPT-2 124M, 8 prompts of U[16,64] random ids, 32 greedy tokens each
  through paged_greedy_generate, block size 16, pool 256 blocks.
* config 2: the decode-attention op alone, 64 sequences, contexts U[16,512]
  (redrawn until they fit the 1,024-block pool), 12 heads, block size 16, Q/K/V
  ~ N(0,1), one query per sequence.
* config 5: one mixed step: 4 prompts of U[512,1024] tokens fed in 256-token
  chunks (chunk 1, start 256) next to 128 decoding sequences at context
  U[64,768]; the reference pads every row to the chunk width.
"""

from __future__ import annotations

import json
import math
import os
import random
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from oracle.gpt2_ref import RefAllocator, RefConfig, build_ref_model, ref_paged_greedy_generate  # noqa: E402
from oracle.paged_ref import RefPagedBatch, cdiv, ref_attention  # noqa: E402
from tokquay_amd import ops  # noqa: E402
from tokquay_amd.generate import paged_forward, paged_greedy_generate  # noqa: E402
from tokquay_amd.kv_cache import BlockAllocator  # noqa: E402
from tokquay_amd.model import GPT2, GPT2Config  # noqa: E402
from tokquay_amd.sequence import Sequence  # noqa: E402
from tokquay_amd.weights import random_state_dict  # noqa: E402

H, D, BS = 12, 64, 16


def timed(fn, reps, sync=True):
    out = []
    for _ in range(reps):
        if sync:
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        if sync:
            torch.cuda.synchronize()
        out.append(time.perf_counter() - t0)
    return statistics.median(out)


def config1(sd):
    rng = random.Random(1)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(16, 64))] for _ in range(8)]
    m = GPT2(GPT2Config())
    m.load_state_dict(sd)
    m = m.cuda().eval()
    paged_greedy_generate(m, BlockAllocator(m.cfg, 256, BS, device="cuda"), prompts, 4)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    got = paged_greedy_generate(m, BlockAllocator(m.cfg, 256, BS, device="cuda"), prompts, 32)
    torch.cuda.synchronize()
    hip_s = time.perf_counter() - t0
    res = {}
    for dev in ("cuda", "cpu"):
        ref = build_ref_model(RefConfig(), sd, device=dev)
        ref_paged_greedy_generate(ref, RefAllocator(RefConfig(), 256, BS, device=dev), prompts, 2)
        if dev == "cuda":
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        want = ref_paged_greedy_generate(ref, RefAllocator(RefConfig(), 256, BS, device=dev), prompts, 32)
        if dev == "cuda":
            torch.cuda.synchronize()
        res[dev] = (time.perf_counter() - t0, want)
    return {"config": 1, "hip_s": round(hip_s, 4), "gather_gpu_s": round(res["cuda"][0], 4),
            "gather_cpu_s": round(res["cpu"][0], 3), "ids_identical_gpu_vs_cpu_oracle": got == res["cpu"][1],
            "decode_steps": 31}  # fmt: skip


def config2():
    s = 0
    while True:
        rng = random.Random(s)
        ctx = [rng.randint(16, 512) for _ in range(64)]
        if sum(cdiv(c, BS) for c in ctx) <= 1024:
            break
        s += 1
    g = torch.Generator().manual_seed(2)
    pool = torch.randn(1024, 1, 2, H, BS, D, generator=g)
    perm = torch.randperm(1024, generator=g).tolist()
    tables, i = [], 0
    for c in ctx:
        tables.append(perm[i : i + cdiv(c, BS)])
        i += cdiv(c, BS)
    q = torch.randn(64, H, 1, D, generator=g)
    nbytes = sum(2 * c * H * D * 4 for c in ctx) + 2 * 64 * H * D * 4 + sum(cdiv(c, BS) * 4 for c in ctx) + 64 * 4
    # HIP op alone (the new token's K/V are part of the pool already).
    pg = pool.cuda()
    bt = torch.zeros(64, max(len(t) for t in tables), dtype=torch.int32)
    for r, t in enumerate(tables):
        bt[r, : len(t)] = torch.tensor(t)
    bt, cl = bt.cuda(), torch.tensor(ctx, dtype=torch.int32, device="cuda")
    qg = q[:, :, 0].contiguous().cuda()
    out = torch.empty_like(qg)
    run = lambda: ops.paged_decode(out, qg, pg, 0, bt, cl, max(ctx))  # noqa: E731
    for _ in range(5):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(True), torch.cuda.Event(True)
    e0.record()
    for _ in range(100):
        run()
    e1.record()
    torch.cuda.synchronize()
    hip_us = e0.elapsed_time(e1) / 100 * 1e3
    res = {}
    for dev in ("cuda", "cpu"):
        p = pool.to(dev)
        qq = q.to(dev)
        batch = RefPagedBatch(p, BS, tables, [c - 1 for c in ctx], [1] * 64)

        def step():
            k, v = batch.gather(0)
            return ref_attention(qq, k, v, batch.mask)

        want = step()
        res[dev] = timed(step, 20, sync=dev == "cuda")
        if dev == "cpu":
            err = float((out.cpu() - want[:, :, 0]).abs().max())
    return {"config": 2, "hip_us": round(hip_us, 2), "hip_GBs": round(nbytes / hip_us / 1e3, 1),
            "gather_gpu_us": round(res["cuda"] * 1e6, 1), "gather_cpu_us": round(res["cpu"] * 1e6, 1),
            "algorithmic_MB": round(nbytes / 1e6, 2), "max_abs_diff_vs_cpu_oracle": err, "seed_used": s}  # fmt: skip


def config5(sd):
    rng = random.Random(5)
    prompts_len = [rng.randint(512, 1024) for _ in range(4)]
    dec_ctx = [rng.randint(64, 768) for _ in range(128)]
    m = GPT2(GPT2Config())
    m.load_state_dict(sd)
    m = m.cuda().eval()
    alloc = BlockAllocator(m.cfg, 8192, BS, device="cuda")
    prompts = [Sequence(i, [rng.randrange(50256) for _ in range(n)]) for i, n in enumerate(prompts_len)]
    decs = [Sequence(4 + i, [rng.randrange(50256) for _ in range(c - 1)]) for i, c in enumerate(dec_ctx)]
    for s_ in prompts + decs:
        alloc.allocate(s_)
    for i in range(0, 128, 32):
        nxt = paged_forward(m, alloc, decs[i : i + 32]).argmax(-1).tolist()
        for s_, t in zip(decs[i : i + 32], nxt):
            s_.append_token(t)
            alloc.append_slot(s_)
    paged_forward(m, alloc, prompts, [256] * 4)  # chunk 0
    # Snapshot the state of chunk 1 for the reference path.
    tables = [list(s_.block_table) for s_ in prompts + decs]
    starts = [s_.num_cached_tokens for s_ in prompts + decs]
    lens = [256] * 4 + [1] * 128
    ids = [s_.token_ids[st : st + n] for s_, st, n in zip(prompts + decs, starts, lens)]
    pool_copy = alloc.pool.clone()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    paged_forward(m, alloc, prompts + decs, lens)
    torch.cuda.synchronize()
    hip_s = time.perf_counter() - t0
    res = {}
    for dev in ("cuda", "cpu"):
        ref = build_ref_model(RefConfig(), sd, device=dev)

        def step():
            p = pool_copy if dev == "cuda" else pool_cpu
            batch = RefPagedBatch(p, BS, tables, starts, lens)
            x = torch.tensor([r + [0] * (256 - len(r)) for r in ids], device=dev)
            with torch.no_grad():
                return ref(x, batch, last_only=True)

        if dev == "cpu":
            pool_cpu = pool_copy.cpu()
        step()
        res[dev] = timed(step, 3 if dev == "cuda" else 1, sync=dev == "cuda")
    return {"config": 5, "chunk": 1, "hip_step_ms": round(hip_s * 1e3, 2), "gather_gpu_step_ms": round(res["cuda"] * 1e3, 2),
            "gather_cpu_step_s": round(res["cpu"], 2)}  # fmt: skip


def main():
    torch.manual_seed(0)
    print(json.dumps({"cpu_threads": torch.get_num_threads()}), flush=True)
    sd = random_state_dict(GPT2Config(), seed=0)
    for fn in (lambda: config2(), lambda: config1(sd), lambda: config5(sd)):
        print(json.dumps(fn()), flush=True)


if __name__ == "__main__":
    main()
