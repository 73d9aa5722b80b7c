"""Decode throughput of the paged-attention engine on one MI355X.

Workload (the decode-throughput configuration): GPT-2 124M, random-init fp32
weights (normal std 0.02), 256 concurrent sequences, block size 16, KV pool of
16,384 blocks (262,144 slots, 18 GiB). Each sequence draws a context c ~
U[256 + K/2, 1024 - K/2] (seeded; K timed steps) and its prompt of random token
ids is sized so that the K timed decode steps run at contexts c - K/2 ... c +
K/2 - 1: the timed window is centred on the draw, its contexts lie in
[256, 1024] and their mean is the draws' (~640). Prompts are prefilled through
the engine (untimed); then W warm-up and K timed decode steps run through
``Engine.step`` (scheduler + paged forward + sampling + the step's one sync).
The decode kernel's own timing runs eagerly over the same K contexts, from the
same state, before the timed steps (the engine's state is rewound in between).

Prints one JSON line: decode tok/s (``value``), the decode-attention kernel's
roofline (algorithmic bytes / live HIP-event kernel time vs 8 TB/s), and beside
them:

* ``cpu_baseline`` / ``gpu_gather_baseline``: the reference's gather-and-attend
  paged path (the oracle's restatement of it) on this host's CPU cores and, with
  torch, on the same GPU, from the same state, with greedy-id agreement;
* ``decode_op_alone``: the decode kernel alone on the 64-sequence op shape;
* ``prefill``: the prefill kernel's fp32 MFMA utilisation over mixed
  chunked-prefill + decode steps; ``mixed_attention``: the same steps' attention
  as one launch per layer for both kinds of row (its combined HBM + MFMA
  roofline, against two launches); ``mixed_engine``: the same scenario through
  ``Engine.step`` with chunked prefill and with the reference's alternating
  policy;
* ``itl`` / ``itl_chunked`` / ``saturated``: the 300-request serving trace
  (p50 / p99 inter-token latency) with each policy, and all requests at t=0.

Other modes (each prints one JSON line and exits): ``--small-batch N`` (decode
step p50 at N sequences), ``--configs`` (the small configurations side by side
with the gather path), ``--prefill-op`` (the prefill kernel alone on synthetic
shapes, also part of the main line as ``prefill_op_alone``), ``--pmc-probe`` (a
short run for counter collection).
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import random
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode tok/s (1 GPU); paged-attn HBM GB/s as % of peak; p50 ITL"
HBM_PEAK_GBS = 8000.0
MFMA_FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
N_SEQS, CTX_LO, CTX_HI, BLOCK, POOL_BLOCKS = 256, 256, 1024, 16, 16384
N_HEAD, D_HEAD = 12, 64
# HBM bytes the decode kernel moves per algorithmic byte on this workload, from two rocprofv3
# counter runs on ``bench.py --pmc-probe`` (FETCH_SIZE scaled x2.0 and WRITE_SIZE x1.0, the factors
# a 1 GiB copy kernel of known size gives): 999.95 MB read + 2.36 MB written per launch for
# 996.43 MB algorithmic (an earlier pair of runs on another box read 1,008.00 MB: 1.0140). The
# excess is the masked tail of each wave's last 16-position chunk.
DECODE_TRAFFIC_PER_ALGO_BYTE = 1.0059
# Greedy ids may differ from a reference run only where that run picked its token by a top-1 /
# top-2 logit gap below this (fp32 logits of two implementations differ by a few 1e-6).
MARGIN_BOUND = 1e-4


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def decode_bytes(ctxs: list[int], n_head: int = N_HEAD, d: int = D_HEAD, bs: int = BLOCK, write: bool = True) -> int:
    """Algorithmic HBM bytes of one decode-attention layer call: every K and V row of the context
    read once, q in and out, the block-table entries and context lengths, and (``write``, the
    engine's tq_paged_decode_write) the new token's K and V written into the pool."""
    kv = sum(2 * c * n_head * d * 4 for c in ctxs)
    new_kv = 2 * len(ctxs) * n_head * d * 4 if write else 0
    qo = 2 * len(ctxs) * n_head * d * 4
    meta = sum(cdiv(c, bs) * 4 for c in ctxs) + 4 * len(ctxs)
    return kv + new_kv + qo + meta


def prefill_flops(starts: list[int], lens: list[int], n_head: int = N_HEAD, d: int = D_HEAD) -> int:
    """Causal-exact flops of one prefill layer call: QK^T and PV over the visible keys only."""
    return sum(4 * n_head * d * (n * s + n * (n + 1) // 2) for s, n in zip(starts, lens))


# A spin of this many shader clock cycles (~0.2 ms on MI355X) per launch to be queued: the
# op-alone measurement enqueues its launches behind one long spin so that they run back to back
# (a launch that finds the GPU idle starts its 8 XCDs up to ~4 us apart, measured with per-wave
# timestamps, which inflates a 15 us launch by a tenth).
QUEUE_AHEAD_CYCLES = 500_000


class LaunchTimer:
    """Times attention launches per kind - "decode", "prefill", or "mixed" (both kinds of row in one
    tq_paged_mixed launch) - with HIP events that the launch itself records at the start and end of
    its kernels (tq_set_timing_events), and adds up each kind's algorithmic decode bytes and prefill
    flops. Its bookkeeping is O(rows) per launch, so an eager step's host work stays short and the
    launches run close together as in the graph-replayed steps."""

    def __init__(self, *kinds: str):
        import torch

        from tokquay_amd import _lib

        self.torch, self.lib = torch, _lib.lib()
        self.pairs = {k: [] for k in kinds}
        self.bytes = dict.fromkeys(kinds, 0)
        self.flops = dict.fromkeys(kinds, 0)

    def __call__(self, batch, kind):
        if kind not in self.pairs:
            return
        start, stop = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
        start.record()  # creates the events; the kernel launch records them again at its own start / end
        stop.record()
        self.lib.tq_set_timing_events(start.cuda_event, stop.cuda_event)
        self.pairs[kind].append((start, stop))
        starts, lens = batch.start, batch.new_lens  # lists; batch.context_lens builds a new one per access
        if kind in ("decode", "mixed"):
            self.bytes[kind] += decode_bytes([s + 1 for s, n in zip(starts, lens) if n == 1])
        if kind in ("prefill", "mixed"):
            pre = [(s, n) for s, n in zip(starts, lens) if n != 1]
            self.flops[kind] += prefill_flops([s for s, _ in pre], [n for _, n in pre])

    def launches(self, kind: str) -> int:
        return len(self.pairs[kind])

    def total_ms(self, kind: str) -> float:
        return sum(a.elapsed_time(b) for a, b in self.pairs[kind])


def load_model(seed: int = 0):
    from tokquay_amd.model import GPT2, GPT2Config
    from tokquay_amd.weights import random_state_dict

    model = GPT2(GPT2Config())
    model.load_state_dict(random_state_dict(model.cfg, seed=seed))
    return model.cuda().eval()


def window_draws(window: int, seed: int = 0) -> tuple[list[int], int, int]:
    """Each sequence's context at the middle of a ``window``-step decode window, uniform on [lo, hi]
    with lo = 256 + window // 2 and hi = 1024 - (window - 1 - window // 2): the window's contexts
    c - window // 2 ... c + window - 1 - window // 2 then stay inside [256, 1024]. Stratified: the
    i-th of the 256 draws is uniform on the i-th 1/256 of the range, and the draws are shuffled, so
    each is still uniform on [lo, hi] while their mean is the range's to within a position
    (256 independent draws put it anywhere within about +-27 of it, at two standard deviations)."""
    lo, hi = CTX_LO + window // 2, CTX_HI - (window - 1 - window // 2)
    rng = random.Random(seed + 4)
    width = (hi - lo + 1) / N_SEQS
    draws = [lo + int((i + rng.random()) * width) for i in range(N_SEQS)]
    rng.shuffle(draws)
    return draws, lo, hi


def build_engine(prompt_lens: list[int], max_tokens: int, seed: int = 0):
    """The engine with one running sequence per prompt length (random token ids), prefilled
    (untimed): each has its prompt cached and its first output token pending."""
    import torch

    from tokquay_amd.engine import Engine
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.scheduler import SchedulerConfig
    from tokquay_amd.sequence import SamplingParams

    model = load_model(seed)
    alloc = BlockAllocator(model.cfg, POOL_BLOCKS, BLOCK, device="cuda")
    engine = Engine(model, alloc, SchedulerConfig(max_num_seqs=N_SEQS, max_num_batched_tokens=32768, max_model_len=1024))
    rng = random.Random(seed + 5)
    for n in prompt_lens:
        prompt = [rng.randrange(50256) for _ in range(max(1, n))]
        engine.add_request(prompt, SamplingParams(max_tokens=max_tokens, ignore_eos=True))
    t0 = time.perf_counter()
    while engine.scheduler.waiting:
        engine.step()  # prefill-only steps: admission comes first while the queue is not empty
    torch.cuda.synchronize()
    log(f"prefilled {N_SEQS} sequences in {time.perf_counter() - t0:.2f} s")
    return engine, model


def engine_state(engine) -> tuple:
    """What decode steps change in the host state of an engine with nothing in flight and no
    request waiting: the free list, the ref counts, the running list and each running sequence's
    outputs, table, cached count and status. (The pool needs no copy: a step writes position p's
    K/V before anything reads it, and a rewound run writes those slots again.)"""
    alloc, sched = engine.allocator, engine.scheduler
    assert engine._inflight is None and not sched.waiting
    seqs = [(s, list(s.output_token_ids), list(s.block_table), s.num_cached_tokens, s.status, s.finish_reason)
            for s in sched.running]  # fmt: skip
    return list(alloc._free), list(alloc.ref_counts), list(sched.running), seqs


def rewind(engine, state: tuple) -> None:
    """Put a drained engine back in ``engine_state``'s state; sequences that finished by length
    since are running again (no request may have arrived or been evicted in between)."""
    engine.drain()
    free, refs, running, seqs = state
    sched = engine.scheduler
    assert not sched.waiting and set(map(id, sched.running)) <= set(map(id, running))
    engine.allocator._free[:] = free
    engine.allocator.ref_counts[:] = refs
    sched.running[:] = running
    for s, out, table, cached, status, reason in seqs:
        s.output_token_ids[:] = out
        s.block_table[:] = table
        s.num_cached_tokens = cached
        s.status, s.finish_reason = status, reason


def host_cpu_name() -> str:
    """The host CPU's model name (what ``lscpu`` prints as "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def margin_agreement(got: list[list[int]], want: list[list[int]], margins: list[list[float]]) -> dict:
    """Per-step greedy ids of two runs fed the same tokens: how many agree, and whether every
    disagreement sits where the reference run's pick had a top-1 / top-2 gap below MARGIN_BOUND."""
    total = same = 0
    near_ties, violations = [], []
    for s, (g, w, m) in enumerate(zip(got, want, margins)):
        for i, (a, b, gap) in enumerate(zip(g, w, m)):
            total += 1
            if a == b:
                same += 1
            else:
                (near_ties if gap < MARGIN_BOUND else violations).append((s, i, round(gap, 7)))
    return {"ids_compared": total, "ids_identical": same, "near_tie_mismatches": len(near_ties),
            "mismatches_above_margin_bound": len(violations), "margin_bound": MARGIN_BOUND,
            "min_reference_margin": round(min(min(m) for m in margins), 7)}  # fmt: skip


# ------------------------------------------------------------------------------ HIP path measurements
def decode_op_alone(seed: int = 2) -> dict:
    """The decode kernel alone on the op-alone shape: 64 sequences, 12 heads, head_dim 64,
    contexts U[16, 512] (redrawn with seeds 0, 1, ... until they fit the 1,024-block pool), block
    size 16, block tables a seeded random permutation, Q and the pool ~ N(0, 1), one query per
    sequence; a 1-layer pool. Median of 200 launches timed with HIP events the launch records around
    its kernels, enqueued behind one long spin kernel so that they run back to back as in a model
    step; the median of 200 launches paced by the host (each one finding the GPU idle, its events
    recorded around the call) is reported beside it."""
    import torch

    from tokquay_amd import _lib, ops

    draw = 0
    while True:
        rng = random.Random(draw)
        ctx = [rng.randint(16, 512) for _ in range(64)]
        if sum(cdiv(c, BLOCK) for c in ctx) <= 1024:
            break
        draw += 1
    g = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.randn(1024, 1, 2, N_HEAD, BLOCK, D_HEAD, device="cuda", generator=g)
    perm = torch.randperm(1024, device="cuda", generator=g).tolist()
    tables = torch.zeros(64, max(cdiv(c, BLOCK) for c in ctx), dtype=torch.int32)
    i = 0
    for r, c in enumerate(ctx):
        n = cdiv(c, BLOCK)
        tables[r, :n] = torch.tensor(perm[i : i + n], dtype=torch.int32)
        i += n
    tables = tables.cuda()
    lens = torch.tensor(ctx, dtype=torch.int32, device="cuda")
    order = torch.tensor(sorted(range(64), key=lambda r: -ctx[r]), dtype=torch.int32, device="cuda")
    q = torch.randn(64, N_HEAD * D_HEAD, device="cuda", generator=g)
    out = torch.empty_like(q)
    call = lambda: ops.paged_decode(out, q, pool, 0, tables, lens, max(ctx), seq_order=order)  # noqa: E731
    for _ in range(10):
        call()
    lib = _lib.lib()
    torch.cuda.synchronize()
    torch.cuda._sleep(200 * QUEUE_AHEAD_CYCLES)  # ~40 ms: the host enqueues all 200 launches behind it
    queued = []
    for _ in range(200):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        b.record()
        lib.tq_set_timing_events(a.cuda_event, b.cuda_event)  # re-recorded at the kernel's start and end
        call()
        queued.append((a, b))
    torch.cuda.synchronize()
    paced = []
    for _ in range(200):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        call()
        b.record()
        paced.append((a, b))
    torch.cuda.synchronize()
    us = statistics.median(a.elapsed_time(b) for a, b in queued) * 1e3
    us_paced = statistics.median(a.elapsed_time(b) for a, b in paced) * 1e3
    nbytes = decode_bytes(ctx, write=False)
    return {"workload": f"decode op alone: 64 sequences, ctx U[16,512] (draw seed {draw}, {sum(ctx)} positions), "
                        "12 heads x 64, block 16, 1,024-block pool (1 layer), random block permutation; "
                        "launches queued back to back",
            "draw_seed": draw,
            "kernel": "tq_paged_decode", "us_per_call": round(us, 2), "bytes_per_call": nbytes,
            "achieved_GBs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "us_per_call_host_paced": round(us_paced, 2)}  # fmt: skip


def prefill_batch(seed: int = 32, reps: int = 3) -> dict:
    """The prefill kernel on a large launch, as the engine's prefill steps run it: one prefill step of
    32 prompts of U[256,1024] random tokens (block size 16) through the model, every layer's
    tq_paged_prefill launch timed by the events it records; causal-exact flops over the launch time
    against the fp32 MFMA peak. The step runs reps times from the same state (its cache writes are the
    same each time); the median per layer over all runs."""
    import torch

    from tokquay_amd import kv_cache
    from tokquay_amd.generate import paged_forward
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.sequence import Sequence

    model = load_model()
    alloc = BlockAllocator(model.cfg, 4096, BLOCK, device="cuda")
    rng = random.Random(seed)
    seqs = [Sequence(i, [rng.randrange(50256) for _ in range(rng.randint(256, 1024))]) for i in range(32)]
    for sq in seqs:
        alloc.allocate(sq)
    lens = [sq.num_tokens for sq in seqs]
    flops = prefill_flops([0] * len(lens), lens)
    paged_forward(model, alloc, seqs)  # warm-up
    times = []
    try:
        for _ in range(reps):
            for sq in seqs:
                sq.num_cached_tokens = 0
            timer = LaunchTimer("prefill")
            kv_cache.PagedBatch.launch_hook = timer
            paged_forward(model, alloc, seqs)
            torch.cuda.synchronize()
            kv_cache.PagedBatch.launch_hook = None
            times += [a.elapsed_time(b) * 1e3 for a, b in timer.pairs["prefill"]]
    finally:
        kv_cache.PagedBatch.launch_hook = None
    alloc.check_device_errors()
    us = statistics.median(times)
    return {"workload": f"one prefill step: 32 prompts U[256,1024] at start 0 ({sum(lens)} rows), block 16, "
                        "12 layers; median launch over the layers of 3 runs",
            "kernel": "tq_paged_prefill (fp32 MFMA 16x16x4; one wave per workgroup, two query tiles per wave)",
            "bound": "mfma", "us_per_launch": round(us, 2), "mflop_per_launch": round(flops / 1e6, 1),
            "achieved": round(flops / us / 1e6, 2), "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(flops / us / 1e6 / MFMA_FP32_PEAK_TFLOPS, 4)}  # fmt: skip


def hbm_copy(reps: int = 20) -> dict:
    """A reference for the HBM bandwidth this box sustains: torch's device-to-device copy of 1 GiB
    (1 GiB read + 1 GiB written), each copy bracketed by events; median."""
    import torch

    x = torch.randn(1 << 28, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    pairs = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        y.copy_(x)
        b.record()
        pairs.append((a, b))
    torch.cuda.synchronize()
    us = statistics.median(a.elapsed_time(b) for a, b in pairs) * 1e3
    moved = 2 << 30
    return {"workload": "torch copy_ of 1 GiB on the device (1 GiB read + 1 GiB written), median of 20",
            "us": round(us, 1), "GBs": round(moved / us / 1e3, 1), "frac": round(moved / us / 1e3 / HBM_PEAK_GBS, 4)}


def prefill_op_alone(reps: int = 25) -> dict:
    """The prefill kernel alone (``tq_paged_prefill`` on a one-layer pool with seeded random K/V, q
    and block tables dealt from a random permutation of the pool), each shape launched ``reps`` times
    back to back, every launch timed by the events it records; median per shape. Shapes: config 5's
    four chunks alone (``mixed_chunked_step``'s 4 prompts in 256-token chunks), ``prefill_batch``'s 32
    prompts U[256,1024] at start 0, long prompts (2 x 8192, 16 x 2048 at start 0), whose key loops are
    long enough that launch start and end amortise: the kernel's steady state, and one prompt of one row
    (12 workgroups of one key tile): the span of a launch with almost nothing to do."""
    import torch

    from tokquay_amd import _lib, ops

    lib = _lib.lib()

    def shapes():
        rng = random.Random(5)  # mixed_chunked_step's draws: each prompt's length, then its token ids
        plen = []
        for _ in range(4):
            plen.append(rng.randint(512, 1024))
            for _ in range(plen[-1]):
                rng.randrange(50256)
        for k in range(4):
            starts = [256 * k for p in plen if p > 256 * k]
            yield f"config 5 chunk {k}", starts, [min(256, p - 256 * k) for p in plen if p > 256 * k]
        rng = random.Random(32)  # prefill_batch's draws: each prompt's length, then its token ids
        lens = []
        for _ in range(32):
            lens.append(rng.randint(256, 1024))
            for _ in range(lens[-1]):
                rng.randrange(50256)
        yield "32 prompts U[256,1024] (prefill_batch's prompts)", [0] * 32, lens
        yield "2 prompts x 8192", [0, 0], [8192, 8192]
        yield "1 prompt x 1 row (launch span)", [0], [1]
        yield "16 prompts x 2048", [0] * 16, [2048] * 16

    out = []
    g = torch.Generator(device="cuda").manual_seed(11)
    for name, starts, lens in shapes():
        # The 32-prompt shape also runs in the natural sequence order, on the same inputs, its
        # launches alternating with the ordered ones.
        compare = name.startswith("32 prompts")
        nblk = [cdiv(s + n, BLOCK) for s, n in zip(starts, lens)]
        nb = sum(nblk) + 8
        pool = torch.randn(nb, 1, 2, N_HEAD, BLOCK, D_HEAD, device="cuda", generator=g)
        perm = torch.randperm(nb, generator=torch.Generator().manual_seed(12)).tolist()
        tables = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
        i = 0
        for r, n in enumerate(nblk):
            tables[r, :n] = torch.tensor(perm[i : i + n], dtype=torch.int32)
            i += n
        rows = sum(lens)
        q = torch.randn(rows, N_HEAD * D_HEAD, device="cuda", generator=g)
        o = torch.empty_like(q)
        cu = torch.tensor([0] + list(itertools.accumulate(lens)), dtype=torch.int32, device="cuda")
        st = torch.tensor(starts, dtype=torch.int32, device="cuda")
        tables = tables.cuda()
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        # The batch view's dispatch order: most causal work first (stable).
        work = [n * (2 * s + n + 1) for s, n in zip(starts, lens)]
        order = torch.tensor(sorted(range(len(lens)), key=lambda b: -work[b]), dtype=torch.int32, device="cuda")
        variants = [(name, order)] + ([(name + ", natural order", None)] if compare else [])
        for _ in range(3):
            for _, so in variants:
                ops.paged_prefill(o, q, pool, 0, tables, cu, st, max(lens), d_error=err, seq_order=so)
        torch.cuda.synchronize()
        pairs = [[] for _ in variants]
        for _ in range(reps):
            for i, (_, so) in enumerate(variants):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                b.record()
                lib.tq_set_timing_events(a.cuda_event, b.cuda_event)
                ops.paged_prefill(o, q, pool, 0, tables, cu, st, max(lens), d_error=err, seq_order=so)
                pairs[i].append((a, b))
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        flops = prefill_flops(starts, lens)
        for (vname, _), ps in zip(variants, pairs):
            us = statistics.median(a.elapsed_time(b) for a, b in ps) * 1e3
            out.append({"shape": vname, "rows": rows, "mflop": round(flops / 1e6, 1), "us": round(us, 2),
                        "tflops": round(flops / us / 1e6, 2),
                        "frac": round(flops / us / 1e6 / MFMA_FP32_PEAK_TFLOPS, 4)})  # fmt: skip
        del pool, q, o
    return {"workload": "tq_paged_prefill alone on a one-layer pool (random K/V, q, permuted tables, the batch "
                        f"view's most-work-first sequence order unless named), launched {reps} times back to back per "
                        "shape; median launch", "shapes": out}


def mixed_chunked_step(seed: int = 5) -> tuple[dict, dict]:
    """Mixed chunked-prefill + decode steps: 4 prompts of U[512,1024] random tokens fed in 256-token
    chunks (chunk k starts at 256k) next to 128 sequences decoding at context U[64,768], block size 16.
    Each chunk step runs twice from the same state: with the step's attention as two launches per
    layer (decode rows, then prefill rows; each timed) and as one tq_paged_mixed launch. Returns the
    prefill kernel's fp32 MFMA utilisation (causal-exact flops / launch time / peak) in the two-launch
    runs, and the one launch's combined roofline: the time the decode rows' bytes take at HBM peak
    plus the time the prefill flops take at MFMA peak, over the measured launch time."""
    import torch

    from tokquay_amd import kv_cache
    from tokquay_amd.generate import paged_forward
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.sequence import Sequence

    model = load_model()
    alloc = BlockAllocator(model.cfg, 8192, BLOCK, device="cuda")
    rng = random.Random(seed)
    prompts = [Sequence(i, [rng.randrange(50256) for _ in range(rng.randint(512, 1024))]) for i in range(4)]
    decoders = [Sequence(4 + i, [rng.randrange(50256) for _ in range(rng.randint(64, 768) - 1)]) for i in range(128)]
    for s in prompts + decoders:
        alloc.allocate(s)
    for i in range(0, 128, 32):  # prefill the decoding sequences' contexts (untimed)
        nxt = paged_forward(model, alloc, decoders[i : i + 32]).argmax(-1).tolist()
        for s, t in zip(decoders[i : i + 32], nxt):
            s.append_token(t)
            alloc.append_slot(s)
    chunks, mixed = [], []
    same = compared = 0
    max_diff = 0.0
    try:
        for k in range(4):
            live = [p for p in prompts if p.num_cached_tokens < p.num_tokens]
            seqs = live + decoders
            lens = [min(256, p.num_tokens - p.num_cached_tokens) for p in live] + [1] * len(decoders)
            starts = [p.num_cached_tokens for p in live]
            cached = [s.num_cached_tokens for s in seqs]
            runs = {}
            for one in (False, True):  # the same step from the same state (the K/V it writes are the same)
                for s, c in zip(seqs, cached):
                    s.num_cached_tokens = c
                kv_cache.PagedBatch.one_launch_mixed = one
                timer = LaunchTimer("decode", "prefill", "mixed")
                kv_cache.PagedBatch.launch_hook = timer
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                logits = paged_forward(model, alloc, seqs, lens)
                torch.cuda.synchronize()
                runs[one] = (timer, logits, (time.perf_counter() - t0) * 1e3)
                kv_cache.PagedBatch.launch_hook = None
            two, one = runs[False][0], runs[True][0]
            ids_two, ids_one = runs[False][1].argmax(-1).tolist(), runs[True][1].argmax(-1).tolist()
            same += sum(a == b for a, b in zip(ids_two, ids_one))
            compared += len(ids_one)
            max_diff = max(max_diff, float((runs[False][1] - runs[True][1]).abs().max()))
            for s, t in zip(decoders, ids_one[len(live) :]):
                s.append_token(t)
                alloc.append_slot(s)
            n = two.launches("prefill")
            pre_us = two.total_ms("prefill") / n * 1e3
            dec_us = two.total_ms("decode") / two.launches("decode") * 1e3
            mix_us = one.total_ms("mixed") / one.launches("mixed") * 1e3
            flops = two.flops["prefill"] / n
            nbytes = one.bytes["mixed"] / one.launches("mixed")
            ideal_us = nbytes / (HBM_PEAK_GBS * 1e3) + flops / (MFMA_FP32_PEAK_TFLOPS * 1e6)
            chunks.append({"chunk": k, "prompt_rows": len(live), "starts": starts, "prefill_us": round(pre_us, 2),
                           "mflop_per_launch": round(flops / 1e6, 1), "tflops": round(flops / pre_us / 1e6, 2),
                           "frac": round(flops / pre_us / 1e6 / MFMA_FP32_PEAK_TFLOPS, 4),
                           "step_ms": round(runs[False][2], 3)})  # fmt: skip
            mixed.append({"chunk": k, "decode_mb": round(nbytes / 1e6, 1), "prefill_mflop": round(flops / 1e6, 1),
                          "ideal_us": round(ideal_us, 2), "one_launch_us": round(mix_us, 2),
                          "two_launch_us": round(dec_us + pre_us, 2), "decode_us": round(dec_us, 2),
                          "frac": round(ideal_us / mix_us, 4), "two_launch_frac": round(ideal_us / (dec_us + pre_us), 4),
                          "step_ms": round(runs[True][2], 3)})  # fmt: skip
    finally:
        kv_cache.PagedBatch.one_launch_mixed = True
        kv_cache.PagedBatch.launch_hook = None
    alloc.check_device_errors()
    workload = "4 prompts U[512,1024] in 256-token chunks + 128 decoding sequences, ctx U[64,768], block 16"
    tot_f = sum(c["mflop_per_launch"] for c in chunks)
    tot_us = sum(c["prefill_us"] for c in chunks)
    prefill = {
        "workload": workload,
        "kernel": "tq_paged_prefill (fp32 MFMA 16x16x4), launched on its own",
        "bound": "mfma",
        "achieved": round(tot_f / tot_us, 2),
        "peak": MFMA_FP32_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tot_f / tot_us / MFMA_FP32_PEAK_TFLOPS, 4),
        "chunks": chunks,
    }
    ideal = sum(m["ideal_us"] for m in mixed)
    one_us = sum(m["one_launch_us"] for m in mixed)
    two_us = sum(m["two_launch_us"] for m in mixed)
    mixed_attention = {
        "workload": workload,
        "kernel": "tq_paged_mixed (decode rows and prefill tiles in one launch per layer)",
        "bound": "hbm + mfma: decode bytes at 8 TB/s plus prefill flops at 157.3 TFLOP/s",
        "ideal_us": round(ideal, 2),
        "one_launch_us": round(one_us, 2),
        "frac": round(ideal / one_us, 4),
        "two_launch_us": round(two_us, 2),
        "two_launch_frac": round(ideal / two_us, 4),
        "speedup_over_two_launches": round(two_us / one_us, 3),
        "greedy_ids_vs_two_launches": {"ids_compared": compared, "ids_identical": same,
                                       "max_abs_logit_diff": max_diff},  # fmt: skip
        "chunks": mixed,
    }
    return prefill, mixed_attention


def mixed_engine(chunked: bool, seed: int = 5) -> dict:
    """The mixed scenario through ``Engine.step``: 128 sequences decode (context U[64,768]) when 4
    prompts of U[512,1024] tokens arrive. With chunked prefill the prompts are fed 256 tokens per
    step next to the decode rows; with the reference's alternating policy (2,048 padded tokens per
    step) the prompts are prefilled in steps of their own while the decode rows wait. Reports the
    steps and wall time from the prompts' arrival until every prompt has its first token, and the
    longest wait a decoding sequence saw for a token from the prompts' arrival until each decoding
    sequence has had a token after the last prompt's first."""
    import torch

    from tokquay_amd.engine import Engine
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.scheduler import SchedulerConfig
    from tokquay_amd.sequence import SamplingParams

    model = load_model()
    cfg = SchedulerConfig(max_num_seqs=256, max_num_batched_tokens=2048, chunked_prefill=chunked,
                          prefill_chunk_tokens=256)  # fmt: skip
    engine = Engine(model, BlockAllocator(model.cfg, 8192, BLOCK, device="cuda"), cfg)
    rng = random.Random(seed)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(512, 1024))] for _ in range(4)]
    for _ in range(128):
        engine.add_request([rng.randrange(50256) for _ in range(rng.randint(64, 768) - 1)],
                           SamplingParams(max_tokens=128, ignore_eos=True))  # fmt: skip
    while engine.scheduler.waiting or any(s.num_uncached_tokens > 1 for s in engine.scheduler.running):
        engine.step()
    for _ in range(8):  # decode steps: graphs captured, pipeline in steady state
        engine.step()
    decoders = {s.seq_id for s in engine.scheduler.running}
    long_ids = {engine.add_request(p, SamplingParams(max_tokens=1, ignore_eos=True)).seq_id for p in prompts}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last: dict[int, float] = {i: t0 for i in decoders}  # the stall counts from the prompts' arrival
    worst_gap, steps, pending, prompts_done_s = 0.0, 0, set(long_ids), None
    after: set[int] = set()  # decoders that emitted after the last prompt's first token
    while (pending or after != decoders) and steps < 1000:
        events = engine.step()
        now = time.perf_counter()
        steps += 1
        for ev in events:
            pending.discard(ev.seq_id)
            if ev.seq_id in last:
                worst_gap = max(worst_gap, now - last[ev.seq_id])
                last[ev.seq_id] = now
                if prompts_done_s is not None:
                    after.add(ev.seq_id)
        if not pending and prompts_done_s is None:
            prompts_done_s, done_steps = now - t0, steps
    engine.drain()
    engine.allocator.check_device_errors()
    return {"policy": "chunked prefill (256-token chunks)" if chunked else "alternating (reference)",
            "steps_until_prompts_done": done_steps, "ms_until_prompts_done": round(prompts_done_s * 1e3, 2),
            "max_decode_gap_ms": round(worst_gap * 1e3, 2)}  # fmt: skip


def itl_trace(seed: int = 0, rate: float = 8.0, n: int = 300, chunked: bool = False) -> dict:
    import torch

    from tokquay_amd.engine import Engine
    from tokquay_amd.harness import run_trace, summarize
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.scheduler import SchedulerConfig
    from tokquay_amd.workload import make_workload

    model = load_model(seed)
    cfg = SchedulerConfig(max_num_seqs=64, max_num_batched_tokens=2048, chunked_prefill=chunked)
    # Warm-up trace (untimed) so kernels, graphs and library heuristics are ready.
    warm = Engine(model, BlockAllocator(model.cfg, 1024, 16, device="cuda"), cfg)
    run_trace(warm, make_workload(math.inf, 12, seed=999, prompt_len=(16, 128), output_len=(8, 16)))
    del warm
    torch.cuda.synchronize()
    alloc = BlockAllocator(model.cfg, 1024, 16, device="cuda")
    engine = Engine(model, alloc, cfg)
    res = run_trace(engine, make_workload(rate, n, seed=seed))
    s = summarize(res, alloc.bytes_per_block // 16)
    st = s["stalls"]
    out = {
        "requests": s["requests"],
        "rate_req_s": rate if math.isfinite(rate) else "all at t=0",
        "policy": "chunked prefill" if chunked else "alternating (reference)",
        "throughput_tok_s": round(s["throughput_tok_s"], 1),
        "itl_p50_ms": round(s["itl_ms"]["p50"], 3),
        "itl_p99_ms": round(s["itl_ms"]["p99"], 3),
        "ttft_p50_ms": round(s["ttft_ms"]["p50"], 2),
        "ttft_p99_ms": round(s["ttft_ms"]["p99"], 2),
        "decode_step_p50_ms": round(st.get("decode_step_ms", {}).get("p50", float("nan")), 3),
        "preemptions": s["stats"]["num_preemptions"],
    }
    if "frac_gaps_stalled_by_prefill" in st:
        out["gaps_with_a_prefill_step"] = round(st["frac_gaps_stalled_by_prefill"], 4)
        out["itl_clean_p50_p99_ms"] = [round(st["itl_ms_clean"]["p50"], 3), round(st["itl_ms_clean"]["p99"], 3)]
        out["itl_stalled_p50_p99_ms"] = [round(st["itl_ms_stalled"]["p50"], 3), round(st["itl_ms_stalled"]["p99"], 3)]
    return out


def small_batch(nseqs: int, steps: int, prompt: int = 300) -> dict:
    """Decode-step wall time at a small batch: ``nseqs`` sequences with ``prompt``-token prompts of
    random ids decode ``steps`` greedy tokens each (graph replay + pipelining, the engine's
    default). Steps are timed with perf_counter around ``Engine.step()``; the first and last five
    are dropped."""
    import torch

    from tokquay_amd.engine import Engine
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.scheduler import SchedulerConfig
    from tokquay_amd.sequence import SamplingParams

    model = load_model()
    engine = Engine(model, BlockAllocator(model.cfg, 4096, BLOCK, device="cuda"),
                    SchedulerConfig(max_model_len=1024, max_num_seqs=max(nseqs, 1)))  # fmt: skip
    rng = random.Random(0)
    for _ in range(nseqs):
        engine.add_request([rng.randrange(50256) for _ in range(prompt)], SamplingParams(max_tokens=steps, ignore_eos=True))
    times = []
    with torch.no_grad():
        while engine.has_unfinished():
            t0 = time.perf_counter()
            engine.step()
            times.append(time.perf_counter() - t0)
    kept = times[5:-5]
    return {"mode": "small-batch decode steps", "sequences": nseqs, "prompt_tokens": prompt, "steps": len(times),
            "step_p50_ms": round(statistics.median(kept) * 1e3, 3),
            "step_p99_ms": round(float(sorted(kept)[int(0.99 * (len(kept) - 1))]) * 1e3, 3)}  # fmt: skip


# ------------------------------------------------------------------------------ baseline leg
# The reference's own algorithm (the oracle's restatement of tokquay's gather-and-attend paged
# path, tokquay/kv_cache.py:228-242 and tokquay/model.py:94-96), timed beside the HIP path. It is
# the baseline being compared against, never part of what `value` measures.
def snapshot_for_cpu(engine, seqs, n_cpu: int, spare_per_seq: int):
    """Copy the first n_cpu running sequences' blocks into a compact CPU pool (oracle layout),
    with ``spare_per_seq`` empty blocks each for the positions the CPU steps append."""
    import torch

    pool = engine.allocator.pool
    picked = seqs[:n_cpu]
    used = sorted({b for s in picked for b in s.block_table})
    remap = {b: i for i, b in enumerate(used)}
    cpu_pool = torch.empty((len(used) + spare_per_seq * len(picked),) + tuple(pool.shape[1:]), dtype=pool.dtype)
    for i in range(0, len(used), 512):
        idx = torch.tensor(used[i : i + 512], device=pool.device)
        cpu_pool[i : i + len(idx)].copy_(pool.index_select(0, idx))
    spare = iter(range(len(used), cpu_pool.shape[0]))
    state = []
    for s in picked:
        table = [remap[b] for b in s.block_table] + [next(spare) for _ in range(spare_per_seq)]
        state.append((table, s.num_cached_tokens, list(s.token_ids)))
    return cpu_pool, state


def baseline_cpu(cpu_pool, state, weights, steps: int) -> dict:
    """Time the oracle gather path on this host's CPU cores: ``steps`` decode steps after one
    warm-up, each sequence feeding the token it picked in the previous step."""
    import torch

    from oracle.gpt2_ref import RefConfig, build_ref_model
    from oracle.paged_ref import RefPagedBatch

    threads = torch.get_num_threads()
    model = build_ref_model(RefConfig(), weights)
    tables = [list(t) for t, _, _ in state]
    cached = [c for _, c, _ in state]
    tokens = [list(t) for _, _, t in state]
    times, first_ids, first_margins = [], None, None
    for step in range(steps + 1):  # the first step is the warm-up
        batch = RefPagedBatch(cpu_pool, BLOCK, tables, cached, [1] * len(cached))
        ids = torch.tensor([[t[c]] for t, c in zip(tokens, cached)])
        t0 = time.perf_counter()
        with torch.no_grad():
            logits = model(ids, batch, last_only=True)[:, 0]
        nxt = logits.argmax(-1).tolist()
        dt = time.perf_counter() - t0
        if step == 0:
            first_ids = nxt
            top2 = logits.topk(2, dim=-1).values
            first_margins = (top2[:, 0] - top2[:, 1]).tolist()
        else:
            times.append(dt)
        for i, t in enumerate(nxt):
            tokens[i].append(t)
            cached[i] += 1
    return {"step_s": statistics.median(times), "threads": threads, "first_ids": first_ids,
            "first_margins": first_margins}  # fmt: skip


def baseline_gpu_gather(pool, state, tables_after, hip_steps: list[list[int]], weights, steps: int) -> dict:
    """The oracle gather path with torch on the GPU, from the state the HIP engine's first measured
    step started from (``state``: block table, cached positions, tokens per sequence; the pool holds
    every position cached then). Step j feeds the token the HIP engine picked at its step j - 1, so
    the two runs see the same inputs every step; its ids are compared with the HIP engine's step j
    under the margin rule. Blocks for the new positions are the ones the engine used
    (``tables_after``). Timed: ``steps`` steps after one warm-up, median."""
    import torch

    from oracle.gpt2_ref import RefConfig, build_ref_model
    from oracle.paged_ref import RefPagedBatch

    model = build_ref_model(RefConfig(), weights, device="cuda")
    n = len(state)
    cached = [c for _, c, _ in state]
    feed = [t[c] for _, c, t in state]
    got, margins, times = [], [], []
    for step in range(steps + 1):
        tables = [full[: cdiv(c + 1, BLOCK)] for full, c in zip(tables_after, cached)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.no_grad():
            batch = RefPagedBatch(pool, BLOCK, tables, cached, [1] * n)
            ids = torch.tensor([[t] for t in feed], device="cuda")
            logits = model(ids, batch, last_only=True)[:, 0]
            nxt = logits.argmax(-1).tolist()
        times.append(time.perf_counter() - t0)
        top2 = logits.topk(2, dim=-1).values
        margins.append((top2[:, 0] - top2[:, 1]).tolist())
        got.append(nxt)
        feed = hip_steps[step]  # teacher forcing: the HIP engine's pick is the next input
        cached = [c + 1 for c in cached]
    step_s = statistics.median(times[1:])
    agree = margin_agreement(hip_steps[: steps + 1], got, margins)
    return {"value": round(n / step_s, 1), "unit": "tok/s", "step_ms": round(step_s * 1e3, 3),
            "kind": "port", "sample": f"{steps} decode steps (median, after 1 warm-up) of all {n} sequences from the "
            "HIP run's state, oracle gather-and-attend path (write + gather + masked softmax) in fp32 torch on "
            "this GPU, fed the HIP engine's tokens", "greedy_ids": agree}  # fmt: skip


def baseline_configs() -> list[dict]:
    """The small configurations side by side: HIP path vs the gather path on this GPU and on this
    host's CPU cores (``--configs``)."""
    import torch

    from oracle.gpt2_ref import RefAllocator, RefConfig, build_ref_model, ref_paged_greedy_generate
    from oracle.paged_ref import RefPagedBatch, ref_attention
    from tokquay_amd import ops
    from tokquay_amd.generate import paged_forward, paged_greedy_generate
    from tokquay_amd.kv_cache import BlockAllocator
    from tokquay_amd.sequence import Sequence
    from tokquay_amd.weights import random_state_dict

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

    rows = [{"cpu": host_cpu_name(), "cpu_threads": torch.get_num_threads()}]
    sd = random_state_dict(load_model().cfg, seed=0)
    m = load_model()

    # Config 1: 8 prompts U[16,64], 32 greedy tokens each, pool 256 blocks.
    rng = random.Random(1)
    prompts = [[rng.randrange(50256) for _ in range(rng.randint(16, 64))] for _ in range(8)]
    paged_greedy_generate(m, BlockAllocator(m.cfg, 256, BLOCK, device="cuda"), prompts, 4)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    got = paged_greedy_generate(m, BlockAllocator(m.cfg, 256, BLOCK, device="cuda"), prompts, 32)
    torch.cuda.synchronize()
    hip_s = time.perf_counter() - t0
    ref_t = {}
    for dev in ("cuda", "cpu"):
        ref = build_ref_model(RefConfig(), sd, device=dev)
        ref_paged_greedy_generate(ref, RefAllocator(RefConfig(), 256, BLOCK, device=dev), prompts, 2)
        ref_t[dev] = timed(lambda: ref_paged_greedy_generate(ref, RefAllocator(RefConfig(), 256, BLOCK, device=dev),
                                                             prompts, 32), 1, sync=dev == "cuda")  # fmt: skip
    want = ref_paged_greedy_generate(build_ref_model(RefConfig(), sd), RefAllocator(RefConfig(), 256, BLOCK), prompts, 32)
    rows.append({"config": 1, "hip_s": round(hip_s, 4), "gather_gpu_s": round(ref_t["cuda"], 4),
                 "gather_cpu_s": round(ref_t["cpu"], 3), "ids_identical_to_cpu_oracle": got == want})  # fmt: skip

    # Config 2: the decode op alone (HIP figures from decode_op_alone, same draw).
    op = decode_op_alone()
    rng = random.Random(op["draw_seed"])
    ctx = [rng.randint(16, 512) for _ in range(64)]
    g = torch.Generator().manual_seed(2)
    pool = torch.randn(1024, 1, 2, N_HEAD, BLOCK, D_HEAD, generator=g)
    perm = torch.randperm(1024, generator=g).tolist()
    tables, i = [], 0
    for c in ctx:
        tables.append(perm[i : i + cdiv(c, BLOCK)])
        i += cdiv(c, BLOCK)
    q = torch.randn(64, N_HEAD, 1, D_HEAD, generator=g)
    t = {}
    for dev in ("cuda", "cpu"):
        p, qq = pool.to(dev), q.to(dev)
        batch = RefPagedBatch(p, BLOCK, tables, [c - 1 for c in ctx], [1] * 64)

        def step():
            k, v = batch.gather(0)
            return ref_attention(qq, k, v, batch.mask)

        step()
        t[dev] = timed(step, 20, sync=dev == "cuda")
    rows.append({"config": 2, "hip_us": op["us_per_call"], "hip_GBs": op["achieved_GBs"],
                 "gather_gpu_us": round(t["cuda"] * 1e6, 1), "gather_cpu_us": round(t["cpu"] * 1e6, 1)})  # fmt: skip

    # Config 5: one mixed step (chunk 1 of 4 prompts U[512,1024] next to 128 decode rows).
    rng = random.Random(5)
    plen = [rng.randint(512, 1024) for _ in range(4)]
    dctx = [rng.randint(64, 768) for _ in range(128)]
    alloc = BlockAllocator(m.cfg, 8192, BLOCK, device="cuda")
    pr = [Sequence(i, [rng.randrange(50256) for _ in range(n)]) for i, n in enumerate(plen)]
    de = [Sequence(4 + i, [rng.randrange(50256) for _ in range(c - 1)]) for i, c in enumerate(dctx)]
    for s in pr + de:
        alloc.allocate(s)
    for i in range(0, 128, 32):
        nxt = paged_forward(m, alloc, de[i : i + 32]).argmax(-1).tolist()
        for s, tok in zip(de[i : i + 32], nxt):
            s.append_token(tok)
            alloc.append_slot(s)
    paged_forward(m, alloc, pr, [256] * 4)  # chunk 0
    tables = [list(s.block_table) for s in pr + de]
    starts = [s.num_cached_tokens for s in pr + de]
    lens = [256] * 4 + [1] * 128
    ids = [s.token_ids[st : st + n] for s, st, n in zip(pr + de, starts, lens)]
    pool_copy = alloc.pool.clone()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    paged_forward(m, alloc, pr + de, lens)
    torch.cuda.synchronize()
    hip_ms = (time.perf_counter() - t0) * 1e3
    t = {}
    for dev in ("cuda", "cpu"):
        ref = build_ref_model(RefConfig(), sd, device=dev)
        p = pool_copy if dev == "cuda" else pool_copy.cpu()

        def step():
            batch = RefPagedBatch(p, BLOCK, tables, starts, lens)
            x = torch.tensor([r + [0] * (256 - len(r)) for r in ids], device=dev)
            with torch.no_grad():
                return ref(x, batch, last_only=True)

        step()
        t[dev] = timed(step, 3 if dev == "cuda" else 1, sync=dev == "cuda")
    rows.append({"config": 5, "chunk": 1, "hip_step_ms": round(hip_ms, 2), "gather_gpu_step_ms": round(t["cuda"] * 1e3, 2),
                 "gather_cpu_step_s": round(t["cpu"], 2)})  # fmt: skip
    return rows


# ------------------------------------------------------------------------------ main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--partition-tokens", type=int, default=0, help="decode partition size (0: automatic)")
    ap.add_argument("--cpu-seqs", type=int, default=256, help="sequences in the CPU baseline sample (0: skip)")
    ap.add_argument("--cpu-steps", type=int, default=4, help="timed CPU baseline steps (after one warm-up)")
    ap.add_argument("--gather-steps", type=int, default=3, help="timed GPU gather-path steps (0: skip)")
    ap.add_argument("--no-itl", action="store_true", help="skip the 300-request serving traces")
    ap.add_argument("--no-prefill", action="store_true", help="skip the mixed chunked-prefill measurements")
    ap.add_argument("--small-batch", type=int, default=0, metavar="N",
                    help="only measure decode-step wall time at N sequences (300-token prompts) and exit")
    ap.add_argument("--small-batch-steps", type=int, default=80, help="tokens per sequence for --small-batch")
    ap.add_argument("--prefill-op", action="store_true",
                    help="only time the prefill kernel alone (chunks, a 32-prompt batch, long prompts) and exit")
    ap.add_argument("--configs", action="store_true",
                    help="only run the small configurations beside the gather path (GPU and CPU) and exit")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="run 3 copies of a known size (1 GiB read + 1 GiB write), 3 decode steps and the mixed "
                    "chunked-prefill steps, then exit; for rocprofv3 --pmc runs")  # fmt: skip
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.", file=sys.stderr)
        return 2

    import torch

    from tokquay_amd import kv_cache
    from tokquay_amd.weights import random_state_dict

    torch.manual_seed(0)
    if args.small_batch:
        print(json.dumps(small_batch(args.small_batch, args.small_batch_steps)), flush=True)
        return 0
    if args.prefill_op:
        print(json.dumps(prefill_op_alone()), flush=True)
        return 0
    if args.configs:
        for row in baseline_configs():
            print(json.dumps(row), flush=True)
        return 0

    # Step accounting, from the prefilled state (prompt P cached, one token pending). The W warm-up
    # calls complete W steps and the drain one more: P + W + 1 cached (state S). From S the timed
    # run completes one step untimed, whose call launches the next ahead; the K timed calls then
    # hold the GPU work of the steps at contexts P + W + 4 ... P + W + K + 3. The prompt is sized so
    # that this window is centred on the sequence's draw c: P = c - W - 4 - K // 2.
    K, W = args.steps, args.warmup
    drawn_ctx, draw_lo, draw_hi = window_draws(K)
    # max_tokens: the run's last step emits each sequence's last token (prompt + max_tokens - 1
    # = c + K - 1 - K // 2 <= 1024, the engine's limit).
    engine, model = build_engine([c - W - 4 - K // 2 for c in drawn_ctx], max_tokens=W + K + 4)
    engine.allocator.decode_partition_tokens = args.partition_tokens

    for _ in range(W):
        engine.step()
    engine.drain()  # nothing in flight: every sequence's tokens are on the host
    if args.pmc_probe:
        x = torch.randn(1 << 28, device="cuda")  # 1 GiB
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)  # calibration: reads exactly 1 GiB, writes exactly 1 GiB
        first_ctx = [s.num_cached_tokens + 1 for s in engine.scheduler.running]  # contexts of the next decode step
        for _ in range(3):
            engine.step()
        torch.cuda.synchronize()
        del engine, x, y
        torch.cuda.empty_cache()
        # The 4-prompt chunked-prefill steps beside 128 decoding sequences, as two launches and as one.
        _, mixed = mixed_chunked_step()
        print(json.dumps({"pmc_probe": True, "copy_bytes": 1 << 30,
                          "decode_bytes_first_step": decode_bytes(first_ctx),
                          "mixed_chunks": [{k: c[k] for k in ("chunk", "prefill_mflop", "decode_mb")} for c in mixed["chunks"]]}),
              flush=True)  # fmt: skip
        return 0
    running = list(engine.scheduler.running)
    assert len(running) == N_SEQS, f"{len(running)} sequences running, expected {N_SEQS}"
    # State S, the one the next step starts from: the baselines start from it too.
    state = [(list(s.block_table), s.num_cached_tokens, list(s.token_ids)) for s in running]
    order = {s.seq_id: i for i, s in enumerate(running)}
    start = engine_state(engine)

    cpu_state = None
    if args.cpu_seqs > 0:
        t0 = time.perf_counter()
        cpu_state = snapshot_for_cpu(engine, running, args.cpu_seqs, spare_per_seq=args.cpu_steps // 16 + 2)
        log(f"copied {cpu_state[0].shape[0]} blocks for the CPU sample in {time.perf_counter() - t0:.1f} s")

    def by_row(events) -> list[int]:
        ids = [0] * N_SEQS
        for ev in events:
            ids[order[ev.seq_id]] = ev.token_id
        return ids

    # Kernel timing: the K decode steps of the timed window run eagerly from S (two untimed steps
    # first, to reach the window), every decode launch timed by HIP events the launch itself
    # records at the start and end of its kernels. Then the engine is rewound to S.
    graphs, engine.graphs = engine.graphs, None
    for _ in range(2):
        engine.step()
    eager_ctx = [s.num_cached_tokens + 1 for s in running]
    timer = LaunchTimer("decode")
    kv_cache.PagedBatch.launch_hook = timer
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(K):
        engine.step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t1) * 1e3 / K
    kv_cache.PagedBatch.launch_hook = None
    engine.graphs = graphs
    engine.allocator.check_device_errors()
    rewind(engine, start)

    # The step after S. The engine launches the following step ahead, so the timed region starts
    # in steady state.
    hip_steps = [by_row(engine.step())]

    # Timed region: K decode steps through Engine.step, replayed from the captured HIP graph.
    # The step in flight at the start is finished before the clock starts; the step launched
    # ahead by the last call is finished inside it: K steps of GPU work, K steps of tokens.
    # Context of each row in the first step of GPU work inside the timed region (the step launched
    # ahead is already counted in num_cached_tokens).
    timed_ctx = [s.num_cached_tokens + 1 for s in running]
    assert timed_ctx == eager_ctx, "the kernel-timing steps ran another window"
    offsets = {c + K // 2 - d for d, c in zip((drawn_ctx[s.seq_id] for s in running), timed_ctx)}
    assert offsets == {0}, f"timed window not centred on the draws: offsets {sorted(offsets)}"
    assert max(timed_ctx) + K - 1 <= CTX_HI and min(timed_ctx) >= CTX_LO
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    emitted = []
    for k in range(args.steps):
        emitted.append(engine.step())
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    n_tokens = sum(len(e) for e in emitted)
    assert n_tokens == N_SEQS * args.steps, n_tokens
    hip_steps += [by_row(e) for e in emitted]
    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = n_tokens / elapsed
    mean_ctx_timed = statistics.mean(timed_ctx) + (args.steps - 1) / 2
    # The blocks every position of the window went to (read before the drain: the drained step
    # emits each sequence's last token, and finishing frees its table).
    tables_after = [list(s.block_table) for s in running]
    engine.drain()
    engine.allocator.check_device_errors()
    n_launch = timer.launches("decode")
    kern_ms = timer.total_ms("decode") / n_launch
    bytes_per_launch = timer.bytes["decode"] / n_launch
    achieved = bytes_per_launch / (kern_ms * 1e-3) / 1e9
    log(f"decode (graph replay): {ms_per_step:.3f} ms/step, {tok_s:.0f} tok/s; kernel-timing eager steps "
        f"{eager_ms:.3f} ms/step (every decode launch timed on its own); "
        f"attention {kern_ms * 1e3:.1f} us/launch, {bytes_per_launch / 1e9:.3f} GB/launch, {achieved:.0f} GB/s")  # fmt: skip

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: random-init weights (seed 0), random token ids",
        "config": {
            "workload": "scaled decode: GPT-2 124M fp32, 256 concurrent sequences, block_size 16, pool 16384 blocks "
            f"(262144 slots); each sequence draws c ~ U[{draw_lo},{draw_hi}] (stratified over the 256) and its {K} "
            "timed steps run at "
            f"contexts c - {K // 2} ... c + {K - 1 - K // 2} (inside [256,1024]): mean context "
            f"{mean_ctx_timed:.1f} over the timed steps (the draws' mean: {statistics.mean(drawn_ctx):.1f}); "
            "the kernel-timing eager steps run the same contexts from the same state",
            "num_seqs": N_SEQS,
            "block_size": BLOCK,
            "pool_blocks": POOL_BLOCKS,
            "timed_mean_context": round(mean_ctx_timed, 1),
            "decode_partition_tokens": args.partition_tokens,
            "decode_steps": "HIP-graph replay (one graph per batch bucket); roofline from the same shape run eagerly",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "tq_paged_decode_write (decode_split_kernel: W waves per (sequence, head) splitting its "
            "context, merged in LDS; W = 8 at contexts of 897-1024)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": int(bytes_per_launch * DECODE_TRAFFIC_PER_ALGO_BYTE),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on bench.py --pmc-probe, "
            "scaled by a 1 GiB copy calibration: 1.0059 x algorithmic bytes",
            "kernel_us": round(kern_ms * 1e3, 2),
            "bytes_per_launch": int(bytes_per_launch),
            "launches": n_launch,
        },
    }

    weights = random_state_dict(model.cfg, seed=0)
    if args.gather_steps > 0:
        log(f"GPU gather baseline: {N_SEQS} sequences, {args.gather_steps} timed steps ...")
        gb = baseline_gpu_gather(engine.allocator.pool, state, tables_after, hip_steps, weights, args.gather_steps)
        gb["speedup_of_hip_engine"] = round(tok_s / gb["value"], 2)
        result["gpu_gather_baseline"] = gb
    if cpu_state is not None:
        cpu_pool, cstate = cpu_state
        log(f"CPU baseline: {len(cstate)} sequences, {args.cpu_steps} timed steps ...")
        cb = baseline_cpu(cpu_pool, cstate, weights, args.cpu_steps)
        n = len(cstate)
        agree = margin_agreement([hip_steps[0][:n]], [cb["first_ids"]], [cb["first_margins"]])
        result["cpu_baseline"] = {
            "value": round(n / cb["step_s"], 2),
            "unit": "tok/s",
            "cores": cb["threads"],
            "kind": "port",
            "sample": f"{args.cpu_steps} decode steps (median, after 1 warm-up) of {n} of the 256 sequences from the "
            f"same state, oracle gather-and-attend path in fp32 torch on {cb['threads']} threads",
            "cpu_model": host_cpu_name(),
            "step_s": round(cb["step_s"], 3),
            "greedy_ids_first_step": agree,
        }
        del cpu_pool
    del engine, graphs
    torch.cuda.empty_cache()
    log("decode op alone (64 sequences, ctx U[16,512]) ...")
    result["decode_op_alone"] = decode_op_alone()
    result["hbm_copy"] = hbm_copy()
    if not args.no_prefill:
        log("mixed chunked-prefill + decode steps ...")
        result["prefill"], result["mixed_attention"] = mixed_chunked_step()
        log(f"prefill: {result['prefill']['achieved']} TFLOP/s = {result['prefill']['frac']:.3f} of fp32 MFMA peak; "
            f"mixed launch: {result['mixed_attention']['frac']:.3f} of its combined roofline "
            f"({result['mixed_attention']['two_launch_frac']:.3f} as two launches)")
        log("prefill batch (32 prompts U[256,1024]) ...")
        result["prefill_batch"] = prefill_batch()
        log(f"prefill batch: {result['prefill_batch']['us_per_launch']} us per launch = "
            f"{result['prefill_batch']['frac']:.3f} of fp32 MFMA peak")
        log("prefill kernel alone (chunks, a 32-prompt batch, long prompts) ...")
        result["prefill_op_alone"] = prefill_op_alone()
        result["mixed_engine"] = [mixed_engine(chunked=True), mixed_engine(chunked=False)]
        torch.cuda.empty_cache()
    if not args.no_itl:
        log("serving trace: 300 requests, Poisson 8 req/s, alternating policy ...")
        result["itl"] = itl_trace()
        log("serving trace: 300 requests, Poisson 8 req/s, chunked prefill ...")
        result["itl_chunked"] = itl_trace(chunked=True)
        log("saturated trace: the same 300 requests, all arriving at t=0 ...")
        sat = itl_trace(rate=math.inf)
        # The reference's saturated-throughput run (Documentation/results.md:97-101): same workload
        # shape (300 requests, prompt and output lengths U[16,256], fixed-length outputs, 1,024 x 16
        # KV slots, 64 sequences at most), pretrained weights, RTX 3050 Laptop, PyTorch 2.6 + CUDA.
        sat["reference_published_tok_s"] = 916.1
        result["saturated"] = sat
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
