"""Decode-step wall time at small and large batches (not collected by pytest).

Run on a GPU box:

    python tests/measure_decode_steps.py              # p50 step time per batch size and mode
    python tests/measure_decode_steps.py --profile 8  # 200 steps of 8 sequences (for a kernel trace)

Workload: GPT-2 124M (random init, seed 0), block size 16; every sequence has a
prompt of U[200,400] random ids (``--profile``: 300) and decodes 80 greedy
tokens (``--profile``: 200) with ``ignore_eos``. Modes: HIP-graph decode steps
with pipelining ("graphs+pipeline", the engine's default), graphs without
pipelining, and eager steps. Steps are timed with ``perf_counter`` around
``Engine.step()`` (which ends in the step's host synchronisation); the first and
last five steps (prefill, ramp) are dropped.
"""

from __future__ import annotations

import argparse
import json
import os
import random
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from tokquay_amd.engine import Engine  # noqa: E402
from tokquay_amd.kv_cache import BlockAllocator  # noqa: E402
from tokquay_amd.model import GPT2, GPT2Config  # noqa: E402
from tokquay_amd.scheduler import SchedulerConfig  # noqa: E402
from tokquay_amd.sequence import SamplingParams  # noqa: E402
from tokquay_amd.weights import random_state_dict  # noqa: E402

MODES = {"graphs+pipeline": (True, True), "graphs": (True, False), "eager": (False, False)}


def model():
    cfg = GPT2Config()
    m = GPT2(cfg)
    m.load_state_dict(random_state_dict(cfg, seed=0))
    return m.cuda().eval()


def engine(m, nseq, mode, prompt=None, max_tokens=80, seed=0):
    use_graphs, pipeline = MODES[mode]
    config = SchedulerConfig(max_model_len=m.cfg.n_positions, max_num_seqs=max(nseq, 1))
    eng = Engine(m, BlockAllocator(m.cfg, 4096, 16, device="cuda"), config, use_graphs=use_graphs, pipeline=pipeline)
    rng = random.Random(seed)
    for _ in range(nseq):
        n = prompt or rng.randint(200, 400)
        eng.add_request([rng.randrange(50256) for _ in range(n)], SamplingParams(max_tokens=max_tokens, ignore_eos=True))
    return eng


def step_times(eng) -> list[float]:
    times = []
    with torch.no_grad():
        while eng.has_unfinished():
            t0 = time.perf_counter()
            eng.step()
            times.append(time.perf_counter() - t0)
    return times[5:-5]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--profile", type=int, default=0, help="only run 200 steps of this many sequences")
    args = ap.parse_args()
    m = model()
    if args.profile:
        eng = engine(m, args.profile, "graphs+pipeline", prompt=300, max_tokens=200)
        t = step_times(eng)
        print(json.dumps({"sequences": args.profile, "steps": len(t) + 10, "step_p50_ms": round(statistics.median(t) * 1e3, 3)}))
        return
    for nseq in (1, 8, 16, 24, 32, 64, 256):
        row = {"sequences": nseq}
        for mode in MODES:
            row[f"{mode}_p50_ms"] = round(statistics.median(step_times(engine(m, nseq, mode))) * 1e3, 3)
        print(json.dumps(row), flush=True)


if __name__ == "__main__":
    main()
