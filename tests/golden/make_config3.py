"""Writes tests/golden/config3_greedy.npz: the oracle's greedy ids for the 300-request serving workload.

Run on a CPU (takes ~7 minutes on 8 cores):

    python tests/golden/make_config3.py

Workload: ``make_workload(8.0, 300, seed=0)`` - 300 requests, prompt and output
lengths U[16, 256] of random token ids (the reference's benchmark workload,
bench/workload.py:24-47, bench/bench.py:204). Model: GPT-2 124M with the
seed-0 random-init fp32 weights (``tokquay_amd.weights.random_state_dict``).
Every request is decoded alone by the oracle (``oracle.gpt2_ref.ref_greedy_generate``:
the reference's batch-of-one contiguous-cache greedy loop, tokquay/generate.py:17-49,
in fp32 on the CPU) for exactly its output length, as the reference benchmark
does with ``ignore_eos`` (bench/harness.py:70).

Stored (no pickles):

* ``ids`` uint16: every request's output ids, concatenated in workload order;
* ``offsets`` int64 [301]: request r's ids are ``ids[offsets[r]:offsets[r+1]]``;
* ``near_tie_index`` int64 / ``near_tie_margin`` float32: every token whose
  top-1 minus top-2 logit gap is below ``NEAR_TIE_STORED`` (position in ``ids``, gap);
  all other tokens were picked by at least that gap;
* ``min_margin`` float32: the smallest gap of all 40 k picks;
* ``workload_sha256``: a hash of the workload's (arrival, prompt, output length)
  triples, so a test notices a changed generator.
"""

from __future__ import annotations

import multiprocessing as mp
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

NEAR_TIE_STORED = 1e-3
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config3_greedy.npz")
WORKERS, THREADS = 4, 2


_model = None


def _init_worker() -> None:
    global _model
    import torch

    from oracle.gpt2_ref import RefConfig, build_ref_model
    from tokquay_amd.weights import random_state_dict

    torch.set_num_threads(THREADS)
    cfg = RefConfig()
    _model = build_ref_model(cfg, random_state_dict(cfg, seed=0))


def _decode(job):
    from oracle.gpt2_ref import ref_greedy_generate

    r, prompt, n = job
    margins: list[float] = []
    ids = ref_greedy_generate(_model, list(prompt), n, margins=margins)
    return r, ids, margins


def main() -> None:
    from tests.golden_ids import workload_sha256
    from tokquay_amd.workload import make_workload

    workload = make_workload(8.0, 300, seed=0)
    jobs = [(r, spec.prompt_ids, spec.output_len) for r, spec in enumerate(workload)]
    jobs.sort(key=lambda j: -(len(j[1]) + j[2]))  # longest first: even load across workers
    results: dict[int, tuple[list[int], list[float]]] = {}
    t0 = time.perf_counter()
    with mp.get_context("spawn").Pool(WORKERS, initializer=_init_worker) as pool:
        for r, ids, margins in pool.imap_unordered(_decode, jobs):
            results[r] = (ids, margins)
            if len(results) % 25 == 0:
                print(f"{len(results)} / {len(jobs)} requests, {time.perf_counter() - t0:.0f} s", flush=True)
    ids = np.concatenate([np.asarray(results[r][0], dtype=np.uint16) for r in range(len(workload))])
    margins = np.concatenate([np.asarray(results[r][1], dtype=np.float64) for r in range(len(workload))])
    offsets = np.cumsum([0] + [len(results[r][0]) for r in range(len(workload))]).astype(np.int64)
    assert offsets[-1] == ids.size == sum(s.output_len for s in workload)
    near = np.flatnonzero(margins < NEAR_TIE_STORED)
    np.savez_compressed(
        OUT,
        ids=ids,
        offsets=offsets,
        near_tie_index=near.astype(np.int64),
        near_tie_margin=margins[near].astype(np.float32),
        near_tie_stored_below=np.float32(NEAR_TIE_STORED),
        min_margin=np.float32(margins.min()),
        workload_sha256=np.array(workload_sha256(workload)),
    )
    print(f"wrote {OUT}: {ids.size} ids, {near.size} below {NEAR_TIE_STORED}, min margin {margins.min():.3e}, "
          f"{time.perf_counter() - t0:.0f} s")  # fmt: skip


if __name__ == "__main__":
    main()
