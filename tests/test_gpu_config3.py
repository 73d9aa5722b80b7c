"""The HIP engine's greedy ids on the 300-request serving workload equal the oracle's.

Workload: ``make_workload(8.0, 300, seed=0)``, the reference benchmark's (bench/workload.py:24-47,
bench/bench.py:204): prompt and output lengths U[16, 256] of random token ids, fixed-length outputs
(bench/harness.py:70). Engine parameters are the reference benchmark's (bench/bench.py:91-101):
1,024 blocks x 16 slots, at most 64 sequences, 2,048 batched tokens, watermark 1 - a pool small
enough that the all-at-once run preempts and recomputes. Expected ids: the committed fixture
``tests/golden/config3_greedy.npz`` (each request decoded alone by the oracle in fp32 on the CPU),
compared with the margin rule of ``tests/golden_ids.py``.
"""

from __future__ import annotations

import math

import pytest
import torch

from tests.golden_ids import MARGIN_BOUND, GoldenIds, workload_sha256
from tokquay_amd.engine import Engine
from tokquay_amd.harness import run_trace
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.scheduler import SchedulerConfig
from tokquay_amd.weights import random_state_dict
from tokquay_amd.workload import make_workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def golden():
    return GoldenIds()


@pytest.fixture(scope="module")
def model():
    m = GPT2(GPT2Config())
    m.load_state_dict(random_state_dict(m.cfg, seed=0))
    return m.cuda().eval()


class VirtualClock:
    def __init__(self):
        self.t = 0.0

    def now(self) -> float:
        return self.t

    def sleep(self, dt: float) -> None:
        self.t += dt


class FixedStepTime:
    """The engine, with every step taking ``dt`` seconds of the virtual clock, so arrivals interleave
    with steps the same way on every run."""

    def __init__(self, engine: Engine, clock: VirtualClock, dt: float):
        self.engine, self.clock, self.dt = engine, clock, dt

    def step(self):
        events = self.engine.step()
        self.clock.t += self.dt
        return events

    def __getattr__(self, name):
        return getattr(self.engine, name)


def run_config3(model, rate: float, chunked: bool = False, step_s: float = 0.01):
    cfg = SchedulerConfig(max_num_seqs=64, max_num_batched_tokens=2048, watermark_blocks=1,
                          chunked_prefill=chunked)  # fmt: skip
    alloc = BlockAllocator(model.cfg, 1024, 16, device="cuda")
    engine = Engine(model, alloc, cfg)
    clock = VirtualClock()
    log = run_trace(FixedStepTime(engine, clock, step_s), make_workload(rate, 300, seed=0), clock=clock.now,
                    sleep=clock.sleep)  # fmt: skip
    torch.cuda.synchronize()
    alloc.check_device_errors()
    assert alloc.num_free_blocks == alloc.num_blocks
    return [log.request_token_ids(r) for r in range(300)], log.stats


@pytest.mark.parametrize(
    "rate, chunked",
    [(8.0, False), (math.inf, False), (math.inf, True)],
    ids=["poisson-8-per-s", "all-at-once", "all-at-once-chunked"],
)
def test_config3_greedy_ids_match_the_oracle(model, golden, rate, chunked):
    assert workload_sha256(make_workload(8.0, 300, seed=0)) == golden.workload_sha256
    outputs, stats = run_config3(model, rate, chunked)
    res = golden.compare(outputs)
    print(f"\n{rate} req/s chunked={chunked}: {res['tokens_compared']} of {res['tokens_total']} tokens compared, "
          f"{len(res['near_tie_divergences'])} near-tie divergences (margin < {MARGIN_BOUND}): "
          f"{res['near_tie_divergences']}, preemptions {stats['num_preemptions']}, "
          f"fixture min margin {golden.min_margin:.2e}")  # fmt: skip
    assert not res["violations"], res["violations"][:10]
    if rate == math.inf and not chunked:
        assert stats["num_preemptions"] > 0  # the pool is small enough to force recompute
