"""Workload generator and serving metrics (bench/workload.py, bench/harness.py in the reference),
checked on a scripted server with a virtual clock where every number can be worked out by hand
(tests/test_phase6_bench.py:35-203 in the reference), plus engine-side sampling helpers."""

from __future__ import annotations

import math
import types

import numpy as np
import pytest
import torch

from tokquay_amd.engine import EngineStats, KVSnapshot, StepInfo, TokenEvent, sample_token
from tokquay_amd.harness import TraceLog, percentiles, prefill_stall_analysis, run_trace, summarize, token_gaps
from tokquay_amd.sequence import SamplingParams
from tokquay_amd.workload import VOCAB_SIZE, RequestSpec, make_workload


def test_workload_is_deterministic_and_in_range():
    a, b = make_workload(2.0, 300, seed=5), make_workload(2.0, 300, seed=5)
    assert a == b and make_workload(2.0, 300, seed=6) != a
    assert all(16 <= len(r.prompt_ids) <= 256 and 16 <= r.output_len <= 256 for r in a)
    assert all(0 <= t < VOCAB_SIZE - 1 for r in a for t in r.prompt_ids)
    assert [r.arrival for r in a] == sorted(r.arrival for r in a)


def test_workload_first_request_is_the_documented_draw():
    """The generator's draw order (length, ids, output length; gaps from seed + 1_000_003)."""
    import random

    content, gaps = random.Random(0), random.Random(1_000_003)
    n = content.randint(16, 256)
    prompt = tuple(content.randrange(VOCAB_SIZE - 1) for _ in range(n))
    out = content.randint(16, 256)
    first = make_workload(8.0, 1, seed=0)[0]
    assert first == RequestSpec(gaps.expovariate(1.0) / 8.0, prompt, out)


def test_rates_compress_the_same_requests_in_time():
    slow, fast = make_workload(1.0, 200, seed=3), make_workload(4.0, 200, seed=3)
    assert [(r.prompt_ids, r.output_len) for r in slow] == [(r.prompt_ids, r.output_len) for r in fast]
    for s, f in zip(slow, fast):
        assert s.arrival == pytest.approx(4 * f.arrival)


def test_arrivals_are_poisson_at_the_requested_rate():
    w = make_workload(2.5, 6000, seed=1)
    gaps = np.diff([0.0] + [r.arrival for r in w])
    assert gaps.mean() == pytest.approx(0.4, rel=0.05) and gaps.std() == pytest.approx(0.4, rel=0.08)
    assert make_workload(math.inf, 5, seed=1)[-1].arrival == 0.0
    for bad in ({"rate": 0, "n": 5}, {"rate": 1, "n": 0}):
        with pytest.raises(ValueError):
            make_workload(**bad)


class FakeClock:
    def __init__(self):
        self.t = 0.0

    def now(self):
        return self.t

    def sleep(self, dt):
        self.t += dt


class FakeSystem:
    """2 slots, FCFS; a step that admits is a 0.5 s prefill, otherwise a 0.1 s decode."""

    def __init__(self, clock):
        self.clock, self.slots = clock, 2
        self.waiting, self.running = [], []
        self.stats, self.last_step, self._n = EngineStats(), None, 0

    def add_request(self, prompt_ids, params):
        seq = types.SimpleNamespace(seq_id=self._n, left=params.max_tokens)
        self._n += 1
        self.waiting.append(seq)
        return seq

    def has_unfinished(self):
        return bool(self.waiting or self.running)

    def step(self):
        admit = []
        while self.waiting and len(self.running) + len(admit) < self.slots:
            admit.append(self.waiting.pop(0))
        self.running += admit
        batch, prefill = (admit, True) if admit else (list(self.running), False)
        self.clock.t += 0.5 if prefill else 0.1
        events = []
        for s in batch:
            s.left -= 1
            events.append(TokenEvent(s.seq_id, 7, "length" if s.left == 0 else None))
        kv = KVSnapshot(len(self.running) * 100, len(self.running) * 10, len(self.running))
        self.last_step = StepInfo(prefill, len(batch), 3 * len(batch) if prefill else len(batch), kv)
        self.running = [s for s in self.running if s.left > 0]
        return events


def scenario():
    clock = FakeClock()
    w = [RequestSpec(0.0, (1,), 3), RequestSpec(0.25, (1,), 2), RequestSpec(5.0, (1,), 1)]
    return run_trace(FakeSystem(clock), w, clock=clock.now, sleep=clock.sleep)


def test_tokens_are_stamped_when_their_step_ends():
    log = scenario()
    assert log.request_token_times(0) == pytest.approx([0.5, 1.1, 1.2])
    assert log.request_token_times(1) == pytest.approx([1.0, 1.1])
    assert log.request_token_times(2) == pytest.approx([5.5])
    assert log.request_token_ids(0) == [7, 7, 7]


def test_summary_metrics_match_a_hand_calculation():
    m = summarize(scenario(), bytes_per_token=2**20)
    assert m["ttft_ms"]["p50"] == pytest.approx(500) and m["ttft_ms"]["p99"] == pytest.approx(745)
    assert m["itl_ms"]["p50"] == pytest.approx(100) and m["itl_ms"]["mean"] == pytest.approx(800 / 3)
    assert m["output_tokens"] == 6 and m["duration_s"] == pytest.approx(5.5)
    assert m["throughput_tok_s"] == pytest.approx(6 / 5.5)
    assert m["latency_ms"]["p50"] == pytest.approx(850)
    assert m["max_concurrent"] == 2 and m["steps"] == 5
    assert m["peak_kv_allocated_mib"] == 200 and m["peak_kv_live_mib"] == 20
    assert m["kv_utilization"] == pytest.approx(70 / 700)


def test_stall_analysis_splits_gaps_by_prefill():
    st = summarize(scenario(), 1)["stalls"]
    assert st["frac_gaps_stalled_by_prefill"] == pytest.approx(1 / 3)
    assert st["itl_ms_stalled"]["p50"] == pytest.approx(600) and st["itl_ms_clean"]["p50"] == pytest.approx(100)
    assert st["num_prefill_steps"] == 3 and st["num_decode_steps"] == 2
    assert "prefill_ms_per_padded_token" not in st


def test_prefill_cost_per_token_is_recovered():
    log, t = TraceLog(arrivals=[0.0], prompt_lens=[1], output_lens=[2]), 0.0
    for tokens in (100, 400, 900, 2000):
        dur = (20 + 0.05 * tokens) / 1e3
        log.steps.append((t, t + dur, True, 1, tokens, 0, 0, 1))
        t += dur
    log.token_request, log.token_step, log.token_ids = [0, 0], [0, 1], [5, 6]
    out = prefill_stall_analysis(log)
    assert out["prefill_ms_per_padded_token"] == pytest.approx(0.05) and out["prefill_ms_fixed"] == pytest.approx(20)


def test_percentiles_and_gaps():
    p = percentiles(list(range(1, 101)))
    assert p == {"p50": pytest.approx(50.5), "p99": pytest.approx(99.01), "mean": pytest.approx(50.5)}
    assert all(math.isnan(v) for v in percentiles([]).values())
    assert list(token_gaps(scenario())[2].round(3)) == [0.6, 0.1, 0.1]


def test_a_stuck_system_raises():
    class Stuck:
        stats, last_step = EngineStats(), None

        def add_request(self, ids, params):
            return types.SimpleNamespace(seq_id=0)

        def has_unfinished(self):
            return True

        def step(self):
            return []

    with pytest.raises(RuntimeError, match="deadlock"):
        run_trace(Stuck(), [RequestSpec(0.0, (1,), 1)])


def test_sample_token_top_k_and_temperature():
    logits = torch.tensor([5.0, 4.0, 3.0, 0.0, -1.0, -2.0, -3.0, -4.0])
    gen = torch.Generator().manual_seed(0)
    assert {sample_token(logits, SamplingParams(temperature=2.0, top_k=3), gen) for _ in range(300)} == {0, 1, 2}
    assert {sample_token(logits, SamplingParams(temperature=0.01), gen) for _ in range(50)} == {0}
    assert sample_token(logits, SamplingParams(), None) == 0
    assert len({sample_token(logits, SamplingParams(temperature=50.0), gen) for _ in range(400)}) >= 6


def test_sampling_params_validation():
    for bad in ({"max_tokens": 0}, {"temperature": -1.0}, {"top_k": -1}):
        with pytest.raises(ValueError):
            SamplingParams(**bad)
