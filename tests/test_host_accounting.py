"""The engine's work and memory accounting, with and without pipelined decode, on the CPU.

Restates tests/test_phase6_accounting.py:32-89 (positions computed = the
necessary positions + the preemption discards; ``StepInfo.kv`` taken after the
forward and before finished sequences free their blocks) over the toy decoder of
``test_host_pipeline``, once with the synchronous engine and once with the
pipelined one, and adds: EOS stops and aborts keep the identity (rows computed
ahead and discarded are counted apart, in ``positions_dropped``), and both
engines report the same ``StepInfo`` after every ``step()`` call.
"""

from __future__ import annotations

import random

import pytest

from tests.test_host_pipeline import VOCAB, make_engine, random_arrivals
from tokquay_amd.engine import KVSnapshot, StepInfo
from tokquay_amd.sequence import SamplingParams

pytestmark = pytest.mark.timeout(120)

TEXT = [random.Random(11).randrange(VOCAB) for _ in range(400)]


def greedy(n):
    return SamplingParams(max_tokens=n, ignore_eos=True)


def needed_positions(specs):
    """Each prompt, plus every generated token but the last (never fed back)."""
    return sum(len(p) + n - 1 for p, n in specs)


@pytest.mark.parametrize("pipeline", [False, True])
def test_positions_computed_is_exactly_the_necessary_work_when_nothing_is_preempted(pipeline):
    specs = [(TEXT[i * 9 : i * 9 + 8 + 3 * i], 6 + 2 * i) for i in range(5)]
    eng = make_engine(pipeline, num_blocks=64, block_size=16)
    for p, n in specs:
        eng.add_request(p, greedy(n))
    eng.run_until_done()
    st = eng.stats
    assert st.num_preemptions == 0 and st.positions_discarded == 0
    assert st.positions_computed == needed_positions(specs)
    assert st.positions_padded >= st.positions_computed
    assert st.positions_dropped == 0  # nothing stops on EOS: every row launched ahead was needed
    assert (st.lookahead_steps > 0) == pipeline


@pytest.mark.parametrize("pipeline", [False, True])
def test_preemption_adds_exactly_the_discarded_positions(pipeline):
    specs = [(TEXT[i * 9 : i * 9 + 18 + 3 * i], 24 + 2 * i) for i in range(5)]
    eng = make_engine(pipeline, num_blocks=8, block_size=16)  # 128 slots for 5 requests wanting ~45 each
    for p, n in specs:
        eng.add_request(p, greedy(n))
    eng.run_until_done()
    st = eng.stats
    assert st.num_preemptions > 0 and st.positions_discarded > 0, "the pool was meant to be too small"
    assert st.positions_computed == needed_positions(specs) + st.positions_discarded
    assert st.positions_discarded == eng.scheduler.num_discarded_positions
    if pipeline:
        assert st.lookahead_steps > 0


@pytest.mark.parametrize("pipeline", [False, True])
def test_last_step_and_kv_snapshot_describe_the_step_that_just_ran(pipeline):
    eng = make_engine(pipeline, num_blocks=64, block_size=16)
    assert eng.last_step is None and eng.kv_snapshot().num_seqs == 0
    eng.add_request(TEXT[:5], greedy(4))
    eng.add_request(TEXT[10:30], greedy(4))

    eng.step()  # prefill of both
    assert (eng.last_step.is_prefill, eng.last_step.num_seqs) == (True, 2)
    assert eng.last_step.padded_tokens == 2 * 20
    snap = eng.last_step.kv
    assert snap == eng.kv_snapshot()
    assert snap.num_seqs == 2 and snap.live_tokens == 5 + 20
    assert snap.allocated_tokens == (1 + 2) * 16
    assert snap.live_tokens <= snap.allocated_tokens

    eng.step()  # decode of both
    assert (eng.last_step.is_prefill, eng.last_step.num_seqs, eng.last_step.padded_tokens) == (False, 2, 2)
    eng.run_until_done()
    assert eng.kv_snapshot() == KVSnapshot(0, 0, 0)
    eng.step()
    assert eng.last_step is None


@pytest.mark.parametrize("pipeline", [False, True])
def test_step_snapshot_is_taken_at_the_peak_before_finished_sequences_free_their_blocks(pipeline):
    eng = make_engine(pipeline, num_blocks=64, block_size=16)
    eng.add_request(TEXT[:5], greedy(2))  # finishes on the first decode step
    eng.add_request(TEXT[10:30], greedy(6))
    eng.step()  # prefill
    eng.step()  # decode: the first request emits its 2nd token and is done
    at_peak, after = eng.last_step.kv, eng.kv_snapshot()
    assert at_peak.num_seqs == 2 and after.num_seqs == 1
    assert at_peak.allocated_tokens == after.allocated_tokens + 16
    assert at_peak.live_tokens == (5 + 1) + (20 + 1)


@pytest.mark.parametrize("pipeline", [False, True])
def test_step_after_a_finish_excludes_the_finished_sequence(pipeline):
    """5 + 20 prompt tokens, max 2 and 6 tokens, 4-slot blocks: the third step runs the second
    request alone, so it holds 22 live slots in 6 blocks, whether or not the step was launched
    before the first request's last token was read."""
    eng = make_engine(pipeline, num_blocks=64, block_size=4)
    eng.add_request(TEXT[:5], greedy(2))
    eng.add_request(TEXT[10:30], greedy(6))
    infos = []
    for _ in range(3):
        eng.step()
        infos.append(eng.last_step)
    assert infos[1] == StepInfo(False, 2, 2, KVSnapshot(32, 27, 2))
    assert infos[2] == StepInfo(False, 1, 1, KVSnapshot(24, 22, 1))
    if pipeline:  # the fourth step is in flight already: the live state is a step further on
        assert eng.stats.lookahead_steps > 0 and eng.kv_snapshot() == KVSnapshot(24, 23, 1)
    else:
        assert eng.kv_snapshot() == KVSnapshot(24, 22, 1)


def run_calls(pipeline: bool, arrivals: dict, aborts: dict | None = None, **kw):
    """Drive ``step()`` to the end with every request queued up front; abort ``aborts[k]`` (request
    numbers) before call k. Returns the engine, the requests and ``last_step`` after every call."""
    eng = make_engine(pipeline, **kw)
    reqs = [eng.add_request(p, params) for p, params in arrivals[0]]
    infos, k = [], 0
    while eng.has_unfinished():
        for r in (aborts or {}).get(k, []):
            eng.abort_request(reqs[r])
        eng.step()
        infos.append(eng.last_step)
        k += 1
        assert k < 10_000
    return eng, reqs, infos


@pytest.mark.parametrize("seed", range(4))
def test_eos_stops_keep_the_identity_and_the_step_records(seed):
    """Requests that stop on EOS: rows launched ahead for them are dropped, counted apart, and
    the pipelined engine's step records equal the synchronous engine's call by call."""
    arr = random_arrivals(seed, 14, 0)
    runs = {p: run_calls(p, arr) for p in (False, True)}
    for pipeline, (eng, reqs, infos) in runs.items():
        st = eng.stats
        needed = sum(len(s.prompt_token_ids) + len(s.output_token_ids) - 1 for s in reqs)
        assert st.positions_computed == needed + st.positions_discarded, pipeline
        assert st.positions_dropped == 0 or pipeline
    (e0, _, i0), (e1, _, i1) = runs[False], runs[True]
    assert i1 == i0
    for f in ("steps", "prefill_steps", "decode_steps", "tokens_generated", "max_batch", "peak_used_blocks",
              "num_preemptions", "positions_computed", "positions_padded", "positions_discarded"):  # fmt: skip
        assert getattr(e1.stats, f) == getattr(e0.stats, f), f
    assert e1.stats.lookahead_steps > 0
    # Some sequence of these seeds stops on EOS with a row already launched ahead.
    if seed in (0, 1):
        assert e1.stats.positions_dropped > 0


def test_aborts_between_calls_keep_the_step_records():
    arr = random_arrivals(5, 10, 0, ignore_eos_every=1)
    aborts = {4: [2], 9: [0, 5], 15: [7]}
    (e0, _, i0), (e1, _, i1) = (run_calls(p, arr, aborts) for p in (False, True))
    assert i1 == i0
    assert e1.stats.positions_computed == e0.stats.positions_computed
    assert e1.stats.positions_dropped > 0  # the aborted rows launched ahead
    assert e1.allocator.num_free_blocks == e1.allocator.num_blocks


def test_preemption_records_match_under_the_pipeline():
    arr = {0: [([i % VOCAB] * 10, greedy(30)) for i in range(6)]}
    (e0, _, i0), (e1, _, i1) = (run_calls(p, arr, num_blocks=24, block_size=4, watermark_blocks=1)
                                for p in (False, True))  # fmt: skip
    assert e0.stats.num_preemptions > 0
    assert i1 == i0
    assert e1.stats.positions_computed == e0.stats.positions_computed


def test_a_step_launched_ahead_whose_rows_all_stop_is_dropped_whole():
    """One request that stops on EOS after its first decode token: the step launched ahead for
    its next token is discarded, uncounted, and the engine reports idle afterwards."""
    from tests.test_host_pipeline import EOS, ideal

    rng = random.Random(0)
    for _ in range(10_000):
        prompt = [rng.randrange(VOCAB) for _ in range(rng.randint(1, 12))]
        out, why = ideal(prompt, SamplingParams(max_tokens=10))
        if why == "stop" and len(out) == 3:
            break
    else:
        pytest.fail("no prompt stops on EOS at its third token")
    runs = {}
    for pipeline in (False, True):
        eng = make_engine(pipeline)
        eng.add_request(prompt, SamplingParams(max_tokens=10))
        infos = []
        while eng.has_unfinished():
            ev = eng.step()
            infos.append((eng.last_step, [e.token_id for e in ev]))
        runs[pipeline] = (eng, infos)
    (e0, i0), (e1, i1) = runs[False], runs[True]
    assert i1 == i0 and i0[-1][1][-1] == EOS
    assert e1.stats.positions_dropped == 1 and e1.stats.steps == e0.stats.steps
    eng = e1
    eng.step()
    assert eng.last_step is None and not eng.has_unfinished()
