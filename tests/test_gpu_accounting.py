"""The GPU engine's work and memory accounting, synchronous and pipelined, and its pool edge cases.

Restates tests/test_phase6_accounting.py:32-89 through ``Engine`` on the HIP
path (graph-replayed decode steps; pipelined and not), with random-init GPT-2
124M weights, and tests/test_phase4_engine.py:119-140 (an oversized request is
rejected without blocking the others; a request whose context is exactly the
whole pool completes) under both engines, against the oracle's greedy ids.
"""

from __future__ import annotations

import random

import pytest

from oracle.gpt2_ref import RefConfig, build_ref_model, ref_greedy_generate
from tokquay_amd.engine import Engine, KVSnapshot, StepInfo
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2, GPT2Config
from tokquay_amd.scheduler import RequestRejected
from tokquay_amd.sequence import SamplingParams, SequenceStatus
from tokquay_amd.weights import random_state_dict

pytestmark = pytest.mark.gpu

TEXT = [random.Random(21).randrange(50256) for _ in range(400)]


@pytest.fixture(scope="module")
def weights():
    return random_state_dict(GPT2Config(), seed=0)


@pytest.fixture(scope="module")
def gpu_model(weights):
    m = GPT2(GPT2Config())
    m.load_state_dict(weights)
    return m.cuda().eval()


@pytest.fixture(scope="module")
def ref_model(weights):
    return build_ref_model(RefConfig(), weights)


_memo: dict = {}


def reference(ref_model, prompt, n):
    key = (tuple(prompt), n)
    if key not in _memo:
        _memo[key] = ref_greedy_generate(ref_model, list(prompt), n)
    return _memo[key]


def greedy(n):
    return SamplingParams(max_tokens=n, ignore_eos=True)


def make_engine(model, num_blocks, block_size, pipeline, **kw):
    eng = Engine(model, BlockAllocator(model.cfg, num_blocks, block_size, device="cuda"), pipeline=pipeline, **kw)
    assert eng.graphs is not None and eng.pipeline == pipeline
    return eng


def needed_positions(specs):
    return sum(len(p) + n - 1 for p, n in specs)


def run(engine, arrivals, max_steps=5000):
    """``arrivals``: (call index, prompt, params). Returns the sequences and ``last_step`` per call."""
    pending = sorted(arrivals, key=lambda a: a[0])
    seqs, infos = [], []
    for k in range(max_steps):
        while pending and pending[0][0] <= k:
            _, prompt, params = pending.pop(0)
            seqs.append(engine.add_request(prompt, params))
        if not pending and not engine.has_unfinished():
            engine.allocator.check_device_errors()
            return seqs, infos
        engine.step()
        infos.append(engine.last_step)
    pytest.fail("engine did not finish")


@pytest.mark.parametrize("pipeline", [False, True])
def test_positions_computed_is_exactly_the_necessary_work(gpu_model, pipeline):
    specs = [(TEXT[i * 9 : i * 9 + 8 + 3 * i], 6 + 2 * i) for i in range(5)]
    eng = make_engine(gpu_model, 64, 16, pipeline)
    run(eng, [(0, p, greedy(n)) for p, n in specs])
    st = eng.stats
    assert st.num_preemptions == 0 and st.positions_discarded == 0 and st.positions_dropped == 0
    assert st.positions_computed == needed_positions(specs)
    assert st.positions_padded >= st.positions_computed
    assert (st.lookahead_steps > 0) == pipeline


@pytest.mark.parametrize("pipeline", [False, True])
def test_preemption_adds_exactly_the_discarded_positions(gpu_model, ref_model, pipeline):
    specs = [(TEXT[i * 9 : i * 9 + 18 + 3 * i], 24 + 2 * i) for i in range(5)]
    eng = make_engine(gpu_model, 8, 16, pipeline)
    seqs, _ = run(eng, [(0, p, greedy(n)) for p, n in specs])
    st = eng.stats
    assert st.num_preemptions > 0 and st.positions_discarded > 0
    assert st.positions_computed == needed_positions(specs) + st.positions_discarded
    assert st.positions_discarded == eng.scheduler.num_discarded_positions
    for seq, (p, n) in zip(seqs, specs):
        assert seq.output_token_ids == reference(ref_model, p, n)


@pytest.mark.parametrize("pipeline", [False, True])
def test_last_step_and_kv_snapshot(gpu_model, pipeline):
    eng = make_engine(gpu_model, 64, 16, pipeline)
    assert eng.last_step is None and eng.kv_snapshot().num_seqs == 0
    eng.add_request(TEXT[:5], greedy(4))
    eng.add_request(TEXT[10:30], greedy(4))
    eng.step()
    assert eng.last_step == StepInfo(True, 2, 40, KVSnapshot((1 + 2) * 16, 5 + 20, 2)) and eng.last_step.kv == eng.kv_snapshot()
    eng.step()
    assert (eng.last_step.is_prefill, eng.last_step.num_seqs, eng.last_step.padded_tokens) == (False, 2, 2)
    eng.run_until_done()
    assert eng.kv_snapshot() == KVSnapshot(0, 0, 0)
    eng.step()
    assert eng.last_step is None


@pytest.mark.parametrize("pipeline", [False, True])
def test_snapshot_at_the_peak_and_after_a_finish(gpu_model, pipeline):
    eng = make_engine(gpu_model, 64, 4, pipeline)
    eng.add_request(TEXT[:5], greedy(2))
    eng.add_request(TEXT[10:30], greedy(6))
    infos = []
    for _ in range(3):
        eng.step()
        infos.append(eng.last_step)
    assert infos[1] == StepInfo(False, 2, 2, KVSnapshot(32, (5 + 1) + (20 + 1), 2))
    assert infos[2] == StepInfo(False, 1, 1, KVSnapshot(24, 22, 1))
    assert (eng.stats.lookahead_steps > 0) == pipeline
    eng.run_until_done()


def test_eos_stops_keep_the_identity_and_the_step_records(gpu_model, ref_model):
    """The EOS id is set to a token the oracle emits part-way through two of the requests, so
    they stop there; the other rows run on. Both engines emit the oracle's ids up to the stop,
    keep positions_computed = needed + discarded, and report the same StepInfo call by call."""
    prompts = [TEXT[40 * i : 40 * i + 7 + 5 * i] for i in range(6)]
    refs = [reference(ref_model, p, 12) for p in prompts]
    eos = refs[1][4]
    params = SamplingParams(max_tokens=12)
    runs = {}
    for pipeline in (False, True):
        eng = make_engine(gpu_model, 64, 16, pipeline, eos_token_id=eos)
        seqs, infos = run(eng, [(0, p, params) for p in prompts])
        for seq, want in zip(seqs, refs):
            cut = want.index(eos) + 1 if eos in want else len(want)
            assert seq.output_token_ids == want[:cut]
            assert seq.finish_reason == ("stop" if eos in want else "length")
        needed = sum(len(s.prompt_token_ids) + len(s.output_token_ids) - 1 for s in seqs)
        assert eng.stats.positions_computed == needed + eng.stats.positions_discarded
        runs[pipeline] = (eng, infos)
    (e0, i0), (e1, i1) = runs[False], runs[True]
    assert i1 == i0
    assert e1.stats.positions_computed == e0.stats.positions_computed
    assert e1.stats.lookahead_steps > 0 and e1.stats.positions_dropped > 0


@pytest.mark.parametrize("pipeline", [False, True])
def test_oversized_request_is_rejected_and_does_not_block_the_others(gpu_model, ref_model, pipeline):
    eng = make_engine(gpu_model, 16, 16, pipeline)  # 256 slots
    ok = [eng.add_request(TEXT[i * 8 : i * 8 + 12], greedy(20)) for i in range(3)]
    with pytest.raises(RequestRejected):
        eng.add_request(TEXT[:300], greedy(1))  # 19 blocks; the pool has 16
    assert eng.scheduler.num_preemptions == 0 and len(eng.scheduler.waiting) == 3
    eng.run_until_done()
    for i, seq in enumerate(ok):
        assert seq.output_token_ids == reference(ref_model, TEXT[i * 8 : i * 8 + 12], 20)
    assert eng.allocator.num_free_blocks == 16


@pytest.mark.parametrize("pipeline", [False, True])
def test_request_that_needs_the_entire_pool_still_completes(gpu_model, ref_model, pipeline):
    """Context 200 + 57 - 1 = 256 = all 16 blocks of 16: the steps near its end have no free block
    for a step launched ahead, and the other requests must wait or be preempted around it."""
    eng = make_engine(gpu_model, 16, 16, pipeline)
    big = TEXT[:200]
    arrivals = [(0, big, greedy(57))] + [(1, TEXT[300 + 10 * i : 310 + 10 * i], greedy(25)) for i in range(3)]
    seqs, _ = run(eng, arrivals)
    assert seqs[0].output_token_ids == reference(ref_model, big, 57)
    for i, seq in enumerate(seqs[1:]):
        assert seq.output_token_ids == reference(ref_model, TEXT[300 + 10 * i : 310 + 10 * i], 25)
    assert all(s.status is SequenceStatus.FINISHED for s in seqs)
    assert eng.allocator.num_free_blocks == 16 and eng.stats.peak_used_blocks == 16
