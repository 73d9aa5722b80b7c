"""Scheduler policy without a model (tokquay/scheduler.py:1-190), restating the reference's
model-free tests (tests/test_phase4_scheduler.py) against this package. ``fake_step`` stands in
for the forward: it marks every uncached token cached and appends a dummy token."""

from __future__ import annotations

import pytest
from hypothesis import given, settings, strategies as st

from tokquay_amd.kv_cache import BlockAllocator, cdiv
from tokquay_amd.model import GPT2Config
from tokquay_amd.scheduler import RequestRejected, Scheduler, SchedulerConfig
from tokquay_amd.sequence import SamplingParams, Sequence, SequenceStatus

pytestmark = pytest.mark.timeout(60)

TINY = GPT2Config(vocab_size=8, n_positions=64, n_embd=4, n_layer=1, n_head=1)


def make(num_blocks=64, block_size=4, **cfg):
    cfg.setdefault("max_model_len", 10_000)
    cfg.setdefault("max_num_batched_tokens", 10_000)
    cfg.setdefault("watermark_blocks", 0)
    return Scheduler(BlockAllocator(TINY, num_blocks, block_size, device="cpu"), SchedulerConfig(**cfg))


def req(sched, seq_id, prompt_len, max_tokens):
    seq = Sequence(seq_id, [1] * prompt_len, sampling=SamplingParams(max_tokens=max_tokens))
    sched.add_request(seq)
    return seq


def fake_step(sched):
    batch = sched.schedule()
    if batch is None:
        return None
    for s in batch.seqs:
        s.num_cached_tokens = s.num_tokens
        s.append_token(0)
        if len(s.output_token_ids) >= s.sampling.max_tokens:
            sched.finish(s, "length")
    return batch


def ids(seqs):
    return [s.seq_id for s in seqs]


def test_fcfs_admission_and_prefill_priority():
    sched = make()
    seqs = [req(sched, i, 5, 10) for i in range(3)]
    batch = fake_step(sched)
    assert batch.is_prefill and ids(batch.seqs) == [0, 1, 2]
    assert all(s.status is SequenceStatus.RUNNING for s in seqs)
    assert not fake_step(sched).is_prefill


def test_arrival_mid_generation_is_admitted_on_the_next_step():
    sched = make()
    a = req(sched, 0, 5, 30)
    for _ in range(4):
        fake_step(sched)
    b = req(sched, 1, 5, 30)
    batch = fake_step(sched)
    assert batch.is_prefill and ids(batch.seqs) == [1] and a.status is SequenceStatus.RUNNING
    assert ids(fake_step(sched).seqs) == [0, 1]
    assert b.status is SequenceStatus.RUNNING


def test_finished_requests_leave_immediately():
    sched = make(num_blocks=8)
    short, long = req(sched, 0, 4, 2), req(sched, 1, 4, 20)
    fake_step(sched)
    fake_step(sched)
    assert short.status is SequenceStatus.FINISHED and short.block_table == []
    assert ids(fake_step(sched).seqs) == [1]
    assert sched.allocator.num_used_blocks == len(long.block_table)


def test_max_num_seqs_and_fcfs_reuse():
    sched = make(max_num_seqs=2)
    seqs = [req(sched, i, 4, 3) for i in range(5)]
    assert ids(fake_step(sched).seqs) == [0, 1]
    later = []
    while sched.has_unfinished():
        batch = fake_step(sched)
        assert len(sched.running) <= 2
        if batch.is_prefill:
            later += ids(batch.seqs)
    assert later == [2, 3, 4] and all(s.status is SequenceStatus.FINISHED for s in seqs)


def test_padded_token_budget_and_no_queue_jumping():
    sched = make(max_num_batched_tokens=64)
    for i in range(3):
        req(sched, i, 30, 2)
    assert ids(fake_step(sched).seqs) == [0, 1]
    sched = make(max_num_batched_tokens=64)
    req(sched, 0, 30, 2)
    req(sched, 1, 60, 2)
    req(sched, 2, 5, 2)
    batch = fake_step(sched)
    assert ids(batch.seqs) == [0] and batch.padded_tokens <= 64


def preemption_scenario():
    sched = make(num_blocks=6, block_size=4)
    seqs = req(sched, 0, 8, 16), req(sched, 1, 8, 16), req(sched, 2, 4, 16)
    assert fake_step(sched).is_prefill and sched.allocator.num_free_blocks == 1
    return (sched, *seqs)


def test_preemption_evicts_the_newest_and_requeues_it_at_the_front():
    sched, a, b, c = preemption_scenario()
    req(sched, 3, 10, 2)
    batch = sched.schedule()
    assert ids(batch.seqs) == [0, 1] and ids(batch.preempted) == [2]
    assert c.status is SequenceStatus.WAITING and c.block_table == [] and c.num_cached_tokens == 0
    assert c.output_token_ids == [0]
    assert ids(sched.waiting) == [2, 3] and sched.num_preemptions == 1


def test_preempted_sequence_recomputes_and_finishes():
    sched, a, b, c = preemption_scenario()
    sched.schedule()
    while sched.has_unfinished():
        fake_step(sched)
    assert all(s.status is SequenceStatus.FINISHED and len(s.output_token_ids) == 16 for s in (a, b, c))
    assert sched.allocator.num_free_blocks == sched.allocator.num_blocks


def test_newest_sequence_evicts_itself_when_it_alone_needs_a_block():
    sched = make(num_blocks=3, block_size=4)
    req(sched, 0, 7, 4)
    b = req(sched, 1, 4, 4)
    fake_step(sched)
    batch = sched.schedule()
    assert ids(batch.seqs) == [0] and ids(batch.preempted) == [1] and b.status is SequenceStatus.WAITING


def test_watermark_applies_only_while_others_run():
    sched = make(num_blocks=8, block_size=4, watermark_blocks=2)
    a = req(sched, 0, 12, 4)
    fake_step(sched)
    b = req(sched, 1, 16, 4)
    assert not fake_step(sched).is_prefill and b.status is SequenceStatus.WAITING
    while a.status is not SequenceStatus.FINISHED:
        fake_step(sched)
    assert fake_step(sched).is_prefill and b.status is SequenceStatus.RUNNING


def test_up_front_rejection():
    sched = make(num_blocks=16, block_size=16, max_model_len=1024)
    with pytest.raises(RequestRejected, match="KV blocks"):
        req(sched, 0, 300, 1)
    with pytest.raises(RequestRejected, match="model supports"):
        req(sched, 1, 900, 200)
    sched = make(num_blocks=64, block_size=16, max_num_batched_tokens=128)
    with pytest.raises(RequestRejected, match="max_num_batched_tokens"):
        req(sched, 2, 100, 50)
    assert not sched.waiting and not sched.running


def test_max_context_boundary_is_exact():
    sched = make(num_blocks=4, block_size=4)
    req(sched, 0, 10, 7)  # 16 positions fit exactly
    with pytest.raises(RequestRejected):
        req(sched, 1, 10, 8)


def test_abort_anywhere_frees_blocks():
    sched = make(num_blocks=8, block_size=4)
    a, b = req(sched, 0, 8, 10), req(sched, 1, 8, 10)
    fake_step(sched)
    waiting = req(sched, 2, 20, 4)  # 6 blocks: cannot be admitted next to A and B
    sched.abort(a)
    sched.abort(waiting)
    sched.abort(a)  # finished: no-op
    assert a.finish_reason == "abort" and waiting.finish_reason == "abort"
    assert ids(sched.running) == [1] and not sched.waiting
    assert sched.allocator.num_used_blocks == len(b.block_table)


@settings(deadline=None, max_examples=200)
@given(
    workload=st.lists(st.tuples(st.integers(1, 40), st.integers(1, 40), st.integers(0, 25)), min_size=1, max_size=14),
    num_blocks=st.integers(3, 20),
    block_size=st.sampled_from([1, 2, 4, 8]),
    max_num_seqs=st.integers(1, 8),
    budget=st.integers(8, 200),
    watermark=st.integers(0, 3),
)
def test_random_workloads_never_deadlock_or_leak(workload, num_blocks, block_size, max_num_seqs, budget, watermark):
    sched = make(num_blocks=num_blocks, block_size=block_size, max_num_seqs=max_num_seqs,
                 max_num_batched_tokens=max(budget, max_num_seqs), watermark_blocks=watermark)  # fmt: skip
    alloc = sched.allocator
    pending = sorted(enumerate(workload), key=lambda x: x[1][2])
    accepted = []
    step = 0
    while True:
        while pending and pending[0][1][2] <= step:
            i, (p, m, _) = pending.pop(0)
            seq = Sequence(i, [1] * p, sampling=SamplingParams(max_tokens=m))
            if sched.rejection_reason(seq):
                with pytest.raises(RequestRejected):
                    sched.add_request(seq)
            else:
                sched.add_request(seq)
                accepted.append(seq)
        if not pending and not sched.has_unfinished():
            break
        batch = fake_step(sched)
        assert batch is not None or pending
        step += 1
        assert step < 50_000
        if batch is not None:
            assert batch.padded_tokens <= sched.config.max_num_batched_tokens
        assert len(sched.running) <= max_num_seqs
        order = [s.seq_id for s in accepted]
        assert ids(sched.running) == sorted(ids(sched.running), key=order.index)
        assert ids(sched.waiting) == sorted(ids(sched.waiting), key=order.index)
        owned = [b for s in sched.running for b in s.block_table]
        assert len(owned) == len(set(owned)) and alloc.num_free_blocks + len(owned) == alloc.num_blocks
        for s in sched.running:
            assert len(s.block_table) >= cdiv(s.num_cached_tokens, block_size)
    assert all(s.status is SequenceStatus.FINISHED and len(s.output_token_ids) == s.sampling.max_tokens for s in accepted)
    assert alloc.num_free_blocks == alloc.num_blocks


# ------------------------------------------------------------------- chunked prefill (mixed steps)
def fake_step_chunked(sched):
    """The forward consumed new_lens[i] tokens of each sequence; complete ones append a token."""
    batch = sched.schedule()
    if batch is None:
        return None
    for s, n in zip(batch.seqs, batch.new_lens):
        s.num_cached_tokens += n
        if s.num_cached_tokens == s.num_tokens:
            s.append_token(0)
            if len(s.output_token_ids) >= s.sampling.max_tokens:
                sched.finish(s, "length")
    return batch


def test_chunked_prompt_is_fed_next_to_decoding_sequences_without_stalling_them():
    sched = make(num_blocks=64, block_size=4, max_num_batched_tokens=40, max_num_seqs=8, chunked_prefill=True, prefill_chunk_tokens=32)
    a = req(sched, 0, 6, 30)
    fake_step_chunked(sched)  # A prefills (6 tokens) and samples
    b = req(sched, 1, 100, 3)  # longer than the whole per-step budget
    feeds = []
    for _ in range(4):
        batch = fake_step_chunked(sched)
        assert batch.padded_tokens <= 40
        rows = dict(zip(ids(batch.seqs), batch.new_lens))
        assert rows[0] == 1  # A decodes in every step
        feeds.append(rows.get(1))
    assert feeds == [32, 32, 32, 4]  # B's prompt in chunks, capped by the chunk size and then what is left
    assert len(b.output_token_ids) == 1 and len(a.output_token_ids) == 5


def test_chunked_budget_is_shared_oldest_prefill_first_then_fcfs_admission():
    sched = make(num_blocks=64, block_size=4, max_num_batched_tokens=48, max_num_seqs=8, chunked_prefill=True, prefill_chunk_tokens=32)
    req(sched, 0, 50, 2)
    req(sched, 1, 20, 2)
    req(sched, 2, 8, 2)
    batch = fake_step_chunked(sched)
    assert list(zip(ids(batch.seqs), batch.new_lens)) == [(0, 32), (1, 16)]  # 48 tokens; request 2 waits
    batch = fake_step_chunked(sched)
    assert list(zip(ids(batch.seqs), batch.new_lens)) == [(0, 18), (1, 4), (2, 8)]
    assert batch.is_prefill


def test_chunked_mode_admits_prompts_longer_than_the_budget():
    sched = make(num_blocks=64, block_size=16, max_num_batched_tokens=128, chunked_prefill=True)
    req(sched, 0, 300, 5)  # alternating mode rejects this (tests/test_phase4_scheduler.py:221-224)
    while sched.has_unfinished():
        fake_step_chunked(sched)
    assert sched.allocator.num_free_blocks == 64


@settings(deadline=None, max_examples=200)
@given(
    workload=st.lists(st.tuples(st.integers(1, 60), st.integers(1, 30), st.integers(0, 25)), min_size=1, max_size=14),
    num_blocks=st.integers(4, 24),
    block_size=st.sampled_from([1, 2, 4, 8]),
    max_num_seqs=st.integers(1, 8),
    budget=st.integers(8, 120),
    chunk=st.integers(1, 48),
    watermark=st.integers(0, 3),
)
def test_chunked_random_workloads_never_deadlock_or_leak(workload, num_blocks, block_size, max_num_seqs, budget,
                                                         chunk, watermark):  # fmt: skip
    sched = make(num_blocks=num_blocks, block_size=block_size, max_num_seqs=max_num_seqs,
                 max_num_batched_tokens=max(budget, max_num_seqs), watermark_blocks=watermark,
                 chunked_prefill=True, prefill_chunk_tokens=chunk)  # fmt: skip
    alloc = sched.allocator
    pending = sorted(enumerate(workload), key=lambda x: x[1][2])
    accepted = []
    step = 0
    while True:
        while pending and pending[0][1][2] <= step:
            i, (p, m, _) = pending.pop(0)
            seq = Sequence(i, [1] * p, sampling=SamplingParams(max_tokens=m))
            if sched.rejection_reason(seq):
                with pytest.raises(RequestRejected):
                    sched.add_request(seq)
            else:
                sched.add_request(seq)
                accepted.append(seq)
        if not pending and not sched.has_unfinished():
            break
        batch = fake_step_chunked(sched)
        assert batch is not None or pending, "deadlock: work remains but nothing is schedulable"
        step += 1
        assert step < 50_000, "livelock"
        if batch is not None:
            assert batch.padded_tokens <= sched.config.max_num_batched_tokens
            assert all(1 <= n <= max(1, chunk) or n == 1 for n in batch.new_lens)
        assert len(sched.running) <= max_num_seqs
        owned = [b for s in sched.running for b in s.block_table]
        assert len(owned) == len(set(owned)) and alloc.num_free_blocks + len(owned) == alloc.num_blocks
        for s in sched.running:
            assert len(s.block_table) >= cdiv(s.num_cached_tokens, block_size)
    assert all(s.status is SequenceStatus.FINISHED and len(s.output_token_ids) == s.sampling.max_tokens for s in accepted)
    assert alloc.num_free_blocks == alloc.num_blocks
