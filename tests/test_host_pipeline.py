"""Pipelined decode in ``Engine`` on the CPU, with a toy decoder in place of the model.

The toy's next token is a fixed function of a sequence's whole history, so an
engine that feeds every sequence its own previous token at the right position
emits exactly the toy's greedy continuation of each prompt, whatever the
batching, pipelining, admission timing or preemption. Every run is checked
against that continuation computed directly (``ideal``). ``ToyGraphs`` stands in
for the captured decode graphs: it asserts, at every launch, the contract the
real graphs rely on (running sequence, one pending or source-row token, a block
table that covers the fed position).
"""

from __future__ import annotations

import random

import pytest
import torch

from tokquay_amd.engine import Engine
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2Config
from tokquay_amd.scheduler import SchedulerConfig
from tokquay_amd.sequence import SamplingParams, SequenceStatus

pytestmark = pytest.mark.timeout(120)

VOCAB = 40
EOS = 7
TINY = GPT2Config(vocab_size=VOCAB, n_positions=256, n_embd=4, n_layer=1, n_head=1)


def toy_next(history: list[int]) -> int:
    h = 0
    for t in history:
        h = (h * 31 + t + 1) % 1_000_003
    return h % VOCAB


def one_hot(ids: list[int]) -> torch.Tensor:
    out = torch.zeros(len(ids), VOCAB)
    out[torch.arange(len(ids)), torch.tensor(ids, dtype=torch.int64)] = 10.0
    return out


def ideal(prompt: list[int], params: SamplingParams) -> tuple[list[int], str]:
    toks = list(prompt)
    out: list[int] = []
    while True:
        t = toy_next(toks)
        toks.append(t)
        out.append(t)
        if not params.ignore_eos and t == EOS:
            return out, "stop"
        if len(out) >= params.max_tokens:
            return out, "length"


class ToyGraphs:
    capacity = 64

    def __init__(self, alloc: BlockAllocator):
        self.alloc = alloc
        self.tokens = torch.zeros(self.capacity, dtype=torch.int64)
        self.rows: list[tuple[object, int]] = []  # (sequence, fed position) of every launched row
        self.src_launches = 0

    def launch(self, seqs, src_rows=None, logits=True):
        """Like DecodeGraphs.launch: ``logits=False`` returns only the ids (the fused-head graph)."""
        prev = self.tokens.clone()
        out = []
        for i, s in enumerate(seqs):
            assert s.status is SequenceStatus.RUNNING
            p = s.num_cached_tokens
            if src_rows is None:
                assert s.num_tokens - p == 1
                fed = s.token_ids[p]
            else:
                assert s.num_tokens == p  # the previous step's token is still pending on the host
                fed = int(prev[src_rows[i]])
            assert self.alloc.blocks_needed(p + 1) <= len(s.block_table)
            out.append(toy_next(s.token_ids[:p] + [fed]))
            self.rows.append((s, p))
            s.num_cached_tokens += 1
        self.src_launches += src_rows is not None
        self.tokens[: len(seqs)] = torch.tensor(out, dtype=torch.int64)
        return (one_hot(out) if logits else None), self.tokens[: len(seqs)]


class ToyEngine(Engine):
    def _eager_forward(self, seqs, new_lens):
        new_lens = new_lens or [s.num_uncached_tokens for s in seqs]
        nxt = []
        for s, n in zip(seqs, new_lens):
            assert self.allocator.blocks_needed(s.num_cached_tokens + n) <= len(s.block_table)
            s.num_cached_tokens += n
            nxt.append(toy_next(s.token_ids[: s.num_cached_tokens]))
        return one_hot(nxt)


def make_engine(pipeline: bool, num_blocks=256, block_size=4, **cfg):
    cfg.setdefault("max_num_seqs", 16)
    cfg.setdefault("max_num_batched_tokens", 512)
    cfg.setdefault("max_model_len", 256)
    alloc = BlockAllocator(TINY, num_blocks, block_size, device="cpu")
    model = type("ToyModel", (), {"cfg": TINY})()
    eng = ToyEngine(model, alloc, SchedulerConfig(**cfg), eos_token_id=EOS, use_graphs=False, pipeline=pipeline)
    eng.graphs = ToyGraphs(alloc)
    return eng


def drive(eng, arrivals: dict[int, list[tuple[list[int], SamplingParams]]], aborts: dict[int, list[int]] = ()):
    """Call ``step()`` until done, adding the requests ``arrivals[k]`` and aborting the sequences
    ``aborts[k]`` (by request number) before call k. Returns (requests, outputs, reasons)."""
    reqs, outs, reasons = [], {}, {}
    k = 0
    last = max(list(arrivals) + list(dict(aborts)) + [0])
    while k <= last or eng.has_unfinished():
        for prompt, params in arrivals.get(k, []):
            reqs.append((eng.add_request(prompt, params), prompt, params))
        for r in dict(aborts).get(k, []):
            eng.abort_request(reqs[r][0])
        for ev in eng.step():
            outs.setdefault(ev.seq_id, []).append(ev.token_id)
            if ev.finish_reason:
                reasons[ev.seq_id] = ev.finish_reason
        k += 1
        assert k < 10_000
    assert eng.allocator.num_free_blocks == eng.allocator.num_blocks  # every block came back
    for seq, p in eng.graphs.rows:
        # Output j > 1 comes from feeding position len(prompt) + j - 2. One row past the last
        # output is a dropped row: only a sequence that stopped on EOS (or was aborted) has one.
        last = len(seq.prompt_token_ids) + len(seq.output_token_ids) - 2
        assert p <= last or (p == last + 1 and seq.finish_reason in ("stop", "abort")), (seq.seq_id, p)
    return reqs, outs, reasons


def random_arrivals(seed: int, n: int, spread: int, ignore_eos_every: int = 3):
    rng = random.Random(seed)
    arr: dict[int, list] = {}
    for i in range(n):
        prompt = [rng.randrange(VOCAB) for _ in range(rng.randint(1, 20))]
        params = SamplingParams(max_tokens=rng.randint(1, 40), ignore_eos=i % ignore_eos_every == 0)
        arr.setdefault(rng.randrange(spread) if spread else 0, []).append((prompt, params))
    return arr


def check_ideal(reqs, outs, reasons, aborted=()):
    for i, (seq, prompt, params) in enumerate(reqs):
        want, why = ideal(prompt, params)
        got = outs.get(seq.seq_id, [])
        if i in aborted:
            assert got == want[: len(got)]
            continue
        assert got == want, f"request {i}"
        assert reasons[seq.seq_id] == why


@pytest.mark.parametrize("pipeline", [False, True])
def test_all_at_once_matches_ideal(pipeline):
    eng = make_engine(pipeline)
    reqs, outs, reasons = drive(eng, random_arrivals(0, 12, 0))
    check_ideal(reqs, outs, reasons)
    if pipeline:
        assert eng.stats.lookahead_steps > 0 and eng.graphs.src_launches == eng.stats.lookahead_steps
        # Rows of sequences that had stopped on EOS while the step was in flight were computed and dropped.
        dropped = sum(1 for s, p in eng.graphs.rows if p == len(s.prompt_token_ids) + len(s.output_token_ids) - 1)
        assert dropped > 0
    else:
        assert eng.stats.lookahead_steps == 0


@pytest.mark.parametrize("seed", range(6))
def test_staggered_arrivals_and_aborts(seed):
    arr = random_arrivals(seed, 20, 60)
    aborts = {15 + seed: [1], 30: [4, 5]}
    for pipeline in (False, True):
        eng = make_engine(pipeline)
        reqs, outs, reasons = drive(eng, arr, aborts)
        check_ideal(reqs, outs, reasons, aborted={1, 4, 5})
    assert eng.stats.lookahead_steps > 0


def test_preemption_under_a_tiny_pool():
    arr = {0: [([i % VOCAB] * 10, SamplingParams(max_tokens=30, ignore_eos=True)) for i in range(6)]}
    for pipeline in (False, True):
        eng = make_engine(pipeline, num_blocks=24, block_size=4, watermark_blocks=1)
        reqs, outs, reasons = drive(eng, arr)
        check_ideal(reqs, outs, reasons)
        assert eng.stats.num_preemptions > 0
        if pipeline:
            assert eng.stats.lookahead_steps > 0


def test_chunked_prefill_mode():
    arr = random_arrivals(7, 16, 40)
    for pipeline in (False, True):
        eng = make_engine(pipeline, chunked_prefill=True, prefill_chunk_tokens=8, max_num_batched_tokens=24)
        reqs, outs, reasons = drive(eng, arr)
        check_ideal(reqs, outs, reasons)


def test_sampled_rows_are_never_launched_ahead():
    arr = random_arrivals(3, 6, 0)
    arr[0].append(([1, 2, 3], SamplingParams(max_tokens=10, temperature=1.0, seed=5, ignore_eos=True)))
    results = []
    for pipeline in (False, True):
        eng = make_engine(pipeline)
        reqs, outs, reasons = drive(eng, arr)
        greedy = [r for r in reqs if r[2].temperature == 0]
        check_ideal(greedy, outs, reasons)
        results.append(outs[reqs[-1][0].seq_id])
    assert results[0] == results[1]  # same seed, same draws


def test_max_tokens_one_and_single_sequence():
    arr = {0: [([5, 6], SamplingParams(max_tokens=1))], 3: [([9] * 3, SamplingParams(max_tokens=25, ignore_eos=True))]}
    eng = make_engine(True)
    reqs, outs, reasons = drive(eng, arr)
    check_ideal(reqs, outs, reasons)
    assert eng.stats.lookahead_steps > 0
