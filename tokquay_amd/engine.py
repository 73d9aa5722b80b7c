"""One continuous-batching iteration per ``step()`` (tokquay/engine.py:95-197).

schedule -> ``paged_forward`` (gfx950 attention) -> batched greedy argmax, plus
per-row temperature / top-k sampling -> one device-to-host sync -> append and
stop checks. Not thread safe: one thread drives it.

Pipelined decode (on by default with HIP graphs). When a decode step is all
greedy rows, ``step()`` launches it, then - before reading its tokens back -
schedules and launches the next decode step, whose graph takes each row's input
token from the argmax the previous replay left on the device. Only then does it
wait for the first step's ids, append them and run the stop checks, so the host
work of one step overlaps the GPU work of the next. Each ``step()`` call still
returns the tokens of exactly one step, in order.

The next step is launched ahead only when the synchronous engine would run the
same decode step anyway: no request is waiting, every running sequence is in
the batch, and the pool has room for every row's next slot without preempting.
A row that will stop by length is left out; a row whose token turns out to be
EOS (or whose request is aborted before the step is read) is computed and
discarded: its sequence is finished by then, so it emits nothing. Greedy ids per
sequence are therefore those of the synchronous engine; the block ids a sequence
receives may differ when a finishing sequence would have returned its blocks
first.

Accounting follows the synchronous engine. A step launched ahead is settled at
the start of the ``step()`` call that returns its tokens, once the previous
step's finishes and any abort between the calls are applied: only then is it
counted in ``stats`` and given its ``StepInfo``, over the rows whose sequences are
still running (the rows the synchronous engine would have scheduled), with the
KV snapshot of that moment. Its discarded rows go to ``positions_dropped``, so
``positions_computed`` is the reference's count (needed + preemption-discarded
positions); a step whose every row is discarded is dropped whole and the call
schedules afresh, as the synchronous engine would.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from tokquay_amd import ops
from tokquay_amd.generate import paged_forward
from tokquay_amd.graphs import DecodeGraphs
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2
from tokquay_amd.scheduler import ScheduledBatch, Scheduler, SchedulerConfig
from tokquay_amd.sequence import SamplingParams, Sequence, SequenceStatus

GPT2_EOS_TOKEN_ID = 50256


@dataclass
class TokenEvent:
    seq_id: int
    token_id: int
    finish_reason: str | None = None


@dataclass
class EngineStats:
    steps: int = 0
    prefill_steps: int = 0
    decode_steps: int = 0
    tokens_generated: int = 0
    max_batch: int = 0
    peak_used_blocks: int = 0
    num_preemptions: int = 0
    positions_computed: int = 0  # real positions fed (prompt + recomputed + decoded)
    positions_padded: int = 0  # batch x longest row, the reference's padded work measure
    positions_discarded: int = 0  # cached positions thrown away by preemption
    lookahead_steps: int = 0  # decode steps launched before the previous step's tokens were read
    positions_dropped: int = 0  # rows computed ahead, then discarded (their sequence had stopped)


@dataclass
class KVSnapshot:
    allocated_tokens: int
    live_tokens: int
    num_seqs: int


@dataclass
class StepInfo:
    is_prefill: bool
    num_seqs: int
    padded_tokens: int
    kv: KVSnapshot  # taken after the forward, before finished sequences free their blocks


@dataclass
class _InFlight:
    """A launched decode step whose tokens the host has not read yet."""

    seqs: list[Sequence]
    ids: torch.Tensor  # host int64 [n] the step's greedy ids are copied into
    ready: torch.cuda.Event | None  # recorded after that copy (None on the CPU)
    info: StepInfo | None  # None until a step launched ahead is settled


def finish_reason_for(seq: Sequence, token: int, eos_token_id: int) -> str | None:
    if not seq.sampling.ignore_eos and token == eos_token_id:
        return "stop"
    if len(seq.output_token_ids) >= seq.sampling.max_tokens:
        return "length"
    return None


def sample_token(logits: torch.Tensor, params: SamplingParams, generator: torch.Generator | None) -> int:
    """Greedy, or temperature + optional top-k sampling from one row ``[vocab]`` (tokquay/engine.py:83-92)."""
    if params.temperature == 0:
        return int(logits.argmax())
    logits = logits / params.temperature
    if params.top_k > 0:
        kth = torch.topk(logits, min(params.top_k, logits.numel())).values[-1]
        logits = logits.masked_fill(logits < kth, float("-inf"))
    probs = torch.softmax(logits, dim=-1)
    return int(torch.multinomial(probs, 1, generator=generator))


class Engine:
    def __init__(
        self,
        model: GPT2,
        allocator: BlockAllocator,
        config: SchedulerConfig | None = None,
        eos_token_id: int = GPT2_EOS_TOKEN_ID,
        use_graphs: bool | None = None,
        pipeline: bool | None = None,
    ):
        """``use_graphs`` (default: on when the pool is on a HIP device) replays decode steps
        from captured HIP graphs; prefill and mixed steps always run eagerly. ``pipeline``
        (default: ``use_graphs``) launches the next greedy decode step before reading the
        current one's tokens."""
        if config is None:
            config = SchedulerConfig(max_model_len=model.cfg.n_positions)
        if config.max_model_len > model.cfg.n_positions:
            raise ValueError("max_model_len exceeds the model's context window")
        self.model = model
        self.allocator = allocator
        self.scheduler = Scheduler(allocator, config)
        self.eos_token_id = eos_token_id
        self.stats = EngineStats()
        self.last_step: StepInfo | None = None
        self._next_id = 0
        self._rngs: dict[int, torch.Generator] = {}
        if use_graphs is None:
            use_graphs = allocator.pool.is_cuda
        self.graphs = DecodeGraphs(model, allocator, config.max_num_seqs) if use_graphs else None
        self.pipeline = bool(use_graphs) if pipeline is None else pipeline
        self._inflight: _InFlight | None = None
        self._host_ids: list[torch.Tensor] | None = None  # two alternating token buffers
        self._flip = 0

    def add_request(self, prompt_token_ids: list[int], params: SamplingParams | None = None) -> Sequence:
        seq = Sequence(self._next_id, list(prompt_token_ids), sampling=params or SamplingParams())
        self.scheduler.add_request(seq)  # may raise; the id is only consumed on success
        self._next_id += 1
        if seq.sampling.temperature > 0:
            gen = torch.Generator(device=self.allocator.pool.device)
            gen.manual_seed(seq.sampling.seed if seq.sampling.seed is not None else torch.seed() % 2**63)
            self._rngs[seq.seq_id] = gen
        return seq

    def abort_request(self, seq: Sequence) -> None:
        self.scheduler.abort(seq)
        self._rngs.pop(seq.seq_id, None)

    def has_unfinished(self) -> bool:
        # A step in flight whose every row is discarded is not work left: step() drops it.
        live = self._inflight is not None and any(s.status is SequenceStatus.RUNNING for s in self._inflight.seqs)
        return live or self.scheduler.has_unfinished()

    def kv_snapshot(self) -> KVSnapshot:
        running = self.scheduler.running
        return KVSnapshot(
            allocated_tokens=self.allocator.num_used_blocks * self.allocator.block_size,
            live_tokens=sum(s.num_cached_tokens for s in running),
            num_seqs=len(running),
        )

    @torch.no_grad()
    def step(self) -> list[TokenEvent]:
        cur, self._inflight = self._inflight, None
        if cur is not None and not self._settle(cur):
            cur = None  # every row of the step launched ahead was discarded: schedule afresh
        if cur is None:
            batch = self.scheduler.schedule()
            if batch is None:
                self.last_step = None
                return []
            self._count(batch.seqs, batch.is_prefill, batch.new_lens or [s.num_uncached_tokens for s in batch.seqs],
                        batch.padded_tokens)  # fmt: skip
            if batch.is_prefill or not self._can_pipeline(batch.seqs):
                return self._run(batch)
            cur = self._launch(batch.seqs, None, batch.padded_tokens)
        self._inflight = self._lookahead(cur)
        events = self._complete(cur)
        nxt = self._inflight
        if nxt is not None and not any(s.status is SequenceStatus.RUNNING for s in nxt.seqs):
            self._settle(nxt)  # every row launched ahead stopped in `cur`: counted as dropped
            self._inflight = None
        return events

    def _count(self, seqs: list[Sequence], is_prefill: bool, fed: list[int], padded: int) -> None:
        st = self.stats
        st.steps += 1
        st.prefill_steps += is_prefill
        st.decode_steps += not is_prefill
        st.max_batch = max(st.max_batch, len(seqs))
        st.peak_used_blocks = max(st.peak_used_blocks, self.allocator.num_used_blocks)
        st.num_preemptions = self.scheduler.num_preemptions
        st.positions_discarded = self.scheduler.num_discarded_positions
        st.positions_computed += sum(fed)
        st.positions_padded += padded

    def _eager_forward(self, seqs: list[Sequence], new_lens: list[int] | None) -> torch.Tensor:
        return paged_forward(self.model, self.allocator, seqs, new_lens)

    def _run(self, batch: ScheduledBatch) -> list[TokenEvent]:
        """One step, synchronously: forward, sample, append, stop checks."""
        greedy = None
        if self.graphs is not None and not batch.is_prefill:
            # All-greedy steps need only ids: small buckets then never write logits.
            want_logits = any(s.sampling.temperature > 0 for s in batch.seqs)
            logits, greedy = self.graphs.launch(batch.seqs, logits=want_logits)
        else:
            logits = self._eager_forward(batch.seqs, batch.new_lens)
        self.last_step = StepInfo(batch.is_prefill, len(batch.seqs), batch.padded_tokens, self.kv_snapshot())
        # A sequence samples once all its tokens are cached; a chunked prompt part-way through does not.
        done = [i for i, s in enumerate(batch.seqs) if s.num_cached_tokens == s.num_tokens]
        if len(done) < len(batch.seqs):
            if logits is None:  # ids-only decode step (every row is done after a decode step anyway)
                greedy = greedy[torch.tensor(done, device=greedy.device)]
            else:
                logits = logits[done]
                greedy = None
        seqs = [batch.seqs[i] for i in done]
        tokens = self._sample(seqs, logits, greedy) if seqs else []
        return self._emit(seqs, tokens)

    def _emit(self, seqs: list[Sequence], tokens: list[int]) -> list[TokenEvent]:
        events = []
        for seq, tok in zip(seqs, tokens):
            if seq.status is not SequenceStatus.RUNNING:
                continue  # finished or aborted while its step was in flight: the row is discarded
            seq.append_token(tok)
            reason = finish_reason_for(seq, tok, self.eos_token_id)
            if reason:
                self.scheduler.finish(seq, reason)
                self._rngs.pop(seq.seq_id, None)
            events.append(TokenEvent(seq.seq_id, tok, reason))
        self.stats.tokens_generated += len(events)
        return events

    # ---- pipelined decode ------------------------------------------------------------
    def _can_pipeline(self, seqs: list[Sequence]) -> bool:
        return self.pipeline and self.graphs is not None and all(s.sampling.temperature == 0 for s in seqs)

    def _launch(self, seqs: list[Sequence], src_rows: list[int] | None, padded: int | None) -> _InFlight:
        """Enqueue one graph decode step and the copy of its greedy ids to the host. ``padded`` is
        None for a step launched ahead: its StepInfo is made when it is settled."""
        _, ids = self.graphs.launch(seqs, src_rows, logits=False)
        if self._host_ids is None:
            cap = self.graphs.capacity
            self._host_ids = [torch.empty(cap, dtype=torch.int64, pin_memory=ids.is_cuda) for _ in range(2)]
        host = self._host_ids[self._flip][: len(seqs)]
        self._flip ^= 1
        host.copy_(ids, non_blocking=True)
        ready = None
        if ids.is_cuda:
            ready = torch.cuda.Event()
            ready.record()
        info = None if padded is None else StepInfo(False, len(seqs), padded, self.kv_snapshot())
        return _InFlight(seqs, host, ready, info)

    def _lookahead(self, cur: _InFlight) -> _InFlight | None:
        """Launch the decode step after ``cur`` if the synchronous engine would run it unchanged."""
        sched, alloc = self.scheduler, self.allocator
        if not self._can_pipeline(cur.seqs) or sched.waiting:
            return None  # admission is decided once the tokens are known
        live = [s for s in cur.seqs if s.status is SequenceStatus.RUNNING]
        if len(live) != len(sched.running):
            return None  # other sequences (prompts part-way through) run too
        # Rows whose token from `cur` will not end them by length; each feeds position num_cached_tokens.
        rows = [i for i, s in enumerate(cur.seqs)
                if s.status is SequenceStatus.RUNNING and len(s.output_token_ids) + 1 < s.sampling.max_tokens]  # fmt: skip
        if not rows:
            return None
        seqs = [cur.seqs[i] for i in rows]
        need = sum(max(0, alloc.blocks_needed(s.num_cached_tokens + 1) - len(s.block_table)) for s in seqs)
        if need > alloc.num_free_blocks:
            return None  # the step may preempt: decided once the tokens are known
        for s in seqs:
            alloc.append_slot(s, s.num_cached_tokens + 1)
        self.stats.lookahead_steps += 1
        return self._launch(seqs, rows, None)

    def _settle(self, cur: _InFlight) -> bool:
        """Count a step launched ahead, now that the previous step's finishes are applied: its
        rows of still-running sequences are the step the synchronous engine schedules here.
        Returns False if no such row is left (the step is then dropped, uncounted)."""
        if cur.info is not None:
            return True
        live = [s for s in cur.seqs if s.status is SequenceStatus.RUNNING]
        self.stats.positions_dropped += len(cur.seqs) - len(live)
        if not live:
            return False
        self._count(live, False, [1] * len(live), len(live))
        cur.info = StepInfo(False, len(live), len(live), self.kv_snapshot())
        return True

    def _complete(self, cur: _InFlight) -> list[TokenEvent]:
        if cur.ready is not None:
            cur.ready.synchronize()
        self.last_step = cur.info
        return self._emit(cur.seqs, cur.ids.tolist())

    def drain(self) -> list[TokenEvent]:
        """Read back the step launched ahead, if any, without launching another; afterwards every
        running sequence's tokens are on the host."""
        cur, self._inflight = self._inflight, None
        if cur is None or not self._settle(cur):
            return []
        return self._complete(cur)

    def run_until_done(self) -> list[TokenEvent]:
        events = []
        while self.has_unfinished():
            events.extend(self.step())
        return events

    def _sample(self, seqs: list[Sequence], logits: torch.Tensor, greedy: torch.Tensor | None = None) -> list[int]:
        """Greedy ids for every row (``greedy`` if the caller has them already), then temperature /
        top-k draws for the sampled rows (tokquay/engine.py:189-194)."""
        if greedy is None:
            greedy = ops.argmax_rows(logits) if logits.is_cuda else logits.argmax(-1)
        tokens = greedy
        sampled = [i for i, s in enumerate(seqs) if s.sampling.temperature > 0]
        if sampled:
            tokens = greedy.clone()
            for i in sampled:
                tokens[i] = sample_token(logits[i], seqs[i].sampling, self._rngs[seqs[i].seq_id])
        return tokens.tolist()  # the step's single device-to-host sync
