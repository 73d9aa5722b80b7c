"""FCFS continuous-batching scheduler (policies of tokquay/scheduler.py:1-31).

* Alternating, prefill-priority steps: if a waiting request can be admitted the
  step prefills only the newly admitted requests, otherwise it decodes every
  running sequence.
* FCFS admission with no skipping: admission stops at the first waiting request
  that does not fit (sequence cap, padded-token budget, or blocks + watermark).
* Preemption by recompute: when a decode step cannot grow some sequence's block
  table, the newest running sequence is evicted and requeued at the front.
* Up-front rejection of requests whose worst case can never fit.
* Watermark: while others run, admission keeps ``watermark_blocks`` free.

The scheduler grows block tables before the forward, which fixes the block
tables the paged-attention kernels read.

``chunked_prefill=True`` replaces the alternation with mixed steps (not in the
reference, whose batches are padded): every running sequence that is decoding
feeds its one token, and the remaining per-step budget - counted in real tokens,
since the packed batch has no padding - goes to prefills in chunks of at most
``prefill_chunk_tokens``: first the sequences already part-way through their
prompt (oldest first), then new admissions (FCFS, same block and watermark
rules). A prompt longer than the budget is then admissible: it is simply fed
over several steps. Preemption is unchanged (newest first, recompute).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.sequence import Sequence, SequenceStatus


class RequestRejected(ValueError):
    """The request can never be served by this engine configuration."""


@dataclass
class SchedulerConfig:
    max_num_seqs: int = 64
    # Per-step budget in padded tokens (batch size x longest row), as in the reference.
    max_num_batched_tokens: int = 2048
    max_model_len: int = 1024
    watermark_blocks: int = 1
    chunked_prefill: bool = False  # mixed prefill + decode steps with chunked prompts
    prefill_chunk_tokens: int = 256  # most prompt tokens one sequence feeds per step (chunked mode)

    def __post_init__(self) -> None:
        if self.prefill_chunk_tokens < 1:
            raise ValueError("prefill_chunk_tokens must be >= 1")
        if self.max_num_seqs < 1 or self.max_num_batched_tokens < self.max_num_seqs:
            raise ValueError("need max_num_seqs >= 1 and max_num_batched_tokens >= max_num_seqs")


@dataclass
class ScheduledBatch:
    seqs: list[Sequence]
    is_prefill: bool  # the step feeds prompt tokens (alone, or next to decode rows in chunked mode)
    preempted: list[Sequence] = field(default_factory=list)
    new_lens: list[int] | None = None  # tokens each sequence feeds (None: all its uncached tokens)
    padded_tokens: int = field(init=False)

    def __post_init__(self) -> None:
        if self.new_lens is None:
            self.padded_tokens = len(self.seqs) * max(s.num_uncached_tokens for s in self.seqs)
        else:
            self.padded_tokens = sum(self.new_lens)  # packed rows: nothing is padded


class Scheduler:
    def __init__(self, allocator: BlockAllocator, config: SchedulerConfig | None = None):
        self.allocator = allocator
        self.config = config or SchedulerConfig()
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []  # admission order; the last one is the newest
        self.num_preemptions = 0
        self.num_discarded_positions = 0

    # ---- requests ------------------------------------------------------------------
    def max_context(self, seq: Sequence) -> int:
        """Most positions the sequence will ever cache (its last token never needs K/V)."""
        return len(seq.prompt_token_ids) + seq.sampling.max_tokens - 1

    def rejection_reason(self, seq: Sequence) -> str | None:
        ctx, cfg = self.max_context(seq), self.config
        if ctx > cfg.max_model_len:
            return f"prompt + max_tokens needs {ctx} positions but the model supports {cfg.max_model_len}"
        blocks = self.allocator.blocks_needed(ctx)
        if blocks > self.allocator.num_blocks:
            return f"needs {blocks} KV blocks but the pool only has {self.allocator.num_blocks}"
        if ctx > cfg.max_num_batched_tokens and not cfg.chunked_prefill:
            return f"needs {ctx} tokens in one step but max_num_batched_tokens is {cfg.max_num_batched_tokens}"
        return None

    def add_request(self, seq: Sequence) -> None:
        reason = self.rejection_reason(seq)
        if reason:
            raise RequestRejected(reason)
        seq.status = SequenceStatus.WAITING
        self.waiting.append(seq)

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running)

    def finish(self, seq: Sequence, reason: str) -> None:
        self.running.remove(seq)
        self.allocator.free(seq)
        seq.status = SequenceStatus.FINISHED
        seq.finish_reason = reason

    def abort(self, seq: Sequence) -> None:
        """Drop a request wherever it is; a no-op once it has finished."""
        if seq.status is SequenceStatus.FINISHED:
            return
        if seq in self.running:
            self.running.remove(seq)
        else:
            self.waiting.remove(seq)
        self.allocator.free(seq)
        seq.status = SequenceStatus.FINISHED
        seq.finish_reason = "abort"

    # ---- one decision --------------------------------------------------------------
    def schedule(self) -> ScheduledBatch | None:
        if self.config.chunked_prefill:
            return self._schedule_chunked()
        if self.waiting:
            admitted = self._admit()
            if admitted:
                self.running.extend(admitted)
                return ScheduledBatch(admitted, is_prefill=True)
        if not self.running:
            return None
        return self._schedule_decode()

    def _admit(self) -> list[Sequence]:
        cfg, alloc = self.config, self.allocator
        admitted: list[Sequence] = []
        longest = 0
        while self.waiting and len(self.running) + len(admitted) < cfg.max_num_seqs:
            seq = self.waiting[0]
            n = seq.num_tokens  # all uncached: prompt (+ output when recomputing)
            if (len(admitted) + 1) * max(longest, n) > cfg.max_num_batched_tokens:
                break
            reserve = cfg.watermark_blocks if (self.running or admitted) else 0
            if alloc.blocks_needed(n) + reserve > alloc.num_free_blocks:
                break  # never skip the head of the queue
            self.waiting.popleft()
            alloc.allocate(seq)
            seq.status = SequenceStatus.RUNNING
            longest = max(longest, n)
            admitted.append(seq)
        return admitted

    def _schedule_decode(self) -> ScheduledBatch:
        alloc, running = self.allocator, self.running
        preempted: list[Sequence] = []
        i = 0
        while i < len(running):
            seq = running[i]
            evicted_self = False
            while not alloc.can_append_slot(seq):
                victim = running.pop()  # newest; may be `seq` itself
                self._preempt(victim)
                preempted.append(victim)
                if victim is seq:
                    evicted_self = True
                    break
            if not evicted_self:
                alloc.append_slot(seq)
                i += 1
        # The oldest sequence is only evicted when alone, and then the whole pool is free
        # for it (rejection guarantees it fits), so the batch cannot be empty.
        assert running, "scheduler evicted every running sequence"
        return ScheduledBatch(list(running), is_prefill=False, preempted=preempted)

    def _grow_decoders(self, decoders: list[Sequence]) -> list[Sequence]:
        """Make room for each decoding sequence's next token, evicting the newest running sequences
        (decoding or part-way through their prompt) when the pool is exhausted."""
        alloc, running = self.allocator, self.running
        preempted: list[Sequence] = []
        for seq in decoders:
            if seq not in running:
                continue  # evicted while making room for an older one
            while not alloc.can_append_slot(seq):
                victim = running.pop()
                self._preempt(victim)
                preempted.append(victim)
                if victim is seq:
                    break
            else:
                alloc.append_slot(seq)
        return preempted

    def _schedule_chunked(self) -> ScheduledBatch | None:
        cfg, alloc = self.config, self.allocator
        decoders = [s for s in self.running if s.num_uncached_tokens == 1 and s.num_cached_tokens > 0]
        preempted = self._grow_decoders(decoders)
        decoders = [s for s in decoders if s in self.running]
        budget = cfg.max_num_batched_tokens - len(decoders)
        chunks: list[tuple[Sequence, int]] = []
        # Sequences part-way through their prompt (or recompute), oldest first.
        for seq in self.running:
            if budget <= 0:
                break
            if seq in decoders:
                continue
            n = min(seq.num_uncached_tokens, cfg.prefill_chunk_tokens, budget)
            chunks.append((seq, n))
            budget -= n
        # New admissions, FCFS: blocks for the whole prompt are taken at admission.
        while self.waiting and budget > 0 and len(self.running) < cfg.max_num_seqs:
            seq = self.waiting[0]
            reserve = cfg.watermark_blocks if self.running else 0
            if alloc.blocks_needed(seq.num_tokens) + reserve > alloc.num_free_blocks:
                break
            self.waiting.popleft()
            alloc.allocate(seq)
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
            n = min(seq.num_uncached_tokens, cfg.prefill_chunk_tokens, budget)
            chunks.append((seq, n))
            budget -= n
        if not decoders and not chunks:
            return None
        order = {id(s): i for i, s in enumerate(self.running)}  # keep admission order in the batch
        rows = sorted([(s, 1) for s in decoders] + chunks, key=lambda sn: order[id(sn[0])])
        return ScheduledBatch([s for s, _ in rows], is_prefill=bool(chunks), preempted=preempted,
                              new_lens=[n for _, n in rows])  # fmt: skip

    def _preempt(self, seq: Sequence) -> None:
        self.num_discarded_positions += seq.num_cached_tokens
        self.allocator.free(seq)
        seq.reset_for_recompute()
        self.waiting.appendleft(seq)
        self.num_preemptions += 1
