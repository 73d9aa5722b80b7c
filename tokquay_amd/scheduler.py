"""Continuous-batching scheduler: which sequences run in the next step, and with how many tokens.

Policies are the reference's (tokquay/scheduler.py:1-31), because they decide
which block tables the paged-attention kernels read and the reference's tests
pin them:

* first come, first served, and never past the head of the queue: admission
  stops at the first waiting request that does not fit;
* the default step kind alternates: a step that can admit someone prefills only
  the newly admitted requests, any other step decodes every running sequence;
* a step's budget counts padded tokens (rows x longest row);
* when the pool cannot give a running sequence its next slot, the newest running
  sequence is evicted, forgets its cache and goes back to the front of the queue
  (recomputed later, prompt + output);
* while others run, admission keeps ``watermark_blocks`` blocks free;
* a request whose worst case can never fit is refused at ``add_request``.

How the decisions are organised here:

* one admission routine for both step kinds (``_take_from_queue``): the caller
  passes the token-budget test and how many tokens a new row feeds;
* one growth routine (``_make_room``): every decoding sequence, oldest first,
  gets its next slot, evicting from the newest end of ``running`` until it fits;
* ``running`` is always in admission order, so "newest" is its last element.

``chunked_prefill=True`` (not in the reference, whose rows are padded so it
cannot mix) builds mixed steps: every decoding sequence feeds one token and the
rest of the budget - real tokens, as the packed batch has no padding - goes to
prompts in chunks of at most ``prefill_chunk_tokens``, sequences part-way
through their prompt first (oldest first), then admissions from the queue.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Callable

from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.sequence import Sequence, SequenceStatus


class RequestRejected(ValueError):
    """The request can never be served by this engine configuration."""


@dataclass
class SchedulerConfig:
    max_num_seqs: int = 64
    # Token budget per step: padded tokens (rows x longest row) in the alternating mode, real tokens
    # in the chunked mode.
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
        # Fixed now: the sequences' uncached counts change once the step has run.
        if self.new_lens is not None:
            self.padded_tokens = sum(self.new_lens)  # packed rows: nothing is padded
        else:
            widest = max(s.num_uncached_tokens for s in self.seqs)
            self.padded_tokens = widest * len(self.seqs)


class Scheduler:
    def __init__(self, allocator: BlockAllocator, config: SchedulerConfig | None = None):
        self.allocator = allocator
        self.config = config or SchedulerConfig()
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []  # admission order: running[-1] is the newest
        self.num_preemptions = 0
        self.num_discarded_positions = 0  # cached positions thrown away by evictions

    # ---- requests ------------------------------------------------------------------
    def max_context(self, seq: Sequence) -> int:
        """Positions the sequence can ever hold in the pool: the token sampled last is returned,
        never fed, so it needs no K/V."""
        return seq.sampling.max_tokens + len(seq.prompt_token_ids) - 1

    def rejection_reason(self, seq: Sequence) -> str | None:
        """Why ``seq`` can never run here, or None. Checked in this order: model window, pool size,
        then (alternating mode, where a recomputed sequence must be re-fed in one step) the budget."""
        cfg, ctx = self.config, self.max_context(seq)
        blocks = self.allocator.blocks_needed(ctx)
        problems = (
            (ctx > cfg.max_model_len,
             f"prompt + max_tokens needs {ctx} positions but the model supports {cfg.max_model_len}"),
            (blocks > self.allocator.num_blocks,
             f"needs {blocks} KV blocks but the pool only has {self.allocator.num_blocks}"),
            (not cfg.chunked_prefill and ctx > cfg.max_num_batched_tokens,
             f"needs {ctx} tokens in one step but max_num_batched_tokens is {cfg.max_num_batched_tokens}"),
        )  # fmt: skip
        return next((msg for bad, msg in problems if bad), None)

    def add_request(self, seq: Sequence) -> None:
        reason = self.rejection_reason(seq)
        if reason is not None:
            raise RequestRejected(reason)
        seq.status = SequenceStatus.WAITING
        self.waiting.append(seq)

    def has_unfinished(self) -> bool:
        return len(self.waiting) + len(self.running) > 0

    def _retire(self, seq: Sequence, reason: str) -> None:
        self.allocator.free(seq)  # a queued sequence holds no blocks: a no-op then
        seq.status = SequenceStatus.FINISHED
        seq.finish_reason = reason

    def finish(self, seq: Sequence, reason: str) -> None:
        self.running.remove(seq)
        self._retire(seq, reason)

    def abort(self, seq: Sequence) -> None:
        """Drop a request wherever it is (queued, requeued after an eviction, running); a no-op once
        it has finished."""
        if seq.status is SequenceStatus.FINISHED:
            return
        (self.running if seq in self.running else self.waiting).remove(seq)
        self._retire(seq, "abort")

    # ---- building blocks -------------------------------------------------------------
    def _evict_newest(self) -> Sequence:
        victim = self.running.pop()
        self.num_discarded_positions += victim.num_cached_tokens
        self.allocator.free(victim)
        victim.reset_for_recompute()  # status WAITING, no blocks, nothing cached; outputs kept
        self.waiting.appendleft(victim)  # ahead of later arrivals: arrival order is kept
        self.num_preemptions += 1
        return victim

    def _make_room(self, decoders: list[Sequence]) -> list[Sequence]:
        """Give each sequence in ``decoders`` (oldest first) the slot its next token needs. When the
        pool is short, evict from the newest end of ``running`` - possibly the sequence itself - until
        it fits. Returns the evicted sequences in eviction order."""
        alloc = self.allocator
        evicted: list[Sequence] = []
        for seq in decoders:
            while seq.status is SequenceStatus.RUNNING and not alloc.can_append_slot(seq):
                evicted.append(self._evict_newest())
            if seq.status is SequenceStatus.RUNNING:
                alloc.append_slot(seq)
        return evicted

    def _take_from_queue(self, fits_budget: Callable[[Sequence], bool], on_admit: Callable[[Sequence], None]) -> None:
        """Admit queue heads while the sequence cap, ``fits_budget(head)`` and the free blocks (less
        the watermark while anyone else holds blocks) allow; stop at the first head that does not fit.
        An admitted sequence gets blocks for all its tokens and joins ``running``."""
        cfg, alloc = self.config, self.allocator
        while self.waiting and len(self.running) < cfg.max_num_seqs:
            head = self.waiting[0]
            if not fits_budget(head):
                return
            keep_free = cfg.watermark_blocks if self.running else 0
            if alloc.num_free_blocks - keep_free < alloc.blocks_needed(head.num_tokens):
                return
            self.waiting.popleft()
            alloc.allocate(head)
            head.status = SequenceStatus.RUNNING
            self.running.append(head)
            on_admit(head)

    # ---- one decision --------------------------------------------------------------
    def schedule(self) -> ScheduledBatch | None:
        if self.config.chunked_prefill:
            return self._mixed_step()
        admitted = self._prefill_admissions()
        if admitted:
            return ScheduledBatch(admitted, is_prefill=True)
        if not self.running:
            return None
        evicted = self._make_room(list(self.running))
        # Only a lone sequence is ever evicted for its own sake, and then the whole pool is free for
        # it (rejection guarantees it fits), so a decode batch is never empty.
        assert self.running, "scheduler evicted every running sequence"
        return ScheduledBatch(list(self.running), is_prefill=False, preempted=evicted)

    def _prefill_admissions(self) -> list[Sequence]:
        """Alternating mode: the requests a prefill-only step admits (all their uncached tokens:
        prompt, plus outputs after an eviction), within the padded-token budget."""
        admitted: list[Sequence] = []
        widest = [0]

        def fits(head: Sequence) -> bool:
            width = max(widest[0], head.num_tokens)
            return width * (len(admitted) + 1) <= self.config.max_num_batched_tokens

        def admit(head: Sequence) -> None:
            widest[0] = max(widest[0], head.num_tokens)
            admitted.append(head)

        self._take_from_queue(fits, admit)
        return admitted

    def _mixed_step(self) -> ScheduledBatch | None:
        """Chunked mode: every decoding sequence's token, then prompt chunks in the remaining budget."""
        cfg = self.config
        decoders = [s for s in self.running if s.num_cached_tokens > 0 and s.num_uncached_tokens == 1]
        evicted = self._make_room(decoders)
        feeds: dict[int, int] = {id(s): 1 for s in decoders if s.status is SequenceStatus.RUNNING}
        num_decoding = len(feeds)
        room = [cfg.max_num_batched_tokens - num_decoding]

        def chunk(seq: Sequence) -> None:
            n = min(seq.num_uncached_tokens, cfg.prefill_chunk_tokens, room[0])
            feeds[id(seq)] = n
            room[0] -= n

        for seq in list(self.running):  # prompts already part-way through, oldest first
            if room[0] <= 0:
                break
            if id(seq) not in feeds:
                chunk(seq)
        self._take_from_queue(lambda head: room[0] > 0, chunk)
        if not feeds:
            return None
        rows = [s for s in self.running if id(s) in feeds]  # admission order
        return ScheduledBatch(rows, is_prefill=len(feeds) > num_decoding, preempted=evicted,
                              new_lens=[feeds[id(s)] for s in rows])  # fmt: skip
