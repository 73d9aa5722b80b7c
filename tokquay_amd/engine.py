"""One continuous-batching iteration per ``step()`` (tokquay/engine.py:95-197).

schedule -> ``paged_forward`` (gfx950 attention) -> batched greedy argmax, plus
per-row temperature / top-k sampling -> one device-to-host sync -> append and
stop checks. Synchronous and not thread safe: one thread drives it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from tokquay_amd.generate import paged_forward
from tokquay_amd.graphs import DecodeGraphs
from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2
from tokquay_amd.scheduler import Scheduler, SchedulerConfig
from tokquay_amd.sequence import SamplingParams, Sequence

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
    ):
        """``use_graphs`` (default: on when the pool is on a HIP device) replays decode steps
        from captured HIP graphs; prefill and mixed steps always run eagerly."""
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
        return self.scheduler.has_unfinished()

    def kv_snapshot(self) -> KVSnapshot:
        running = self.scheduler.running
        return KVSnapshot(
            allocated_tokens=self.allocator.num_used_blocks * self.allocator.block_size,
            live_tokens=sum(s.num_cached_tokens for s in running),
            num_seqs=len(running),
        )

    @torch.no_grad()
    def step(self) -> list[TokenEvent]:
        batch = self.scheduler.schedule()
        if batch is None:
            self.last_step = None
            return []
        st = self.stats
        st.steps += 1
        st.prefill_steps += batch.is_prefill
        st.decode_steps += not batch.is_prefill
        st.max_batch = max(st.max_batch, len(batch.seqs))
        st.peak_used_blocks = max(st.peak_used_blocks, self.allocator.num_used_blocks)
        st.num_preemptions = self.scheduler.num_preemptions
        st.positions_discarded = self.scheduler.num_discarded_positions
        fed = batch.new_lens or [s.num_uncached_tokens for s in batch.seqs]
        st.positions_computed += sum(fed)
        st.positions_padded += batch.padded_tokens

        if self.graphs is not None and not batch.is_prefill:
            logits = self.graphs.forward(batch.seqs)
        else:
            logits = paged_forward(self.model, self.allocator, batch.seqs, batch.new_lens)
        self.last_step = StepInfo(batch.is_prefill, len(batch.seqs), batch.padded_tokens, self.kv_snapshot())
        # A sequence samples once all its tokens are cached; a chunked prompt part-way through does not.
        done = [i for i, s in enumerate(batch.seqs) if s.num_cached_tokens == s.num_tokens]
        if len(done) < len(batch.seqs):
            logits = logits[done]
        seqs = [batch.seqs[i] for i in done]
        tokens = self._sample(seqs, logits) if seqs else []

        events = []
        for seq, tok in zip(seqs, tokens):
            seq.append_token(tok)
            reason = finish_reason_for(seq, tok, self.eos_token_id)
            if reason:
                self.scheduler.finish(seq, reason)
                self._rngs.pop(seq.seq_id, None)
            events.append(TokenEvent(seq.seq_id, tok, reason))
        st.tokens_generated += len(events)
        return events

    def run_until_done(self) -> list[TokenEvent]:
        events = []
        while self.has_unfinished():
            events.extend(self.step())
        return events

    def _sample(self, seqs: list[Sequence], logits: torch.Tensor) -> list[int]:
        tokens = logits.argmax(-1)
        for i, s in enumerate(seqs):
            if s.sampling.temperature > 0:
                tokens[i] = sample_token(logits[i], s.sampling, self._rngs[s.seq_id])
        return tokens.tolist()  # the step's single device-to-host sync
