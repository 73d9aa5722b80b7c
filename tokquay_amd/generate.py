"""Step drivers over the paged pool.

``paged_forward`` is one batched model step (tokquay/generate.py:63-87): build
the step view, right-pad the new ids, run the model, advance
``num_cached_tokens``. ``paged_greedy_generate`` is the scheduler-free driver
of tokquay/generate.py:90-120: prefill all prompts in one batch, decode them
together, free each sequence the moment it has ``max_new_tokens`` tokens.
"""

from __future__ import annotations

import torch

from tokquay_amd.kv_cache import BlockAllocator
from tokquay_amd.model import GPT2
from tokquay_amd.sequence import Sequence, SequenceStatus


@torch.no_grad()
def paged_forward(
    model: GPT2,
    allocator: BlockAllocator,
    seqs: list[Sequence],
    new_lens: list[int] | None = None,
) -> torch.Tensor:
    """One step; returns next-token logits ``[B, vocab]`` and advances each sequence's cache."""
    lens = new_lens or [s.num_uncached_tokens for s in seqs]
    batch = allocator.batch_for(seqs, lens)
    rows = []
    for s, n in zip(seqs, lens):
        row = s.token_ids[s.num_cached_tokens : s.num_cached_tokens + n]
        rows.append(row + [0] * (batch.T - n))
    ids = torch.tensor(rows, dtype=torch.long, pin_memory=allocator.pool.is_cuda).to(
        allocator.pool.device, non_blocking=True
    )
    logits = model(ids, batch, last_only=True)[:, 0]
    for s, n in zip(seqs, lens):
        s.num_cached_tokens += n
    return logits


@torch.no_grad()
def paged_greedy_generate(
    model: GPT2,
    allocator: BlockAllocator,
    prompts: list[list[int]],
    max_new_tokens: int,
) -> list[list[int]]:
    seqs = [Sequence(i, list(p)) for i, p in enumerate(prompts)]
    for s in seqs:
        allocator.allocate(s)
        s.status = SequenceStatus.RUNNING
    running = seqs
    while running:
        next_ids = paged_forward(model, allocator, running).argmax(-1).tolist()
        still = []
        for s, t in zip(running, next_ids):
            s.append_token(t)
            if len(s.output_token_ids) >= max_new_tokens:
                allocator.free(s)
                s.status = SequenceStatus.FINISHED
            else:
                allocator.append_slot(s)  # room for the token just sampled
                still.append(s)
        running = still
    return [s.output_token_ids for s in seqs]
