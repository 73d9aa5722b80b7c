"""Per-request state shared by the allocator, scheduler and engine.

Same fields and meaning as the reference's ``Sequence`` / ``SamplingParams``
(tokquay/sequence.py:15-81): ``num_cached_tokens`` leading positions already
have K/V in the pool, so the next step feeds ``token_ids[num_cached_tokens:]``
(a whole prompt for prefill, one token for decode, prompt + output after a
preemption by recompute).
"""

from __future__ import annotations

import enum
from dataclasses import dataclass, field


class SequenceStatus(enum.Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


@dataclass(frozen=True)
class SamplingParams:
    """``temperature == 0`` is greedy; ``top_k == 0`` disables top-k (tokquay/sequence.py:15-31)."""

    max_tokens: int = 16
    temperature: float = 0.0
    top_k: int = 0
    ignore_eos: bool = False
    seed: int | None = None

    def __post_init__(self) -> None:
        if self.max_tokens < 1:
            raise ValueError("max_tokens must be >= 1")
        if self.temperature < 0:
            raise ValueError("temperature must be >= 0")
        if self.top_k < 0:
            raise ValueError("top_k must be >= 0")


@dataclass
class Sequence:
    seq_id: int
    prompt_token_ids: list[int]
    output_token_ids: list[int] = field(default_factory=list)
    block_table: list[int] = field(default_factory=list)  # block_table[i] holds positions [i*bs, (i+1)*bs)
    status: SequenceStatus = SequenceStatus.WAITING
    num_cached_tokens: int = 0
    sampling: SamplingParams = field(default_factory=SamplingParams)
    finish_reason: str | None = None  # "length", "stop" or "abort"

    def __post_init__(self) -> None:
        if not self.prompt_token_ids:
            raise ValueError("prompt must contain at least one token")

    @property
    def token_ids(self) -> list[int]:
        return self.prompt_token_ids + self.output_token_ids

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    @property
    def num_uncached_tokens(self) -> int:
        return self.num_tokens - self.num_cached_tokens

    def append_token(self, token_id: int) -> None:
        self.output_token_ids.append(token_id)

    def reset_for_recompute(self) -> None:
        """Forget the cache state once the allocator freed our blocks (preemption)."""
        self.block_table = []
        self.num_cached_tokens = 0
        self.status = SequenceStatus.WAITING
