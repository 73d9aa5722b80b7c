"""Seeded serving workload: Poisson arrivals, uniform prompt and output lengths.

Same draws as the reference generator (bench/workload.py:24-47): contents from
``random.Random(seed)`` and unit-rate exponential gaps from
``random.Random(seed + 1_000_003)`` divided by ``rate``, so a seed names the same
requests at every rate. Prompt ids avoid the last vocabulary id (EOS).
"""

from __future__ import annotations

import random
from dataclasses import dataclass

VOCAB_SIZE = 50257


@dataclass(frozen=True)
class RequestSpec:
    arrival: float  # seconds after the start of the run
    prompt_ids: tuple[int, ...]
    output_len: int


def make_workload(
    rate: float,
    n: int,
    seed: int = 0,
    prompt_len: tuple[int, int] = (16, 256),
    output_len: tuple[int, int] = (16, 256),
) -> list[RequestSpec]:
    """``n`` requests arriving as a Poisson process of ``rate`` per second (``inf``: all at t=0)."""
    if rate <= 0 or n < 1:
        raise ValueError("need rate > 0 and n >= 1")
    content, gaps = random.Random(seed), random.Random(seed + 1_000_003)
    t = 0.0
    specs = []
    for _ in range(n):
        t += gaps.expovariate(1.0)
        length = content.randint(*prompt_len)
        prompt = tuple(content.randrange(VOCAB_SIZE - 1) for _ in range(length))
        specs.append(RequestSpec(t / rate, prompt, content.randint(*output_len)))
    return specs
