"""The committed greedy-id fixture of the 300-request serving workload, and the margin-aware rule
tests use to compare an engine run with it.

Rule: fp32 implementations of the same model disagree in the last bits of their logits (the
oracle's fp32 logits differ from float64 by at most ~3.3e-6 on a 500-token prompt), so a pick whose
top-1 / top-2 gap is smaller than that can legitimately flip. A request must therefore reproduce
every oracle token picked by a gap of at least ``MARGIN_BOUND``; it may diverge only at a token
picked by less, and its later tokens are then not compared (the two histories differ from there on).
"""

from __future__ import annotations

import hashlib
import os

import numpy as np

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config3_greedy.npz")
MARGIN_BOUND = 1e-4  # logit units: ~30x the measured fp32 logit error


def workload_sha256(workload) -> str:
    """Hash of a workload's (arrival, prompt, output length) triples."""
    h = hashlib.sha256()
    for spec in workload:
        h.update(repr((round(spec.arrival, 9), spec.prompt_ids, spec.output_len)).encode())
    return h.hexdigest()


class GoldenIds:
    def __init__(self, path: str = FIXTURE):
        with np.load(path) as z:  # allow_pickle is False by default: the file holds arrays only
            self.ids = z["ids"].astype(np.int64)
            self.offsets = z["offsets"]
            self.near_index = z["near_tie_index"]
            self.near_margin = z["near_tie_margin"].astype(np.float64)
            self.stored_below = float(z["near_tie_stored_below"])
            self.min_margin = float(z["min_margin"])
            self.workload_sha256 = str(z["workload_sha256"])
        self._near = dict(zip(self.near_index.tolist(), self.near_margin.tolist()))

    @property
    def num_requests(self) -> int:
        return self.offsets.size - 1

    def request(self, r: int) -> list[int]:
        return self.ids[self.offsets[r] : self.offsets[r + 1]].tolist()

    def margin(self, r: int, i: int) -> float:
        """The oracle's top-1 / top-2 gap at token ``i`` of request ``r`` (a lower bound,
        ``near_tie_stored_below``, when the fixture did not store it)."""
        return self._near.get(int(self.offsets[r]) + i, self.stored_below)

    def compare(self, outputs: list[list[int]], bound: float = MARGIN_BOUND) -> dict:
        """Check ``outputs[r]`` (an engine's ids for request r) against the fixture with the
        margin rule. Returns counts; ``violations`` lists (request, token, got, want, margin) of
        mismatches the rule does not allow, plus wrong lengths."""
        assert len(outputs) == self.num_requests
        violations, near_tie_divergences, compared = [], [], 0
        for r, got in enumerate(outputs):
            want = self.request(r)
            if len(got) != len(want):
                violations.append((r, None, len(got), len(want), None))
                continue
            for i, (a, b) in enumerate(zip(got, want)):
                compared += 1
                if a == b:
                    continue
                m = self.margin(r, i)
                (near_tie_divergences if m < bound else violations).append((r, i, a, b, m))
                break
        return {
            "requests": len(outputs),
            "tokens_compared": compared,
            "tokens_total": int(self.ids.size),
            "near_tie_divergences": near_tie_divergences,
            "violations": violations,
        }
