"""Open-loop serving driver and the serving metrics computed from what it logged.

Metric definitions follow the reference's benchmark harness (bench/harness.py:54-177),
so that ITL, TTFT and throughput mean the same thing here:

* requests arrive when the workload says, whether or not the system keeps up;
  latencies count from the scheduled arrival;
* a token is stamped when the ``step()`` that produced it returns (a step ends
  with the engine's one device-to-host sync);
* inter-token latency pools the gaps between consecutive tokens of every request;
* percentiles are numpy's linear interpolation.

How it is organised: ``TraceDriver`` appends one row per step to a step log and
one row per emitted token (request index, step index, token id) to a token log.
Times live on the step log only, since a token's time is its step's end. Every
metric is computed afterwards from those columns with numpy: per-request token
times by a stable sort on the request column, prefill stalls by prefix sums over
the step log.
"""

from __future__ import annotations

import math
import time
from dataclasses import asdict, dataclass, field

import numpy as np

from tokquay_amd.sequence import SamplingParams
from tokquay_amd.workload import RequestSpec

# Step-log columns: the order of each TraceLog.steps tuple.
STEP_FIELDS = ("t_start", "t_end", "is_prefill", "num_seqs", "padded_tokens", "kv_allocated_tokens",
               "kv_live_tokens", "kv_num_seqs")  # fmt: skip


@dataclass
class TraceLog:
    """Everything one run produced. Requests are indexed by their position in the workload."""

    arrivals: list[float] = field(default_factory=list)
    prompt_lens: list[int] = field(default_factory=list)
    output_lens: list[int] = field(default_factory=list)
    steps: list[tuple] = field(default_factory=list)  # one STEP_FIELDS tuple per step
    token_request: list[int] = field(default_factory=list)
    token_step: list[int] = field(default_factory=list)
    token_ids: list[int] = field(default_factory=list)
    stats: dict = field(default_factory=dict)  # the system's own counters at the end
    wall_s: float = 0.0

    def step_column(self, name: str) -> np.ndarray:
        i = STEP_FIELDS.index(name)
        return np.array([row[i] for row in self.steps], dtype=float)

    def token_times(self) -> np.ndarray:
        """Time of every logged token (its step's end), in log order."""
        ends = self.step_column("t_end")
        return ends[np.asarray(self.token_step, dtype=np.int64)] if self.token_step else np.zeros(0)

    def by_request(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """(request index, time, log position) of every token, grouped by request, each request's
        tokens in order."""
        req = np.asarray(self.token_request, dtype=np.int64)
        order = np.argsort(req, kind="stable")  # the log is in time order, so this keeps it per request
        return req[order], self.token_times()[order], order

    def request_token_times(self, r: int) -> list[float]:
        req, times, _ = self.by_request()
        return times[req == r].tolist()

    def request_token_ids(self, r: int) -> list[int]:
        req = np.asarray(self.token_request, dtype=np.int64)
        ids = np.asarray(self.token_ids, dtype=np.int64)
        return ids[req == r].tolist()


class TraceDriver:
    """Feeds a workload to anything with the engine interface (``add_request``, ``step``,
    ``has_unfinished``, ``last_step``, ``stats``) in real time, on ``clock``."""

    def __init__(self, system, workload: list[RequestSpec], *, clock=time.perf_counter, sleep=time.sleep,
                 idle_quantum: float = 0.005, time_limit: float | None = None):  # fmt: skip
        self.system, self.workload = system, workload
        self.clock, self.sleep, self.idle_quantum = clock, sleep, idle_quantum
        self.time_limit = math.inf if time_limit is None else time_limit
        self.log = TraceLog()
        self._next = 0  # first request not yet handed to the system
        self._request_of: dict[int, int] = {}  # the system's seq_id -> request index

    def _hand_over_arrivals(self, now: float) -> None:
        while self._next < len(self.workload) and self.workload[self._next].arrival <= now:
            spec = self.workload[self._next]
            seq = self.system.add_request(list(spec.prompt_ids),
                                          SamplingParams(max_tokens=spec.output_len, ignore_eos=True))  # fmt: skip
            self._request_of[seq.seq_id] = self._next
            self.log.arrivals.append(spec.arrival)
            self.log.prompt_lens.append(len(spec.prompt_ids))
            self.log.output_lens.append(spec.output_len)
            self._next += 1

    def _run_one_step(self, t0: float) -> None:
        t_start = self.clock() - t0
        events = self.system.step()
        t_end = self.clock() - t0
        info = self.system.last_step
        if info is None:
            raise RuntimeError("the system has unfinished requests but nothing it can run (deadlock)")
        step_index = len(self.log.steps)
        self.log.steps.append((t_start, t_end, info.is_prefill, info.num_seqs, info.padded_tokens,
                               info.kv.allocated_tokens, info.kv.live_tokens, info.kv.num_seqs))  # fmt: skip
        for ev in events:
            self.log.token_request.append(self._request_of[ev.seq_id])
            self.log.token_step.append(step_index)
            self.log.token_ids.append(ev.token_id)

    def run(self) -> TraceLog:
        t0 = self.clock()
        while True:
            now = self.clock() - t0
            if now > self.time_limit:
                break
            self._hand_over_arrivals(now)
            busy = self.system.has_unfinished()
            if busy:
                self._run_one_step(t0)
            elif self._next < len(self.workload):  # idle until the next arrival, in small naps
                self.sleep(max(0.0, min(self.workload[self._next].arrival - now, self.idle_quantum)))
            else:
                break
        self.log.stats = asdict(self.system.stats)
        self.log.wall_s = self.clock() - t0
        return self.log


def run_trace(system, workload: list[RequestSpec], **kwargs) -> TraceLog:
    """Drive ``system`` through ``workload`` in real time (see ``TraceDriver`` for the keywords;
    ``time_limit`` in seconds stops admitting and stepping once exceeded)."""
    return TraceDriver(system, workload, **kwargs).run()


# ------------------------------------------------------------------------------ metrics
def percentiles(values, qs=(50, 99)) -> dict[str, float]:
    """p50 / p99 (numpy linear interpolation) and the mean; NaN for no values."""
    arr = np.asarray(values, dtype=float)
    if arr.size == 0:
        return dict({f"p{q}": math.nan for q in qs}, mean=math.nan)
    return dict({f"p{q}": float(np.percentile(arr, q)) for q in qs}, mean=float(arr.mean()))


def _ms(stats: dict[str, float]) -> dict[str, float]:
    return {k: 1e3 * v for k, v in stats.items()}


def token_gaps(log: TraceLog) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Every gap between two consecutive tokens of one request, as (first token's step, second
    token's step, length in seconds) arrays."""
    req, times, order = log.by_request()
    steps = np.asarray(log.token_step, dtype=np.int64)[order]
    same = req[1:] == req[:-1]
    return steps[:-1][same], steps[1:][same], (times[1:] - times[:-1])[same]


def prefill_stall_analysis(log: TraceLog) -> dict:
    """Split token gaps by whether a prefill step ran inside them, and fit prefill step time against
    the tokens it fed. Steps run one after another, so the steps that end inside the gap between
    tokens of steps i < j are exactly steps i+1 .. j: a gap is stalled when that range holds a
    prefill step (a prefix sum over the step log)."""
    prefill = log.step_column("is_prefill").astype(bool)
    out: dict = {"num_prefill_steps": int(prefill.sum()), "num_decode_steps": int((~prefill).sum())}
    first, second, gap = token_gaps(log)
    if gap.size:
        ran_before = np.concatenate(([0], np.cumsum(prefill)))  # prefill steps among steps 0 .. k-1
        stalled = ran_before[second + 1] - ran_before[first + 1] > 0
        out["frac_gaps_stalled_by_prefill"] = float(stalled.mean())
        out["itl_ms_clean"] = _ms(percentiles(gap[~stalled]))
        out["itl_ms_stalled"] = _ms(percentiles(gap[stalled]))
    durations = log.step_column("t_end") - log.step_column("t_start")
    if (~prefill).any():
        out["decode_step_ms"] = _ms(percentiles(durations[~prefill]))
    tokens = log.step_column("padded_tokens")[prefill]
    if tokens.size >= 2 and np.unique(tokens).size >= 2:
        ms = durations[prefill] * 1e3
        design = np.stack([tokens, np.ones_like(tokens)], axis=1)
        (per_token, fixed), *_ = np.linalg.lstsq(design, ms, rcond=None)
        out["prefill_ms_per_padded_token"] = float(per_token)
        out["prefill_ms_fixed"] = float(fixed)
        out["prefill_step_ms"] = percentiles(ms)
        out["prefill_padded_tokens"] = percentiles(tokens)
        out["prefill_max_step_ms"] = float(ms.max())
    return out


def summarize(log: TraceLog, bytes_per_token: int) -> dict:
    """The serving metrics of one run: times in ms, KV memory in MiB (``bytes_per_token`` is one
    cache slot across all layers)."""
    req, times, _ = log.by_request()
    arrivals = np.asarray(log.arrivals, dtype=float)
    served = np.unique(req)
    first_at = np.searchsorted(req, served, side="left")
    last_at = np.searchsorted(req, served, side="right") - 1
    ttft = (times[first_at] - arrivals[served]) * 1e3
    latency = (times[last_at] - arrivals[served]) * 1e3
    span = times.max() - arrivals.min() if times.size else math.nan
    allocated = log.step_column("kv_allocated_tokens")
    live = log.step_column("kv_live_tokens")
    mib = bytes_per_token / 2**20
    return {
        "requests": len(log.arrivals),
        "output_tokens": int(times.size),
        "duration_s": float(span),
        "throughput_tok_s": float(times.size / span),
        "ttft_ms": percentiles(ttft),
        "itl_ms": _ms(percentiles(token_gaps(log)[2])),
        "latency_ms": percentiles(latency),
        "peak_kv_allocated_mib": float(allocated.max() * mib) if allocated.size else 0.0,
        "peak_kv_live_mib": float(live.max() * mib) if live.size else 0.0,
        "kv_utilization": float(live.sum() / allocated.sum()) if allocated.sum() else math.nan,
        "max_concurrent": int(log.step_column("kv_num_seqs").max()) if log.steps else 0,
        "steps": len(log.steps),
        "stats": log.stats,
        "stalls": prefill_stall_analysis(log),
    }
