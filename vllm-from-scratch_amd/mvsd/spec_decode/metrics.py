"""Acceptance statistics: per step (minivllm/spec_decode/metrics.py:30-63) and aggregated
over logging intervals (:66-146)."""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass, field


@dataclass
class SpecDecodingStats:
    num_spec_tokens: int
    num_drafts: int = 0
    num_draft_tokens: int = 0
    num_accepted_tokens: int = 0
    num_accepted_tokens_per_pos: list[int] = field(default_factory=list)
    num_draft_tokens_per_pos: list[int] = field(default_factory=list)

    @classmethod
    def new(cls, num_spec_tokens: int) -> "SpecDecodingStats":
        return cls(num_spec_tokens=num_spec_tokens,
                   num_accepted_tokens_per_pos=[0] * num_spec_tokens,
                   num_draft_tokens_per_pos=[0] * num_spec_tokens)

    def observe_draft(self, num_draft_tokens: int, num_accepted_tokens: int) -> None:
        self.num_drafts += 1
        self.num_draft_tokens += num_draft_tokens
        self.num_accepted_tokens += num_accepted_tokens
        assert num_accepted_tokens <= self.num_spec_tokens
        for i in range(num_accepted_tokens):
            self.num_accepted_tokens_per_pos[i] += 1
        for i in range(num_draft_tokens):
            self.num_draft_tokens_per_pos[i] += 1


def stats_from_outputs(outputs: list[list[int]], num_draft_tokens: list[int],
                       num_spec_tokens: int) -> SpecDecodingStats:
    """Fill a SpecDecodingStats from parsed verification outputs the way the scheduler
    does (minivllm/core/sched/scheduler.py:637-657): a request with K_i > 0 drafts that
    produced n tokens accepted n - 1 of them."""
    stats = SpecDecodingStats.new(num_spec_tokens)
    for tokens, k in zip(outputs, num_draft_tokens):
        if k > 0:
            stats.observe_draft(k, max(len(tokens) - 1, 0))
    return stats


class SpecDecodingLogging:
    """Aggregates per-step SpecDecodingStats between two ``log`` calls
    (minivllm/spec_decode/metrics.py:66-146): ``observe(stats)`` adds one step, ``len()`` is
    the number of steps observed, ``log()`` reports the totals through ``log_fn`` and returns
    them as a dict, then starts a new interval; ``reset()`` starts one without reporting.

    Running totals are kept rather than every step's stats, so a caller that reuses or mutates
    a SpecDecodingStats after observing it does not change what was observed.  The
    per-position totals cover the longest per-position list observed; acceptance rate =
    accepted / drafted tokens, mean acceptance length = 1 + accepted tokens per draft, and the
    throughputs divide by the time since the interval started."""

    def __init__(self, log_fn=None) -> None:
        self._log_fn = log_fn if log_fn is not None else logging.getLogger(__name__).info
        self.reset()

    def reset(self) -> None:
        self._steps = 0
        self._drafts = 0
        self._draft_tokens = 0
        self._accepted = 0
        self._accepted_per_pos: list[int] = []
        self._draft_per_pos: list[int] = []
        self.last_log_time = time.monotonic()

    def observe(self, stats: SpecDecodingStats) -> None:
        self._steps += 1
        self._drafts += stats.num_drafts
        self._draft_tokens += stats.num_draft_tokens
        self._accepted += stats.num_accepted_tokens
        for totals, step in ((self._accepted_per_pos, stats.num_accepted_tokens_per_pos),
                             (self._draft_per_pos, stats.num_draft_tokens_per_pos)):
            if len(step) > len(totals):
                totals.extend([0] * (len(step) - len(totals)))
            for j, n in enumerate(step):
                totals[j] += n

    def __len__(self) -> int:
        return self._steps

    def log(self) -> dict:
        """The interval's totals, also passed to ``log_fn`` as one line; starts a new interval.
        With no step observed, the empty totals are returned and nothing is logged."""
        if self._steps == 0:
            return {"num_drafts": 0, "num_draft_tokens": 0, "num_accepted_tokens": 0,
                    "accepted_tokens_per_pos": [], "draft_tokens_per_pos": [],
                    "acceptance_rate": None, "mean_acceptance_length": None}
        seconds = max(time.monotonic() - self.last_log_time, 1e-12)
        width = max(len(self._accepted_per_pos), len(self._draft_per_pos))
        pad = lambda xs: xs + [0] * (width - len(xs))  # noqa: E731
        rate = self._accepted / self._draft_tokens if self._draft_tokens else None
        mean_len = 1 + self._accepted / self._drafts if self._drafts else None
        totals = {"num_drafts": self._drafts, "num_draft_tokens": self._draft_tokens,
                  "num_accepted_tokens": self._accepted,
                  "accepted_tokens_per_pos": pad(list(self._accepted_per_pos)),
                  "draft_tokens_per_pos": pad(list(self._draft_per_pos)),
                  "acceptance_rate": rate, "mean_acceptance_length": mean_len,
                  "draft_throughput": self._draft_tokens / seconds,
                  "accepted_throughput": self._accepted / seconds}
        self._log_fn(
            "SpecDecoding metrics: Mean acceptance length: %.2f, "
            "Accepted throughput: %.2f tokens/s, Drafted throughput: %.2f tokens/s, "
            "Accepted: %d tokens, Drafted: %d tokens, Avg Draft acceptance rate: %s",
            mean_len if mean_len is not None else float("nan"),
            totals["accepted_throughput"], totals["draft_throughput"], self._accepted,
            self._draft_tokens, "N/A" if rate is None else f"{rate * 100:.1f}%")
        self.reset()
        return totals
