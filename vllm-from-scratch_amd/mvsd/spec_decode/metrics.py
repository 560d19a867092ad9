"""Per-step acceptance statistics (minivllm/spec_decode/metrics.py:30-63)."""

from __future__ import annotations

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
