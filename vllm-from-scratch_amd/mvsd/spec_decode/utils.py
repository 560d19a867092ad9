"""Scheduler-side helpers of the ngram path (minivllm/spec_decode/utils.py)."""

from __future__ import annotations

from dataclasses import dataclass

PADDING_SLOT_ID = -1
PADDING_TOKEN_ID = 0


@dataclass(frozen=True)
class TargetRows:
    """One request's target-side facts for this step (minivllm/spec_decode/utils.py:33-59)."""

    req_id: str
    row: int
    start: int
    target_rows: int
    num_rejected: int
    history_end: int
    next_token_id: int
    ready: bool

    @property
    def num_valid(self) -> int:
        return self.target_rows - self.num_rejected


def update_scheduler_for_invalid_drafts(spec_token_ids: list[int],
                                        num_valid_draft_tokens: int | None) -> list[int]:
    """Trim fixed-width drafts to their valid prefix and drop any -1 that remains
    (minivllm/spec_decode/utils.py:403-420)."""
    if num_valid_draft_tokens is None:
        return list(spec_token_ids)
    valid = max(0, min(int(num_valid_draft_tokens), len(spec_token_ids)))
    return [token for token in spec_token_ids[:valid] if token >= 0]


def unconditional_to_conditional_rates(rates: list[float]) -> list[float]:
    """``c_i = p_i / p_{i-1}`` with ``p_{-1} = 1`` and 0 where the denominator is 0
    (minivllm/spec_decode/utils.py:528-545)."""
    out = []
    prev = 1.0
    for rate in rates:
        out.append(rate / prev if prev > 0.0 else 0.0)
        prev = rate
    return out
