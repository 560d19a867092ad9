"""Output containers of the verification path (minivllm/outputs.py:97-135)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class DraftTokenIds:
    """Next-step drafts handed back to the scheduler (minivllm/outputs.py:97-117).

    ``num_valid_draft_tokens`` is set by fixed-width proposers (``[B, K]`` padded with -1):
    it is the valid prefix length of each row; ``None`` means every listed draft is valid.
    """

    req_ids: list[str]
    draft_token_ids: list[list[int]]
    draft_probs: torch.Tensor | None = None
    num_valid_draft_tokens: list[int] | None = None


@dataclass
class SamplerOutput:
    """Sampled ids ``[B, max_spec_len + 1]`` int32, -1 padded (minivllm/outputs.py:119-135)."""

    sampled_token_ids: torch.Tensor
    logprobs_tensors: object | None = None
