"""Output containers of the verification path (minivllm/outputs.py:97-135, :209-323)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple, Sequence

import numpy as np
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


class LogprobsTensors(NamedTuple):
    """Device logprobs of the output positions (minivllm/outputs.py:209-294): column 0 is the
    sampled token, columns 1..k the top-k; ``selected_token_ranks`` is the sampled token's rank
    in its row's distribution."""

    logprob_token_ids: torch.Tensor     # [num_positions, k + 1] int32
    logprobs: torch.Tensor              # [num_positions, k + 1] fp32
    selected_token_ranks: torch.Tensor  # [num_positions] int32
    cu_num_generated_tokens: list[int] | None = None

    @staticmethod
    def cat(tensors: Sequence["LogprobsTensors"],
            cu_num_generated_tokens: list[int] | None = None) -> "LogprobsTensors":
        assert tensors
        assert cu_num_generated_tokens is not None or all(
            t.cu_num_generated_tokens is None for t in tensors)
        if len(tensors) == 1:
            t = tensors[0]
            return t if cu_num_generated_tokens is None else t._replace(
                cu_num_generated_tokens=cu_num_generated_tokens)
        return LogprobsTensors(torch.cat([t.logprob_token_ids for t in tensors]),
                               torch.cat([t.logprobs for t in tensors]),
                               torch.cat([t.selected_token_ranks for t in tensors]),
                               cu_num_generated_tokens)

    def tolists(self, cu_num_generated_tokens: list[int] | None = None) -> "LogprobsLists":
        return LogprobsLists(self.logprob_token_ids.cpu().numpy(), self.logprobs.cpu().numpy(),
                             self.selected_token_ranks.cpu().numpy(),
                             cu_num_generated_tokens if cu_num_generated_tokens is not None
                             else self.cu_num_generated_tokens)

    def filter(self, mask) -> "LogprobsTensors":
        """Rows where ``mask`` is true (the valid mask of parse_output)."""
        assert self.cu_num_generated_tokens is None, \
            "filter cannot be combined with cu_num_generated_tokens"
        if not isinstance(mask, torch.Tensor):
            mask = torch.as_tensor(np.asarray(mask, dtype=bool))
        mask = mask.to(self.logprobs.device)
        return LogprobsTensors(self.logprob_token_ids[mask], self.logprobs[mask],
                               self.selected_token_ranks[mask])


class LogprobsLists(NamedTuple):
    """Host logprobs (minivllm/outputs.py:297-323); ``cu_num_generated_tokens[i]`` is request
    i's first row."""

    logprob_token_ids: np.ndarray
    logprobs: np.ndarray
    sampled_token_ranks: np.ndarray
    cu_num_generated_tokens: list[int] | None = None

    def slice_request(self, req_idx: int, num_positions: int) -> "LogprobsLists":
        if self.cu_num_generated_tokens is not None:
            req_idx = self.cu_num_generated_tokens[req_idx]
        end_idx = req_idx + num_positions
        return LogprobsLists(self.logprob_token_ids[req_idx:end_idx],
                             self.logprobs[req_idx:end_idx],
                             self.sampled_token_ranks[req_idx:end_idx], None)
