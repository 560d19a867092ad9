"""Index tensors of one verification step (minivllm/spec_decode/metadata.py:62-81).

All index tensors are int32 device tensors; the cumulative sums carry NO leading 0
(``cu_num_draft_tokens = [3, 3, 5, 5, 6]`` for K = [3, 0, 2, 0, 1]).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class SpecDecodeMetadata:
    draft_token_ids: torch.Tensor          # [P] int32
    num_draft_tokens: list[int]            # [B] host list
    cu_num_draft_tokens: torch.Tensor      # [B] int32, inclusive, no leading 0
    cu_num_sampled_tokens: torch.Tensor    # [B] int32, inclusive sums of K_i + 1
    target_logits_indices: torch.Tensor    # [P] rows of the compact [P+B, V] logits
    bonus_logits_indices: torch.Tensor     # [B]
    logits_indices: torch.Tensor           # [P+B] rows of the forward output

    def __post_init__(self):
        # max over requests; an empty batch is an error as in the reference (:79-81)
        self.max_spec_len = max(self.num_draft_tokens)
