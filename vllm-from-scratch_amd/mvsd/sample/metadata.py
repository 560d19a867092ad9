"""Row-aligned sampling parameters (minivllm/sample/metadata.py:34-150).

Only the fields the verification path reads are meaningful here; the rest are kept so that
objects built by the reference's runner can be passed through unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

# temperatures below this are greedy (minivllm/sample/metadata.py:34)
SAMPLING_EPS = 1e-5


@dataclass
class SamplingMetadata:
    # None when every row is greedy; otherwise [num_rows] fp32
    temperature: torch.Tensor | None
    all_greedy: bool
    all_random: bool
    top_k: torch.Tensor | None                 # [num_rows] int64; None = no top-k
    top_p: torch.Tensor | None                 # [num_rows] fp32;  None = no top-p
    generators: dict[int, torch.Generator] = field(default_factory=dict)
    no_penalties: bool = True
    prompt_token_ids: list[list[int]] = field(default_factory=list)
    output_token_ids: list[list[int]] = field(default_factory=list)
    presence_penalties: torch.Tensor | None = None
    frequency_penalties: torch.Tensor | None = None
    repetition_penalties: torch.Tensor | None = None
    min_tokens: list[int] = field(default_factory=list)
    stop_token_ids: list[list[int]] = field(default_factory=list)
    spec_token_ids: list[list[int]] = field(default_factory=list)
    max_num_logprobs: int | None = None
    logprobs_mode: str = "raw_logprobs"
    min_p: torch.Tensor | None = None
    allowed_token_ids_mask: torch.Tensor | None = None
    bad_words_token_ids: list[list[int]] | None = None
    thinking_budget_state_holder: object | None = None

    @property
    def num_rows(self) -> int:
        if self.temperature is not None:
            return int(self.temperature.shape[0])
        for tensor in (self.top_k, self.top_p, self.presence_penalties, self.min_p):
            if tensor is not None:
                return int(tensor.shape[0])
        return len(self.min_tokens)
