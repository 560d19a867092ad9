"""The V2 sampler's output (minivllm/worker/gpu/sample/output.py): the sampled tokens with
the per-request counts that the V2 runner's bookkeeping reads."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ....outputs import LogprobsTensors


@dataclass
class SamplerOutput:
    """``sampled_token_ids [num_reqs, K + 1]`` int64 (entries at or past ``num_sampled[r]``
    undefined); ``num_sampled`` / ``num_rejected [num_reqs]`` int32 (0 for a request still
    prefilling); ``num_nans`` per-row NaN counts when the runner computes them, else None;
    ``sampling_mask_tensors`` is the runner's structured-output mask handle (not produced on
    the verification path)."""

    sampled_token_ids: torch.Tensor
    logprobs_tensors: LogprobsTensors | None
    num_nans: torch.Tensor | None
    num_sampled: torch.Tensor | None = None
    num_rejected: torch.Tensor | None = None
    sampling_mask_tensors: object | None = None
