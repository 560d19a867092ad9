"""top-k / top-p masking (drop-in for minivllm/sample/ops/topk_topp_sampler.py:48-79).

One HIP workgroup per row (``mvsd_apply_top_k_top_p``): the k-th largest value from the
entries at or above the k-th largest per-thread maximum, gathered and sorted in LDS; the
top-p crossing from a logarithmic mass histogram and the entries of the crossing bin; then one
masking pass -- no sort of the vocabulary.
"""

from __future__ import annotations

import torch

from ... import _native as nat

SAMPLING_EPS = 1e-5


def apply_top_k_top_p(logits: torch.Tensor, k: torch.Tensor | None,
                      p: torch.Tensor | None) -> torch.Tensor:
    """Set non-candidate logits to -inf in place and return ``logits``; ``None`` disables a
    filter.

    Reference semantics (:48-79): keep every value >= the k-th largest (ties kept); then over
    the top-k-masked row drop the ascending prefix whose cumulative probability is <= 1 - p,
    always keeping the largest entry.  Equal values are ordered by index (a stable sort).
    ``logits`` must be a 2-D fp32 device tensor whose rows are contiguous; the reference's
    callers guarantee 0 < k < V, and here k >= V (rows without top-k) keeps the row.  p >= 1
    keeps the row (the reference's p = 1 masks only entries whose fp32 probability is 0).
    """
    if k is None and p is None:
        return logits
    assert logits.ndim == 2 and logits.dtype == torch.float32, "fp32 [N, V] logits expected"
    nat.require_device_tensor(logits, "logits")
    if logits.stride(1) != 1:
        raise ValueError("apply_top_k_top_p needs rows with unit stride")
    n, V = logits.shape
    device = logits.device
    kk = None if k is None else k.to(device=device, dtype=torch.int64).contiguous()
    pp = None if p is None else p.to(device=device, dtype=torch.float32).contiguous()
    if kk is not None:
        assert kk.numel() == n
    if pp is not None:
        assert pp.numel() == n
    nat.check(nat.lib().mvsd_apply_top_k_top_p(
        logits.data_ptr(), logits.stride(0), None if kk is None else kk.data_ptr(),
        None if pp is None else pp.data_ptr(), n, V, nat.stream_of(device)),
        "mvsd_apply_top_k_top_p")
    return logits
