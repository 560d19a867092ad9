"""Build a SpecDecodeMetadata the way the runner does (minivllm/testing/spec_metadata.py:19-81,
minivllm/worker/gpu_model_runner.py:959-1045).

Layout per request i with K_i drafts: the forward computes K_i + 1 query rows
``[b][d1..dK]``; the compact logits keep all of them, so request i owns compact rows
``[S_i, S_i + K_i]`` where ``S_i = sum_{j<i} (K_j + 1)``.  Verify row k of request i is compact
row ``S_i + k`` and the bonus row is ``S_i + K_i``.
"""

from __future__ import annotations

import numpy as np
import torch

from ..spec_decode.metadata import SpecDecodeMetadata


def _inclusive_and_local(counts: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(inclusive prefix sums, position of each element inside its own group)."""
    inclusive = np.cumsum(counts, dtype=np.int64)
    starts = inclusive - counts
    local = np.arange(int(counts.sum()), dtype=np.int64) - np.repeat(starts, counts)
    return inclusive, local


def make_metadata(draft_token_ids: list[list[int]],
                  num_scheduled: list[int] | None = None,
                  input_ids: list[int] | None = None,
                  device: str | torch.device = "cpu") -> SpecDecodeMetadata:
    ks = np.array([len(d) for d in draft_token_ids], dtype=np.int64)
    if num_scheduled is None:
        num_scheduled = [int(k) + 1 if k else 1 for k in ks]
    scheduled = np.array(num_scheduled, dtype=np.int64)
    sampled = ks + 1
    if input_ids is None:
        input_ids = [tok for draft in draft_token_ids for tok in [0, *draft]]
    if len(input_ids) != int(scheduled.sum()):
        raise ValueError(f"input_ids has {len(input_ids)} rows but {int(scheduled.sum())} "
                         "are scheduled")

    cu_sampled, local_sampled = _inclusive_and_local(sampled)
    cu_scheduled = np.cumsum(scheduled)
    # the last K_i + 1 scheduled rows of each request are sampled
    logits_indices = np.repeat(cu_scheduled - sampled, sampled) + local_sampled
    bonus_logits_indices = cu_sampled - 1
    cu_draft, local_draft = _inclusive_and_local(ks)
    target_logits_indices = np.repeat(cu_sampled - sampled, ks) + local_draft

    gathered = np.asarray(input_ids, dtype=np.int64)[logits_indices]
    drafts = gathered[target_logits_indices + 1] if len(target_logits_indices) else np.zeros(0)
    expected = [tok for draft in draft_token_ids for tok in draft]
    if [int(t) for t in drafts] != expected:
        raise ValueError("input_ids layout does not match the drafts")

    def dev(a):
        return torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32), device=device)

    return SpecDecodeMetadata(
        draft_token_ids=dev(drafts),
        num_draft_tokens=[int(k) for k in ks],
        cu_num_draft_tokens=dev(cu_draft),
        cu_num_sampled_tokens=dev(cu_sampled),
        target_logits_indices=dev(target_logits_indices),
        bonus_logits_indices=dev(bonus_logits_indices),
        logits_indices=dev(logits_indices),
    )
