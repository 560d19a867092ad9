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


def sampling_metadata(temperatures, drafts, *, device="cpu", max_num_logprobs=None,
                      logprobs_mode="raw_logprobs", output_token_ids=None,
                      prompt_token_ids=None, top_k=None, top_p=None, min_p=None,
                      no_penalties=True, presence_penalties=None, frequency_penalties=None,
                      repetition_penalties=None, min_tokens=None, stop_token_ids=None,
                      generators=None):
    """A row-aligned SamplingMetadata from plain lists (the keyword set of the reference's
    test builder, tests/step68/spec68_helpers.py:22-51): temperatures below 1e-5 are greedy;
    missing histories, min_tokens and stop lists default to empty."""
    from ..sample.metadata import SAMPLING_EPS, SamplingMetadata

    def tensor(values, dtype=torch.float32):
        return None if values is None else torch.tensor(values, dtype=dtype, device=device)

    n = len(temperatures)
    all_greedy = all(t < SAMPLING_EPS for t in temperatures)
    return SamplingMetadata(
        temperature=None if all_greedy else tensor(temperatures),
        all_greedy=all_greedy, all_random=all(t >= SAMPLING_EPS for t in temperatures),
        top_k=tensor(top_k, torch.int64), top_p=tensor(top_p), min_p=tensor(min_p),
        generators=dict(generators or {}), no_penalties=no_penalties,
        prompt_token_ids=prompt_token_ids or [[] for _ in range(n)],
        output_token_ids=output_token_ids or [[] for _ in range(n)],
        min_tokens=min_tokens or [0] * n,
        stop_token_ids=stop_token_ids or [[] for _ in range(n)],
        spec_token_ids=[list(d) for d in drafts],
        presence_penalties=tensor(presence_penalties),
        frequency_penalties=tensor(frequency_penalties),
        repetition_penalties=tensor(repetition_penalties),
        max_num_logprobs=max_num_logprobs, logprobs_mode=logprobs_mode)
