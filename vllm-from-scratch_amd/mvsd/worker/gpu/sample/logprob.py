"""``compute_topk_scores`` of the V2 sampler on the HIP logprobs kernel (csrc/logprobs.hip,
C ABI ``mvsd_topk_scores``).

Replaces minivllm/worker/gpu/sample/logprob.py:140-216 on the path without per-request
logprob token ids (the only path the V2 verification reaches): for every row n of
``logits [N, V]`` and its token ``sampled_token_ids[n]``,

* ``logprob_token_ids[n] = [token, top-k ids of the raw logits]`` (int64; equal logits in
  index order, where the reference's ``torch.topk`` leaves their order unspecified);
* ``logprobs[n]`` = the fp32 log-softmax at those ids (``_topk_log_softmax_kernel``,
  :44-83), or the logits themselves in ``logits_mode``;
* ``selected_token_ranks[n] = #{i : logits[n, i] >= logits[n, token]}`` (``_ranks_kernel``,
  :86-104), int64.

One workgroup per row reads the row once for its max and sum and once per 32 top-k keys.
"""

from __future__ import annotations

import torch

from ...._native import check, lib, require_device_tensor, stream_of
from ....outputs import LogprobsTensors


def compute_topk_scores(
    logits: torch.Tensor,
    num_logprobs: int,
    sampled_token_ids: torch.Tensor,
    cu_num_logits: list[int] | None = None,
    logprob_token_ids_state=None,
    expanded_idx_mapping: torch.Tensor | None = None,
    max_per_req_token_ids: int = 0,
    logits_mode: bool = False,
) -> LogprobsTensors:
    assert num_logprobs >= 0
    if max_per_req_token_ids != 0:
        # The reference refuses per-request logprob token ids when the request is made, so
        # its slow path (:164-200) has no caller on the verification path.
        raise NotImplementedError("per-request logprob token ids are not supported")
    require_device_tensor(logits, "logits")
    require_device_tensor(sampled_token_ids, "sampled_token_ids")
    num_rows, vocab_size = logits.shape
    device = logits.device
    if num_logprobs > vocab_size:
        raise ValueError(f"num_logprobs={num_logprobs} exceeds the vocabulary ({vocab_size})")
    x = logits
    if x.dtype != torch.float32 or x.stride(-1) != 1:
        x = x.to(torch.float32).contiguous()
    tokens = sampled_token_ids.reshape(-1)
    if tokens.numel() != num_rows:
        raise ValueError(f"{tokens.numel()} sampled tokens for {num_rows} logits rows")
    tokens = tokens.to(torch.int32).contiguous()
    ids = torch.empty(num_rows, num_logprobs + 1, dtype=torch.int32, device=device)
    scores = torch.empty(num_rows, num_logprobs + 1, dtype=torch.float32, device=device)
    ranks = torch.empty(num_rows, dtype=torch.int32, device=device)
    check(lib().mvsd_topk_scores(ids.data_ptr(), scores.data_ptr(), ranks.data_ptr(),
                                 x.data_ptr(), x.stride(0), tokens.data_ptr(), num_rows,
                                 vocab_size, num_logprobs, int(bool(logits_mode)),
                                 stream_of(device)), "mvsd_topk_scores")
    return LogprobsTensors(
        logprob_token_ids=ids.to(torch.int64),
        logprobs=scores,
        selected_token_ranks=ranks.to(torch.int64),
        cu_num_generated_tokens=cu_num_logits,
    )
