"""CPU oracle of the speculative logprobs — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline may use this
module, as the checker.

``get_logprobs_tensors`` restates RejectionSampler._get_logprobs_tensors
(minivllm/sample/rejection_sampler.py:269-300) on torch-CPU: the compact ``final_logits`` with
the verify rows at ``target_logits_indices`` and the bonus rows at ``bonus_logits_indices``;
position j of request i reads row ``start_i + j`` clamped to the last row; placeholder ids
read token 0; ``compute_logprobs`` is the fp32 log-softmax (sampler.py:313-315) unless the
mode reports logits; ``gather_logprobs`` (sampler.py:330-349) puts the sampled token first,
then the top-k, and the rank is ``#{logprobs >= the token's}`` (sampler.py:318-327).  The top-k
here is ordered by value, then index (a stable descending sort); the reference's torch.topk
leaves the order of exactly equal values unspecified.

Pinned by the reference's known answers for the row indexing and parse_output filtering
(tests/step68/test_spec_logprobs.py:229-279, :352-390, held in
tests/golden/reference_kats.json) and by closed forms (tests/test_oracle_logprobs.py).
"""

from __future__ import annotations

import torch

PLACEHOLDER_TOKEN_ID = -1


def compute_logprobs(rows: torch.Tensor) -> torch.Tensor:
    return rows.log_softmax(dim=-1, dtype=torch.float32)


def gather_logprobs(logprobs: torch.Tensor, k: int, token_ids: torch.Tensor):
    """(ids [N, k+1] int32, logprobs [N, k+1] fp32, ranks [N] int32)."""
    values, order = torch.sort(logprobs, dim=-1, descending=True, stable=True)
    top_v, top_i = values[:, :k], order[:, :k]
    token_ids = token_ids.to(torch.int64).unsqueeze(-1)
    token_lp = logprobs.gather(-1, token_ids)
    ranks = (logprobs >= token_lp).sum(-1)
    ids = torch.cat((token_ids, top_i), dim=1).to(torch.int32)
    lps = torch.cat((token_lp, top_v), dim=1)
    return ids, lps, ranks.to(torch.int32)


def rank_slack(logprobs: torch.Tensor, token_ids: torch.Tensor, ulps: int = 4) -> torch.Tensor:
    """Per row, the entries other than the token whose value lies within `ulps` fp32 ulps of
    the token's: the rank #{x >= x_token} may count them or not depending on the rounding of
    two otherwise correct fp32 log-softmax evaluations, so a rank computed elsewhere may
    differ from this one by at most that many."""
    token_lp = logprobs.gather(-1, token_ids.to(torch.int64).unsqueeze(-1))
    ulp = torch.nextafter(token_lp.abs(), torch.tensor(float("inf"))) - token_lp.abs()
    near = (logprobs - token_lp).abs() <= ulps * ulp
    return (near.sum(-1) - 1).clamp(min=0).to(torch.int32)


def get_logprobs_tensors(k: int, cu_num_sampled_tokens, target_logits_indices,
                         bonus_logits_indices, target_rows: torch.Tensor,
                         bonus_rows: torch.Tensor, sampled_token_ids: torch.Tensor,
                         logits_mode: bool = False, return_slack: bool = False):
    target_rows = torch.as_tensor(target_rows).to(torch.float32).cpu()
    bonus_rows = torch.as_tensor(bonus_rows).to(torch.float32).cpu()
    t_idx = torch.as_tensor(target_logits_indices).cpu().to(torch.int64)
    b_idx = torch.as_tensor(bonus_logits_indices).cpu().to(torch.int64)
    n_rows = int(t_idx.numel() + b_idx.numel())
    final = torch.zeros((n_rows, bonus_rows.shape[-1]), dtype=torch.float32)
    final[t_idx] = target_rows
    final[b_idx] = bonus_rows
    cu = torch.as_tensor(cu_num_sampled_tokens).cpu().to(torch.int64)
    starts = torch.zeros_like(cu)
    starts[1:] = cu[:-1]
    sampled = torch.as_tensor(sampled_token_ids).cpu()
    width = sampled.shape[-1]
    idx = (starts.unsqueeze(1) + torch.arange(width).unsqueeze(0)).flatten()
    idx = idx.clamp(max=n_rows - 1)
    tokens = sampled.clone().flatten().to(torch.int64)
    tokens[tokens == PLACEHOLDER_TOKEN_ID] = 0
    rows = final[idx]
    lps = rows if logits_mode else compute_logprobs(rows)
    out = gather_logprobs(lps, k, tokens)
    if return_slack:
        return (*out, rank_slack(lps, tokens))
    return out


def topk_scores(logits, k: int, token_ids, logits_mode: bool = False):
    """V2 ``compute_topk_scores`` (minivllm/worker/gpu/sample/logprob.py:140-216), the path
    without per-request logprob token ids: row n scores ``[token_n, top-k of the raw logits]``
    with the fp32 log-softmax (``_topk_log_softmax_kernel``, :44-83: (x - max) - log(sum
    exp(x - max))) or the logits themselves, and ranks the token by ``#{x_i >= x_token}`` over
    the raw logits (``_ranks_kernel``, :86-104).  Equal logits are taken in index order.
    Returns (ids [N, k+1] int64, scores [N, k+1] fp32, ranks [N] int64)."""
    x = torch.as_tensor(logits).to(torch.float32).cpu()
    tok = torch.as_tensor(token_ids).cpu().to(torch.int64).reshape(-1, 1)
    _, order = torch.sort(x, dim=-1, descending=True, stable=True)
    ids = torch.cat((tok, order[:, :k]), dim=1)
    if logits_mode:
        scores = x.gather(-1, ids)
    else:
        m = x.max(dim=-1, keepdim=True).values
        lse = torch.log(torch.exp(x - m).sum(dim=-1, keepdim=True))
        scores = (x.gather(-1, ids) - m) - lse
    ranks = (x >= x.gather(-1, tok)).sum(-1)
    return ids, scores, ranks
