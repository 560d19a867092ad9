"""CPU oracle of top-k / top-p masking — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline may use this
module, as the checker.

``apply_top_k_top_p`` restates minivllm/sample/ops/topk_topp_sampler.py:48-79 with torch-CPU
ops in the reference's order: ascending sort, k-th-largest threshold with ``<`` masking
(:61-69), fp32 softmax + cumsum over the sorted row with ``<= 1 - p`` masking and the largest
entry always kept (:71-77), scatter back (:79).  The sort is stable, so equal values keep index
order (the order a stable GPU radix sort produces).

``brute_force_mask`` is the definition written out for tiny rows in float64 with exact
tie order, used to pin the restatement (tests/test_oracle_topk_topp.py).
"""

from __future__ import annotations

import numpy as np
import torch


def apply_top_k_top_p(logits: torch.Tensor, k: torch.Tensor | None,
                      p: torch.Tensor | None) -> torch.Tensor:
    """Returns a masked copy of fp32 ``logits [N, V]`` (the reference masks in place)."""
    logits = logits.to(torch.float32).clone()
    if k is None and p is None:
        return logits
    logits_sort, logits_idx = logits.sort(dim=-1, descending=False, stable=True)
    if k is not None:
        top_k_index = logits_sort.size(1) - k.to(torch.long)
        thresh = logits_sort.gather(1, top_k_index.unsqueeze(dim=1))
        logits_sort.masked_fill_(logits_sort < thresh, -float("inf"))
    if p is not None:
        probs_sort = logits_sort.softmax(dim=-1)
        probs_sum = torch.cumsum(probs_sort, dim=-1)
        top_p_mask = probs_sum <= 1 - p.to(torch.float32).unsqueeze(dim=1)
        top_p_mask[:, -1] = False
        logits_sort.masked_fill_(top_p_mask, -float("inf"))
    return logits.scatter_(dim=-1, index=logits_idx, src=logits_sort)


def brute_force_mask(row: np.ndarray, k: int | None, p: float | None) -> np.ndarray:
    """Boolean keep-mask of one row by the definition, float64 sums, stable tie order."""
    v = np.asarray(row, dtype=np.float64)
    n = v.size
    order = sorted(range(n), key=lambda i: (v[i], i))        # ascending, ties by index
    keep = np.ones(n, dtype=bool)
    if k is not None:
        kth = v[order[n - k]]
        keep &= v >= kth
    if p is not None:
        x = np.where(keep, v, -np.inf)
        m = x.max()
        e = np.where(keep, np.exp(x - m), 0.0)
        probs = e / e.sum()
        t = np.float32(1.0) - np.float32(p)
        csum = 0.0
        for pos, i in enumerate(order):
            csum += probs[i]
            if pos < n - 1 and csum <= float(t):
                keep[i] = False
    return keep


def near_boundary(row: np.ndarray, k: int | None, p: float | None, tol: float = 1e-5) -> np.ndarray:
    """Entries whose top-p decision depends on rounding: |cumsum - (1 - p)| < tol at them."""
    v = np.asarray(row, dtype=np.float64)
    n = v.size
    flag = np.zeros(n, dtype=bool)
    if p is None:
        return flag
    order = sorted(range(n), key=lambda i: (v[i], i))
    keep = np.ones(n, dtype=bool)
    if k is not None:
        keep &= v >= v[order[n - k]]
    x = np.where(keep, v, -np.inf)
    e = np.where(keep, np.exp(x - x.max()), 0.0)
    probs = e / e.sum()
    t = float(np.float32(1.0) - np.float32(p))
    csum = 0.0
    for i in order:
        csum += probs[i]
        if abs(csum - t) < tol:
            flag[i] = True
    return flag
