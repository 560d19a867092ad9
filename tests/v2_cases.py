"""Seeded input builder for the V2 verification tests (CPU tensors; shapes as the V2 runner
passes them, minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py:935-962)."""

from __future__ import annotations

import numpy as np
import torch


def make_case(drafts_per_req, temps, K, V, *, seed=0, draft_logits=True, states=None,
              greedy_match=0.5, invalid=(), dtype=torch.float32):
    """drafts_per_req[r] drafts for request r (<= K); temps[r] its temperature (0 = greedy).
    ``invalid`` lists (request, step) pairs whose draft id is set to -1."""
    g = torch.Generator().manual_seed(seed)
    R = len(drafts_per_req)
    S = states if states is not None else R + 3
    perm = torch.randperm(S, generator=g)[:R].to(torch.int32)
    counts = [n + 1 for n in drafts_per_req]
    cu = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32)
    num_logits = int(cu[-1])
    target = (torch.randn(num_logits, V, generator=g) * 2.0).to(dtype)
    dl = None
    if draft_logits:
        dl = (torch.randn(S, K, V, generator=g) * 2.0)
    exp_idx = torch.empty(num_logits, dtype=torch.int32)
    local = torch.empty(num_logits, dtype=torch.int32)
    pos = torch.empty(num_logits, dtype=torch.int64)
    draft_sampled = torch.zeros(num_logits, dtype=torch.int32)
    temperature = torch.zeros(S, dtype=torch.float32)
    seeds = torch.randint(0, 2**62, (S,), generator=g, dtype=torch.int64)
    for r in range(R):
        st = int(perm[r])
        temperature[st] = temps[r]
        start = int(cu[r])
        for j in range(counts[r]):
            exp_idx[start + j] = st
            local[start + j] = j
            pos[start + j] = 1000 * r + 37 + j
        for i in range(drafts_per_req[r]):
            row = target[start + i].float()
            if dl is not None:
                # the target leans towards the draft so that chains get accepted
                target[start + i] = (0.7 * dl[st, i] + 0.6 * row).to(dtype)
                row = target[start + i].float()
            if temps[r] == 0.0 and torch.rand(1, generator=g).item() < greedy_match:
                tok = int(row.argmax())
            elif dl is not None:
                p = torch.softmax(dl[st, i] / max(temps[r], 1e-3), -1)
                tok = int(torch.multinomial(p, 1, generator=g))
            else:
                tok = int(torch.randint(0, V, (1,), generator=g))
            draft_sampled[start + i + 1] = -1 if (r, i) in invalid else tok
    if dl is not None:
        dl = dl.to(dtype)
    return dict(target_logits=target, draft_logits=dl, draft_sampled=draft_sampled,
                cu_num_logits=cu, pos=pos, idx_mapping=perm,
                expanded_idx_mapping=exp_idx, expanded_local_pos=local,
                temperature=temperature, seed=seeds, num_speculative_steps=K)


def oracle_args(case):
    out = {}
    for k, v in case.items():
        if isinstance(v, torch.Tensor):
            out[k] = v.float().numpy() if v.is_floating_point() else v.numpy()
        else:
            out[k] = v
    return out


def repeat_case(target, draft, tokens, temp, n, *, seed=0):
    """``n`` requests with the same rows (target [K+1, V], draft [K, V] or None, draft ids
    ``tokens``) and temperature, each with its own state, seed and positions: n independent
    draws of one design (the layout of tests/step75/test_block_verification.py:176-204)."""
    target = torch.as_tensor(np.asarray(target, np.float32))
    K = len(tokens)
    rows = K + 1
    g = torch.Generator().manual_seed(seed)
    ds = torch.zeros(n * rows, dtype=torch.int32)
    for i, tok in enumerate(tokens):
        ds[i + 1::rows] = tok
    return dict(
        target_logits=target.repeat(n, 1).contiguous(),
        draft_logits=None if draft is None else
        torch.as_tensor(np.asarray(draft, np.float32))[None].repeat(n, 1, 1).contiguous(),
        draft_sampled=ds, cu_num_logits=torch.arange(0, (n + 1) * rows, rows, dtype=torch.int32),
        pos=torch.arange(n * rows, dtype=torch.int64) + 100,
        idx_mapping=torch.arange(n, dtype=torch.int32),
        expanded_idx_mapping=torch.arange(n, dtype=torch.int32).repeat_interleave(rows),
        expanded_local_pos=torch.arange(rows, dtype=torch.int32).repeat(n),
        temperature=torch.full((n,), float(temp)),
        seed=torch.randint(0, 2**62, (n,), generator=g, dtype=torch.int64),
        num_speculative_steps=K)


def near_tie(margins, windows, gap, gap_window) -> bool:
    """A request's output may differ from the oracle's only when one of its decisions was
    within its fp32 flip window (oracle.v2_rejection.flip_window: 8 fp32 ulps of the terms'
    magnitudes, from the hardware exp2 / log2 error of at most 3 ulp and the sums' roundings),
    or when the best two resampling scores were."""
    return any(m < w for m, w in zip(margins, windows)) or gap < gap_window
