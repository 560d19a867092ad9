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
