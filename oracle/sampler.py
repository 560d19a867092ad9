"""CPU oracle of the regular (bonus-row) sampler — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline may use this
module, as the checker.

``forward`` restates Sampler.forward (minivllm/sample/sampler.py:73-120) on torch-CPU fp32,
with the exponential noise supplied by the caller instead of drawn:
  * the raw logprobs (log-softmax) or raw logits are kept first when logprobs are asked for
    (:88-95);
  * penalties (:122-157) over the committed output, plus every draft when
    ``predict_bonus_token`` (:159-175), by oracle/penalties.apply_all_penalties; then
    min_tokens (:177-190): rows whose committed output is shorter than min_tokens get their
    stop tokens at -inf;
  * ``sample`` (:243-278): greedy argmax before any temperature; all-greedy batches return the
    processed logits / logprobs as they are; otherwise divide by the temperature (rows below
    SAMPLING_EPS divide by 1), ``apply_min_p`` (:280-293: probs < max(probs) * min_p -> -inf),
    top-k / top-p (oracle/topk_topp.py), the exponential race argmax(softmax / noise)
    (ops/topk_topp_sampler.py:82-115), and rows below SAMPLING_EPS take the greedy token;
  * logprobs: -1 hands back the full rows; k >= 0 is oracle/logprobs.gather_logprobs.
``race_scores`` returns the race's scores so that a test can accept a device argmax that
differs only on a near tie.

Pinned by the reference's known answers (tests/step68/test_spec_sampling_constraints.py:39-98,
:138-161, :262-296, held in tests/golden/reference_kats.json) and by closed forms
(tests/test_oracle_sampler.py).
"""

from __future__ import annotations

import numpy as np
import torch

from . import logprobs as olp
from . import penalties as opn
from . import topk_topp as otk

SAMPLING_EPS = 1e-5


def _vec(values, n, default):
    if values is None:
        return np.full(n, default, np.float32)
    return np.asarray(torch.as_tensor(values).cpu(), dtype=np.float32)


def apply_logits_processors(x: torch.Tensor, sm, predict_bonus_token: bool) -> torch.Tensor:
    n = x.shape[0]
    if not sm.no_penalties:
        outs = [list(o) for o in sm.output_token_ids]
        if predict_bonus_token and sm.spec_token_ids is not None:
            outs = [[*o, *s] if s else o for o, s in zip(outs, sm.spec_token_ids)]
        x = torch.from_numpy(opn.apply_all_penalties(
            x.numpy(), [list(p) for p in sm.prompt_token_ids], outs,
            _vec(sm.presence_penalties, n, 0.0), _vec(sm.frequency_penalties, n, 0.0),
            _vec(sm.repetition_penalties, n, 1.0)))
    x = x.clone()
    for row, (min_tokens, stop_ids) in enumerate(zip(sm.min_tokens, sm.stop_token_ids)):
        if row < n and stop_ids and len(sm.output_token_ids[row]) < min_tokens:
            x[row, list(stop_ids)] = -float("inf")
    return x


def apply_min_p(x: torch.Tensor, min_p) -> torch.Tensor:
    if min_p is None:
        return x
    probs = torch.softmax(x, dim=-1)
    adjusted = probs.amax(dim=-1, keepdim=True) * torch.as_tensor(min_p).float().cpu()[:, None]
    return x.masked_fill(probs < adjusted, -float("inf"))


def race_scores(x: torch.Tensor, noise: torch.Tensor) -> torch.Tensor:
    return torch.softmax(x, dim=-1, dtype=torch.float32) / noise


def sample(x: torch.Tensor, sm, noise: torch.Tensor, mode: str):
    """(tokens int64 [N], processed rows or None, race scores or None); ``x`` is not
    modified."""
    x = x.clone()
    greedy = None if sm.all_random else x.argmax(dim=-1)
    if sm.all_greedy:
        processed = None
        if sm.max_num_logprobs is not None:
            if mode == "processed_logits":
                processed = x
            elif mode == "processed_logprobs":
                processed = olp.compute_logprobs(x)
        return greedy, processed, None
    t = torch.as_tensor(sm.temperature).float().cpu()
    safe = torch.where(t < SAMPLING_EPS, torch.ones_like(t), t)
    x = x / safe[:, None]
    x = apply_min_p(x, sm.min_p)
    k = None if sm.top_k is None else torch.as_tensor(sm.top_k).cpu()
    p = None if sm.top_p is None else torch.as_tensor(sm.top_p).cpu()
    x = otk.apply_top_k_top_p(x, k, p)
    processed = None
    if mode == "processed_logits":
        processed = x
    elif mode == "processed_logprobs":
        processed = olp.compute_logprobs(x)
    scores = race_scores(x, noise.float().cpu())
    random = scores.argmax(dim=-1)
    if greedy is None:
        return random, processed, scores
    return torch.where(t < SAMPLING_EPS, greedy, random), processed, scores


def forward(logits: torch.Tensor, sm, noise: torch.Tensor | None, mode: str = "raw_logprobs",
            predict_bonus_token: bool = False):
    """(sampled int64 [N], logprobs triple / full rows / None, race scores or None)."""
    x = torch.as_tensor(logits).cpu().to(torch.float32)
    k = sm.max_num_logprobs
    kept = None
    if k is not None:
        if mode == "raw_logprobs":
            kept = olp.compute_logprobs(x)
        elif mode == "raw_logits":
            kept = x.clone()
    x = apply_logits_processors(x, sm, predict_bonus_token)
    sampled, processed, scores = sample(x, sm, noise, mode)
    if processed is not None:
        kept = processed
    if k is None:
        return sampled, None, scores
    if k == -1:
        return sampled, kept, scores
    return sampled, olp.gather_logprobs(kept, k, sampled), scores
