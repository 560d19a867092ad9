"""CPU oracle of the verify-row logits processors — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline may use this
module, as the checker.

Restates, in numpy fp32 with the reference's operation order:
  * ``combine_outputs_with_spec_tokens`` — RejectionSampler._combine_outputs_with_spec_tokens,
    minivllm/sample/rejection_sampler.py:387-406: per request with drafts, the rows
    out, out + spec[:1], ..., out + spec[:K-1]; requests without drafts give no rows;
  * ``apply_all_penalties`` — minivllm/sample/ops/penalties.py:51-72: bin counts of prompt and
    output tokens per row; ``logits *= where(logits > 0, 1 / scaling, scaling)`` with
    ``scaling = repetition`` where the token occurs in prompt or output, else 1; then
    ``logits -= frequency * counts``; then ``logits -= presence * (counts > 0)``;
  * ``apply_min_tokens_for_spec_decode`` — minivllm/sample/sampler.py:192-228: the first
    clamp(min_tokens - len(output), 0, K_i) rows of request i get its stop tokens at -inf;
  * ``apply_logits_processors`` — rejection_sampler.py:338-356: penalties with the combined
    histories (prompts repeated per row, penalties expanded per row), then min_tokens.

Pinned by the reference's known answers (tests/step68/test_spec_sampling_constraints.py:104-136
and :167-181, held in tests/golden/reference_kats.json) and by the closed forms the formulas
fix (tests/test_oracle_penalties.py).
"""

from __future__ import annotations

import numpy as np


def combine_outputs_with_spec_tokens(output_token_ids, spec_token_ids):
    if spec_token_ids is None:
        return [list(o) for o in output_token_ids]
    rows = []
    for out, spec in zip(output_token_ids, spec_token_ids):
        if len(spec) == 0:
            continue
        rows.append(list(out))
        for i in range(len(spec) - 1):
            rows.append([*rows[-1], spec[i]])
    return rows


def _bin_counts(rows, vocab_size):
    counts = np.zeros((len(rows), vocab_size), dtype=np.int64)
    for r, tokens in enumerate(rows):
        for t in tokens:
            counts[r, t] += 1
    return counts


def apply_all_penalties(logits, prompt_token_ids, output_token_ids, presence, frequency,
                        repetition):
    """Returns a penalised copy of fp32 ``logits [R, V]``; per-row lists and [R] penalties."""
    x = np.array(logits, dtype=np.float32, copy=True)
    vocab_size = x.shape[1]
    prompt_mask = _bin_counts(prompt_token_ids, vocab_size) > 0
    out_counts = _bin_counts(output_token_ids, vocab_size)
    out_mask = out_counts > 0
    rep = np.asarray(repetition, dtype=np.float32)[:, None]
    scaling = np.where(prompt_mask | out_mask, rep, np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scaling).astype(np.float32)
    x = (x * np.where(x > 0, inv, scaling)).astype(np.float32)
    freq = np.asarray(frequency, dtype=np.float32)[:, None]
    x = (x - (freq * out_counts.astype(np.float32)).astype(np.float32)).astype(np.float32)
    pres = np.asarray(presence, dtype=np.float32)[:, None]
    x = (x - (pres * out_mask.astype(np.float32)).astype(np.float32)).astype(np.float32)
    return x


def apply_min_tokens_for_spec_decode(logits, min_tokens, stop_token_ids, output_token_ids,
                                     num_draft_tokens):
    x = np.array(logits, dtype=np.float32, copy=True)
    if not min_tokens:
        return x
    offset = 0
    for i, k in enumerate(num_draft_tokens):
        stop_ids = stop_token_ids[i] if i < len(stop_token_ids) else []
        if stop_ids:
            remaining = min_tokens[i] - len(output_token_ids[i])
            n_mask = int(min(max(remaining, 0), k))
            for row in range(offset, offset + n_mask):
                for t in stop_ids:
                    x[row, t] = -np.inf
        offset += k
    return x


def apply_logits_processors(logits, num_draft_tokens, *, no_penalties=True,
                            prompt_token_ids=(), output_token_ids=(), spec_token_ids=None,
                            presence=None, frequency=None, repetition=None, min_tokens=(),
                            stop_token_ids=()):
    """Penalties over the hypothetical histories, then min_tokens, on fp32 verify rows."""
    x = np.array(logits, dtype=np.float32, copy=True)
    if not no_penalties:
        histories = combine_outputs_with_spec_tokens(output_token_ids, spec_token_ids)
        prompts = [list(p) for p, k in zip(prompt_token_ids, num_draft_tokens) for _ in range(k)]

        def per_row(values, default):
            v = np.full(len(num_draft_tokens), default, np.float32) if values is None else \
                np.asarray(values, dtype=np.float32)
            return np.repeat(v, num_draft_tokens)

        x = apply_all_penalties(x, prompts, histories, per_row(presence, 0.0),
                                per_row(frequency, 0.0), per_row(repetition, 1.0))
    return apply_min_tokens_for_spec_decode(x, list(min_tokens), list(stop_token_ids),
                                            list(output_token_ids), list(num_draft_tokens))
