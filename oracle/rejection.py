"""CPU oracle of the verification path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module, and only as the checker (or the timed CPU baseline).  The product path
(``mvsd``) never imports it and has no CPU fallback.

A restatement, on torch-CPU / numpy, of the reference's algorithm in the reference's order:
    temperature divide          minivllm/sample/rejection_sampler.py:553-561 (expand :574-597)
    target softmax (fp32)       rejection_sampler.py:502; torch_rejection_sampler.py:111
    greedy argmax               rejection_sampler.py:485; torch_rejection_sampler.py:112
    exponential noise -> 1/E    rejection_sampler.py:646-655; torch_rejection_sampler.py:267-274
    recovered scores + argmax   rejection_sampler.py:850-928; torch_rejection_sampler.py:276-289
    greedy chain                rejection_sampler.py:678-740
    random chain                rejection_sampler.py:744-822; torch_rejection_sampler.py:131-167
The randomness (fp64 uniforms, Exp(1) noise rows or recovered ids) is always supplied.

Pinning (see tests/test_oracle_rejection.py): the reference's hand-computed KATs
(tests/step59/test_rejection.py, transcribed in tests/golden/reference_kats.json), the
distribution theorems the reference tests statistically (output ~ p, recovered ~ max(p-q,0)),
softmax against a float64 computation, argmax against numpy's first-index rule, and a
brute-force float64 recovered argmax on tiny vocabularies.

Acceptance precision: the production kernel divides p[d] / q[d] in fp32 and compares with the
fp64 uniform (rejection_sampler.py:806); ``ratio="fp64"`` gives the torch reference's form
(torch_rejection_sampler.py:159-165).  They differ only when |u - p/q| is at rounding level.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

PLACEHOLDER_TOKEN_ID = -1


def expand_batch_to_tokens(x, cu_num_tokens, num_tokens: int, replace_from=0, replace_to=0):
    """``[B] -> [num_tokens]`` by request ranges [cu[i-1], cu[i]) (rejection_sampler.py:574-597,
    expand_kernel :826-847)."""
    x = np.asarray(x)
    cu = np.asarray(cu_num_tokens, dtype=np.int64)
    out = np.empty(num_tokens, dtype=x.dtype)
    start = 0
    for i in range(len(x)):
        v = replace_to if x[i] == replace_from else x[i]
        out[start:cu[i]] = v
        start = cu[i]
    return out


def request_of_row(num_draft_tokens) -> np.ndarray:
    return np.repeat(np.arange(len(num_draft_tokens)), np.asarray(num_draft_tokens, dtype=np.int64))


def row_temperatures(temperature, num_draft_tokens, all_greedy: bool,
                     apply_temperature: bool) -> torch.Tensor | None:
    """Per-row divisor: T of the row's request with T == 0 -> 1 (rejection_sampler.py:553-559);
    None when no divide happens (all greedy, or temperature already applied)."""
    if all_greedy or not apply_temperature:
        return None
    t = np.asarray(torch.as_tensor(temperature).cpu().numpy(), dtype=np.float32)
    rows = t[request_of_row(num_draft_tokens)]
    rows = np.where(rows == 0.0, np.float32(1.0), rows)
    return torch.from_numpy(rows.astype(np.float32))


def target_probs(target_logits: torch.Tensor, row_temperature: torch.Tensor | None) -> torch.Tensor:
    """fp32 softmax over V after the fp32 temperature divide (rejection_sampler.py:502,561)."""
    x = target_logits.to(torch.float32)
    if row_temperature is not None:
        x = x / row_temperature.to(torch.float32).unsqueeze(-1)
    return torch.softmax(x, dim=-1, dtype=torch.float32)


def recovered_scores(probs: torch.Tensor, draft_probs: torch.Tensor | None,
                     draft_token_ids: torch.Tensor, exp_noise: torch.Tensor,
                     num_draft_tokens) -> torch.Tensor:
    """``max(p - q, 0) * (1 / E)[request]``; point-mass drafts use p with the draft id zeroed
    (rejection_sampler.py:882-918, torch_rejection_sampler.py:274-288)."""
    inv = torch.reciprocal(exp_noise.to(torch.float32))
    if draft_probs is None:
        weights = probs.clone()
        rows = torch.arange(weights.shape[0])
        weights[rows, draft_token_ids.long()] = 0.0
    else:
        weights = torch.clamp_min(probs - draft_probs.to(torch.float32), 0.0)
    req = torch.from_numpy(request_of_row(num_draft_tokens))
    return weights * inv[req]


def recovered_token_ids(scores: torch.Tensor) -> torch.Tensor:
    """First-index argmax clamped to V - 1 (rejection_sampler.py:921-927)."""
    if scores.shape[0] == 0:
        return torch.zeros(0, dtype=torch.int32)
    ids = torch.argmax(scores, dim=-1)
    return torch.clamp(ids, max=scores.shape[1] - 1).to(torch.int32)


@dataclass
class OracleResult:
    output_token_ids: np.ndarray      # [B, max_spec_len + 1] int32
    ratio: np.ndarray                 # [P] p[d]/q[d] as compared (nan for greedy rows)
    uniforms: np.ndarray              # [P] fp64 (nan when not supplied)
    top1: np.ndarray                  # [P] best recovered score (nan when not computed)
    top2: np.ndarray                  # [P] second best recovered score
    greedy_rows: np.ndarray           # [P] bool
    top1_p: np.ndarray | None = None  # [P] target probability at the best recovered index
    top1_q: np.ndarray | None = None  # [P] draft probability there (0 for point-mass drafts)
    top1_scale: np.ndarray | None = None  # [P] |x / T| + |max(x) / T| there (exponent scale)


def rejection_sample(draft_token_ids, num_draft_tokens, max_spec_len, draft_probs,
                     target_logits, bonus_token_ids, *, temperature=None, all_greedy: bool,
                     uniforms=None, exp_noise=None, recovered=None, synthetic_rates=None,
                     apply_temperature: bool = False, ratio: str = "fp32") -> OracleResult:
    """Reference-order restatement of ``rejection_sample`` with supplied randomness.

    ``target_logits`` [P, V] (any float dtype, upcast to fp32), ``draft_probs`` [P, V] fp32 or
    None, ``exp_noise`` [B, V] (or ``recovered`` [P]), ``uniforms`` [P] fp64.
    """
    draft_ids = torch.as_tensor(draft_token_ids).cpu().to(torch.int64)
    num_draft_tokens = [int(k) for k in num_draft_tokens]
    B = len(num_draft_tokens)
    P = int(draft_ids.shape[0])
    logits = torch.as_tensor(target_logits).cpu()
    V = int(logits.shape[-1])
    bonus = torch.as_tensor(bonus_token_ids).cpu().reshape(-1).numpy().astype(np.int64)
    out = np.full((B, max_spec_len + 1), PLACEHOLDER_TOKEN_ID, dtype=np.int32)
    temps = None if temperature is None else torch.as_tensor(temperature).cpu().to(torch.float32)
    greedy_req = (np.ones(B, dtype=bool) if all_greedy
                  else (temps.numpy() == 0.0))                    # rejection_sampler.py:469-473
    req_row = request_of_row(num_draft_tokens)
    greedy_rows = greedy_req[req_row] if P else np.zeros(0, dtype=bool)
    u = (np.full(P, np.nan) if uniforms is None
         else torch.as_tensor(uniforms).cpu().to(torch.float64).numpy())
    ratio_out = np.full(P, np.nan)
    top1 = np.full(P, np.nan)
    top2 = np.full(P, np.nan)
    top1_p = np.full(P, np.nan)
    top1_q = np.zeros(P)
    top1_scale = np.zeros(P)

    argmax = torch.argmax(logits.to(torch.float32), dim=-1).numpy() if P else np.zeros(0, int)
    probs = None
    rec = None
    if not all_greedy and P:
        probs = target_probs(logits, row_temperatures(temps, num_draft_tokens, all_greedy,
                                                       apply_temperature))
        if recovered is not None:
            rec = torch.as_tensor(recovered).cpu().numpy().astype(np.int64)
        else:
            dp = None if draft_probs is None else torch.as_tensor(draft_probs).cpu()
            scores = recovered_scores(probs, dp, draft_ids, torch.as_tensor(exp_noise).cpu(),
                                      num_draft_tokens)
            rec = recovered_token_ids(scores).numpy().astype(np.int64)
            if V >= 2:
                top = torch.topk(scores, 2, dim=-1).values.numpy()
                top1, top2 = top[:, 0].astype(np.float64), top[:, 1].astype(np.float64)
                rows = torch.arange(P)
                ridx = torch.from_numpy(rec)
                top1_p = probs[rows, ridx].to(torch.float64).numpy()
                rt = row_temperatures(temps, num_draft_tokens, all_greedy, apply_temperature)
                xs = logits.to(torch.float32)
                if rt is not None:
                    xs = xs / rt.unsqueeze(-1)
                top1_scale = (xs[rows, ridx].abs() + xs.max(dim=-1).values.abs()).to(
                    torch.float64).numpy()
                if dp is not None:
                    top1_q = dp[rows, ridx].to(torch.float64).numpy()
    rates = None if synthetic_rates is None else np.asarray(
        torch.as_tensor(synthetic_rates).cpu().numpy(), dtype=np.float32)
    dp_np = None if draft_probs is None else torch.as_tensor(draft_probs).cpu().to(
        torch.float32).numpy()
    probs_np = None if probs is None else probs.numpy()

    start = 0
    for r, k in enumerate(num_draft_tokens):
        rejected = False
        for pos in range(k):
            row = start + pos
            d = int(draft_ids[row])
            if greedy_req[r]:
                if rates is not None:
                    accepted = bool(u[row] < float(rates[pos]) and d >= 0)
                    token = d if accepted else int(argmax[row])
                else:
                    token = int(argmax[row])
                    accepted = d == token
            else:
                if d < 0:
                    accepted = False
                elif rates is not None:
                    accepted = bool(u[row] < float(rates[pos]))
                elif d >= V:
                    accepted = False
                else:
                    q = np.float32(1.0) if dp_np is None else np.float32(dp_np[row, d])
                    p = np.float32(probs_np[row, d])
                    if ratio == "fp32":
                        rr = float(np.float32(p) / q) if q > 0 else np.nan
                    else:
                        rr = float(p) / float(q) if q > 0 else np.nan
                    ratio_out[row] = rr
                    accepted = bool(q > 0 and rr >= u[row])
                token = d if accepted else int(rec[row])
            out[r, pos] = token
            if not accepted:
                rejected = True
                break
        if not rejected:
            out[r, k] = int(bonus[r])
        start += k
    return OracleResult(out, ratio_out, u, top1, top2, greedy_rows, top1_p, top1_q, top1_scale)


@dataclass
class ParityReport:
    requests: int
    mismatched: int
    accept_flips: int
    recovered_flips: int
    unexplained: list


def recovered_window(p: float, q: float, scale: float = 0.0) -> float:
    """Relative gap between the two best recovered scores below which fp32 rounding may swap
    them.  Two fp32 softmax evaluations of one row (torch's exp(x / T - max) against the
    kernel's exp2((x - M) log2(e) / T - log2 S), different summation orders) agree in p to
    about 2^-22 (scale + |ln p| + 16) relative, where scale = |x / T| + |M / T|: the
    exponent's absolute rounding error grows with the magnitudes rounded on the way (x / T is
    rounded before the maximum is subtracted), and the normaliser's sum over the vocabulary
    adds a few ulp.  The score (p - q) / E carries that error amplified by p / (p - q); both
    candidates can move, hence the factor 2."""
    if not (p > 0.0) or not (p > q):
        return 0.0
    eps = 2.0 ** -22 * (scale + abs(np.log(p)) + 16.0)
    return 2.0 * eps * p / (p - q)


def compare(out_device: np.ndarray, res: OracleResult, draft_token_ids, num_draft_tokens, *,
            accept_tol: float = 1e-6, recovered_rel_tol: float | None = None) -> ParityReport:
    """Compare device output with the oracle request by request.

    A mismatch is allowed only where the first differing position is
      * an accept/reject flip with |u - p/q| < accept_tol, or
      * a rejection in both with different recovered ids whose top-2 scores are within the
        row's rounding window (``recovered_window`` of p and q at the best index; a fixed
        relative ``recovered_rel_tol`` when given or when the oracle did not record p, q);
    and it is counted.  Greedy rows must match exactly.
    """
    out_device = np.asarray(out_device)
    draft_ids = np.asarray(torch.as_tensor(draft_token_ids).cpu().numpy(), dtype=np.int64)
    acc = rec = mism = 0
    bad = []
    start = 0
    for r, k in enumerate(num_draft_tokens):
        a, b = out_device[r], res.output_token_ids[r]
        if not np.array_equal(a, b):
            mism += 1
            j = int(np.argmax(a != b))
            row = start + j
            if j >= k or row >= len(draft_ids) or res.greedy_rows[row]:
                bad.append((r, j, "greedy/bonus mismatch"))
            else:
                d = draft_ids[row]
                ka, kb = a[j] == d, b[j] == d
                if ka != kb:
                    if abs(res.uniforms[row] - res.ratio[row]) < accept_tol:
                        acc += 1
                    else:
                        bad.append((r, j, f"accept flip u={res.uniforms[row]!r} "
                                          f"ratio={res.ratio[row]!r}"))
                else:
                    t1, t2 = res.top1[row], res.top2[row]
                    if recovered_rel_tol is not None or res.top1_p is None:
                        tol = 1e-5 if recovered_rel_tol is None else recovered_rel_tol
                    else:
                        tol = recovered_window(float(res.top1_p[row]), float(res.top1_q[row]),
                                               float(res.top1_scale[row]))
                    if np.isfinite(t1) and t1 - t2 <= tol * abs(t1):
                        rec += 1
                    else:
                        bad.append((r, j, f"recovered {a[j]} vs {b[j]} top1={t1!r} top2={t2!r}"))
        start += k
    return ParityReport(len(num_draft_tokens), mism, acc, rec, bad)
