"""CPU restatement of the V2 speculative-decoding verification (test infrastructure only).

This module is the checker for ``mvsd.worker.gpu.spec_decode.rejection_sampler_utils`` and is
imported only by ``tests/`` (never by the product path).  It follows, step by step:

* ``rejection_sample`` (minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py:935-1201):
  per-block logits statistics (:206-316), the per-request chain (:497-706), the Gumbel-max
  resampling of the rejected/bonus row (:709-866) and its insertion (:869-932); for block
  verification also the running joint ratio (:318-384), the look-ahead residual mass
  (:387-446, :60-104), the threshold of the chain's block branch (:608-640) and the
  p_tau-shifted residual (:820-829);
* the counter-based draws of minivllm/worker/gpu/sample/gumbel.py: ``tl_rand32`` (:87-91),
  ``tl_rand64`` (:72-83) and ``gumbel_noised_argmax`` (:95-131), whose generator is Triton's
  ``tl.randint4x`` / ``tl.rand`` (Philox4x32, 10 rounds; triton/language/random.py of the
  installed Triton 3.6.0 — the reference pins 3.7.1, whose generator is the same published
  algorithm: Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011).

Block sizes are the reference's (8192 for the statistics, 1024 for the resampling); the
HIP kernels use their own decomposition, which changes only the rounding of the log-sum-exp
(first-index ties are decomposition-independent).

Pinning:
* ``philox4x32`` — the Random123 known-answer vectors for Philox4x32-10 and values of
  Triton's ``tl.randint4x`` / ``tl.rand`` produced by Triton's CPU interpreter
  (``tests/golden/v2_philox.json``, made by ``tests/golden/make_v2_philox.py``);
* the chain and the resampling — closed forms on small vocabularies (greedy accept iff
  draft == argmax; random accept iff log p(d) > log u + log q(d); the residual argmax
  equals brute force over max(p - q, 0) with the same noise) and the semantics pins of the
  reference's tests (tests/step73/test_v2_rejection_diff.py:318-327, :357-360);
* block verification — the hand-computed values of the reference's tests
  (tests/step75/test_block_verification.py:80-170) against float64 closed forms, and an
  exhaustive losslessness check on tiny vocabularies (Sun et al. 2024: summed over draft
  sequences, acceptance lengths and residuals, the output is distributed as the target),
  which a dropped p_tau shift or a threshold without the look-ahead mass fails
  (tests/test_oracle_v2_block.py);
* float rounding of exp/log is not pinned bit for bit (numpy vs device libm): decisions are
  compared with a margin and near-ties are counted.
"""

from __future__ import annotations

import numpy as np

M32 = np.uint64(0xFFFFFFFF)
_KEY_A, _KEY_B = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_ROUND_A, _ROUND_B = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
RAND32_MIN = np.float32(4.6566127342e-10)  # gumbel.py:24
RAND32_SCALE = np.float32(4.6566127342e-10)
RAND64_SCALE = 5.421010862427522170037e-20  # gumbel.py:79
F64_TINY = 2.2250738585072014e-308
STATS_BLOCK = 8192    # rejection_sampler_utils.py:981
RESAMPLE_BLOCK = 1024  # rejection_sampler_utils.py:1158


def philox4x32(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Philox4x32 rounds as in triton/language/random.py ``philox_impl`` (uint32 arrays)."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint32).astype(np.uint64) for c in (c0, c1, c2, c3))
    k0 = np.asarray(k0, dtype=np.uint32).astype(np.uint64)
    k1 = np.asarray(k1, dtype=np.uint32).astype(np.uint64)
    for _ in range(rounds):
        p0 = _ROUND_B * c2  # B * c2 (64-bit product of 32-bit values)
        p2 = _ROUND_A * c0
        n0 = (p0 >> np.uint64(32)) ^ c1 ^ k0
        n2 = (p2 >> np.uint64(32)) ^ c3 ^ k1
        c1 = p0 & M32
        c3 = p2 & M32
        c0, c2 = n0 & M32, n2 & M32
        k0 = (k0 + np.uint64(_KEY_A)) & M32
        k1 = (k1 + np.uint64(_KEY_B)) & M32
    return tuple(c.astype(np.uint32) for c in (c0, c1, c2, c3))


def randint4x(seed, offset):
    """``tl.randint4x(seed, offset)``: key = (seed lo, seed hi), counter = (offset lo, offset hi
    if the offset is 64-bit else 0, 0, 0).  ``offset`` is int64 or int32 (its dtype decides)."""
    s = np.asarray(seed).astype(np.int64).astype(np.uint64)
    off = np.asarray(offset)
    lo = (off.astype(np.int64).astype(np.uint64) & M32).astype(np.uint32)
    if off.dtype.itemsize > 4:
        hi = ((off.astype(np.int64).astype(np.uint64) >> np.uint64(32)) & M32).astype(np.uint32)
    else:
        hi = np.zeros_like(lo)
    z = np.zeros_like(lo)
    return philox4x32(lo, hi, z, z, (s & M32).astype(np.uint32), (s >> np.uint64(32)).astype(np.uint32))


def uint_to_uniform_f32(x):
    """triton/language/random.py ``uint_to_uniform_float`` for 32-bit inputs."""
    i = np.asarray(x, dtype=np.uint32).view(np.int32).astype(np.int64)
    i = np.where(i < 0, -i - 1, i).astype(np.int32)
    return (i.astype(np.float32) * RAND32_SCALE).astype(np.float32)


def tl_rand32(seed, offset, includes_zero: bool = False):
    """gumbel.py:87-91."""
    u = uint_to_uniform_f32(randint4x(seed, offset)[0])
    return u if includes_zero else np.maximum(u, RAND32_MIN)


def tl_rand64(seed, offset, includes_zero: bool = False):
    """gumbel.py:72-83."""
    lo, hi, _, _ = randint4x(seed, offset)
    r = (hi.astype(np.uint64) << np.uint64(32)) | lo.astype(np.uint64)
    u = r.astype(np.float64) * RAND64_SCALE
    return u if includes_zero else np.maximum(u, F64_TINY)


def gumbel_argmax(logits_f32, seed: int, pos: int, temp: float, use_fp64: bool):
    """``gumbel_noised_argmax`` with APPLY_TEMPERATURE=False over a whole row
    (gumbel.py:95-131): returns (index, value)."""
    x = np.asarray(logits_f32, dtype=np.float32)
    if use_fp64:
        x = x.astype(np.float64)
    if temp != 0.0:
        gseed = np.int64(randint4x(np.int64(seed), np.int64(pos))[0])  # tl.randint: uint32 seed
        keys = np.arange(x.shape[0], dtype=np.int32)
        with np.errstate(divide="ignore"):
            if use_fp64:
                u = tl_rand64(gseed, keys)
                noise = -np.log(-np.log(u))
            else:
                u = tl_rand32(gseed, keys)
                noise = (-np.log(-np.log1p(-u))).astype(np.float32)
        x = x + noise
    i = int(np.argmax(x))
    return i, x[i]


def _max_sumexp(x):
    m = np.float32(x.max())
    s = np.float32(np.exp(x - m).sum(dtype=np.float32)) if m > -np.inf else np.float32(0.0)
    return m, s


def _lse(maxes, sums):
    g = np.float32(maxes.max())
    return np.float32(g + np.log(np.float32((sums * np.exp(maxes - g)).sum(dtype=np.float32))))


class Stats:
    """Per-block statistics of every verify row (rejection_sampler_utils.py:206-316): the
    greedy rows' (max, first argmax), the random rows' (max, sum exp) of the target row and of
    the temperature-scaled draft row."""

    def __init__(self, t, dl, exp_idx, exp_local, temp_all, K, V):
        num_logits = t.shape[0]
        nb = -(-V // STATS_BLOCK)
        self.tmax = np.full((num_logits, nb), -np.inf, np.float32)
        self.targ = np.zeros((num_logits, nb), np.int64)
        self.tsum = np.zeros((num_logits, nb), np.float32)
        self.dmax = np.full((num_logits, nb), -np.inf, np.float32)
        self.dsum = np.zeros((num_logits, nb), np.float32)
        for row in range(num_logits):
            step = int(exp_local[row])
            if step >= K:
                continue
            st = int(exp_idx[row])
            tt = temp_all[st]
            for b in range(nb):
                blk = t[row, b * STATS_BLOCK:min(V, (b + 1) * STATS_BLOCK)]
                if tt == 0.0:
                    j = int(np.argmax(blk))
                    self.tmax[row, b], self.targ[row, b] = blk[j], b * STATS_BLOCK + j
                else:
                    self.tmax[row, b], self.tsum[row, b] = _max_sumexp(blk)
                    if dl is not None:
                        cols = slice(b * STATS_BLOCK, min(V, (b + 1) * STATS_BLOCK))
                        d = (dl[st, step, cols] / tt).astype(np.float32)
                        self.dmax[row, b], self.dsum[row, b] = _max_sumexp(d)

    def target_lse(self, row):
        return _lse(self.tmax[row], self.tsum[row])

    def draft_lse(self, row):
        return _lse(self.dmax[row], self.dsum[row])


def _valid(d, V):
    """A draft id the chain verifies: -1 is the reference's placeholder; ids >= V are treated
    as placeholders too (the HIP path refuses to read past the row)."""
    return 0 <= d < V


def _logprobs_at(t, dl, stats, row, st, step, tt, tok):
    """(log p(tok), log q(tok)) of verify row ``row`` (rejection_sampler_utils.py:134-203);
    log q = 0 for one-hot drafts."""
    tlp = np.float32(t[row, tok] - stats.target_lse(row))
    if dl is None:
        return tlp, np.float32(0.0)
    return tlp, np.float32(np.float32(dl[st, step, tok] / tt) - stats.draft_lse(row))


def cumulative_log_p(t, dl, ds, cu, idx_mapping, temp_all, stats, V):
    """log of the running joint ratio, _compute_cumulative_log_p_kernel
    (rejection_sampler_utils.py:318-384): for every random request, row start + i holds
    min(log p_i + log p(d) - log q(d), 0) after draft i; placeholder drafts carry the value.
    Rows of greedy requests and bonus rows stay NaN (never read)."""
    cum = np.full(t.shape[0], np.nan, np.float32)
    for r in range(cu.shape[0] - 1):
        st = int(idx_mapping[r])
        tt = temp_all[st]
        if tt == 0.0:
            continue
        start, end = int(cu[r]), int(cu[r + 1])
        log_p = np.float32(0.0)
        for step in range(end - start - 1):
            li = start + step
            d = int(ds[li + 1])
            if _valid(d, V):
                tlp, dlp = _logprobs_at(t, dl, stats, li, st, step, tt, d)
                log_p = np.float32(min(np.float32(log_p + np.float32(tlp - dlp)), np.float32(0.0)))
            cum[li] = log_p
    return cum


def local_residual_mass(t, dl, ds, cum, exp_idx, exp_local, temp_all, K, stats, V):
    """Residual mass sum_x max(p_i M_b(x) - M_s(x), 0) of the rows that the block threshold
    looks ahead to, _compute_local_residual_mass_kernel (rejection_sampler_utils.py:387-446),
    summed over the reference's 8192-column blocks in fp32 as _compute_global_residual_mass
    does (:60-85).  Only rows at draft step 1..K-1 whose own draft is verifiable, of random
    requests; other rows stay NaN."""
    num_logits = t.shape[0]
    mass = np.full(num_logits, np.nan, np.float32)
    nb = -(-V // STATS_BLOCK)
    for row in range(num_logits):
        step = int(exp_local[row])
        if step == 0 or step >= K or row + 1 >= num_logits or not _valid(int(ds[row + 1]), V):
            continue
        st = int(exp_idx[row])
        tt = temp_all[st]
        if tt == 0.0:
            continue
        prefix = np.float32(np.exp(cum[row - 1]))
        t_lse, d_lse = stats.target_lse(row), stats.draft_lse(row)
        total = np.float32(0.0)
        for b in range(nb):
            cols = slice(b * STATS_BLOCK, min(V, (b + 1) * STATS_BLOCK))
            m_b = np.exp((t[row, cols] - t_lse).astype(np.float32)).astype(np.float32)
            d = (dl[st, step, cols] / tt).astype(np.float32)
            m_s = np.exp((d - d_lse).astype(np.float32)).astype(np.float32)
            part = np.maximum((prefix * m_b - m_s).astype(np.float32), np.float32(0.0))
            total = np.float32(total + part.sum(dtype=np.float32))
        mass[row] = total
    return mass


def block_threshold(prefix, residual_mass):
    """Acceptance threshold h of a block position with a verifiable next draft
    (rejection_sampler_utils.py:633-634): R / (R + 1 - p_i), or 1 when that denominator is
    not positive (p_i = 1 and R = 0: the draft equals the target)."""
    prefix, residual_mass = np.float32(prefix), np.float32(residual_mass)
    denom = np.float32(np.float32(residual_mass + np.float32(1.0)) - prefix)
    return np.float32(residual_mass / denom) if denom > 0.0 else np.float32(1.0)


def residual_logits(row, rej, t_lse=0.0, d_row=None, d_lse=0.0, log_p_tau=0.0):
    """Logits the rejected row is resampled from (rejection_sampler_utils.py:800-842).
    ``row`` is the target row [V]; ``d_row`` the temperature-scaled draft row or None
    (one-hot drafts); ``rej`` the rejected draft id, or a negative value for the bonus row or
    a placeholder (then the target row itself).  With draft logits the result is
    log max(p_tau p - q, 0), where ``log_p_tau`` is 0 outside block verification."""
    row = np.asarray(row, dtype=np.float32)
    V = row.shape[0]
    if rej < 0:
        return row
    if d_row is None:
        return np.where(np.arange(V) != rej, row, -np.inf).astype(np.float32)
    tlp = ((row - np.float32(t_lse)).astype(np.float32) + np.float32(log_p_tau)).astype(np.float32)
    dlp = (np.asarray(d_row, dtype=np.float32) - np.float32(d_lse)).astype(np.float32)
    ratio = np.exp(dlp - tlp).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(ratio < 1.0, tlp + np.log1p(-ratio), -np.inf).astype(np.float32)


# fp32 evaluation error allowed between this restatement (numpy libm, float64 where it helps)
# and a device build that computes the same quantities in fp32 with the hardware exp2 / log2
# (each within 3 ulp) and reduced sums: DEVICE_ULPS fp32 ulps of every magnitude that enters a
# decision.
DEVICE_ULPS = 8
EPS32 = 2.0 ** -23


def flip_window(magnitude: float) -> float:
    """Width below which a decision margin (or a resampling gap) whose terms sum to
    ``magnitude`` in absolute value may be flipped by fp32 evaluation differences."""
    return DEVICE_ULPS * EPS32 * float(magnitude)


def rejection_sample(target_logits, draft_logits, draft_sampled, cu_num_logits, pos, idx_mapping,
                     expanded_idx_mapping, expanded_local_pos, temperature, seed,
                     num_speculative_steps: int, synthetic_conditional_rates=None,
                     use_fp64: bool = False, use_block_verification: bool = False,
                     return_margins: bool = False, return_details: bool = False,
                     return_windows: bool = False):
    """V2 ``rejection_sample`` on numpy arrays, standard or block verification.

    Returns ``(sampled [R, K+1] int64, num_sampled [R] int32)`` where entries at or past
    ``num_sampled[r]`` are -1 (the reference leaves them undefined).  With ``return_margins``
    also returns, per request, the list of decision margins of the random steps that were
    decided (|log p - log u - log q| for the standard test, |u - h| for the block test), and
    the gap between the best and second-best resampled scores (a near-tie measure).  With
    ``return_windows`` (and ``return_margins``) also returns, in the same shapes, the width
    below which a margin or gap may be flipped by fp32 evaluation differences between this
    restatement and a device build (``flip_window``).  With
    ``return_details`` (block verification) the last element returned is a dict with the
    per-request thresholds ``h``, the ``cumulative_log_p`` and ``residual_mass`` arrays and
    the ``stats``."""
    t = np.asarray(target_logits, dtype=np.float32)
    num_logits, V = t.shape
    dl = None if draft_logits is None else np.asarray(draft_logits, dtype=np.float32)
    if dl is not None:
        V = min(V, dl.shape[-1])
    ds = np.asarray(draft_sampled).astype(np.int64)
    cu = np.asarray(cu_num_logits).astype(np.int64)
    pos = np.asarray(pos).astype(np.int64)
    temp_all = np.asarray(temperature, dtype=np.float32)
    seed_all = np.asarray(seed).astype(np.int64)
    K = int(num_speculative_steps)
    R = cu.shape[0] - 1
    rates = None if synthetic_conditional_rates is None else np.asarray(
        synthetic_conditional_rates, dtype=np.float32)
    block = bool(use_block_verification)
    if block:
        assert rates is None, "Block verification is incompatible with synthetic acceptance rates."

    stats = Stats(t, dl, expanded_idx_mapping, expanded_local_pos, temp_all, K, V)
    cum = mass = None
    if block:
        cum = cumulative_log_p(t, dl, ds, cu, idx_mapping, temp_all, stats, V)
        if dl is not None:
            mass = local_residual_mass(t, dl, ds, cum, expanded_idx_mapping,
                                       expanded_local_pos, temp_all, K, stats, V)

    sampled = np.full((R, K + 1), -1, np.int64)
    num_sampled = np.zeros(R, np.int32)
    margins = [[] for _ in range(R)]
    windows = [[] for _ in range(R)]
    thresholds = [[] for _ in range(R)]
    gaps = np.full(R, np.inf)
    gap_windows = np.zeros(R)

    def lse_mag(row):
        m = abs(float(stats.target_lse(row)))
        return m + (abs(float(stats.draft_lse(row))) if dl is not None else 0.0)
    for r in range(R):
        st = int(idx_mapping[r])
        start, end = int(cu[r]), int(cu[r + 1])
        nd = end - start - 1
        s, tt = seed_all[st], temp_all[st]
        greedy = tt == 0.0
        acc, verifying = 0, True
        t_lse = d_lse = np.float32(0.0)
        for i in range(nd):
            li = start + i
            d = int(ds[li + 1])
            valid = _valid(d, V)
            d = d if valid else 0
            if not greedy:
                verifying &= valid
            if not verifying:
                continue
            u = tl_rand32(s, np.int64(pos[li]))
            if greedy:
                m = np.where(np.isnan(stats.tmax[li]), -np.inf, stats.tmax[li])
                am = int(stats.targ[li, int(np.argmax(m))])
                ok = (u < rates[i]) if rates is not None else (am == d)
                ok = bool(ok) and valid
                verifying = ok
                acc += ok
                sampled[r, i] = d if ok else am
            elif block:
                # Block verification (:608-640): accept i + 1 tokens when u <= h; the last
                # position that passes decides.
                prefix = np.float32(np.exp(cum[li]))
                nxt = int(ds[li + 2]) if i < nd - 1 else -1
                if _valid(nxt, V):
                    if dl is not None:
                        res = mass[li + 1]
                    else:
                        # one-hot drafts: p_i (1 - M_b(next)) in closed form (:87-104)
                        m_b = np.float32(np.exp(np.float32(t[li + 1, nxt] - stats.target_lse(li + 1))))
                        res = np.float32(prefix * np.float32(1.0 - m_b))
                    h = block_threshold(prefix, res)
                else:
                    h = prefix
                thresholds[r].append(float(h))
                margins[r].append(abs(float(u) - float(h)))
                if return_windows:
                    # h is a function of exp(cum) and the next row's residual: its relative
                    # error follows the log-space error of every row up to the next one
                    mag = abs(float(cum[li])) + sum(lse_mag(j) for j in range(start, min(li + 2, end - 1)))
                    windows[r].append(flip_window(mag + 1.0))
                if u <= h:
                    acc = i + 1
                sampled[r, i] = d
            else:
                t_lse = stats.target_lse(li)
                tlp = np.float32(t[li, d] - t_lse)
                if dl is not None:
                    d_lse = stats.draft_lse(li)
                    dlp = np.float32(np.float32(dl[st, i, d] / tt) - d_lse)
                else:
                    dlp, d_lse = np.float32(0.0), np.float32(0.0)
                rhs = np.float32(np.float32(np.log(u)) + dlp)
                if rates is not None:
                    ok = bool(u < rates[i])
                else:
                    ok = bool(tlp > rhs)
                    margins[r].append(abs(float(tlp) - float(rhs)))
                    if return_windows:
                        windows[r].append(flip_window(
                            abs(float(tlp)) + abs(float(t_lse)) + abs(float(np.log(u)))
                            + abs(float(dlp)) + abs(float(d_lse)) + 1.0))
                verifying = ok
                acc += ok
                sampled[r, i] = d
        num_sampled[r] = acc
        if block and not greedy and acc < nd:
            # (:683-700) the statistics of the row the block rejected
            t_lse = stats.target_lse(start + acc)
            d_lse = stats.draft_lse(start + acc) if dl is not None else np.float32(0.0)

        # Resample the rejected or bonus row (:709-866) and insert it (:869-932).
        ri = start + acc
        is_bonus = ri == end - 1
        if greedy and not is_bonus:
            num_sampled[r] = acc + 1
            continue
        rej = int(ds[ri + 1]) if not is_bonus else -1
        rej = rej if _valid(rej, V) else -1
        d_row = None if (dl is None or rej < 0) else (dl[st, acc, :V] / tt).astype(np.float32)
        log_p_tau = np.float32(cum[ri - 1]) if (block and acc > 0) else np.float32(0.0)
        resid = residual_logits(t[ri, :V], rej, t_lse, d_row, d_lse, log_p_tau)
        tok, _ = gumbel_argmax(resid, int(s), int(pos[ri]), float(tt), use_fp64)
        if return_margins and tt != 0.0:
            x = np.asarray(resid, dtype=np.float64)
            gseed = np.int64(randint4x(np.int64(s), np.int64(pos[ri]))[0])
            keys = np.arange(V, dtype=np.int32)
            with np.errstate(divide="ignore", invalid="ignore"):
                if use_fp64:
                    sc = x - np.log(-np.log(tl_rand64(gseed, keys)))
                else:
                    sc = x - np.log(-np.log1p(-tl_rand32(gseed, keys).astype(np.float64)))
            finite = np.flatnonzero(np.isfinite(sc))
            best = finite[np.argsort(sc[finite], kind="stable")[-2:]]
            if best.size == 2:
                gaps[r] = float(sc[best[1]] - sc[best[0]])
                if return_windows:
                    noise = np.abs(x[best] - sc[best]).sum()
                    gap_windows[r] = flip_window(
                        np.abs(sc[best]).sum() + noise + 2.0 * (abs(float(t_lse)) + abs(float(d_lse))
                                                                + abs(float(log_p_tau))) + 1.0)
        sampled[r, acc] = tok
        num_sampled[r] = acc + 1
    out = (sampled, num_sampled)
    if return_margins:
        out = out + (margins, gaps)
        if return_windows:
            out = out + (windows, gap_windows)
    if return_details:
        out = out + (dict(h=thresholds, cumulative_log_p=cum, residual_mass=mass, stats=stats),)
    return out


def flatten_sampled(sampled, num_sampled, cu_num_logits, num_logits):
    """``flatten_sampled`` (minivllm/worker/gpu/spec_decode/rejection_sampler.py:73-108): row
    ``cu[r] + j`` holds ``sampled[r, j]`` for ``j < num_sampled[r]``; every other row is 0."""
    flat = np.zeros(int(num_logits), np.int64)
    cu = np.asarray(cu_num_logits).astype(np.int64)
    for r in range(cu.shape[0] - 1):
        n = int(num_sampled[r])
        flat[cu[r]:cu[r] + n] = np.asarray(sampled)[r, :n]
    return flat
