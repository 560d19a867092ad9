"""CPU restatement of the V2 speculative-decoding verification (test infrastructure only).

This module is the checker for ``mvsd.worker.gpu.spec_decode.rejection_sampler_utils`` and is
imported only by ``tests/`` (never by the product path).  It follows, step by step:

* ``rejection_sample`` (minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py:935-1201),
  non-block path: per-block logits statistics (:206-316), the per-request chain (:497-706),
  the Gumbel-max resampling of the rejected/bonus row (:709-866) and its insertion (:869-932);
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


def rejection_sample(target_logits, draft_logits, draft_sampled, cu_num_logits, pos, idx_mapping,
                     expanded_idx_mapping, expanded_local_pos, temperature, seed,
                     num_speculative_steps: int, synthetic_conditional_rates=None,
                     use_fp64: bool = False, return_margins: bool = False):
    """V2 ``rejection_sample`` (non-block) on numpy arrays.

    Returns ``(sampled [R, K+1] int64, num_sampled [R] int32)`` where entries at or past
    ``num_sampled[r]`` are -1 (the reference leaves them undefined).  With ``return_margins``
    also returns, per request, the list of acceptance margins |log p - log u - log q| of the
    random steps that were decided, and the gap between the best and second-best resampled
    scores (a near-tie measure)."""
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
    nb = -(-V // STATS_BLOCK)

    # Per-block statistics (rejection_sampler_utils.py:206-316).
    tmax = np.full((num_logits, nb), -np.inf, np.float32)
    targ = np.zeros((num_logits, nb), np.int64)
    tsum = np.zeros((num_logits, nb), np.float32)
    dmax = np.full((num_logits, nb), -np.inf, np.float32)
    dsum = np.zeros((num_logits, nb), np.float32)
    for row in range(num_logits):
        step = int(expanded_local_pos[row])
        if step >= K:
            continue
        st = int(expanded_idx_mapping[row])
        tt = temp_all[st]
        for b in range(nb):
            blk = t[row, b * STATS_BLOCK:min(V, (b + 1) * STATS_BLOCK)]
            if tt == 0.0:
                j = int(np.argmax(blk))
                tmax[row, b], targ[row, b] = blk[j], b * STATS_BLOCK + j
            else:
                tmax[row, b], tsum[row, b] = _max_sumexp(blk)
                if dl is not None:
                    d = (dl[st, step, b * STATS_BLOCK:min(V, (b + 1) * STATS_BLOCK)] / tt).astype(np.float32)
                    dmax[row, b], dsum[row, b] = _max_sumexp(d)

    sampled = np.full((R, K + 1), -1, np.int64)
    num_sampled = np.zeros(R, np.int32)
    margins = [[] for _ in range(R)]
    gaps = np.full(R, np.inf)
    rates = None if synthetic_conditional_rates is None else np.asarray(
        synthetic_conditional_rates, dtype=np.float32)
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
            valid = d >= 0
            d = max(0, d)
            if not greedy:
                verifying &= valid
            if not verifying:
                continue
            u = tl_rand32(s, np.int64(pos[li]))
            if greedy:
                m = np.where(np.isnan(tmax[li]), -np.inf, tmax[li])
                am = int(targ[li, int(np.argmax(m))])
                ok = (u < rates[i]) if rates is not None else (am == d)
                ok = bool(ok) and valid
                verifying = ok
                acc += ok
                sampled[r, i] = d if ok else am
            else:
                t_lse = _lse(tmax[li], tsum[li])
                tlp = np.float32(t[li, d] - t_lse)
                if dl is not None:
                    d_lse = _lse(dmax[li], dsum[li])
                    dlp = np.float32(np.float32(dl[st, i, d] / tt) - d_lse)
                else:
                    dlp, d_lse = np.float32(0.0), np.float32(0.0)
                rhs = np.float32(np.float32(np.log(u)) + dlp)
                if rates is not None:
                    ok = bool(u < rates[i])
                else:
                    ok = bool(tlp > rhs)
                    margins[r].append(abs(float(tlp) - float(rhs)))
                verifying = ok
                acc += ok
                sampled[r, i] = d
        num_sampled[r] = acc

        # Resample the rejected or bonus row (:709-866) and insert it (:869-932).
        ri = start + acc
        is_bonus = ri == end - 1
        if greedy and not is_bonus:
            num_sampled[r] = acc + 1
            continue
        rej = int(ds[ri + 1]) if not is_bonus else 0
        row = t[ri, :V]
        if is_bonus or rej < 0:
            resid = row
        elif dl is not None:
            d = (dl[st, acc, :V] / tt).astype(np.float32)
            tlp = (row - t_lse).astype(np.float32)
            dlp = (d - d_lse).astype(np.float32)
            ratio = np.exp(dlp - tlp).astype(np.float32)
            with np.errstate(divide="ignore", invalid="ignore"):
                resid = np.where(ratio < 1.0, tlp + np.log1p(-ratio), -np.inf).astype(np.float32)
        else:
            resid = np.where(np.arange(V) != rej, row, -np.inf).astype(np.float32)
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
            top2 = np.sort(sc[np.isfinite(sc)])[-2:]
            if top2.size == 2:
                gaps[r] = float(top2[1] - top2[0])
        sampled[r, acc] = tok
        num_sampled[r] = acc + 1
    if return_margins:
        return sampled, num_sampled, margins, gaps
    return sampled, num_sampled
