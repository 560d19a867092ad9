"""Pins the block-verification path of the CPU restatement (oracle/v2_rejection.py) without
the GPU.

* Known answers: the hand-computed thresholds, acceptance-length distributions and residuals
  the reference's own tests state for their small cases (V = 8;
  tests/step75/test_block_verification.py:80-95 residual case, :103-117 one-hot case,
  :128-135 K = 1 case, :141-152 zero-probability draft, :158-170 draft equal to target).
* Losslessness, exhaustively (Sun et al. 2024, arXiv:2403.10444, block verification is a
  valid verification): on tiny vocabularies, summing over every draft sequence (weighted by
  the draft distribution, or each fixed sequence for one-hot drafts), every acceptance length
  (its probability from the thresholds) and the residual distribution at that length, the
  output extended by the target's own later positions is distributed exactly as the target.
  A dropped p_tau shift, a wrong prefix index or a threshold without the look-ahead mass all
  break this identity (the planted-mistake tests below show it).
* K = 1 reduces block verification to the standard test (h = min(1, p/q), p_0 = 1), so the
  two paths agree request by request away from rounding ties.
* The main routine composes the pieces as the tests do: its acceptance length is the last
  position whose uniform passes its threshold, its resampled token the Gumbel argmax of the
  residual at that length.
"""

import itertools

import numpy as np
import pytest

from oracle import v2_rejection as o
from v2_cases import make_case, oracle_args


def _request(target, draft, tokens, temp=1.0, seed=1234, pos0=100):
    """Oracle arguments of one request: target rows [K+1, V], draft rows [K, V] or None."""
    target = np.asarray(target, np.float32)
    K = len(tokens)
    ds = np.zeros(K + 1, np.int64)
    ds[1:] = tokens
    return dict(
        target_logits=target,
        draft_logits=None if draft is None else np.asarray(draft, np.float32)[None],
        draft_sampled=ds, cu_num_logits=np.array([0, K + 1]),
        pos=np.arange(K + 1) + pos0, idx_mapping=np.array([0]),
        expanded_idx_mapping=np.zeros(K + 1, np.int64),
        expanded_local_pos=np.arange(K + 1), temperature=np.array([temp], np.float32),
        seed=np.array([seed]), num_speculative_steps=K)


def _details(args):
    *_, det = o.rejection_sample(**args, use_block_verification=True, return_details=True)
    return det


def _softmax(x):
    x = np.asarray(x, np.float64)
    m = x[np.isfinite(x)].max()
    e = np.exp(x - m)
    return e / e.sum()


def _tau_distribution(h):
    """P(tau = n) = h[n - 1] prod_{j >= n} (1 - h[j]) (the last position that passes wins)."""
    K = len(h)
    return np.array([(h[n - 1] if n > 0 else 1.0) * np.prod([1.0 - h[j] for j in range(n, K)])
                     for n in range(K + 1)])


def _residual_logits(args, det, tokens, tau):
    """Logits the oracle resamples from at acceptance length tau."""
    t = args["target_logits"]
    K = len(tokens)
    if tau == K:
        return t[K]
    st = det["stats"]
    dl = args["draft_logits"]
    temp = float(args["temperature"][0])
    d_row = None if dl is None else (dl[0, tau] / np.float32(temp)).astype(np.float32)
    lp = det["cumulative_log_p"][tau - 1] if tau > 0 else 0.0
    return o.residual_logits(t[tau], tokens[tau], st.target_lse(tau), d_row,
                             st.draft_lse(tau) if dl is not None else 0.0, lp)


def _residual_probs(args, det, tokens, tau):
    return _softmax(_residual_logits(args, det, tokens, tau))


# ------------------------------------------------------------------ known answers ------

V8 = 8
RESIDUAL_TARGET = [[0.0] * V8, [1.0, 0.5, 0.0, -1.0, 0.0, 0.5, 1.5, 0.0],
                   [4.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]]
RESIDUAL_DRAFT = [[0.0, 0.6, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                  [0.0, 0.0, 0.0, 2.0, 0.0, 0.0, 0.0, 0.0]]


def test_residual_case_known_answers():
    """tests/step75/test_block_verification.py:80-95, K = 2 with draft logits: the closed forms
    in float64 (p_1 = p(t1)/q(t1), M = sum max(p_1 M_b - M_s, 0) over row 1, h_1 = M/(M + 1 -
    p_1), h_2 = p_2 = p_1 M_b(t3)/M_s(t3), the residual max(p_1 M_b - M_s, 0)/M), and the
    reference's four-digit hand values (p = 0.6052, M = 0.1801, h = (0.3134, 0.0313), tau
    distribution (0.6651, 0.3036, 0.0313), block residual at tau = 1; the standard residual
    of the same row, which differs by TV 0.19)."""
    args = _request(RESIDUAL_TARGET, RESIDUAL_DRAFT, [1, 3])
    det = _details(args)
    mb0, ms0 = _softmax(RESIDUAL_TARGET[0]), _softmax(RESIDUAL_DRAFT[0])
    mb1, ms1 = _softmax(RESIDUAL_TARGET[1]), _softmax(RESIDUAL_DRAFT[1])
    p1 = mb0[1] / ms0[1]
    mass = np.maximum(p1 * mb1 - ms1, 0).sum()
    p2 = p1 * mb1[3] / ms1[3]
    h = det["h"][0]
    assert np.exp(det["cumulative_log_p"][:2]) == pytest.approx([p1, p2], rel=1e-5)
    assert det["residual_mass"][1] == pytest.approx(mass, rel=1e-5)
    assert h == pytest.approx([mass / (mass + 1 - p1), p2], rel=1e-5)
    blk = _residual_probs(args, det, [1, 3], 1)
    assert blk == pytest.approx(np.maximum(p1 * mb1 - ms1, 0) / mass, abs=1e-6)
    # the reference's hand values (rounded to four digits there)
    assert p1 == pytest.approx(0.6052, abs=2e-4) and mass == pytest.approx(0.1801, abs=2e-4)
    assert h == pytest.approx([0.3134, 0.0313], abs=2e-4)
    assert _tau_distribution(h) == pytest.approx([0.6651, 0.3036, 0.0313], abs=2e-4)
    assert blk == pytest.approx([0.2728, 0.0137, 0, 0, 0, 0.0137, 0.6999, 0], abs=2e-4)
    std = _softmax(o.residual_logits(args["target_logits"][1], 3,
                                     det["stats"].target_lse(1),
                                     np.asarray(RESIDUAL_DRAFT[1], np.float32),
                                     det["stats"].draft_lse(1), 0.0))
    assert std == pytest.approx([0.2599, 0.1015, 0.0054, 0, 0.0054, 0.1015, 0.521, 0.0054],
                                abs=1e-3)
    assert 0.5 * np.abs(blk - std).sum() == pytest.approx(0.1917, abs=1e-3)


def test_one_hot_case_known_answers():
    """tests/step75/test_block_verification.py:103-117: h = (0.4667, 0.0323, 0.03125) from
    the closed-form residual mass p_i (1 - M_b(next draft))."""
    target = np.zeros((4, V8), np.float32)
    target[0, 1] = 2.0
    target[2, 5] = 2.0
    target[2, 1] = 0.5
    target[3, 6] = 3.0
    # the reference's comments round these softmax values: p(t1) of row 0 is e^2/(e^2+7)
    det = _details(_request(target, None, [1, 2, 5]))
    p0 = np.exp(2.0) / (np.exp(2.0) + 7)
    p2 = np.exp(2.0) / (np.exp(2.0) + np.exp(0.5) + 6)
    want_prefix = [p0, p0 / 8, p0 / 8 * p2]
    assert np.exp(det["cumulative_log_p"][:3]) == pytest.approx(want_prefix, rel=1e-5)
    m0 = p0 * (1 - 1 / 8)
    m1 = p0 / 8 * (1 - p2)
    want_h = [m0 / (m0 + 1 - p0), m1 / (m1 + 1 - p0 / 8), p0 / 8 * p2]
    assert det["h"][0] == pytest.approx(want_h, rel=1e-5)
    assert det["h"][0] == pytest.approx([0.4667, 0.0323, 0.03125], abs=2e-2)


def test_k1_last_candidate_and_zero_probability_draft():
    """K = 1 (:128-135): the threshold is p_1 = p(d) with no look-ahead.  A draft the target
    gives probability 0 (:141-152) has h = 0 and is rejected for every seed (u > 0), and the
    rejected token never comes back from the resampling."""
    target = np.zeros((2, V8), np.float32)
    target[0, 3] = 1.0
    target[1, 4] = 2.0
    det = _details(_request(target, None, [3]))
    assert det["h"][0] == pytest.approx([np.e / (np.e + 7)], rel=1e-6)
    target[0, 5] = -np.inf
    for seed in range(40):
        args = _request(target, None, [5], seed=seed)
        s, n, det = o.rejection_sample(**args, use_block_verification=True, return_details=True)
        assert det["h"][0] == [0.0]
        assert n[0] == 1 and s[0, 0] != 5


def test_draft_equal_to_target_accepts_everything():
    """p == q (:158-170): R = 0 and p_i = 1 make the threshold 0/0, which is 1 (the fallback
    branch), so every draft is accepted."""
    rng = np.random.default_rng(75)
    target = (rng.standard_normal((4, V8)) * 2).astype(np.float32)
    draft = target[:3].copy()
    tokens = [int(draft[i].argmax()) for i in range(3)]
    for seed in range(20):
        args = _request(target, draft, tokens, seed=seed)
        _, n, det = o.rejection_sample(**args, use_block_verification=True, return_details=True)
        assert det["h"][0] == [1.0, 1.0, 1.0]
        assert n[0] == 4


# ------------------------------------------------------------------ losslessness -------

def _lossless_error(V, K, temp, one_hot, seed):
    """max |P(extended output = y) - prod_j p_j(y_j)| over y in V^(K+1), exhaustively."""
    rng = np.random.default_rng(seed)
    target = (rng.standard_normal((K + 1, V)) * 1.5).astype(np.float32)
    draft = (rng.standard_normal((K, V)) * 1.5).astype(np.float32)
    p = np.stack([_softmax(target[j]) for j in range(K + 1)])
    q = np.stack([_softmax(draft[j] / np.float64(np.float32(temp))) for j in range(K)])
    want = np.ones([V] * (K + 1))
    for j in range(K + 1):
        want = want * p[j].reshape([V if a == j else 1 for a in range(K + 1)])
    worst = 0.0
    total = np.zeros([V] * (K + 1))
    for xs in itertools.product(range(V), repeat=K):
        args = _request(target, None if one_hot else draft, list(xs), temp=temp)
        det = _details(args)
        taus = _tau_distribution(det["h"][0])
        got = np.zeros([V] * (K + 1))
        for tau in range(K + 1):
            if not np.isfinite(_residual_logits(args, det, list(xs), tau)).any():
                # no residual mass at this length: its threshold made it impossible
                assert taus[tau] < 1e-6, (xs, tau, taus)
                continue
            res = _residual_probs(args, det, list(xs), tau)
            for y in itertools.product(range(V), repeat=K + 1):
                if list(y[:tau]) != list(xs[:tau]):
                    continue
                pr = taus[tau] * res[y[tau]]
                for j in range(tau + 1, K + 1):
                    pr *= p[j][y[j]]
                got[y] += pr
        if one_hot:
            # a fixed draft sequence must already give the target distribution
            worst = max(worst, float(np.abs(got - want).max()))
        else:
            total += np.prod([q[j][xs[j]] for j in range(K)]) * got
    if not one_hot:
        worst = float(np.abs(total - want).max())
    return worst


@pytest.mark.parametrize("V,K,temp,one_hot,seed", [
    (3, 2, 1.0, False, 0), (3, 2, 0.7, False, 1), (3, 3, 1.3, False, 2), (4, 2, 1.0, False, 3),
    (3, 2, 1.0, True, 4), (3, 3, 0.8, True, 5), (4, 2, 1.0, True, 6)])
def test_block_verification_is_lossless(V, K, temp, one_hot, seed):
    assert _lossless_error(V, K, temp, one_hot, seed) < 2e-6


def test_planted_mistakes_break_losslessness(monkeypatch):
    """The identity above catches a dropped p_tau shift in the residual, and a threshold that
    ignores the look-ahead residual mass."""
    assert _lossless_error(3, 2, 1.0, False, 0) < 2e-6
    real = o.residual_logits

    def no_shift(row, rej, t_lse=0.0, d_row=None, d_lse=0.0, log_p_tau=0.0):
        return real(row, rej, t_lse, d_row, d_lse, 0.0)

    monkeypatch.setattr(o, "residual_logits", no_shift)
    assert _lossless_error(3, 2, 1.0, False, 0) > 1e-3
    monkeypatch.setattr(o, "residual_logits", real)
    monkeypatch.setattr(o, "block_threshold", lambda prefix, mass: np.float32(prefix))
    assert _lossless_error(3, 2, 1.0, False, 0) > 1e-3
    assert _lossless_error(3, 2, 1.0, True, 4) > 1e-3


# ------------------------------------------------------------------ reductions ---------

def test_k1_block_equals_standard():
    """With one draft per request the block test is u <= min(1, p/q) and the residual has
    p_tau = 1: the same decisions and tokens as the standard path except at rounding ties."""
    V = 64
    case = make_case([1] * 40 + [0] * 4, [0.9] * 20 + [1.0] * 20 + [0.5] * 4, 1, V, seed=11)
    a = oracle_args(case)
    sb, nb, mb, _ = o.rejection_sample(**a, use_block_verification=True, return_margins=True)
    ss, ns = o.rejection_sample(**a)
    for r in range(len(nb)):
        if mb[r] and min(mb[r]) < 1e-5:
            continue
        assert nb[r] == ns[r] and (sb[r, :nb[r]] == ss[r, :ns[r]]).all(), r
    one_hot = dict(a, draft_logits=None)
    sb, nb, mb, _ = o.rejection_sample(**one_hot, use_block_verification=True, return_margins=True)
    ss, ns = o.rejection_sample(**one_hot)
    for r in range(len(nb)):
        if mb[r] and min(mb[r]) < 1e-5:
            continue
        assert nb[r] == ns[r] and (sb[r, :nb[r]] == ss[r, :ns[r]]).all(), r


def test_greedy_requests_ignore_block_mode():
    """Greedy requests take the argmax path in both modes (:583-606)."""
    V = 64
    case = make_case([3, 2, 3, 0], [0.0] * 4, 3, V, seed=12, invalid={(2, 1)})
    a = oracle_args(case)
    sb, nb = o.rejection_sample(**a, use_block_verification=True)
    ss, ns = o.rejection_sample(**a)
    assert (nb == ns).all() and (sb == ss).all()


def test_block_refuses_synthetic_rates():
    a = oracle_args(make_case([2], [1.0], 2, 16, seed=13))
    with pytest.raises(AssertionError):
        o.rejection_sample(**a, synthetic_conditional_rates=np.array([0.5, 0.5], np.float32),
                           use_block_verification=True)


def test_main_routine_composes_the_pieces():
    """Acceptance length = last position whose uniform passes its threshold (placeholders end
    the chain); the token = Gumbel argmax of the residual at that length, over many seeds."""
    V, K = 16, 3
    rng = np.random.default_rng(21)
    target = (rng.standard_normal((K + 1, V)) * 1.5).astype(np.float32)
    draft = (target[:K] * 0.8 + rng.standard_normal((K, V)).astype(np.float32)).astype(np.float32)
    seen = set()
    for seed in range(60):
        tokens = [int(x) for x in rng.integers(0, V, K)]
        for one_hot in (False, True):
            args = _request(target, None if one_hot else draft, tokens, temp=0.9, seed=seed)
            s, n, det = o.rejection_sample(**args, use_block_verification=True,
                                           return_details=True)
            h = det["h"][0]
            us = [o.tl_rand32(np.int64(seed), np.int64(args["pos"][i])) for i in range(K)]
            tau = max([i + 1 for i in range(K) if us[i] <= h[i]], default=0)
            assert n[0] == tau + 1 and list(s[0, :tau]) == tokens[:tau]
            logits = _residual_logits(args, det, tokens, tau)
            tok, _ = o.gumbel_argmax(logits, seed, int(args["pos"][tau]), 0.9, False)
            assert s[0, tau] == tok
            seen.add(tau)
    assert seen == {0, 1, 2, 3}
