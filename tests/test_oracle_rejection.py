"""Pin the CPU rejection oracle (oracle/rejection.py) to the reference.

Checks, each chosen so that a plausible slip in the oracle fails one of them:
  * the reference's hand-computed KATs (tests/golden/reference_kats.json);
  * the distribution theorems the reference tests statistically
    (tests/step59/test_rejection.py:387-435): outputs ~ p, recovered ~ max(p - q, 0);
  * softmax against a float64 computation, argmax against numpy's first-index rule;
  * the recovered argmax against a brute-force float64 search on tiny vocabularies;
  * special cases that reduce to known answers (q == p accepts everything; a zero q[d]
    always rejects; the point-mass recovered distribution never returns the draft).
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rejection as orc

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def build_case(case):
    """Inputs of a KAT in the layout rejection_sample takes (verify rows only)."""
    drafts = case["drafts"]
    ks = [len(d) for d in drafts]
    flat = [t for d in drafts for t in d]
    if case["kind"] == "argmax":
        V = case["vocab"]
        rows = []
        for target in case["targets"]:
            for t in target:
                row = [0.01] * V
                row[t] = 0.9
                rows.append(row)
        logits = torch.tensor(rows, dtype=torch.float32).log() if rows else torch.zeros((0, V))
        q = None
    else:
        logits = torch.tensor(case["p_rows"], dtype=torch.float32).log()
        q = None if case["q_rows"] is None else torch.tensor(case["q_rows"], dtype=torch.float32)
    temps = case["temperature"]
    all_greedy = all(t < 1e-5 for t in temps)
    return dict(draft_token_ids=torch.tensor(flat, dtype=torch.int32), num_draft_tokens=ks,
                max_spec_len=max(ks), draft_probs=q, target_logits=logits,
                bonus_token_ids=torch.tensor(case["bonus"], dtype=torch.int32).view(-1, 1),
                temperature=torch.tensor(temps, dtype=torch.float32), all_greedy=all_greedy,
                uniforms=(torch.tensor(case["uniforms"], dtype=torch.float64)
                          if "uniforms" in case else None),
                recovered=(torch.tensor(case["recovered"], dtype=torch.int32)
                           if "recovered" in case else None))


@pytest.mark.parametrize("case", KATS["rejection"], ids=lambda c: c["name"])
def test_oracle_matches_reference_kats(case):
    kw = build_case(case)
    res = orc.rejection_sample(**kw)
    assert res.output_token_ids.tolist() == case["expected"]


@pytest.mark.parametrize("case", KATS["expand"], ids=lambda c: c["source"])
def test_expand_kats(case):
    out = orc.expand_batch_to_tokens(np.array(case["x"]), case["cu"], case["num_tokens"],
                                     case["replace_from"], case["replace_to"])
    assert out.tolist() == case["expected"]


def _sample_many(p, q, n, seed):
    """Run the oracle on n independent single-draft requests with fresh randomness."""
    rng = np.random.default_rng(seed)
    drafts = rng.choice(len(q), size=n, p=q)
    logits = torch.tensor([p], dtype=torch.float32).log().repeat(n, 1)
    dp = torch.tensor([q], dtype=torch.float32).repeat(n, 1)
    res = orc.rejection_sample(
        torch.tensor(drafts, dtype=torch.int32), [1] * n, 1, dp, logits,
        torch.full((n, 1), len(p) - 1, dtype=torch.int32),
        temperature=torch.ones(n), all_greedy=False,
        uniforms=torch.from_numpy(rng.random(n)),
        exp_noise=torch.from_numpy(rng.exponential(size=(n, len(p))).astype(np.float32)))
    return res.output_token_ids[:, 0]


def test_output_distribution_equals_target():
    case = KATS["distribution"][0]
    out = _sample_many(case["p"], case["q"], case["samples"], seed=0)
    freq = np.bincount(out, minlength=3) / case["samples"]
    assert np.all(np.abs(freq - np.array(case["p"])) < case["threshold"]), freq


def test_recovered_distribution_is_max_p_minus_q():
    case = KATS["distribution"][1]
    n = case["samples"]
    rng = np.random.default_rng(1)
    probs = torch.tensor([case["p"]], dtype=torch.float32).repeat(n, 1)
    q = torch.tensor([case["q"]], dtype=torch.float32).repeat(n, 1)
    noise = torch.from_numpy(rng.exponential(size=(n, 3)).astype(np.float32))
    scores = orc.recovered_scores(probs, q, torch.zeros(n, dtype=torch.int32), noise, [1] * n)
    ids = orc.recovered_token_ids(scores).numpy()
    freq = np.bincount(ids, minlength=3) / n
    assert freq[0] == 0.0
    assert np.all(np.abs(freq - np.array(case["expected"])) < case["threshold"]), freq


def test_point_mass_recovered_never_returns_the_draft():
    rng = np.random.default_rng(2)
    n, V = 4000, 6
    p = rng.dirichlet(np.ones(V)).astype(np.float32)
    probs = torch.from_numpy(np.tile(p, (n, 1)))
    drafts = torch.from_numpy(rng.integers(0, V, n).astype(np.int32))
    noise = torch.from_numpy(rng.exponential(size=(n, V)).astype(np.float32))
    ids = orc.recovered_token_ids(orc.recovered_scores(probs, None, drafts, noise, [1] * n))
    assert not np.any(ids.numpy() == drafts.numpy())
    # conditional on draft d, the recovered id follows p restricted to v != d
    mask = drafts.numpy() == 0
    freq = np.bincount(ids.numpy()[mask], minlength=V)[1:] / mask.sum()
    assert np.all(np.abs(freq - p[1:] / p[1:].sum()) < 0.06)


def test_equal_draft_and_target_accepts_everything():
    rng = np.random.default_rng(3)
    B, k, V = 16, 5, 50
    logits = torch.from_numpy(rng.normal(size=(B * k, V)).astype(np.float32))
    probs = torch.softmax(logits, -1)
    # q = p up to rounding: the ratio is 1 within an ulp, so any u < 1 - 1e-6 accepts
    res = orc.rejection_sample(
        torch.from_numpy(rng.integers(0, V, B * k).astype(np.int32)), [k] * B, k, probs, logits,
        torch.arange(B, dtype=torch.int32).view(-1, 1), temperature=torch.ones(B),
        all_greedy=False, uniforms=torch.from_numpy(rng.random(B * k) * (1 - 1e-6)),
        exp_noise=torch.ones((B, V)))
    assert (res.output_token_ids[:, k] == np.arange(B)).all()


def test_zero_q_always_rejects():
    # q[d] = 0 rejects even at u = 0; the residual max(p - q, 0) then has all of its mass on
    # the draft id itself (p[1] > q[1] = 0, p[0] < q[0] = 1), so the recovered token is 1
    # and no bonus is appended.
    res = orc.rejection_sample(
        torch.tensor([1], dtype=torch.int32), [1], 1, torch.tensor([[1.0, 0.0]]),
        torch.tensor([[0.0, 10.0]]), torch.tensor([[0]], dtype=torch.int32),
        temperature=torch.ones(1), all_greedy=False, uniforms=torch.tensor([0.0]),
        exp_noise=torch.ones((1, 2)))
    assert res.output_token_ids.tolist() == [[1, -1]]
    assert np.isnan(res.ratio[0])


def test_softmax_matches_float64():
    rng = np.random.default_rng(4)
    x = rng.normal(scale=3.0, size=(8, 1000)).astype(np.float32)
    t = np.full(8, 0.7, dtype=np.float32)
    got = orc.target_probs(torch.from_numpy(x), torch.from_numpy(t)).numpy()
    xd = x.astype(np.float64) / np.float64(0.7)
    ref = np.exp(xd - xd.max(-1, keepdims=True))
    ref /= ref.sum(-1, keepdims=True)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-12)


def test_argmax_is_first_index_with_ties():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0]])
    res = orc.rejection_sample(torch.tensor([0, 3], dtype=torch.int32), [1, 1], 1, None, x,
                               torch.tensor([[9], [9]], dtype=torch.int32), all_greedy=True)
    assert res.output_token_ids[:, 0].tolist() == [1, 0]
    assert np.argmax(x.numpy(), -1).tolist() == [1, 0]


def test_recovered_argmax_matches_float64_brute_force():
    rng = np.random.default_rng(5)
    n, V = 2000, 7
    p = rng.dirichlet(np.ones(V), size=n).astype(np.float32)
    q = rng.dirichlet(np.ones(V), size=n).astype(np.float32)
    e = rng.exponential(size=(n, V)).astype(np.float32)
    ids = orc.recovered_token_ids(orc.recovered_scores(
        torch.from_numpy(p), torch.from_numpy(q), torch.zeros(n, dtype=torch.int32),
        torch.from_numpy(e), [1] * n)).numpy()
    w = np.maximum(p.astype(np.float64) - q.astype(np.float64), 0.0) / e.astype(np.float64)
    brute = []
    for row in w:
        best, bi = -1.0, 0
        for v, s in enumerate(row):
            if s > best:
                best, bi = s, v
        brute.append(bi)
    brute = np.array(brute)
    # identical except where the float64 and fp32 scores tie within rounding
    diff = np.nonzero(brute != ids)[0]
    for i in diff:
        top = np.sort(w[i])[-2:]
        assert top[1] - top[0] <= 1e-6 * top[1]


def test_synthetic_greedy_uses_rates():
    # greedy synthetic: accept iff u < c_pos and d >= 0; replacement is the argmax
    x = torch.tensor([[0.0, 5.0, 0.0]] * 3)
    res = orc.rejection_sample(torch.tensor([2, 2, -1], dtype=torch.int32), [3], 3, None, x,
                               torch.tensor([[0]], dtype=torch.int32), all_greedy=True,
                               uniforms=torch.tensor([0.1, 0.2, 0.0], dtype=torch.float64),
                               synthetic_rates=torch.tensor([0.5, 0.5, 0.5]))
    assert res.output_token_ids.tolist() == [[2, 2, 1, -1]]


def test_compare_counts_only_near_ties():
    res = orc.OracleResult(np.array([[3, -1]], dtype=np.int32), np.array([0.5]),
                           np.array([0.5 + 1e-9]), np.array([1.0]), np.array([0.1]),
                           np.array([False]))
    rep = orc.compare(np.array([[7, 8]], dtype=np.int32), res, [7], [1])
    assert rep.accept_flips == 1 and not rep.unexplained
    rep = orc.compare(np.array([[4, -1]], dtype=np.int32), res, [7], [1])
    assert rep.unexplained


def test_recovered_window_covers_fp32_softmax_disagreement():
    """The near-tie window of oracle.compare assumes two fp32 evaluations of one softmax agree
    to 2^-22 (|x / T| + |M / T| + |ln p| + 16) relative.  Check that on vocabulary-sized
    rows: torch's fp32
    softmax of x / T (the oracle) against an fp32 evaluation in the kernel's form, raw
    maximum M, c1 = fl(log2(e) / T), S = sum of exp2((x - M) c1) in a different order, and
    p = exp2((x - M) c1 - log2 S)."""
    g = torch.Generator().manual_seed(77)
    V = 151936
    worst = 0.0
    for T in (0.3, 0.8, 1.0, 1.5):
        x = torch.randn(4, V, generator=g) * 2.0
        p_torch = torch.softmax(x / T, dim=-1).double().numpy()
        xf = x.numpy().astype(np.float32)
        c1 = np.float32(1.4426950408889634 / T)
        m = xf.max(axis=1, keepdims=True)
        z = ((xf - m) * c1).astype(np.float32)
        e = np.exp2(z).astype(np.float32)
        # a different summation order: 512 interleaved partial sums, then combined
        s = e.reshape(4, -1, 8).sum(axis=1, dtype=np.float32).sum(axis=1, dtype=np.float32)
        nl = (-np.log2(s.astype(np.float64))).astype(np.float32)
        p_kernel = np.exp2((z + nl[:, None]).astype(np.float32)).astype(np.float64)
        big = p_torch >= 1e-30
        rel = np.abs(p_kernel[big] / p_torch[big] - 1.0)
        scale = (np.abs(xf / np.float32(T)) + np.abs(m / np.float32(T)))[big]
        bound = 2.0 ** -22 * (scale + np.abs(np.log(p_torch[big])) + 16.0)
        assert (rel <= bound).all(), (T, (rel / bound).max())
        worst = max(worst, float((rel / bound).max()))
    print(f"worst disagreement / window eps = {worst:.3f}")


def test_recovered_window_shape():
    from oracle.rejection import recovered_window
    # point-mass drafts (q = 0): the p-error alone, twice
    assert recovered_window(0.5, 0.0) == pytest.approx(2 * 2.0 ** -22 * (np.log(2) + 16))
    # cancellation: q = 0.9 p amplifies by 10
    assert recovered_window(0.1, 0.09) == pytest.approx(
        10 * recovered_window(0.1, 0.0), rel=1e-9)
    assert recovered_window(0.1, 0.1) == 0.0 and recovered_window(0.0, 0.0) == 0.0
