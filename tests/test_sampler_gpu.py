"""GPU parity of the bonus-row Sampler (mvsd_sampler_rows, mvsd_apply_logits_processors,
mvsd_apply_top_k_top_p and mvsd_spec_logprobs behind mvsd.sample.Sampler) against
oracle/sampler.py on the same noise.

Bar: greedy tokens, penalised rows and masks equal the oracle's (the kernels perform the
reference's fp32 operations); a random row's token equals the oracle's or is a near tie of the
race (its oracle score within 1e-5 relative of the winner's); logprob ids and ranks equal the
oracle's and values are within 2e-6 absolute + 1e-6 relative (a float reduction in another
order); the reference's known answers."""

import json
import math
from dataclasses import replace
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.sample import Sampler
from mvsd.sample import rejection_sampler as rs
from mvsd.sample import sampler as smp
from mvsd.testing.spec_metadata import make_metadata, sampling_metadata
from oracle import sampler as osm

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())
CASE_KEYS = ("output_token_ids", "prompt_token_ids", "frequency_penalties",
             "presence_penalties", "repetition_penalties", "max_num_logprobs", "min_p",
             "no_penalties")


def kat_rows(case):
    if "log_of_rows" in case:
        return torch.tensor(case["log_of_rows"], dtype=torch.float32).log()
    return torch.tensor([[float(v) for v in row] for row in case["rows"]], dtype=torch.float32)


def kat_value(v):
    return {"-inf": -math.inf, "ln2-2": math.log(2.0) - 2.0}.get(v, v)


@pytest.mark.parametrize("case", KATS["sampler"], ids=lambda c: c["name"])
def test_reference_kats_on_device(case, device):
    rows = kat_rows(case).to(device)
    if case["op"] == "apply_min_p":
        mp = None if case["min_p"] is None else torch.tensor(case["min_p"], device=device)
        out = Sampler.apply_min_p(rows.clone(), mp).cpu()
        want = torch.tensor([[kat_value(v) for v in r] for r in case["expect_rows"]])
        assert torch.equal(out, want)
        return
    kw = {key: case[key] for key in CASE_KEYS if key in case}
    sm = sampling_metadata(case["temperatures"], case["drafts"], device=device,
                           logprobs_mode=case["mode"], **kw)
    out = Sampler(case["mode"]).forward(rows.clone(), sm,
                                        predict_bonus_token=case.get("predict_bonus_token",
                                                                     False))
    if "expect_sampled" in case:
        assert out.sampled_token_ids.flatten().tolist() == case["expect_sampled"]
    t = out.logprobs_tensors
    for e in case.get("expect_values", []):
        column = t.logprob_token_ids[e["row"]].tolist().index(e["token"])
        got, want = float(t.logprobs[e["row"], column]), kat_value(e["value"])
        assert got == want if want == -math.inf else abs(got - want) <= case["tolerance"]


def test_row_ops_match_torch(device):
    """argmax (lowest index on ties, NaN first), log-softmax with -inf entries, min_p rows."""
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.normal(0, 3, (6, 50000)).astype(np.float32))
    x[1, 100] = x[1, 7] = 40.0                 # tie: lowest index wins
    x[2, 31] = float("nan")                    # NaN is the maximum (torch.argmax)
    x[3, ::3] = -math.inf
    xd = x.to(device)
    assert Sampler.greedy_sample(xd).cpu().tolist() == x.argmax(-1).tolist()
    finite = torch.cat([x[:2], x[3:]])
    got = Sampler.compute_logprobs(finite.to(device)).cpu()
    want = finite.log_softmax(-1)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    m = torch.isfinite(want)
    assert torch.allclose(got[m], want[m], atol=2e-6, rtol=1e-6)
    mp = torch.tensor([0.0, 0.3, 0.01, 1e-4, 0.9], dtype=torch.float32)
    got = Sampler.apply_min_p(finite.to(device).clone(), mp.to(device)).cpu()
    want = osm.apply_min_p(finite, mp)
    assert torch.equal(got, want)


@pytest.mark.parametrize("V,pad", [(1000, 0), (8192, 0), (8193, 3), (151936, 0), (151936, 1),
                                   (20001, 0)])
@pytest.mark.parametrize("with_t", [False, True])
def test_race_matches_float64(device, V, pad, with_t):
    """mvsd_sampler_race (through random_sample) against float64 softmax(fl(x / T)) / E: the
    token is the oracle's argmax or within 1e-5 relative of its score.  Chunk edges (V = 8192,
    8193), a scalar-load path (rows padded to an odd stride), a row with a NaN (every score
    NaN: index 0), a row of -inf (index 0) and a row masked but for a few entries."""
    rng = np.random.default_rng(V + pad + 7 * with_t)
    n = 9
    full = torch.from_numpy(rng.normal(0, 3, (n, V + pad)).astype(np.float32))
    full[1, 5] = float("nan")
    full[2, :] = -math.inf
    full[3, :] = -math.inf
    full[3, [V - 1, V // 2, 7]] = torch.tensor([1.0, 1.5, 0.5])
    x = full[:, :V]
    noise = torch.from_numpy(rng.exponential(1.0, (n, V)).astype(np.float32))
    temps = torch.from_numpy(rng.uniform(0.3, 1.7, n).astype(np.float32))
    temps[4] = 1.0
    xd = full.to(device)[:, :V]
    assert xd.stride(0) == V + pad
    smp_noise = noise.to(device)
    orig = smp.generate_sampler_noise
    smp.generate_sampler_noise = lambda shape, gens, dev: smp_noise
    try:
        got = smp.random_sample(xd, {}, temperature=temps.to(device) if with_t else None)
    finally:
        smp.generate_sampler_noise = orig
    got = got.cpu().tolist()
    v = (x / temps[:, None]) if with_t else x          # fl(x / T), as the kernel divides
    scores = torch.softmax(v.double(), dim=-1) / noise.double()
    assert got[1] == 0 and got[2] == 0
    for r in (0, 3, 4, 5, 6, 7, 8):
        want = int(torch.argmax(scores[r]))
        assert got[r] == want or float(scores[r, got[r]]) >= float(scores[r, want]) * (1 - 1e-5), \
            (r, got[r], want)
    assert got[3] in (V - 1, V // 2, 7)


def _random_case(seed, V, n, mode, num_logprobs, *, greedy_rows=(), top_k=False, top_p=False,
                 min_p=False, penalties=False, min_tokens=False, device=None):
    rng = np.random.default_rng(seed)
    logits = torch.from_numpy(rng.normal(0, 2, (n, V)).astype(np.float32))
    temps = [0.0 if i in greedy_rows else float(rng.uniform(0.5, 1.5)) for i in range(n)]
    drafts = [list(rng.integers(0, 64, int(rng.integers(0, 5)))) for _ in range(n)]
    kw = dict(max_num_logprobs=num_logprobs, logprobs_mode=mode)
    if top_k:
        kw["top_k"] = [int(v) for v in rng.integers(1, 200, n)]
    if top_p:
        kw["top_p"] = [float(v) for v in rng.uniform(0.5, 0.95, n)]
    if min_p:
        kw["min_p"] = [0.0 if i % 3 == 0 else float(rng.uniform(0.001, 0.2)) for i in range(n)]
    if penalties:
        logits[:, :64] += 3.0                   # history tokens near the top of the rows
        kw.update(no_penalties=False,
                  prompt_token_ids=[list(rng.integers(0, 64, 6)) for _ in range(n)],
                  output_token_ids=[list(rng.integers(0, 64, int(rng.integers(0, 8))))
                                    for _ in range(n)],
                  presence_penalties=[float(v) for v in rng.uniform(0, 1, n)],
                  frequency_penalties=[float(v) for v in rng.uniform(0, 1, n)],
                  repetition_penalties=[float(v) for v in rng.uniform(1, 2, n)])
    if min_tokens:
        kw["output_token_ids"] = kw.get("output_token_ids",
                                        [[1] * int(rng.integers(0, 4)) for _ in range(n)])
        kw["min_tokens"] = [int(v) for v in rng.integers(0, 6, n)]
        kw["stop_token_ids"] = [[int(np.argmax(logits[i]))] for i in range(n)]
    noise = torch.from_numpy(rng.exponential(1.0, (n, V)).astype(np.float32))
    return logits, noise, temps, drafts, kw


def _check_tokens(got, want, scores, temps, label):
    for row, (g, w) in enumerate(zip(got, want)):
        if g == w:
            continue
        assert scores is not None and temps[row] >= 1e-5, f"{label}: greedy row {row}: {g} != {w}"
        s = scores[row]
        assert float(s[g]) >= float(s[w]) * (1 - 1e-5), f"{label}: row {row}: {g} != {w}"


CASES = [
    # (mode, num_logprobs, options)
    ("raw_logprobs", None, dict(greedy_rows=(0, 3))),
    ("raw_logprobs", 5, dict(greedy_rows=(1,), penalties=True)),
    ("raw_logits", 0, dict(top_k=True, min_p=True)),
    ("processed_logprobs", 20, dict(greedy_rows=(2,), top_k=True, top_p=True, min_p=True)),
    ("processed_logits", -1, dict(top_k=True, penalties=True, min_tokens=True)),
    ("processed_logprobs", 3, dict(greedy_rows=tuple(range(8)), penalties=True)),
    ("raw_logprobs", 1, dict(min_tokens=True, top_p=True)),
]


@pytest.mark.parametrize("V", [1000, 151936])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-{'+'.join(c[2])}")
@pytest.mark.parametrize("bonus", [False, True])
def test_forward_matches_oracle(device, monkeypatch, V, case, bonus):
    mode, num_logprobs, opts = case
    n = 8
    seed = V + 17 * CASES.index(case) + (1000 if bonus else 0)
    logits, noise, temps, drafts, kw = _random_case(seed, V, n, mode, num_logprobs, **opts)
    sm_dev = sampling_metadata(temps, drafts, device=device, **kw)
    sm_cpu = sampling_metadata(temps, drafts, **kw)
    noise_dev = noise.to(device)
    monkeypatch.setattr(smp, "generate_sampler_noise", lambda *a, **k: noise_dev)
    out = Sampler(mode).forward(logits.to(device), sm_dev, predict_bonus_token=bonus)
    want_tok, want_lp, scores = osm.forward(logits, sm_cpu, noise, mode, bonus)
    label = f"V={V} {mode} k={num_logprobs} {opts} bonus={bonus}"
    got_tok = out.sampled_token_ids.flatten().cpu().tolist()
    assert out.sampled_token_ids.shape == (n, 1) and out.sampled_token_ids.dtype == torch.int32
    _check_tokens(got_tok, want_tok.tolist(), scores, temps, label)
    t = out.logprobs_tensors
    if num_logprobs is None:
        assert t is None
        return
    if num_logprobs == -1:
        got = t.logprobs.cpu()
        assert torch.equal(torch.isinf(got), torch.isinf(want_lp)), label
        m = torch.isfinite(want_lp)
        assert torch.allclose(got[m], want_lp[m], atol=2e-6, rtol=1e-6), label
        return
    if got_tok != want_tok.tolist():
        # a near tie went the other way: the logprobs follow the device's token
        from oracle import logprobs as olp
        _, kept, _ = osm.forward(logits, replace(sm_cpu, max_num_logprobs=-1), noise, mode,
                                 bonus)
        want_lp = olp.gather_logprobs(kept, num_logprobs, torch.tensor(got_tok))
    ids, lps, ranks = (x.cpu() for x in tuple(t)[:3])
    assert torch.equal(ids, want_lp[0]), label
    assert torch.equal(ranks, want_lp[2]), label
    assert torch.allclose(lps, want_lp[1], atol=2e-6, rtol=1e-6), label


def test_generators_give_reproducible_rows(device):
    """Rows with their own generators draw the same noise, and so the same tokens, when the
    generators are re-seeded; a row's token does not depend on other rows."""
    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.normal(0, 1, (4, 5000)).astype(np.float32)).to(device)

    def run(rows):
        gens = {i: torch.Generator(device=device).manual_seed(100 + i) for i in range(4)}
        sm = sampling_metadata([1.0] * 4, [[]] * 4, device=device, generators=gens)
        return Sampler().forward(rows.clone(), sm).sampled_token_ids.flatten().tolist()

    first = run(x)
    assert run(x) == first
    y = x.clone()
    y[0] = torch.roll(y[0], 7)
    assert run(y)[1:] == first[1:]


def test_rejection_sampler_with_device_sampler(device, monkeypatch):
    """RejectionSampler(Sampler()) end to end: greedy drafts equal to each verify row's argmax
    are all accepted, and each bonus token is the oracle's bonus-row sample with the penalty
    history extended by every draft."""
    rng = np.random.default_rng(44)
    B, k, V = 6, 3, 4096
    target = torch.from_numpy(rng.normal(0, 2, (B * (k + 1), V)).astype(np.float32))
    target[:, :32] += 4.0
    drafts = [[int(target[i * (k + 1) + j].argmax()) for j in range(k)] for i in range(B)]
    meta = make_metadata(drafts, device=device)
    kw = dict(no_penalties=False, prompt_token_ids=[[1, 2, 3]] * B,
              output_token_ids=[list(rng.integers(0, 32, 3)) for _ in range(B)],
              frequency_penalties=[0.05] * B, presence_penalties=[0.02] * B,
              repetition_penalties=[1.1] * B)
    sm = sampling_metadata([0.0] * B, drafts, device=device, **kw)
    # drafts chosen on the unpenalised rows: check the ones the penalised rows still accept
    out = rs.RejectionSampler(Sampler())(meta, None, target.to(device), sm)
    bonus_rows = target[meta.bonus_logits_indices.cpu()]
    want, _, _ = osm.forward(bonus_rows, sampling_metadata([0.0] * B, drafts, **kw), None,
                             "raw_logprobs", predict_bonus_token=True)
    got = out.sampled_token_ids.cpu()
    accepted = [i for i in range(B) if bool((got[i, :k] == torch.tensor(drafts[i])).all())]
    assert accepted, "no request accepted all its drafts"
    for i in accepted:
        assert int(got[i, k]) == int(want[i]), f"request {i}"


def test_caller_rows_after_forward(device):
    """Which rows the caller holds after Sampler.forward on fp32 logits.  Where something reads
    the divided rows (top-k here), they are divided in place, as in the reference
    (sampler.py:260 ``logits.div_``).  Where nothing does (no min_p, top-k or top-p, raw
    logprobs), the race kernel divides each value as it reads it and the caller's rows stay as
    they were: this build's documented difference, which saves a [B, V] read and write."""
    rng = np.random.default_rng(61)
    temps = [0.7, 1.3, 0.0, 2.0]
    x = torch.from_numpy(rng.normal(0, 2, (4, 3000)).astype(np.float32)).to(device)

    rows = x.clone()
    Sampler().forward(rows, sampling_metadata(temps, [[]] * 4, device=device))
    assert torch.equal(rows, x)

    rows = x.clone()
    Sampler().forward(rows, sampling_metadata(temps, [[]] * 4, device=device, top_k=[50] * 4))
    divisor = torch.tensor([t if t >= 1e-5 else 1.0 for t in temps], device=device)
    divided = x / divisor.unsqueeze(1)
    kept = torch.isfinite(rows)
    assert torch.equal(rows[kept], divided[kept])
    assert kept.sum(1).tolist() == [50] * 4


class _GenericPathSampler(Sampler):
    """The device sampler under another type: RejectionSampler then takes its generic path
    (gathered bonus rows through Sampler.forward)."""


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("temps_kind", ["random", "mixed", "greedy"])
def test_forward_race_only_path_equals_generic_path(device, dtype, temps_kind):
    """RejectionSampler(Sampler()).forward without processors or constraints reads the bonus
    rows in place in one race launch; from the same RNG state (global and per-request
    generators) it must give exactly the generic path's tokens: the same draws in the same
    order, the same keys."""
    rng = np.random.default_rng(62)
    B, V = 48, 5000
    ks = [int(k) for k in rng.integers(0, 5, B)]
    drafts = [list(map(int, rng.integers(0, V, k))) for k in ks]
    meta = make_metadata(drafts, device=device)
    rows = sum(ks) + B
    logits = torch.from_numpy(rng.normal(0, 2, (rows, V)).astype(np.float32)).to(device, dtype)
    for i, d in enumerate(drafts):  # make acceptance likely: drafts near the top of their rows
        for j, tok in enumerate(d):
            logits[int(meta.target_logits_indices[sum(ks[:i]) + j]), tok] += 6.0
    temps = {"random": [float(t) for t in rng.uniform(0.3, 1.5, B)],
             "mixed": [0.0 if i % 3 == 0 else float(rng.uniform(0.3, 1.5)) for i in range(B)],
             "greedy": [0.0] * B}[temps_kind]
    P = sum(ks)
    probs = torch.softmax(torch.from_numpy(rng.normal(0, 2, (P, V)).astype(np.float32)), -1)
    probs = probs.to(device)

    def run(sampler):
        gens = {i: torch.Generator(device=device).manual_seed(500 + i) for i in range(0, B, 5)}
        sm = sampling_metadata(temps, drafts, device=device, generators=gens)
        torch.manual_seed(77)
        return rs.RejectionSampler(sampler)(meta, probs, logits, sm).sampled_token_ids

    fast = run(Sampler())
    generic = run(_GenericPathSampler())
    assert torch.equal(fast, generic)
    got = fast.cpu().numpy()
    assert (got[:, 0] >= 0).all()
    if temps_kind != "greedy":
        assert (got[np.array(ks) > 0, 1] >= 0).any()  # some request accepted a draft


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_race_rows_in_place(device, dtype):
    """mvsd_sampler_race_rows on rows picked by index in a larger 16/32-bit tensor, greedy rows
    (temperature below 1e-5) among random ones, against float64 softmax(fl(x / T)) / E on the
    upcast rows (within 1e-5 relative of the winner's score) and the exact argmax for greedy
    rows; without noise every row is greedy."""
    rng = np.random.default_rng(63)
    V, n = 20001, 12
    table = torch.from_numpy(rng.normal(0, 3, (40, V)).astype(np.float32)).to(dtype)
    idx = torch.from_numpy(rng.choice(40, n, replace=False).astype(np.int32))
    x = table[idx.long()].float()
    noise = torch.from_numpy(rng.exponential(1.0, (n, V)).astype(np.float32))
    temps = torch.from_numpy(rng.uniform(0.3, 1.7, n).astype(np.float32))
    temps[[2, 7]] = 0.0
    temps[5] = 1e-6
    got = smp.race_rows(table.to(device), idx.to(device), noise.to(device),
                        temps.to(device)).cpu().tolist()
    for r in range(n):
        if temps[r] < 1e-5:
            assert got[r] == int(torch.argmax(x[r])), r
            continue
        scores = torch.softmax((x[r] / temps[r]).double(), -1) / noise[r].double()
        want = int(torch.argmax(scores))
        assert got[r] == want or float(scores[got[r]]) >= float(scores[want]) * (1 - 1e-5), r
    greedy = smp.race_rows(table.to(device), idx.to(device), None, temps.to(device))
    assert greedy.cpu().tolist() == [int(torch.argmax(x[r])) for r in range(n)]
