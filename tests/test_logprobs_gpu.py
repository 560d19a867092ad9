"""GPU parity of the speculative logprobs (mvsd_spec_logprobs through
RejectionSampler._get_logprobs_tensors / forward / parse_output) against oracle/logprobs.py.

Bar: the token column, top-k ids and ranks equal the oracle's (random fp32 rows have no ties);
logprob values within 2e-6 absolute + 1e-6 relative (the log-sum is a float reduction in a
different order); the reference's known answers for row indexing and parse_output filtering."""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.outputs import LogprobsTensors, SamplerOutput
from mvsd.sample import rejection_sampler as rs
from mvsd.sample.metadata import SamplingMetadata
from mvsd.testing.spec_metadata import make_metadata
from oracle import logprobs as olp

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


class BonusSampler:
    """Test stand-in for the caller's sampler: argmax of the bonus rows; with
    max_num_logprobs=-1 it hands the bonus rows back as its logprobs, as the reference's
    Sampler does under the raw_logits / processed_logits override."""

    def __init__(self, mode="raw_logprobs"):
        self.logprobs_mode = mode

    def forward(self, logits, sampling_metadata, predict_bonus_token=False,
                logprobs_mode_override=None):
        tensors = None
        if sampling_metadata.max_num_logprobs == -1:
            tensors = LogprobsTensors(torch.empty(0), logits.float(), torch.empty(0))
        return SamplerOutput(sampled_token_ids=logits.argmax(-1).to(torch.int32).view(-1, 1),
                             logprobs_tensors=tensors)


def hand_log_softmax(row):
    top = max(row)
    total = sum(math.exp(v - top) for v in row if v != -math.inf)
    return [v - top - math.log(total) for v in row]


def kat_rows(case):
    if "log_of_rows" in case:
        return torch.tensor(case["log_of_rows"], dtype=torch.float32).log()
    return torch.tensor(case["rows"], dtype=torch.float32)


@pytest.mark.parametrize("case", KATS["spec_logprobs"], ids=lambda c: c["name"])
def test_reference_kats_on_device(case, device):
    meta = make_metadata(case["drafts"], device=device)
    logits = kat_rows(case).to(device)
    sampler = rs.RejectionSampler(BonusSampler())
    sampled = torch.tensor(case["sampled"], dtype=torch.int32, device=device)
    t = sampler._get_logprobs_tensors(case["k"], meta, logits, logits[meta.target_logits_indices],
                                      logits[meta.bonus_logits_indices], sampled)
    rows = kat_rows(case)
    if "expect_token_column" in case:
        assert t.logprob_token_ids[:, 0].cpu().tolist() == case["expect_token_column"]
    for e in case.get("expect_logprob_of", []):
        want = hand_log_softmax(rows[e["row"]].tolist())[e["token"]]
        assert abs(t.logprobs[e["slot"], 0].item() - want) <= case["tolerance"]
    if "expect_parsed" in case:
        parsed, lists = rs.RejectionSampler.parse_output(sampled, case["vocab"],
                                                         logprobs_tensors=t)
        assert parsed == case["expect_parsed"]
        assert lists.cu_num_generated_tokens == case["expect_cu"]
        if "expect_shape" in case:
            assert list(lists.logprob_token_ids.shape) == case["expect_shape"]
        if "expect_filtered_token_column" in case:
            assert lists.logprob_token_ids[:, 0].tolist() == case["expect_filtered_token_column"]
        for e in case.get("expect_filtered_logprob_of", []):
            want = hand_log_softmax(rows[e["row"]].tolist())[e["token"]]
            assert lists.logprob_token_ids[e["filtered_slot"], 0] == e["token"]
            assert abs(lists.logprobs[e["filtered_slot"], 0] - want) <= case["tolerance"]


def _check(got, want, label):
    """ids exact; ranks exact except by at most the oracle's rank slack (entries within 4 ulp
    of the sampled token's logprob, which either fp32 evaluation may round onto either side);
    logprobs within 2e-6 absolute."""
    ids, lps, ranks = (x.cpu() for x in tuple(got)[:3])
    wids, wlps, wranks = want[:3]
    assert torch.equal(ids, wids), f"{label}: ids differ"
    if len(want) > 3 and not torch.equal(ranks, wranks):
        diff = (ranks - wranks).abs()
        slack = want[3]
        assert (diff <= slack).all(), f"{label}: ranks differ beyond the rounding slack"
        print(f"[{label}] {int((diff > 0).sum())} ranks differ within the rounding slack",
              flush=True)
    else:
        assert torch.equal(ranks, wranks), f"{label}: ranks differ"
    assert torch.allclose(lps, wlps, atol=2e-6, rtol=1e-6), \
        f"{label}: max |diff| {float((lps - wlps).abs().max())}"


@pytest.mark.parametrize("k", [0, 1, 5, 20, 32, 33, 50, 100])
@pytest.mark.parametrize("V,mode", [(1000, "raw_logprobs"), (151936, "raw_logprobs"),
                                    (4096, "raw_logits"), (151936, "processed_logprobs")])
def test_random_rows_match_oracle(device, k, V, mode):
    rng = np.random.default_rng(k * 1000 + V % 997)
    drafts = [list(rng.integers(0, V, n)) for n in [3, 0, 5, 1, 4, 2]]
    meta = make_metadata(drafts, device=device)
    B, W = len(drafts), meta.max_spec_len + 1
    logits = torch.from_numpy(rng.normal(0, 2, (meta.target_logits_indices.numel()
                                               + B, V)).astype(np.float32)).to(device)
    sampled = torch.from_numpy(rng.integers(-1, V, (B, W)).astype(np.int32)).to(device)
    target = logits[meta.target_logits_indices]
    bonus = logits[meta.bonus_logits_indices]
    sampler = rs.RejectionSampler(BonusSampler(mode))
    got = sampler._get_logprobs_tensors(k, meta, logits, target, bonus, sampled)
    want = olp.get_logprobs_tensors(k, meta.cu_num_sampled_tokens, meta.target_logits_indices,
                                    meta.bonus_logits_indices, target.cpu(), bonus.cpu(),
                                    sampled.cpu(), logits_mode=mode.endswith("logits"),
                                    return_slack=True)
    _check(got, want, f"k={k} V={V} {mode}")
    # the raw modes can read the verify rows straight from the compact logits
    if mode.startswith("raw"):
        got2 = sampler._get_logprobs_tensors(k, meta, logits, None, bonus, sampled)
        _check(got2, want, f"k={k} V={V} {mode} via target rows")


@pytest.mark.parametrize("mode", ["raw_logprobs", "processed_logprobs", "raw_logits"])
def test_forward_with_logprobs(device, monkeypatch, mode):
    """RejectionSampler.forward with max_num_logprobs: the filtered logprobs hold one row per
    delivered token, whose token column is that token and whose values come from its row."""
    rng = np.random.default_rng(31)
    B, V, k = 12, 2048, 4
    drafts = [list(rng.integers(0, 50, k)) for _ in range(B)]
    meta = make_metadata(drafts, device=device)
    P = B * k
    logits = rng.normal(0, 2, (P + B, V)).astype(np.float32)
    logits[:, :50] += 4.0
    x = torch.from_numpy(logits).to(device)
    temps = torch.full((B,), 0.7, dtype=torch.float32, device=device)
    draft_probs = torch.softmax(torch.from_numpy(rng.normal(0, 2, (P, V)).astype(np.float32)),
                                -1).to(device)
    uniforms = torch.from_numpy(rng.random(P)).to(device)
    noise = torch.from_numpy(rng.exponential(1.0, (B, V)).astype(np.float32)).to(device)
    monkeypatch.setattr(rs, "generate_uniform_probs", lambda *a, **kw: uniforms)
    monkeypatch.setattr(rs, "generate_exponential_noise", lambda *a, **kw: noise)
    sm = SamplingMetadata(temperature=temps, all_greedy=False, all_random=True, top_k=None,
                          top_p=None, max_num_logprobs=3, logprobs_mode=mode,
                          prompt_token_ids=[[] for _ in range(B)],
                          output_token_ids=[[] for _ in range(B)])
    out = rs.RejectionSampler(BonusSampler(mode))(meta, draft_probs, x, sm)
    parsed, lists = rs.RejectionSampler.parse_output(out.sampled_token_ids, V,
                                                     logprobs_tensors=out.logprobs_tensors)
    assert lists.cu_num_generated_tokens[-1] == sum(len(r) for r in parsed)
    assert lists.logprob_token_ids[:, 0].tolist() == [t for r in parsed for t in r]
    # the oracle on the rows the mode reports: raw rows, or the temperature-divided rows
    target = torch.from_numpy(logits[meta.target_logits_indices.cpu().numpy()])
    if mode.startswith("processed"):
        target = target / 0.7
    want = olp.get_logprobs_tensors(3, meta.cu_num_sampled_tokens, meta.target_logits_indices,
                                    meta.bonus_logits_indices, target,
                                    torch.from_numpy(logits[meta.bonus_logits_indices.cpu().numpy()]),
                                    out.sampled_token_ids.cpu(), logits_mode=mode.endswith("logits"))
    _check((out.logprobs_tensors.logprob_token_ids, out.logprobs_tensors.logprobs,
            out.logprobs_tensors.selected_token_ranks), want, f"forward {mode}")


def test_full_vocabulary_logprobs_are_refused(device):
    meta = make_metadata([[1, 2]], device=device)
    logits = torch.zeros((3, 8), device=device)
    sm = SamplingMetadata(temperature=None, all_greedy=True, all_random=False, top_k=None,
                          top_p=None, max_num_logprobs=-1, prompt_token_ids=[[]])
    with pytest.raises(NotImplementedError):
        rs.RejectionSampler(BonusSampler())(meta, None, logits, sm)


@pytest.mark.parametrize("V", [1000, 151936])
def test_masked_rows_match_oracle(device, V):
    """Rows whose entries are mostly -inf (processed rows after top-k / top-p / min_p): the
    masked entries add nothing to the log-sum, whichever lane holds them."""
    rng = np.random.default_rng(V)
    drafts = [[1, 2, 3], [], [4, 5]]
    meta = make_metadata(drafts, device=device)
    B, W = len(drafts), meta.max_spec_len + 1
    n_rows = meta.target_logits_indices.numel() + B
    logits = torch.from_numpy(rng.normal(0, 2, (n_rows, V)).astype(np.float32))
    keep = torch.from_numpy(rng.random((n_rows, V)) < 0.05)
    keep[:, 3] = True
    logits = torch.where(keep, logits, torch.full_like(logits, -math.inf)).to(device)
    sampled = torch.from_numpy(rng.integers(0, 4, (B, W)).astype(np.int32)).to(device)
    target = logits[meta.target_logits_indices]
    bonus = logits[meta.bonus_logits_indices]
    sampler = rs.RejectionSampler(BonusSampler("processed_logprobs"))
    got = sampler._get_logprobs_tensors(5, meta, logits, target, bonus, sampled)
    want = olp.get_logprobs_tensors(5, meta.cu_num_sampled_tokens, meta.target_logits_indices,
                                    meta.bonus_logits_indices, target.cpu(), bonus.cpu(),
                                    sampled.cpu())
    assert not torch.isnan(got.logprobs).any()
    _check(got, want, f"masked V={V}")


@pytest.mark.parametrize("k,V", [(64, 64), (200, 257), (70, 151936)])
def test_large_k_with_ties_match_oracle(device, k, V):
    """k above one 32-key round (up to k = V), on rows with heavy ties, so that round
    boundaries fall inside runs of equal values (order: value, then index)."""
    rng = np.random.default_rng(k + V)
    drafts = [list(rng.integers(0, V, n)) for n in [2, 3, 0, 1]]
    meta = make_metadata(drafts, device=device)
    B, W = len(drafts), meta.max_spec_len + 1
    rows = meta.target_logits_indices.numel() + B
    logits = torch.from_numpy(rng.integers(0, 5, (rows, V)).astype(np.float32)).to(device)
    sampled = torch.from_numpy(rng.integers(-1, V, (B, W)).astype(np.int32)).to(device)
    target = logits[meta.target_logits_indices]
    bonus = logits[meta.bonus_logits_indices]
    sampler = rs.RejectionSampler(BonusSampler("raw_logprobs"))
    got = sampler._get_logprobs_tensors(k, meta, logits, target, bonus, sampled)
    want = olp.get_logprobs_tensors(k, meta.cu_num_sampled_tokens, meta.target_logits_indices,
                                    meta.bonus_logits_indices, target.cpu(), bonus.cpu(),
                                    sampled.cpu(), logits_mode=False, return_slack=True)
    _check(got, want, f"ties k={k} V={V}")
