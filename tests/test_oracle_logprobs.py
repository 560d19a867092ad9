"""The speculative-logprobs oracle (oracle/logprobs.py) against the reference's known answers
for the row indexing, and against closed forms of log-softmax, top-k and rank."""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.testing.spec_metadata import make_metadata
from oracle import logprobs as olp

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


def hand_log_softmax(row):
    """float64 log-softmax written out (the reference tests' hand_log_softmax)."""
    top = max(row)
    total = sum(math.exp(v - top) for v in row if v != -math.inf)
    return [v - top - math.log(total) for v in row]


def kat_rows(case):
    if "log_of_rows" in case:
        return torch.tensor(case["log_of_rows"], dtype=torch.float32).log()
    return torch.tensor(case["rows"], dtype=torch.float32)


def oracle_for(case):
    meta = make_metadata(case["drafts"])
    logits = kat_rows(case)
    return olp.get_logprobs_tensors(
        case["k"], meta.cu_num_sampled_tokens, meta.target_logits_indices,
        meta.bonus_logits_indices, logits[meta.target_logits_indices],
        logits[meta.bonus_logits_indices], torch.tensor(case["sampled"], dtype=torch.int32))


@pytest.mark.parametrize("case", [c for c in KATS["spec_logprobs"] if "expect_logprob_of" in c],
                         ids=lambda c: c["name"])
def test_oracle_row_indexing_kats(case):
    ids, lps, _ = oracle_for(case)
    logits = kat_rows(case)
    if "expect_token_column" in case:
        assert ids[:, 0].tolist() == case["expect_token_column"]
    for e in case["expect_logprob_of"]:
        want = hand_log_softmax(logits[e["row"]].tolist())[e["token"]]
        assert abs(lps[e["slot"], 0].item() - want) <= case["tolerance"]


def test_closed_forms():
    rows = torch.tensor([[1.0, 3.0, 3.0, -2.0, 0.5]], dtype=torch.float32)
    lp = olp.compute_logprobs(rows)
    assert abs(float(lp.exp().sum()) - 1.0) < 1e-6
    ids, lps, ranks = olp.gather_logprobs(lp, 3, torch.tensor([2]))
    # sampled token first; top-3 by value then index: the tie 3.0 / 3.0 keeps index order
    assert ids.tolist() == [[2, 1, 2, 0]]
    assert ranks.tolist() == [2]                      # ties count as >=: rank 2 for token 2
    _, _, ranks = olp.gather_logprobs(lp, 0, torch.tensor([3]))
    assert ranks.tolist() == [5]                      # the smallest entry is last
    want = hand_log_softmax(rows[0].tolist())
    assert np.allclose(lps[0].numpy(), [want[2], want[1], want[2], want[0]], atol=1e-6)
    # logits mode reports the values themselves
    ids, lps, ranks = olp.gather_logprobs(rows, 2, torch.tensor([0]))
    assert lps.tolist() == [[1.0, 3.0, 3.0]] and ranks.tolist() == [3]


def test_rank_slack_counts_only_rounding_neighbours():
    from oracle.logprobs import rank_slack
    lp = torch.tensor([[-1.0, np.nextafter(np.float32(-1.0), np.float32(0)), -1.5, -1.0 - 1e-3]],
                      dtype=torch.float32)
    tok = torch.tensor([0])
    assert rank_slack(lp, tok).tolist() == [1]       # the 1-ulp neighbour only
    assert rank_slack(lp, torch.tensor([2])).tolist() == [0]


def test_v2_topk_scores_closed_forms():
    """oracle.logprobs.topk_scores (V2 compute_topk_scores) against float64: the log-softmax
    at the listed ids, the top-k of the raw logits in (value desc, index asc) order with
    planted ties, and the rank as a brute-force count over the raw logits."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 50, generator=g) * 3
    x[1, 7] = x[1, 3] = x[1].max() + 1.0          # tie at the top: index 3 first
    x[2, :] = 0.5                                  # all equal
    tok = torch.tensor([0, 7, 49, 10, 3, 22])
    ids, sc, rk = olp.topk_scores(x, 5, tok)
    x64 = x.double()
    lsm = x64 - x64.max(-1, keepdim=True).values
    lsm = lsm - torch.log(torch.exp(lsm).sum(-1, keepdim=True))
    assert torch.allclose(sc.double(), lsm.gather(-1, ids), atol=2e-6)
    assert ids[:, 0].tolist() == tok.tolist()
    assert ids[1, 1:3].tolist() == [3, 7]
    assert ids[2, 1:].tolist() == [0, 1, 2, 3, 4]
    for n in range(6):
        row = x[n].tolist()
        order = sorted(range(50), key=lambda i: (-row[i], i))[:5]
        assert ids[n, 1:].tolist() == order
        assert int(rk[n]) == sum(v >= row[int(tok[n])] for v in row)
    ids2, sc2, rk2 = olp.topk_scores(x, 0, tok, logits_mode=True)
    assert ids2.shape == (6, 1) and torch.equal(sc2[:, 0], x.gather(-1, tok[:, None])[:, 0])
    assert torch.equal(rk2, rk)
