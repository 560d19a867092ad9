"""The bonus-row sampler oracle (oracle/sampler.py) against the reference's known answers
for min_p, its place after the temperature, greedy rows and the bonus-row penalty history,
and against closed forms of the exponential race and the processed modes."""

import json
import math
from pathlib import Path

import pytest
import torch

from mvsd.testing.spec_metadata import sampling_metadata
from oracle import sampler as osm

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


def kat_metadata(case, device="cpu"):
    kw = {key: case[key] for key in CASE_KEYS if key in case}
    return sampling_metadata(case["temperatures"], case["drafts"], device=device,
                             logprobs_mode=case["mode"], **kw)


def check_values(case, ids, lps):
    for e in case.get("expect_values", []):
        column = ids[e["row"]].tolist().index(e["token"])
        got, want = float(lps[e["row"], column]), kat_value(e["value"])
        if want == -math.inf:
            assert got == -math.inf
        else:
            assert abs(got - want) <= case["tolerance"]


@pytest.mark.parametrize("case", KATS["sampler"], ids=lambda c: c["name"])
def test_oracle_kats(case):
    rows = kat_rows(case)
    if case["op"] == "apply_min_p":
        out = osm.apply_min_p(rows, None if case["min_p"] is None else torch.tensor(case["min_p"]))
        want = torch.tensor([[kat_value(v) for v in r] for r in case["expect_rows"]])
        assert torch.equal(out, want)
        return
    sm = kat_metadata(case)
    noise = torch.empty(rows.shape).exponential_(generator=torch.Generator().manual_seed(5))
    sampled, (ids, lps, _), _ = osm.forward(rows, sm, noise, case["mode"],
                                            case.get("predict_bonus_token", False))
    if "expect_sampled" in case:
        assert sampled.tolist() == case["expect_sampled"]
    check_values(case, ids, lps)


def test_race_is_argmax_of_probs_over_noise():
    """With unit noise the race picks the argmax; a row with one finite entry always picks it;
    the winner maximises p_i / E_i computed by hand."""
    x = torch.tensor([[0.0, 2.0, 1.0], [-math.inf, 3.0, -math.inf], [1.0, 1.5, 0.5]])
    sm = sampling_metadata([1.0, 1.0, 1.0], [[], [], []])
    noise = torch.tensor([[1.0, 1.0, 1.0], [0.1, 9.0, 0.1], [0.05, 4.0, 1.0]])
    sampled, _, scores = osm.sample(x, sm, noise, "raw_logprobs")
    p2 = [math.exp(v) / sum(math.exp(u) for u in (1.0, 1.5, 0.5)) for v in (1.0, 1.5, 0.5)]
    hand = max(range(3), key=lambda i: p2[i] / [0.05, 4.0, 1.0][i])
    assert sampled.tolist() == [1, 1, hand]
    assert abs(float(scores[2, hand]) - p2[hand] / [0.05, 4.0, 1.0][hand]) < 1e-6


def test_mixed_batch_greedy_rows_ignore_temperature_and_noise():
    x = torch.tensor([[0.0, 5.0, 1.0], [0.0, 5.0, 1.0]])
    sm = sampling_metadata([0.0, 1.0], [[], []])
    noise = torch.tensor([[1.0, 1e9, 1.0], [1.0, 1e9, 1e-9]])   # random row 1 -> token 2
    sampled, _, _ = osm.sample(x, sm, noise, "raw_logprobs")
    assert sampled.tolist() == [1, 2]


def test_processed_logprobs_are_log_softmax_of_the_divided_masked_rows():
    x = torch.tensor([[2.0, 1.0, 0.0, -1.0]])
    sm = sampling_metadata([0.5], [[]], top_k=[2], max_num_logprobs=-1,
                           logprobs_mode="processed_logprobs")
    _, full, _ = osm.forward(x, sm, torch.ones(1, 4), "processed_logprobs")
    z = math.log(math.exp(4.0) + math.exp(2.0))
    assert torch.allclose(full, torch.tensor([[4.0 - z, 2.0 - z, -math.inf, -math.inf]]))


def test_min_tokens_masks_stop_tokens_until_reached():
    x = torch.zeros((2, 5))
    sm = sampling_metadata([0.0, 0.0], [[], []], output_token_ids=[[1], [1, 2, 3]],
                           min_tokens=[3, 3], stop_token_ids=[[0, 4], [0, 4]],
                           max_num_logprobs=-1, logprobs_mode="processed_logits")
    _, full, _ = osm.forward(x, sm, None, "processed_logits")
    assert full[0].tolist() == [-math.inf, 0.0, 0.0, 0.0, -math.inf]
    assert full[1].tolist() == [0.0] * 5
