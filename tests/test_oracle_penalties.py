"""The logits-processor oracle (oracle/penalties.py) against the reference's known answers and
the closed forms of the formulas, and the host-side history summaries of the product path
(per-request distinct tokens, committed counts, prompt flags, min_tokens rows) against the
oracle, without a GPU.

The host summaries are checked by applying them with a numpy statement of the kernel's
per-entry arithmetic (include/mvsd.h, mvsd_apply_logits_processors) and comparing bit for bit
with the oracle on random histories."""

import json
import math
from pathlib import Path

import numpy as np
import pytest

from mvsd.sample.rejection_sampler import _min_tokens_rows, _penalty_entries
from mvsd.sample.metadata import SamplingMetadata
from oracle import penalties as opn

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


def _value(text):
    return {"ln2-1": math.log(2.0) - 1.0, "ln2-2": math.log(2.0) - 2.0, "0": 0.0,
            "-inf": -math.inf, "5": 5.0}[text]


def kat_inputs(case):
    if "log_of_rows" in case:
        logits = np.log(np.asarray(case["log_of_rows"], dtype=np.float32))
    else:
        logits = np.asarray(case["rows"], dtype=np.float32)
    num_draft = [len(d) for d in case["drafts"]]
    kwargs = dict(no_penalties="frequency_penalties" not in case,
                  prompt_token_ids=case["prompt_token_ids"],
                  output_token_ids=case["output_token_ids"], spec_token_ids=case["drafts"],
                  presence=case.get("presence_penalties"),
                  frequency=case.get("frequency_penalties"),
                  repetition=case.get("repetition_penalties"),
                  min_tokens=case["min_tokens"], stop_token_ids=case["stop_token_ids"])
    return logits, num_draft, kwargs


@pytest.mark.parametrize("case", KATS["logits_processors"], ids=lambda c: c["name"])
def test_oracle_matches_reference_kats(case):
    logits, num_draft, kwargs = kat_inputs(case)
    out = opn.apply_logits_processors(logits, num_draft, **kwargs)
    for e in case["expected"]:
        want = _value(e["value"])
        got = float(out[e["row"], e["token"]])
        if math.isinf(want):
            assert got == want
        else:
            assert abs(got - want) <= case["tolerance"] + 1e-7


def test_combined_histories_follow_the_draft_prefix():
    rows = opn.combine_outputs_with_spec_tokens([[1], [], [4, 4]], [[5, 6, 7], [], [8]])
    assert rows == [[1], [1, 5], [1, 5, 6], [4, 4]]


def test_penalty_closed_forms():
    """One row, V = 6: token 0 in the prompt only, token 1 three times in the output, token 2
    once, token 3 nowhere; repetition 2, frequency 0.5, presence 0.25."""
    x = np.array([[3.0, -2.0, 1.5, 4.0, -1.0, 0.0]], dtype=np.float32)
    out = opn.apply_all_penalties(x, [[0]], [[1, 1, 2, 1]], [0.25], [0.5], [2.0])
    assert out[0, 0] == np.float32(3.0) * np.float32(0.5)          # prompt: repetition only
    assert out[0, 1] == np.float32(-2.0 * 2.0 - 0.5 * 3 - 0.25)    # negative: times rep
    assert out[0, 2] == np.float32(1.5 * 0.5 - 0.5 * 1 - 0.25)     # positive: divided by rep
    assert out[0, 3] == np.float32(4.0)                             # outside the history
    assert out[0, 4] == np.float32(-1.0) and out[0, 5] == np.float32(0.0)


def test_min_tokens_rows_closed_form():
    x = np.zeros((7, 4), dtype=np.float32)
    out = opn.apply_min_tokens_for_spec_decode(x, [3, 5, 1], [[1, 2], [0], [3]],
                                               [[9], [], [9, 9]], [2, 4, 1])
    masked = np.isinf(out)
    # request 0 (rows 0-1): 3 - 1 = 2 rows; request 1 (rows 2-5): min(5 - 0, 4) = 4 rows;
    # request 2 (row 6): 1 - 2 < 0, none
    assert masked[0, [1, 2]].all() and masked[1, [1, 2]].all()
    assert masked[2:6, 0].all()
    assert masked.sum() == 2 * 2 + 4


def _apply_host_summaries(logits, num_draft, specs, entries, masks, pres, freq, rep):
    """numpy statement of the kernel's per-entry arithmetic over the host summaries."""
    x = logits.copy()
    off, tok, info = entries if entries is not None else (None, None, None)
    row = 0
    for r, k in enumerate(num_draft):
        for j in range(k):
            if off is not None:
                for e in range(off[r], off[r + 1]):
                    t = int(tok[e])
                    u = int(np.uint32(info[e]))
                    cnt = (u & 0x7FFFFFFF) + sum(1 for m in range(j) if specs[r][m] == t)
                    v = x[row, t]
                    if (u >> 31) or cnt > 0:
                        v = np.float32(v * (np.float32(1.0) / np.float32(rep[r])
                                            if v > 0 else np.float32(rep[r])))
                    v = np.float32(v - np.float32(np.float32(freq[r]) * np.float32(cnt)))
                    v = np.float32(v - np.float32(np.float32(pres[r]) * np.float32(cnt > 0)))
                    x[row, t] = v
            if masks is not None and j < masks[0][r]:
                for s in range(masks[1][r], masks[1][r + 1]):
                    x[row, masks[2][s]] = -np.inf
            row += 1
    return x


@pytest.mark.parametrize("seed", range(6))
def test_host_summaries_reproduce_the_oracle(seed):
    rng = np.random.default_rng(seed)
    B, V = 5, 40
    num_draft = [int(k) for k in rng.integers(0, 5, B)]
    prompts = [list(rng.integers(0, V, rng.integers(0, 8))) for _ in range(B)]
    outputs = [list(rng.integers(0, 12, rng.integers(0, 10))) for _ in range(B)]
    specs = [list(rng.integers(0, 12, k)) for k in num_draft]
    pres = rng.uniform(-1, 1, B).astype(np.float32)
    freq = rng.uniform(-1, 1, B).astype(np.float32)
    rep = rng.uniform(0.5, 2, B).astype(np.float32)
    min_tokens = [int(m) for m in rng.integers(0, 12, B)]
    stops = [list(rng.integers(0, V, rng.integers(0, 3))) for _ in range(B)]
    logits = rng.normal(0, 2, (sum(num_draft), V)).astype(np.float32)

    want = opn.apply_logits_processors(
        logits, num_draft, no_penalties=False, prompt_token_ids=prompts,
        output_token_ids=outputs, spec_token_ids=specs, presence=pres, frequency=freq,
        repetition=rep, min_tokens=min_tokens, stop_token_ids=stops)
    sm = SamplingMetadata(temperature=None, all_greedy=True, all_random=False, top_k=None,
                          top_p=None, no_penalties=False, prompt_token_ids=prompts,
                          output_token_ids=outputs, min_tokens=min_tokens,
                          stop_token_ids=stops, spec_token_ids=specs)
    got = _apply_host_summaries(logits, num_draft, specs, _penalty_entries(prompts, outputs, specs),
                                _min_tokens_rows(sm, num_draft), pres, freq, rep)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
