"""GPU parity of the verify-row logits processors (mvsd_apply_logits_processors through
RejectionSampler.apply_logits_processors / apply_penalties) against oracle/penalties.py.

Bar: bit-exact fp32 rows (the kernel performs the reference's fp32 operations in the
reference's order), the reference's known answers, and RejectionSampler.forward with penalties
and min_tokens equal to the oracle pipeline (processors, temperature, rejection sampling) up to
the counted flips oracle.compare allows."""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.outputs import SamplerOutput
from mvsd.sample import rejection_sampler as rs
from mvsd.sample.metadata import SamplingMetadata
from mvsd.testing.spec_metadata import make_metadata
from oracle import penalties as opn
from oracle import rejection as orc

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())


class ArgmaxBonusSampler:
    """Test stand-in for the caller's bonus sampler: argmax of the bonus rows."""

    logprobs_mode = "raw_logprobs"

    def forward(self, logits, sampling_metadata, predict_bonus_token=False,
                logprobs_mode_override=None):
        return SamplerOutput(sampled_token_ids=logits.argmax(-1).to(torch.int32).view(-1, 1))


def _value(text):
    return {"ln2-1": math.log(2.0) - 1.0, "ln2-2": math.log(2.0) - 2.0, "0": 0.0,
            "-inf": -math.inf, "5": 5.0}[text]


def _sm(device, *, temperature=None, prompts=(), outputs=(), specs=(), pres=None, freq=None,
        rep=None, min_tokens=(), stops=(), no_penalties=False):
    t = lambda v: None if v is None else torch.as_tensor(np.asarray(v, np.float32), device=device)
    temp = t(temperature)
    return SamplingMetadata(
        temperature=temp, all_greedy=temp is None, all_random=temp is not None, top_k=None,
        top_p=None, no_penalties=no_penalties, prompt_token_ids=[list(p) for p in prompts],
        output_token_ids=[list(o) for o in outputs], presence_penalties=t(pres),
        frequency_penalties=t(freq), repetition_penalties=t(rep),
        min_tokens=list(min_tokens), stop_token_ids=[list(s) for s in stops],
        spec_token_ids=[list(s) for s in specs])


@pytest.mark.parametrize("case", KATS["logits_processors"], ids=lambda c: c["name"])
def test_reference_kats_on_device(case, device):
    if "log_of_rows" in case:
        logits = torch.tensor(case["log_of_rows"], dtype=torch.float32).log()
    else:
        logits = torch.tensor(case["rows"], dtype=torch.float32)
    logits = logits.to(device)
    meta = make_metadata(case["drafts"], device=device)
    sm = _sm(device, prompts=case["prompt_token_ids"], outputs=case["output_token_ids"],
             specs=case["drafts"], pres=case.get("presence_penalties"),
             freq=case.get("frequency_penalties"), rep=case.get("repetition_penalties"),
             min_tokens=case["min_tokens"], stops=case["stop_token_ids"],
             no_penalties="frequency_penalties" not in case)
    out = rs.RejectionSampler(ArgmaxBonusSampler()).apply_logits_processors(logits, sm, meta)
    out = out.cpu()
    for e in case["expected"]:
        want = _value(e["value"])
        got = float(out[e["row"], e["token"]])
        if math.isinf(want):
            assert got == want
        else:
            assert abs(got - want) <= case["tolerance"] + 1e-7


def _random_case(seed, B, V, max_k=6, vocab_hist=None):
    rng = np.random.default_rng(seed)
    hv = vocab_hist or V
    num_draft = [int(k) for k in rng.integers(0, max_k + 1, B)]
    prompts = [list(rng.integers(0, V, rng.integers(0, 40))) for _ in range(B)]
    outputs = [list(rng.integers(0, hv, rng.integers(0, 30))) for _ in range(B)]
    specs = [list(rng.integers(0, hv, k)) for k in num_draft]
    pres = rng.uniform(-1, 1, B).astype(np.float32)
    freq = rng.uniform(-1, 1, B).astype(np.float32)
    rep = rng.uniform(0.5, 2, B).astype(np.float32)
    min_tokens = [int(m) for m in rng.integers(0, 30, B)]
    stops = [list(rng.integers(0, V, rng.integers(0, 4))) for _ in range(B)]
    logits = rng.normal(0, 2, (sum(num_draft), V)).astype(np.float32)
    logits[rng.random(logits.shape) < 0.01] = 0.0          # exact zeros: neither side of > 0
    return num_draft, prompts, outputs, specs, pres, freq, rep, min_tokens, stops, logits


@pytest.mark.parametrize("seed,B,V,hist", [(1, 8, 64, 16), (2, 32, 1000, 50),
                                           (3, 64, 151936, 200), (4, 16, 4096, None)])
def test_processors_bit_exact(device, seed, B, V, hist):
    (num_draft, prompts, outputs, specs, pres, freq, rep, min_tokens, stops,
     logits) = _random_case(seed, B, V, vocab_hist=hist)
    want = opn.apply_logits_processors(
        logits, num_draft, no_penalties=False, prompt_token_ids=prompts,
        output_token_ids=outputs, spec_token_ids=specs, presence=pres, frequency=freq,
        repetition=rep, min_tokens=min_tokens, stop_token_ids=stops)
    drafts = [s for s in specs]
    meta = make_metadata(drafts, device=device)
    sm = _sm(device, prompts=prompts, outputs=outputs, specs=specs, pres=pres, freq=freq,
             rep=rep, min_tokens=min_tokens, stops=stops)
    x = torch.from_numpy(logits).to(device)
    got = rs.RejectionSampler(ArgmaxBonusSampler()).apply_logits_processors(x, sm, meta)
    got = got.cpu().numpy()
    diff = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    detail = [(int(i), float(logits.reshape(-1)[i]), float(got.reshape(-1)[i]),
               float(want.reshape(-1)[i])) for i in diff[:4]]
    assert diff.size == 0, f"{diff.size} entries differ (index, input, got, want): {detail}"


def test_min_tokens_only_and_penalties_only(device):
    (num_draft, prompts, outputs, specs, pres, freq, rep, min_tokens, stops,
     logits) = _random_case(7, 24, 512, vocab_hist=40)
    meta = make_metadata(specs, device=device)
    sampler = rs.RejectionSampler(ArgmaxBonusSampler())
    # min_tokens alone (no_penalties): only the stop-token masks
    want = opn.apply_logits_processors(logits, num_draft, output_token_ids=outputs,
                                       min_tokens=min_tokens, stop_token_ids=stops)
    sm = _sm(device, prompts=prompts, outputs=outputs, specs=specs, min_tokens=min_tokens,
             stops=stops, no_penalties=True)
    got = sampler.apply_logits_processors(torch.from_numpy(logits).to(device), sm, meta)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # penalties alone, with one penalty tensor missing (treated as its no-op value)
    want = opn.apply_logits_processors(logits, num_draft, no_penalties=False,
                                       prompt_token_ids=prompts, output_token_ids=outputs,
                                       spec_token_ids=specs, presence=None, frequency=freq,
                                       repetition=rep)
    sm = _sm(device, prompts=prompts, outputs=outputs, specs=specs, freq=freq, rep=rep)
    got = sampler.apply_logits_processors(torch.from_numpy(logits).to(device), sm, meta)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_apply_penalties_with_per_row_histories(device):
    (num_draft, prompts, outputs, specs, pres, freq, rep, _, _,
     logits) = _random_case(9, 20, 700, vocab_hist=60)
    histories = rs.RejectionSampler._combine_outputs_with_spec_tokens(outputs, specs)
    assert histories == opn.combine_outputs_with_spec_tokens(outputs, specs)
    meta = make_metadata(specs, device=device)
    sm = _sm(device, prompts=prompts, outputs=outputs, specs=specs, pres=pres, freq=freq,
             rep=rep)
    got = rs.RejectionSampler.apply_penalties(torch.from_numpy(logits).to(device), sm, meta,
                                              histories)
    row_prompts = [p for p, k in zip(prompts, num_draft) for _ in range(k)]
    want = opn.apply_all_penalties(logits, row_prompts, histories, np.repeat(pres, num_draft),
                                   np.repeat(freq, num_draft), np.repeat(rep, num_draft))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_forward_with_penalties_and_min_tokens(device, monkeypatch):
    """RejectionSampler.forward on the compact [P + B, V] logits with penalties and min_tokens
    (the processed path: gather, processors, temperature, rejection sampling) against the
    oracle run on the same processed rows with the same uniforms and noise."""
    rng = np.random.default_rng(2027)
    B, V, k = 24, 4096, 4
    drafts = [list(rng.integers(0, 200, k)) for _ in range(B)]
    num_draft = [k] * B
    P = B * k
    prompts = [list(rng.integers(0, 200, 30)) for _ in range(B)]
    outputs = [list(rng.integers(0, 200, rng.integers(0, 20))) for _ in range(B)]
    pres = rng.uniform(0, 1, B).astype(np.float32)
    freq = rng.uniform(0, 1, B).astype(np.float32)
    rep = rng.uniform(1, 2, B).astype(np.float32)
    min_tokens = [int(m) for m in rng.integers(0, 25, B)]
    stops = [list(rng.integers(0, 200, 2)) for _ in range(B)]
    temps = rng.uniform(0.5, 1.2, B).astype(np.float32)
    meta = make_metadata(drafts, device=device)
    # compact logits: each request's K verify rows, then its bonus row; tokens < 200 boosted
    # so that the histories matter
    logits = rng.normal(0, 2, (P + B, V)).astype(np.float32)
    logits[:, :200] += 3.0
    x = torch.from_numpy(logits).to(device)
    draft_probs = torch.softmax(torch.from_numpy(rng.normal(0, 2, (P, V)).astype(np.float32)),
                                -1).to(device)
    uniforms = torch.from_numpy(rng.random(P)).to(device)
    noise = torch.from_numpy(rng.exponential(1.0, (B, V)).astype(np.float32)).to(device)
    monkeypatch.setattr(rs, "generate_uniform_probs", lambda *a, **kw: uniforms)
    monkeypatch.setattr(rs, "generate_exponential_noise", lambda *a, **kw: noise)
    sm = _sm(device, temperature=temps, prompts=prompts, outputs=outputs, specs=drafts,
             pres=pres, freq=freq, rep=rep, min_tokens=min_tokens, stops=stops)
    out = rs.RejectionSampler(ArgmaxBonusSampler())(meta, draft_probs, x, sm).sampled_token_ids

    verify_rows = logits[meta.target_logits_indices.cpu().numpy()]
    processed = opn.apply_logits_processors(
        verify_rows, num_draft, no_penalties=False, prompt_token_ids=prompts,
        output_token_ids=outputs, spec_token_ids=drafts, presence=pres, frequency=freq,
        repetition=rep, min_tokens=min_tokens, stop_token_ids=stops)
    bonus = logits[meta.bonus_logits_indices.cpu().numpy()].argmax(-1).astype(np.int32)
    ref = orc.rejection_sample(meta.draft_token_ids.cpu(), num_draft, meta.max_spec_len,
                               draft_probs.cpu(), torch.from_numpy(processed),
                               torch.from_numpy(bonus).view(-1, 1),
                               temperature=torch.from_numpy(temps), all_greedy=False,
                               uniforms=uniforms.cpu(), exp_noise=noise.cpu(),
                               apply_temperature=True)
    rep_ = orc.compare(out.cpu().numpy(), ref, meta.draft_token_ids.cpu(), num_draft)
    print(f"[forward with processors] requests={rep_.requests} mismatched={rep_.mismatched} "
          f"accept_flips={rep_.accept_flips} recovered_flips={rep_.recovered_flips}", flush=True)
    assert not rep_.unexplained, rep_.unexplained[:5]
    # the processors changed something the sampler saw
    assert not np.array_equal(processed, verify_rows)
