"""GPU parity of the fused rejection sampler (libmvsd.so through the C ABI) against the
reference's KATs and the CPU oracle, on the benchmark configurations at full size.

Bar: greedy ids bit-exact; random ids bit-exact except accept/reject flips where
|u - p/q| < 1e-6 and recovered-token flips whose top-2 scores tie within 1e-5 relative — both
counted and printed (probabilities differ from torch's softmax by rounding only).
"""

import json
from dataclasses import replace
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.outputs import SamplerOutput
from mvsd.sample import rejection_sampler as rs
from mvsd.sample.metadata import SamplingMetadata
from mvsd.testing import configs
from mvsd.testing.spec_metadata import make_metadata
from oracle import rejection as orc

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def sm_for(temps, drafts, device, generators=None):
    all_greedy = all(t < 1e-5 for t in temps)
    n = len(temps)
    return SamplingMetadata(
        temperature=None if all_greedy else torch.tensor(temps, dtype=torch.float32,
                                                         device=device),
        all_greedy=all_greedy, all_random=all(t >= 1e-5 for t in temps), top_k=None,
        top_p=None, generators=dict(generators or {}), prompt_token_ids=[[] for _ in range(n)],
        output_token_ids=[[] for _ in range(n)], min_tokens=[0] * n,
        stop_token_ids=[[] for _ in range(n)], spec_token_ids=[list(d) for d in drafts])


def compact_logits(case):
    """[P+B, V] compact logits of a KAT: each request's verify rows then its bonus row."""
    rows = []
    if case["kind"] == "argmax":
        V = case["vocab"]
        for target, bonus in zip(case["targets"], case["bonus"]):
            for t in list(target) + [bonus]:
                row = [0.01] * V
                row[t] = 0.9
                rows.append(row)
    else:
        start = 0
        V = len(case["p_rows"][0])
        for draft, bonus in zip(case["drafts"], case["bonus"]):
            rows.extend(case["p_rows"][start:start + len(draft)])
            onehot = [0.0] * V
            onehot[bonus] = 1.0
            rows.append(onehot)
            start += len(draft)
    return torch.tensor(rows, dtype=torch.float32).log()


def run_kat(case, device, monkeypatch, fused):
    drafts = case["drafts"]
    meta = make_metadata(drafts, device=device)
    logits = compact_logits(case).to(device)
    q = None
    if case["kind"] == "probs" and case["q_rows"] is not None:
        q = torch.tensor(case["q_rows"], dtype=torch.float32, device=device)
    bonus = torch.tensor(case["bonus"], dtype=torch.int32, device=device).view(-1, 1)
    sm = sm_for(case["temperature"], drafts, device)
    if "uniforms" in case:
        u = torch.tensor(case["uniforms"], dtype=torch.float64, device=device)
        monkeypatch.setattr(rs, "generate_uniform_probs", lambda *a, **k: u)
    if "recovered" in case:
        r = torch.tensor(case["recovered"], dtype=torch.int32, device=device)
        monkeypatch.setattr(rs, "sample_recovered_tokens", lambda *a, **k: r)
    if fused:
        return rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens,
                                   meta.max_spec_len, meta.cu_num_draft_tokens, q, logits, bonus,
                                   sm, target_rows=meta.target_logits_indices,
                                   apply_temperature=True)
    target = logits[meta.target_logits_indices.long()]
    return rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, meta.max_spec_len,
                               meta.cu_num_draft_tokens, q, target, bonus, sm)


@pytest.mark.parametrize("fused", [False, True], ids=["reference_signature", "fused_gather"])
@pytest.mark.parametrize("case", KATS["rejection"], ids=lambda c: c["name"])
def test_reference_kats(case, fused, device, monkeypatch):
    out = run_kat(case, device, monkeypatch, fused)
    assert out.dtype == torch.int32
    assert out.cpu().tolist() == case["expected"]


class ArgmaxBonusSampler:
    """Test stand-in for the caller's bonus sampler: argmax of the bonus rows."""

    logprobs_mode = "raw_logprobs"

    def forward(self, logits, sampling_metadata, predict_bonus_token=False,
                logprobs_mode_override=None):
        return SamplerOutput(sampled_token_ids=logits.argmax(-1).to(torch.int32).view(-1, 1))


@pytest.mark.parametrize("case", [c for c in KATS["rejection"] if c["kind"] == "argmax"],
                         ids=lambda c: c["name"])
def test_rejection_sampler_forward_greedy_kats(case, device):
    meta = make_metadata(case["drafts"], device=device)
    logits = compact_logits(case).to(device)
    sm = sm_for(case["temperature"], case["drafts"], device)
    out = rs.RejectionSampler(ArgmaxBonusSampler())(meta, None, logits, sm)
    assert out.sampled_token_ids.cpu().tolist() == case["expected"]
    parsed, _ = rs.RejectionSampler.parse_output(out.sampled_token_ids, case["vocab"])
    assert parsed == [[t for t in row if t != -1] for row in case["expected"]]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [5, 64, 4096 + 8, 151936])
def test_greedy_argmax_at_every_position(device, dtype, V):
    """One row per argmax position (vector-lane 0..7, thread boundaries, chunk boundaries,
    last column), plus ties that must resolve to the first index."""
    positions = sorted({p for p in [0, 1, 2, 3, 4, 7, 8, 9, 1023, 1024, 4095, 4096, 4097,
                                    8191, 8192, V - 2, V - 1] if 0 <= p < V})
    P = len(positions)
    logits = torch.randn((P, V), device=device).clamp(-3, 3).to(dtype)
    for r, pos in enumerate(positions):
        logits[r, pos] = 10.0
    tie = torch.full((2, V), -1.0, device=device, dtype=dtype)
    tie[0, [V - 1, max(V - 3, 0)]] = 5.0
    tie[1, :] = 2.0
    logits = torch.cat([logits, tie])
    drafts = [[0] for _ in range(P + 2)]
    meta = make_metadata(drafts, device=device)
    out = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, 1,
                              meta.cu_num_draft_tokens, None, logits,
                              torch.full((P + 2, 1), 7, dtype=torch.int32, device=device),
                              sm_for([0.0] * (P + 2), drafts, device))
    expect = positions + [max(V - 3, 0), 0]
    got = out[:, 0].cpu().tolist()
    assert got == expect
    assert got == logits.float().argmax(-1).cpu().tolist()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [4096 + 8, 151936])
def test_greedy_16bit_special_values(device, dtype, V):
    """16-bit greedy rows (each sub-chunk's maximum from a tree of maxima, a tree of sums
    flagging NaN for the per-entry rule): NaN ranks first and the first NaN wins whatever its
    sign or payload; -0 and +0 tie; -inf rows give column 0; +inf beats every finite value
    (and, beside -inf, makes the sum NaN); an entry at the last column and one in the partial
    last sub-chunk win.  Expected: the first index of the maximum, NaN above every number."""
    def row(fill=-1.0):
        return torch.full((V,), fill, dtype=torch.float32)
    rows, expect = [], []
    r = row(); r[100] = 5.0; r[3000] = float("nan"); r[3500] = float("nan"); rows.append(r); expect.append(3000)
    r = row(); r[10] = 7.0; rows.append(r); expect.append(10)
    r = row(-float("inf")); rows.append(r); expect.append(0)
    r = row(-2.0); r[40] = -0.0; r[41] = 0.0; r[7] = -0.0; rows.append(r); expect.append(7)
    r = row(); r[V - 1] = float("inf"); r[5] = 60000.0; rows.append(r); expect.append(V - 1)
    r = row(); r[V - 3] = 3.0; rows.append(r); expect.append(V - 3)
    r = row(); r[200] = -float("inf"); r[201] = -0.5; rows.append(r); expect.append(201)
    logits = torch.stack(rows).to(dtype)
    # a NaN with the sign bit set ranks first as well
    bits = logits.view(torch.int16)
    bits[0, 3000] = bits[0, 3000] | -32768
    logits = logits.to(device)
    n = len(rows)
    drafts = [[0] for _ in range(n)]
    meta = make_metadata(drafts, device=device)
    out = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, 1,
                              meta.cu_num_draft_tokens, None, logits,
                              torch.full((n, 1), 7, dtype=torch.int32, device=device),
                              sm_for([0.0] * n, drafts, device))
    got = out[:, 0].cpu().tolist()
    assert got == expect, (got, expect)


def test_greedy_argmax_treats_signed_zeros_as_equal(device):
    """-0.0 == +0.0 for torch.argmax: the first of them is the argmax."""
    logits = torch.tensor([[-1.0, -0.0, 0.0, -2.0], [-3.0, 0.0, -0.0, -0.0]], device=device)
    drafts = [[3], [3]]
    meta = make_metadata(drafts, device=device)
    out = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, 1,
                              meta.cu_num_draft_tokens, None, logits,
                              torch.full((2, 1), 7, dtype=torch.int32, device=device),
                              sm_for([0.0, 0.0], drafts, device))
    assert out[:, 0].cpu().tolist() == [1, 1] == logits.argmax(-1).cpu().tolist()


def test_expand_kats(device):
    for case in KATS["expand"]:
        x = torch.tensor(case["x"], device=device)
        cu = torch.tensor(case["cu"], dtype=torch.int32, device=device)
        out = rs.expand_batch_to_tokens(x, cu, case["num_tokens"], case["replace_from"],
                                        case["replace_to"])
        assert out.cpu().tolist() == case["expected"]
    k = torch.tensor([5, 50, 7], dtype=torch.int64, device=device)
    out = rs.expand_batch_to_tokens(k, torch.tensor([2, 2, 5], dtype=torch.int32, device=device), 5)
    assert out.cpu().tolist() == [5, 5, 7, 7, 7]


# --------------------------------------------------------------------------- oracle parity


def run_workload(w: configs.Workload, *, draft_none=False, synthetic=None):
    sm = SamplingMetadata(temperature=w.temperature, all_greedy=w.all_greedy,
                          all_random=w.all_random, top_k=None, top_p=None)
    return rs.rejection_sample(
        w.draft_token_ids, w.num_draft_tokens, w.max_spec_len, w.cu_num_draft_tokens,
        None if draft_none else w.draft_probs, w.target_logits, w.bonus_token_ids, sm,
        synthetic_mode=synthetic is not None, synthetic_conditional_rates=synthetic,
        uniform_probs=w.uniforms, exp_noise=w.exp_noise, target_rows=w.target_rows,
        apply_temperature=w.apply_temperature)


def oracle_for(w: configs.Workload, *, draft_none=False, synthetic=None, rows=None):
    """Oracle on the verify rows (optionally on a subset of requests)."""
    logits = w.target_logits if w.target_rows is None else w.target_logits[w.target_rows.long()]
    return orc.rejection_sample(
        w.draft_token_ids.cpu(), w.num_draft_tokens, w.max_spec_len,
        None if (draft_none or w.draft_probs is None) else w.draft_probs.cpu(), logits.cpu(),
        w.bonus_token_ids.cpu(), temperature=None if w.temperature is None else w.temperature.cpu(),
        all_greedy=w.all_greedy, uniforms=None if w.uniforms is None else w.uniforms.cpu(),
        exp_noise=None if w.exp_noise is None else w.exp_noise.cpu(),
        apply_temperature=w.apply_temperature,
        synthetic_rates=None if synthetic is None else synthetic.cpu())


def check_parity(w, out, ref, label, **kw):
    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), w.num_draft_tokens, **kw)
    print(f"[{label}] requests={rep.requests} mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}", flush=True)
    assert not rep.unexplained, rep.unexplained[:5]
    return rep


def test_c1_greedy_bit_exact(device):
    w = configs.greedy_c1(device)
    out = run_workload(w)
    ref = oracle_for(w)
    assert np.array_equal(out.cpu().numpy(), ref.output_token_ids)


def test_c1_greedy_larger_batch_bit_exact(device):
    w = configs.greedy_c1(device, B=64, k=6, seed=77)
    out = run_workload(w)
    ref = oracle_for(w)
    assert np.array_equal(out.cpu().numpy(), ref.output_token_ids)


def test_c2_random_parity(device):
    w = configs.random_c2(device)
    rep = check_parity(w, run_workload(w), oracle_for(w), "c2")
    assert rep.mismatched <= 2


def test_headline_parity_full_size(device):
    w = configs.headline(device)
    rep = check_parity(w, run_workload(w), oracle_for(w), "headline B=256 k=4")
    assert rep.mismatched <= 4


def test_point_mass_drafts_parity(device):
    w = configs.random_c2(device, B=32, k=4, seed=4242)
    check_parity(w, run_workload(w, draft_none=True), oracle_for(w, draft_none=True),
                 "point-mass")


def test_bf16_ragged_mixed_parity(device):
    """c4's ragged mixed greedy/random bf16 batch (without its top-k/top-p quartiles)."""
    w = configs.ragged_c4(device, B=128)
    check_parity(w, run_workload(w), oracle_for(w), "c4-recipe B=128 no top-k/p")


def test_eagle_c5_recipe_subset_parity(device):
    w = configs.eagle_c5(device, B=48)
    check_parity(w, run_workload(w), oracle_for(w), "c5-recipe B=48")


def test_synthetic_mode_parity(device):
    w = configs.random_c2(device, B=32, k=4, seed=99)
    rates = torch.tensor([0.9, 0.6, 0.5, 0.3], device=device)
    out = run_workload(w, synthetic=rates)
    ref = oracle_for(w, synthetic=rates)
    # synthetic acceptance never looks at p/q: accept/reject is exact, recovered ids may tie
    check_parity(w, out, ref, "synthetic")


@pytest.mark.parametrize("case", ["headline", "point_mass", "bf16_ragged", "c5_rows",
                                  "one_request", "one_subchunk", "two_subchunks"])
def test_edge_shapes_parity(device, case):
    """Shapes that stress the schedule: one request (fewer tasks than workgroups), rows of one
    or two sub-chunks, point-mass drafts, ragged bf16 batches with greedy requests, K = 7 rows
    in two groups per request."""
    draft_none = case == "point_mass"
    w = {"headline": lambda: configs.headline(device),
         "point_mass": lambda: configs.random_c2(device, B=32, k=4, seed=4243),
         "bf16_ragged": lambda: configs.ragged_c4(device, B=64),
         "c5_rows": lambda: configs.eagle_c5(device, B=40),
         "one_request": lambda: configs.random_c2(device, B=1, k=7, seed=12),
         "one_subchunk": lambda: configs.random_c2(device, B=24, k=5, V=1000, seed=13),
         "two_subchunks": lambda: configs.random_c2(device, B=24, k=5, V=4000, seed=14)}[case]()
    rep = check_parity(w, run_workload(w, draft_none=draft_none),
                       oracle_for(w, draft_none=draft_none), case)
    assert rep.mismatched <= 4


@pytest.mark.parametrize("case", ["c1", "c1_large", "c4_mixed"])
def test_greedy_edge_shapes_bit_exact(device, case):
    """Greedy rows (argmax tasks, target_rows gathers), alone and mixed with random ones."""
    w = {"c1": lambda: configs.greedy_c1(device),
         "c1_large": lambda: configs.greedy_c1(device, B=64, k=6, seed=77),
         "c4_mixed": lambda: configs.ragged_c4(device, B=96, seed=31)}[case]()
    out = run_workload(w)
    if case == "c4_mixed":
        check_parity(w, out, oracle_for(w), "c4 mixed")
    else:
        assert np.array_equal(out.cpu().numpy(), oracle_for(w).output_token_ids)


@pytest.mark.parametrize("B", [1, 6, 7, 14, 28, 29])
def test_greedy_batches_around_one_wave(device, B):
    """All-greedy fp32 batches (k=3) at full vocabulary.  Up to 28 requests every task has a
    workgroup of its own and the launch has no tail (chunks of 2, 3, 5 or 9 sub-chunks as the
    count grows); at 29 the tasks outnumber the 256 resident workgroups and the launch claims
    tickets with a half-chunk tail again.  Bit-exact against the oracle on both sides."""
    w = configs.greedy_c1(device, B=B, k=3, seed=600 + B)
    assert np.array_equal(run_workload(w).cpu().numpy(), oracle_for(w).output_token_ids)


def test_supplied_recovered_ids_take_the_plan_without_scores(device, monkeypatch):
    """Random requests whose recovered ids come from a replaced sample_recovered_tokens give the
    launch no score units (chunks of any sub-chunk count, no tail when its tasks all start at
    once).  The ids supplied are the standalone sampler's on the same noise, so the tokens
    match the in-kernel scores' and the oracle's."""
    w = configs.random_c2(device, B=6, k=3, seed=611)
    ref = oracle_for(w)
    check_parity(w, run_workload(w), ref, "in-kernel scores")
    probs = orc.target_probs(w.target_logits.cpu(), orc.row_temperatures(
        w.temperature.cpu(), w.num_draft_tokens, False, True))
    rec = rs.sample_recovered_tokens(w.max_spec_len, w.num_draft_tokens, w.cu_num_draft_tokens,
                                     w.draft_token_ids, w.draft_probs, probs.to(device), None,
                                     device, exp_noise=w.exp_noise)
    monkeypatch.setattr(rs, "sample_recovered_tokens", lambda *a, **k: rec)
    check_parity(w, run_workload(w), ref, "supplied recovered ids")


def test_more_requests_than_one_launch(device):
    """Batches beyond 4096 requests run as several launches over one workspace (request
    offsets, the first row of a later launch from cu[r0 - 1])."""
    w = configs.random_c2(device, B=4500, k=3, V=1024, seed=71)
    check_parity(w, run_workload(w), oracle_for(w), "B=4500")
    g = configs.greedy_c1(device, B=4200, k=2, V=512, seed=72)
    assert np.array_equal(run_workload(g).cpu().numpy(), oracle_for(g).output_token_ids)


def test_gave_up_waits_poison_and_recover(device):
    """Fail-stop: with the wait limit at 0 every cross-workgroup wait gives up at once (every
    kernel still exits normally).  The output rows of the requests concerned hold MVSD_POISON,
    parse_output raises, the workspace is zero again, and the next call is exact."""
    from mvsd import _native as nat
    w = configs.random_c2(device, B=48, k=4, seed=81)
    g = configs.greedy_c1(device, B=16, k=3, seed=82)
    lib = nat.lib()
    prev = lib.mvsd_set_wait_limit(0)
    try:
        bad = run_workload(w)
        bad_g = run_workload(g)
        torch.cuda.synchronize()
    finally:
        lib.mvsd_set_wait_limit(prev)
    for out, work in ((bad, w), (bad_g, g)):
        arr = out.cpu().numpy()
        has_drafts = np.asarray(work.num_draft_tokens) > 0
        assert (arr[has_drafts] == nat.POISON).all(), "every request with drafts waits"
        with pytest.raises(RuntimeError, match="gave up"):
            rs.RejectionSampler.parse_output(out, work.vocab_size)
    for ws in rs._WORKSPACES.values():
        assert int(ws.view(torch.int32).abs().sum()) == 0
    check_parity(w, run_workload(w), oracle_for(w), "after failure")
    assert np.array_equal(run_workload(g).cpu().numpy(), oracle_for(g).output_token_ids)


def test_repeated_calls_across_shapes(device):
    """Calls of different shapes in a row leave the workspace zeroed for the next one."""
    big = configs.random_c2(device, B=96, k=4, seed=51)
    small = configs.random_c2(device, B=5, k=2, seed=52)
    a = run_workload(big)
    b = run_workload(small)
    c = run_workload(big)
    d = run_workload(small)
    assert torch.equal(a, c) and torch.equal(b, d)
    check_parity(big, a, oracle_for(big), "repeated big")
    check_parity(small, b, oracle_for(small), "repeated small")


@pytest.mark.parametrize("V", [5, 1001, 4097, 8193])
def test_odd_vocab_sizes(device, V):
    """Unaligned rows (scalar loads) and partial last chunks."""
    w = configs.random_c2(device, B=16, k=3, V=V, seed=V)
    check_parity(w, run_workload(w), oracle_for(w), f"V={V}")
    g = configs.greedy_c1(device, B=16, k=3, V=V, seed=V + 1)
    assert np.array_equal(run_workload(g).cpu().numpy(), oracle_for(g).output_token_ids)


@pytest.mark.parametrize("tdtype,ddtype", [(torch.bfloat16, torch.float32),
                                           (torch.bfloat16, torch.bfloat16),
                                           (torch.float16, torch.float32)])
@pytest.mark.parametrize("V", [4097, 8200, 151936])
def test_bf16_target_score_loads(device, V, tdtype, ddtype):
    """Random requests on a 2-byte target (bf16, fp16), so that score tasks run on 2-byte
    targets: 4 columns per lane and load for the target, draft and noise rows, and a tree of
    maxima per lane and sub-chunk.  V = 4097 leaves the rows unaligned (every load
    bounds-checked, element by element), V = 8200 ends each row in a partial sub-chunk (8-byte
    loads where a quad fits, checked loads past it)."""
    w = configs.random_c2(device, B=32, k=4, V=V, seed=V + 17)
    w = replace(w, target_logits=w.target_logits.to(tdtype),
                draft_probs=w.draft_probs.to(ddtype))
    out = run_workload(w)
    ref = oracle_for(w)
    rejected = sum(len([t for t in row if t != -1]) <= k
                   for row, k in zip(ref.output_token_ids.tolist(), w.num_draft_tokens))
    assert rejected > 0, "no request rejected a draft: no score task ran"
    check_parity(w, out, ref, f"{tdtype} target V={V} draft {ddtype}")


def test_repeated_calls_are_identical(device):
    w = configs.random_c2(device, B=32, k=4, seed=5)
    a = run_workload(w)
    b = run_workload(w)
    c = run_workload(configs.greedy_c1(device, B=3, k=2, seed=6))
    d = run_workload(w)
    assert torch.equal(a, b) and torch.equal(a, d) and c.shape == (3, 3)


def test_workspace_is_left_zeroed_across_shapes(device):
    """Calls of different shapes share one cached workspace; each must leave it zeroed (the
    tiny greedy batch runs one task per workgroup and no tail)."""
    big = configs.random_c2(device, B=96, k=4, seed=41)
    small = configs.random_c2(device, B=8, k=2, seed=42)
    greedy = configs.greedy_c1(device, B=40, k=5, seed=43)
    tiny = configs.greedy_c1(device, B=4, k=3, seed=44)
    expect = {id(w): oracle_for(w).output_token_ids for w in (big, small, greedy, tiny)}
    for w in (big, small, greedy, tiny, small, big, tiny, greedy, big):
        out = run_workload(w).cpu().numpy()
        rep = orc.compare(out, orc.OracleResult(expect[id(w)], *([np.full(w.num_tokens, np.nan)] * 4),
                                                np.zeros(w.num_tokens, bool)),
                          w.draft_token_ids.cpu(), w.num_draft_tokens)
        assert rep.mismatched == 0, (w.name, rep)
    torch.cuda.synchronize()
    for ws in rs._WORKSPACES.values():
        assert int(ws.view(torch.int32).abs().sum()) == 0


def test_no_host_synchronisation(device):
    w = configs.random_c2(device, B=16, k=4, seed=8)
    run_workload(w)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        run_workload(w)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()


def test_output_distribution_equals_target(device):
    case = KATS["distribution"][0]
    n = case["samples"]
    drafts = [[int(t)] for t in np.random.default_rng(0).choice(3, size=n, p=case["q"])]
    meta = make_metadata(drafts, device=device)
    target = torch.tensor([case["p"]], dtype=torch.float32, device=device).log().repeat(n, 1)
    q = torch.tensor([case["q"]], dtype=torch.float32, device=device).repeat(n, 1)
    bonus = torch.full((n, 1), 2, dtype=torch.int32, device=device)
    torch.manual_seed(0)
    out = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, 1,
                              meta.cu_num_draft_tokens, q, target, bonus,
                              sm_for([1.0] * n, drafts, device))[:, 0].cpu().numpy()
    freq = np.bincount(out, minlength=3) / n
    assert np.all(np.abs(freq - np.array(case["p"])) < case["threshold"]), freq


def test_recovered_distribution_standalone(device):
    case = KATS["distribution"][1]
    n = case["samples"]
    meta = make_metadata([[0]] * n, device=device)
    p = torch.tensor([case["p"]], dtype=torch.float32, device=device).repeat(n, 1)
    q = torch.tensor([case["q"]], dtype=torch.float32, device=device).repeat(n, 1)
    torch.manual_seed(1)
    rec = rs.sample_recovered_tokens(1, meta.num_draft_tokens, meta.cu_num_draft_tokens,
                                     meta.draft_token_ids, q, p, sm_for([1.0] * n, [[0]] * n,
                                                                        device), device)
    freq = np.bincount(rec.cpu().numpy(), minlength=3) / n
    assert freq[0] == 0.0
    assert np.all(np.abs(freq - np.array(case["expected"])) < case["threshold"]), freq


def test_standalone_recovered_matches_oracle(device):
    w = configs.random_c2(device, B=16, k=4, seed=21)
    probs = orc.target_probs(w.target_logits.cpu(), orc.row_temperatures(
        w.temperature.cpu(), w.num_draft_tokens, False, True))
    rec = rs.sample_recovered_tokens(w.max_spec_len, w.num_draft_tokens, w.cu_num_draft_tokens,
                                     w.draft_token_ids, w.draft_probs, probs.to(device), None,
                                     device, exp_noise=w.exp_noise)
    scores = orc.recovered_scores(probs, w.draft_probs.cpu(), w.draft_token_ids.cpu(),
                                  w.exp_noise.cpu(), w.num_draft_tokens)
    assert torch.equal(rec.cpu(), orc.recovered_token_ids(scores))


def test_seeded_generators_do_not_depend_on_batch(device):
    """K=0 requests consume no randomness (tests/step59/test_rejection.py:466-485)."""
    gen = torch.Generator(device=device).manual_seed(7)
    p = [0.5, 0.5]
    meta = make_metadata([[1], []], device=device)
    logits = torch.tensor([p], dtype=torch.float32, device=device).log().repeat(3, 1)
    q = torch.tensor([p], dtype=torch.float32, device=device)
    bonus = torch.tensor([[0], [1]], dtype=torch.int32, device=device)
    torch.manual_seed(11)
    a = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, 1,
                            meta.cu_num_draft_tokens, q, logits[meta.target_logits_indices.long()],
                            bonus, sm_for([1.0, 1.0], [[1], []], device, {0: gen})).cpu()
    gen.manual_seed(7)
    meta2 = make_metadata([[1]], device=device)
    torch.manual_seed(11)
    b = rs.rejection_sample(meta2.draft_token_ids, [1], 1, meta2.cu_num_draft_tokens, q,
                            logits[:1], bonus[:1], sm_for([1.0], [[1]], device, {0: gen})).cpu()
    assert a[0].tolist() == b[0].tolist()


def test_forward_fast_path_matches_processed_path(device):
    """RejectionSampler.forward folds gather + temperature into the kernel; the reference's
    explicit gather + fp32 + div_ followed by rejection_sample must give the same ids."""
    w = configs.random_c2(device, B=24, k=3, seed=31)
    drafts = w.draft_token_ids.cpu().view(24, 3).tolist()
    meta = make_metadata(drafts, device=device)
    B, k, V = 24, 3, w.vocab_size
    compact = torch.zeros((B * (k + 1), V), device=device)
    compact[meta.target_logits_indices.long()] = w.target_logits
    sm = replace(sm_for([0.8] * B, drafts, device), temperature=w.temperature)
    u, e = w.uniforms, w.exp_noise
    a = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, k,
                            meta.cu_num_draft_tokens, w.draft_probs, compact, w.bonus_token_ids,
                            sm, uniform_probs=u, exp_noise=e,
                            target_rows=meta.target_logits_indices, apply_temperature=True)
    processed = rs.apply_sampling_constraints(compact[meta.target_logits_indices.long()].clone(),
                                              meta.cu_num_draft_tokens, sm)
    b = rs.rejection_sample(meta.draft_token_ids, meta.num_draft_tokens, k,
                            meta.cu_num_draft_tokens, w.draft_probs, processed, w.bonus_token_ids,
                            sm, uniform_probs=u, exp_noise=e)
    assert torch.equal(a, b)


def test_corrected_reciprocal_equals_ieee_division(device):
    """The score kernels compute 1/E with the hardware reciprocal plus one FMA correction;
    it must equal IEEE fp32 division for every normal E with a normal reciprocal."""
    from mvsd import _native as nat
    failures = torch.zeros(1, dtype=torch.int64, device=device)
    nat.check(nat.lib().mvsd_selftest(0, failures.data_ptr(), nat.stream_of(device)),
              "mvsd_selftest")
    assert int(failures.item()) == 0


@pytest.mark.parametrize("ddtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", ["c2", "odd_v", "c4_bf16_target"])
def test_16bit_draft_probs(device, ddtype, case):
    """draft_probs in bf16 / fp16, upcast in the kernel (the reference's kernels load them in
    their own dtype and compute in fp32, rejection_sampler.py:797-806, :882-890): against the
    oracle on the same 16-bit values upcast.  Score tasks load 16-bit drafts 4 columns (8 bytes)
    per lane for every target type; odd V takes the bounds-checked loads."""
    w = {"c2": lambda: configs.random_c2(device, B=48, k=4, seed=301),
         "odd_v": lambda: configs.random_c2(device, B=24, k=3, V=4097, seed=302),
         "c4_bf16_target": lambda: configs.ragged_c4(device, B=96, seed=303)}[case]()
    w = replace(w, draft_probs=w.draft_probs.to(ddtype))
    check_parity(w, run_workload(w), oracle_for(w), f"{case} draft {ddtype}")
