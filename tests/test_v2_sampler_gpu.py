"""GPU tests of the V2 RejectionSampler wrapper (mvsd/worker/gpu/spec_decode/
rejection_sampler.py, after minivllm/worker/gpu/spec_decode/rejection_sampler.py:54-337) and
the kernels it adds: compute_topk_scores (mvsd_topk_scores), flatten_sampled
(mvsd_v2_flatten_sampled) and get_num_sampled_and_rejected
(mvsd_v2_num_sampled_and_rejected), each against the CPU oracle; chunked verification
against the whole batch (the properties of tests/step75/test_logit_chunks.py:218-372).

The V2 runner's sampler and input batch are stand-ins carrying the fields the wrapper reads;
their ``apply_sampling_params`` scales the logits by a constant so that the processed and
raw logprob modes differ.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import logprobs as olp
from oracle import v2_rejection as o
from v2_cases import make_case, near_tie, oracle_args

pytestmark = pytest.mark.gpu

V = 151936


class _Sampler:
    def __init__(self, case, *, k=-1, mode="raw_logprobs", scale=1.0, fp64=False,
                 prefill_len=None):
        dev = "cuda"
        self.logprobs_mode = mode
        self.use_fp64_gumbel = fp64
        self.scale = scale
        states = case["temperature"].numel()
        self.sampling_states = SimpleNamespace(
            temperature=SimpleNamespace(gpu=case["temperature"].to(dev)),
            seeds=SimpleNamespace(gpu=case["seed"].to(dev)),
            max_num_logprobs=lambda idx_np: k)
        pl = torch.zeros(states, dtype=torch.int32) if prefill_len is None else prefill_len
        self.req_states = SimpleNamespace(prefill_len=SimpleNamespace(gpu=pl.to(dev)))

    def apply_sampling_params(self, logits, *_args):
        return logits.to(torch.float32) * self.scale


def _batch(case, *, pad=7, seq_lens=None):
    dev = "cuda"
    cu = case["cu_num_logits"]
    num_logits = int(cu[-1])
    R = cu.numel() - 1
    junk = torch.full((pad,), 12345, dtype=torch.int32)
    input_ids = torch.cat([junk, case["draft_sampled"].to(torch.int32)])
    positions = torch.cat([torch.zeros(pad, dtype=torch.int64), case["pos"]])
    return SimpleNamespace(
        num_reqs=R, cu_num_logits=cu.to(dev), cu_num_logits_np=cu.numpy().astype(np.int64),
        idx_mapping=case["idx_mapping"].to(dev), idx_mapping_np=case["idx_mapping"].numpy(),
        expanded_idx_mapping=case["expanded_idx_mapping"].to(dev),
        expanded_local_pos=case["expanded_local_pos"].to(dev),
        input_ids=input_ids.to(dev), positions=positions.to(dev),
        logits_indices=(torch.arange(num_logits) + pad).to(dev),
        seq_lens=(torch.full((R,), 100, dtype=torch.int32) if seq_lens is None
                  else seq_lens).to(dev))


def _rs(case, method="standard", rates=None, **kw):
    from mvsd.worker.gpu.spec_decode import RejectionSampler
    spec = SimpleNamespace(num_speculative_tokens=case["num_speculative_steps"],
                           rejection_sample_method=method, synthetic_acceptance_rates=rates)
    return RejectionSampler(_Sampler(case, **kw), spec, torch.device("cuda"))


def _dev(case):
    return {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}


def _same_prefix(a, b):
    (sa, na), (sb, nb) = a, b
    na, nb = na.cpu(), nb.cpu()
    assert torch.equal(na, nb), (na.tolist(), nb.tolist())
    sa, sb = sa.cpu(), sb.cpu()
    for r in range(na.numel()):
        n = int(na[r])
        assert torch.equal(sa[r, :n], sb[r, :n]), r


@pytest.mark.parametrize("method", ["standard", "block", "synthetic"])
def test_call_matches_the_verification_and_the_oracle(method):
    temps = [0.8, 0.0, 1.2, 0.9, 0.0, 1.0, 0.7, 1.1]
    case = make_case([4, 3, 4, 0, 2, 4, 1, 4], temps, 4, V, seed=51, states=12)
    rates = [0.9, 0.6, 0.4, 0.2] if method == "synthetic" else None
    rs = _rs(case, method, rates)
    d = _dev(case)
    out = rs(d["target_logits"], _batch(case), d["draft_logits"])
    torch.cuda.synchronize()
    from mvsd.worker.gpu.spec_decode import rejection_sample
    direct = rejection_sample(
        **d, synthetic_conditional_rates=rs.synthetic_conditional_rates,
        use_block_verification=method == "block")
    _same_prefix((out.sampled_token_ids, out.num_sampled), direct)
    rows = np.diff(case["cu_num_logits"].numpy())
    assert out.num_rejected.cpu().tolist() == (rows - out.num_sampled.cpu().numpy()).tolist()
    assert out.logprobs_tensors is None and out.num_nans is None
    okw = {}
    if rates is not None:
        okw["synthetic_conditional_rates"] = rs.synthetic_conditional_rates.cpu().numpy()
    es, en, margins, gaps, wins, gap_wins = o.rejection_sample(
        **oracle_args(case), use_block_verification=method == "block", return_margins=True,
        return_windows=True, **okw)
    s, n = out.sampled_token_ids.cpu().numpy(), out.num_sampled.cpu().numpy()
    for r in range(len(en)):
        if n[r] == en[r] and (s[r, :en[r]] == es[r, :en[r]]).all():
            continue
        assert near_tie(margins[r], wins[r], gaps[r], gap_wins[r]), r


def test_requests_still_prefilling_sample_nothing():
    """get_num_sampled_and_rejected (input_batch.py:507-553): a request whose seq_len is
    below its state's prefill_len reports 0 sampled and 0 rejected."""
    case = make_case([3, 3, 2, 3], [0.9, 0.0, 1.0, 0.8], 3, 4096, seed=52, states=6)
    idx = case["idx_mapping"].tolist()
    prefill = torch.zeros(6, dtype=torch.int32)
    prefill[idx[1]] = 500
    prefill[idx[2]] = 100   # seq_len 100 is not below it: not prefilling
    rs = _rs(case, prefill_len=prefill)
    d = _dev(case)
    out = rs(d["target_logits"], _batch(case), d["draft_logits"])
    ns, nr = out.num_sampled.cpu().tolist(), out.num_rejected.cpu().tolist()
    assert ns[1] == 0 and nr[1] == 0
    rows = np.diff(case["cu_num_logits"].numpy())
    for r in (0, 2, 3):
        assert 1 <= ns[r] <= rows[r] and nr[r] == rows[r] - ns[r]


def _chunked(case, limit, *, k=-1, method="standard", mode="raw_logprobs", scale=1.0,
             draft_logits=True, batch=None):
    rs = _rs(case, method, k=k, mode=mode, scale=scale)
    d = _dev(case)
    b = batch or _batch(case)
    draft_sampled = b.input_ids[b.logits_indices]
    pos = b.positions[b.logits_indices]
    return rs._verify_in_chunks(d["target_logits"], b, d["draft_logits"] if draft_logits else None,
                                draft_sampled, pos, limit, k)


def _same_result(a, b):
    _same_prefix(a[:2], b[:2])
    la, lb = a[2], b[2]
    if la is None or lb is None:
        assert la is None and lb is None
        return
    assert la.cu_num_generated_tokens == lb.cu_num_generated_tokens
    assert torch.equal(la.logprob_token_ids, lb.logprob_token_ids)
    assert torch.equal(la.selected_token_ranks, lb.selected_token_ranks)
    assert torch.equal(la.logprobs, lb.logprobs)


@pytest.mark.parametrize("method", ["standard", "block"])
@pytest.mark.parametrize("draft_logits", [True, False])
def test_chunks_agree_with_the_whole_batch(method, draft_logits):
    """Mixed draft counts (one request without drafts) and scrambled states: every chunk
    limit gives the whole batch's tokens, counts and logprobs (rows and order included)."""
    K = 4
    case = make_case([4, 0, 2, 3, 4, 1], [0.9, 1.0, 0.0, 1.3, 0.7, 1.0], K, 8192, seed=53,
                     states=10, draft_logits=draft_logits)
    whole = _chunked(case, 10**9, k=3, method=method, draft_logits=draft_logits)
    assert whole[2] is not None
    for limit in (1, 2, 5, 6, 9, 12):
        _same_result(whole, _chunked(case, limit, k=3, method=method,
                                     draft_logits=draft_logits))
    cu = case["cu_num_logits"].tolist()
    assert whole[2].cu_num_generated_tokens == cu
    assert whole[2].logprob_token_ids.shape == (cu[-1], 4)


def test_draft_logits_stay_indexed_by_state_across_chunks():
    """Chunking slices the rows but not draft_logits: swapping two states' draft rows changes
    the result, so the chunked run really reads them by state."""
    case = make_case([4, 4], [1.0, 1.0], 4, 4096, seed=54, states=8)
    single = _chunked(case, 10**9)
    chunked = _chunked(case, 5)
    _same_result(single, chunked)
    s0, s1 = case["idx_mapping"].tolist()
    swapped = dict(case)
    dl = case["draft_logits"].clone()
    dl[s0], dl[s1] = case["draft_logits"][s1], case["draft_logits"][s0]
    swapped["draft_logits"] = dl
    other = _chunked(swapped, 5)
    assert not (torch.equal(other[1].cpu(), chunked[1].cpu())
                and torch.equal(other[0].cpu(), chunked[0].cpu()))


def test_stale_host_offsets_do_not_choose_chunks(monkeypatch):
    """A compacted batch keeps stale host prefix sums; when its rows fit the limit the whole
    batch is one chunk and the chunk iterator is never consulted (:227-238)."""
    from mvsd.worker.gpu.spec_decode import rejection_sampler as mod
    case = make_case([4, 4, 4], [0.9, 1.0, 0.8], 4, 4096, seed=55, states=5)
    fresh = _chunked(case, 10**9)
    b = _batch(case)
    b.cu_num_logits_np = b.cu_num_logits_np + np.arange(4) * 2
    calls = []
    real = mod._iter_request_chunks

    def spy(cu, limit):
        for c in real(cu, limit):
            calls.append(c)
            yield c

    monkeypatch.setattr(mod, "_iter_request_chunks", spy)
    stale = _chunked(case, 20, batch=b)
    assert calls == []
    _same_result(fresh, stale)
    _chunked(case, 5)
    assert calls


@pytest.mark.parametrize("mode,scale", [("raw_logprobs", 2.0), ("processed_logprobs", 2.0),
                                        ("raw_logits", 1.0), ("processed_logits", 0.5)])
def test_logprobs_against_the_oracle(mode, scale):
    """The wrapper scores every logits row with the token sampled there (0 past the sampled
    ones), from the raw or the processed logits as the mode says."""
    case = make_case([3, 2, 3, 0], [0.9, 0.0, 1.1, 1.0], 3, V, seed=56, states=6)
    k = 5
    whole = _chunked(case, 10**9, k=k, mode=mode, scale=scale)
    lp = whole[2]
    flat = o.flatten_sampled(whole[0].cpu().numpy(), whole[1].cpu().numpy(),
                             case["cu_num_logits"].numpy(), int(case["cu_num_logits"][-1]))
    src = case["target_logits"].float()
    if mode.startswith("processed"):
        src = src * scale
    ids, sc, rk = olp.topk_scores(src, k, torch.from_numpy(flat),
                                  logits_mode=mode.endswith("logits"))
    assert torch.equal(lp.logprob_token_ids.cpu(), ids)
    assert torch.equal(lp.selected_token_ranks.cpu(), rk)
    assert torch.allclose(lp.logprobs.cpu(), sc, rtol=0, atol=4e-6)


@pytest.mark.parametrize("k", [0, 1, 7, 40])
@pytest.mark.parametrize("logits_mode", [False, True])
def test_compute_topk_scores_full_vocab(k, logits_mode):
    from mvsd.worker.gpu.sample.logprob import compute_topk_scores
    g = torch.Generator().manual_seed(57 + k)
    x = torch.randn(24, V, generator=g) * 3.0
    x[3, 100] = x[3, 5] = x[3].max() + 2.0     # tie at the top
    x[4, :] = 0.25                              # a flat row
    x[5, 17] = float("-inf")                    # a masked entry
    tok = torch.randint(0, V, (24,), generator=g)
    tok[5] = 17
    got = compute_topk_scores(x.cuda(), k, tok.cuda(), [0, 24], logits_mode=logits_mode)
    ids, sc, rk = olp.topk_scores(x, k, tok, logits_mode=logits_mode)
    assert got.cu_num_generated_tokens == [0, 24]
    assert got.logprob_token_ids.dtype == torch.int64
    assert torch.equal(got.logprob_token_ids.cpu(), ids)
    assert torch.equal(got.selected_token_ranks.cpu(), rk)
    fin = torch.isfinite(sc)
    assert torch.equal(fin, torch.isfinite(got.logprobs.cpu()))
    assert torch.allclose(got.logprobs.cpu()[fin], sc[fin], rtol=0, atol=4e-6)
    assert ids[3, 1:3].tolist() == [5, 100][:k]
    # bf16 logits are upcast exactly
    got16 = compute_topk_scores(x.to(torch.bfloat16).cuda(), k, tok.cuda())
    ids16, sc16, rk16 = olp.topk_scores(x.to(torch.bfloat16).float(), k, tok)
    assert torch.equal(got16.logprob_token_ids.cpu(), ids16)
    assert torch.equal(got16.selected_token_ranks.cpu(), rk16)


def test_flatten_sampled_against_the_oracle():
    from mvsd.worker.gpu.spec_decode import flatten_sampled
    g = np.random.default_rng(58)
    R, K = 40, 5
    rows = g.integers(1, K + 2, R)
    cu = np.concatenate(([0], np.cumsum(rows)))
    sampled = g.integers(0, 1000, (R, K + 1))
    ns = np.array([g.integers(0, r + 1) for r in rows])
    got = flatten_sampled(torch.from_numpy(sampled).cuda(), torch.from_numpy(ns).int().cuda(),
                          torch.from_numpy(cu).int().cuda(), int(cu[-1]))
    assert got.cpu().numpy().tolist() == o.flatten_sampled(sampled, ns, cu, cu[-1]).tolist()


def test_flatten_sampled_writes_rows_past_the_last_request():
    """Rows after cu[-1] (padded or compacted logits) hold 0, as after the reference's zero
    fill, even when the output's memory held other values before."""
    from mvsd.worker.gpu.spec_decode import flatten_sampled
    g = np.random.default_rng(59)
    R, K, pad = 12, 4, 9
    rows = g.integers(1, K + 2, R)
    cu = np.concatenate(([0], np.cumsum(rows)))
    n = int(cu[-1]) + pad
    sampled = g.integers(1, 1000, (R, K + 1))
    ns = np.array([g.integers(0, r + 1) for r in rows])
    dirty = torch.full((n,), -5, dtype=torch.int64, device="cuda")
    del dirty  # the caching allocator hands this block to the next allocation of its size
    got = flatten_sampled(torch.from_numpy(sampled).cuda(), torch.from_numpy(ns).int().cuda(),
                          torch.from_numpy(cu).int().cuda(), n)
    want = o.flatten_sampled(sampled, ns, cu, n)
    assert got.cpu().numpy().tolist() == want.tolist()
    assert (want[int(cu[-1]):] == 0).all()
