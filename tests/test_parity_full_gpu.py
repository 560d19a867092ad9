"""Full-size parity of the verification path against the CPU oracle, and the probability bound.

* C4 (B=512, ragged K in 0..8, bf16, half greedy, top-k=50 / top-p=0.9 quartiles) through
  RejectionSampler's fused path (temperature divide and constraints in the kernels) against
  one oracle pipeline: fp32 divide, oracle/topk_topp.py masks, oracle/rejection.py.  A request
  may differ only where oracle.compare allows it (acceptance margin < 1e-6, recovered near-tie
  within the rounding window), or where the kernel's mask of one of its rows differs from the
  oracle's only at top-p decisions whose cumulative mass lies within 1e-5 of 1 - p (both
  counted and printed).
* C5 (B=1024, k=7, bf16 target [8192, V] read through target_rows, fp32 draft probs) at its
  full size.
* The probability bound of the north star, 1e-5 relative in fp32 (bf16 inputs are upcast
  exactly, so the same bound applies to them): mvsd_softmax_rows against a float64 softmax,
  and the verify kernel's own per-row statistics and draft-token probability (the
  debug_row_stats read-out of the values its acceptance test used) against float64.
"""

import numpy as np
import pytest
import torch

from mvsd.sample import rejection_sampler as rs
from mvsd.sample.metadata import SamplingMetadata
from mvsd.testing import configs
from oracle import rejection as orc
from oracle import topk_topp as otp

pytestmark = pytest.mark.gpu

REL = 1e-5          # north_star: probabilities within 1e-5 relative (fp32), for p >= 1e-12
P_MEANINGFUL = 1e-12  # and for the deep tail 1e-30 <= p < 1e-12 alike (there the fp32 exponent
REL_TAIL = 1e-5     # (x - M) / T, up to ~70 in magnitude, carries the largest rounding: the
P_FLOOR = 1e-30     # runs measure at most ~4e-6 relative); below 1e-30 the check is
ABS_FLOOR = 1e-35   # absolute.


def _report(label, rep, extra=""):
    print(f"[{label}] requests={rep.requests} mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}{extra}",
          flush=True)


def test_c4_full_size_against_oracle_pipeline(device):
    w = configs.ragged_c4(device)  # B=512
    sm = SamplingMetadata(temperature=w.temperature, all_greedy=False, all_random=False,
                          top_k=w.top_k, top_p=w.top_p)
    out = rs.rejection_sample(
        w.draft_token_ids, w.num_draft_tokens, w.max_spec_len, w.cu_num_draft_tokens,
        w.draft_probs, w.target_logits, w.bonus_token_ids, sm, uniform_probs=w.uniforms,
        exp_noise=w.exp_noise, apply_temperature=True, apply_top_k_top_p=True)
    masks = rs.sampling_masks(w.target_logits, w.cu_num_draft_tokens, sm)
    torch.cuda.synchronize()

    # the oracle pipeline on the host: divide, mask, verify
    ks = w.num_draft_tokens
    req = orc.request_of_row(ks)
    temps = w.temperature.cpu().numpy()
    row_t = np.where(temps[req] == 0, 1.0, temps[req]).astype(np.float32)
    x = w.target_logits.float().cpu()
    xt = x / torch.from_numpy(row_t).unsqueeze(-1)
    row_k = w.top_k.cpu()[torch.from_numpy(req)]
    row_p = w.top_p.cpu()[torch.from_numpy(req)]
    masked = otp.apply_top_k_top_p(xt, row_k, row_p)
    ref = orc.rejection_sample(w.draft_token_ids.cpu(), ks, w.max_spec_len,
                               w.draft_probs.cpu(), masked, w.bonus_token_ids.cpu(),
                               temperature=w.temperature.cpu(), all_greedy=False,
                               uniforms=w.uniforms.cpu(), exp_noise=w.exp_noise.cpu(),
                               apply_temperature=False)

    # rows whose kernel mask differs from the oracle's, and whether only at the boundary
    m = masks.cpu().numpy()
    a, b = m[:, 0:1], m[:, 1:2]
    j = np.ascontiguousarray(m[:, 2]).view(np.int32)[:, None]
    xn = x.numpy()
    idx = np.arange(xn.shape[1])[None, :]
    kernel_masked = (xn < a) | ((xn < b) & (idx <= j))
    oracle_masked = ~torch.isfinite(masked).numpy() & np.isfinite(xn)
    boundary_reqs = set()
    boundary_entries = 0
    # greedy rows carry no mask unless a mask could change their argmax (a tied maximum);
    # their tokens are still compared below
    greedy_rows = temps[req] == 0
    differ = (kernel_masked != oracle_masked).any(axis=1) & ~greedy_rows
    for row in np.nonzero(differ)[0]:
        k = int(row_k[row])
        k = k if 0 < k < xn.shape[1] else None
        amb = otp.near_boundary(xt[row].numpy(), k, float(row_p[row]))
        diff = kernel_masked[row] != oracle_masked[row]
        assert not (diff & ~amb).any(), f"row {row}: mask differs away from the top-p boundary"
        boundary_entries += int(diff.sum())
        boundary_reqs.add(int(req[row]))

    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), ks)
    unexplained = [u for u in rep.unexplained if u[0] not in boundary_reqs]
    _report("c4 full B=512", rep, f" boundary_requests={len(boundary_reqs)} "
            f"boundary_entries={boundary_entries}")
    assert not unexplained, unexplained[:5]
    assert rep.mismatched <= len(boundary_reqs) + rep.accept_flips + rep.recovered_flips


def test_c5_full_size(device):
    w = configs.eagle_c5(device)  # B=1024, k=7
    sm = SamplingMetadata(temperature=w.temperature, all_greedy=w.all_greedy,
                          all_random=w.all_random, top_k=None, top_p=None)
    out = rs.rejection_sample(
        w.draft_token_ids, w.num_draft_tokens, w.max_spec_len, w.cu_num_draft_tokens,
        w.draft_probs, w.target_logits, w.bonus_token_ids, sm, uniform_probs=w.uniforms,
        exp_noise=w.exp_noise, target_rows=w.target_rows,
        apply_temperature=w.apply_temperature)
    torch.cuda.synchronize()
    logits = w.target_logits[w.target_rows.long()].cpu()
    ref = orc.rejection_sample(w.draft_token_ids.cpu(), w.num_draft_tokens, w.max_spec_len,
                               w.draft_probs.cpu(), logits, w.bonus_token_ids.cpu(),
                               temperature=w.temperature.cpu(), all_greedy=w.all_greedy,
                               uniforms=w.uniforms.cpu(), exp_noise=w.exp_noise.cpu(),
                               apply_temperature=w.apply_temperature)
    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), w.num_draft_tokens)
    outputs, _ = rs.RejectionSampler.parse_output(out, w.vocab_size)
    hist = np.bincount([len(o) - 1 for o in outputs], minlength=w.max_spec_len + 1)
    _report("c5 full B=1024 k=7", rep, f" accept_length_hist={hist.tolist()}")
    assert not rep.unexplained, rep.unexplained[:5]
    assert rep.mismatched <= 8


def _softmax64(x: torch.Tensor, t: np.ndarray) -> np.ndarray:
    x64 = x.double().numpy() / t[:, None].astype(np.float64)
    x64 -= x64.max(axis=1, keepdims=True)
    e = np.exp(x64)
    return e / e.sum(axis=1, keepdims=True)


def _rel_check(got: np.ndarray, want: np.ndarray, label: str):
    big = want >= P_MEANINGFUL
    tail = (want >= P_FLOOR) & ~big
    rel = np.abs(got[big] / want[big] - 1.0)
    rel_tail = np.abs(got[tail] / want[tail] - 1.0)
    absd = np.abs(got[want < P_FLOOR] - want[want < P_FLOOR]).max(initial=0.0)
    print(f"[{label}] entries={want.size} p>={P_MEANINGFUL:g}: max rel={rel.max():.3e} "
          f"median rel={np.median(rel):.3e}; tail max rel={rel_tail.max(initial=0.0):.3e}; "
          f"max abs below {P_FLOOR:g}={absd:.3e}", flush=True)
    assert rel.max() <= REL, (label, rel.max())
    assert rel_tail.max(initial=0.0) <= REL_TAIL, (label, rel_tail.max())
    assert absd <= ABS_FLOOR
    # a systematic bias of 1e-6 would move the median, which rounding alone keeps far below
    assert np.median(rel) <= 5e-7, (label, np.median(rel))
    return rel


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_softmax_rows_probability_bound(device, dtype):
    """mvsd_softmax_rows (the materialised target_probs of the sample_recovered_tokens seam)
    against a float64 softmax of the same rows, with and without temperatures."""
    g = torch.Generator(device=device).manual_seed(5150)
    rows, V = 24, configs.VOCAB
    x = (torch.randn(rows, V, generator=g, device=device) * 2.0).to(dtype)
    t = torch.tensor([0.3, 0.8, 1.0, 1.5] * (rows // 4), device=device)
    for temps in (None, t):
        probs = rs._softmax_rows(x, None, temps)
        torch.cuda.synchronize()
        tn = np.ones(rows, np.float32) if temps is None else temps.cpu().numpy()
        want = _softmax64(x.float().cpu(), tn)
        _rel_check(probs.cpu().double().numpy(), want,
                   f"softmax_rows {dtype} T={'1' if temps is None else 'mixed'}")


@pytest.mark.parametrize("case", ["headline", "c4_bf16"])
def test_verify_kernel_row_statistics(device, case):
    """The verify kernel's own statistics: for every random verify row, the read-out maximum
    M equals the row's maximum, the read-out sum S = sum exp((x - M) / T) is within 1e-5
    relative of float64, and the fp32 p[d] the acceptance test compared is within 1e-5
    relative of the float64 softmax at the draft token."""
    w = configs.headline(device) if case == "headline" else configs.ragged_c4(device, B=256)
    sm = SamplingMetadata(temperature=w.temperature, all_greedy=w.all_greedy,
                          all_random=w.all_random, top_k=None, top_p=None)
    stats = torch.full((w.num_tokens, 3), float("nan"), device=device)
    rs.rejection_sample(w.draft_token_ids, w.num_draft_tokens, w.max_spec_len,
                        w.cu_num_draft_tokens, w.draft_probs, w.target_logits,
                        w.bonus_token_ids, sm, uniform_probs=w.uniforms, exp_noise=w.exp_noise,
                        apply_temperature=True, debug_row_stats=stats)
    torch.cuda.synchronize()
    st = stats.cpu().double().numpy()
    req = orc.request_of_row(w.num_draft_tokens)
    temps = w.temperature.cpu().numpy()
    random_rows = temps[req] != 0
    x = w.target_logits.float().cpu()
    t = temps[req].astype(np.float32)
    t = np.where(t == 0, 1.0, t)
    d = w.draft_token_ids.cpu().numpy()
    xr = x[torch.from_numpy(np.nonzero(random_rows)[0])]
    tr = t[random_rows]
    assert np.isnan(st[~random_rows]).all(), "greedy rows must not be written"
    st = st[random_rows]
    x64 = xr.double().numpy()
    assert np.array_equal(st[:, 0], x64.max(axis=1)), "row maximum"
    s64 = np.exp((x64 - x64.max(axis=1, keepdims=True)) / tr[:, None].astype(np.float64)).sum(axis=1)
    srel = np.abs(st[:, 1] / s64 - 1.0)
    print(f"[{case}] row sums: max rel={srel.max():.3e} median={np.median(srel):.3e}", flush=True)
    assert srel.max() <= REL
    p64 = _softmax64(xr, tr)
    dr = d[random_rows]
    valid = (dr >= 0) & (dr < x.shape[1])
    want = p64[np.nonzero(valid)[0], dr[valid]]
    _rel_check(st[valid, 2], want, f"{case} p[d] as compared")


def test_c5_drop_in_forward_with_bonus_rows(device, monkeypatch):
    """RejectionSampler(Sampler()).forward on C5's compact [8192, V] bf16 logits (B=1024, k=7):
    the bonus rows sampled on the device by the exponential race, the verification with the
    gather and temperature in the kernel.  Every seam is fed known randomness (the bonus rows'
    noise, the uniforms, the recovered-token noise); the bonus tokens must equal the oracle
    sampler's on the bonus rows (a race near-tie within 1e-5 relative allowed and counted),
    and the whole output the oracle verification given those bonus tokens."""
    from mvsd.sample import Sampler
    from mvsd.sample import sampler as smp
    from mvsd.testing.spec_metadata import make_metadata, sampling_metadata
    from oracle import sampler as osm

    w = configs.eagle_c5(device)
    B, k, V = w.batch_size, w.max_spec_len, w.vocab_size
    drafts = w.draft_token_ids.view(B, k).tolist()
    meta = make_metadata(drafts, device=device)
    assert torch.equal(meta.target_logits_indices.long(), w.target_rows.long())
    g = torch.Generator(device=device).manual_seed(5005)
    bonus_noise = torch.empty((B, V), device=device).exponential_(generator=g)
    monkeypatch.setattr(smp, "generate_sampler_noise", lambda *a, **kw: bonus_noise)
    monkeypatch.setattr(rs, "generate_uniform_probs", lambda *a, **kw: w.uniforms)
    monkeypatch.setattr(rs, "generate_exponential_noise", lambda *a, **kw: w.exp_noise)
    sm = sampling_metadata([1.0] * B, drafts, device=device)
    out = rs.RejectionSampler(Sampler())(meta, w.draft_probs, w.target_logits, sm)
    got = out.sampled_token_ids.cpu().numpy()

    bonus_rows = w.target_logits[meta.bonus_logits_indices.long()].float().cpu()
    want_bonus, _, scores = osm.forward(bonus_rows, sampling_metadata([1.0] * B, drafts),
                                        bonus_noise.cpu(), "raw_logprobs",
                                        predict_bonus_token=True)
    want_bonus = want_bonus.numpy()
    all_accepted = got[:, k] >= 0
    bonus = want_bonus.copy()
    ties = 0
    for r in np.nonzero(all_accepted)[0]:
        gb, wb = int(got[r, k]), int(want_bonus[r])
        if gb != wb:
            assert float(scores[r, gb]) >= float(scores[r, wb]) * (1 - 1e-5), (r, gb, wb)
            ties += 1
            bonus[r] = gb
    logits = w.target_logits[w.target_rows.long()].cpu()
    ref = orc.rejection_sample(w.draft_token_ids.cpu(), w.num_draft_tokens, k,
                               w.draft_probs.cpu(), logits, torch.from_numpy(bonus).view(B, 1),
                               temperature=w.temperature.cpu(), all_greedy=False,
                               uniforms=w.uniforms.cpu(), exp_noise=w.exp_noise.cpu(),
                               apply_temperature=True)
    rep = orc.compare(got, ref, w.draft_token_ids.cpu(), w.num_draft_tokens)
    _report("c5 drop-in forward B=1024 k=7", rep,
            f" all_accepted={int(all_accepted.sum())} bonus_near_ties={ties}")
    assert all_accepted.any()
    assert not rep.unexplained, rep.unexplained[:5]
