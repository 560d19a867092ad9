"""GPU parity of top-k / top-p masking (mvsd_apply_top_k_top_p) against oracle/topk_topp.py.

Bar: the kept/masked decision of every entry is identical, except top-p decisions at entries
whose cumulative mass is within 1e-5 of 1 - p (oracle.near_boundary; counted and printed);
kept entries are unchanged bit for bit."""

import numpy as np
import pytest
import torch

from mvsd.sample.ops.topk_topp_sampler import apply_top_k_top_p
from mvsd.sample.rejection_sampler import apply_sampling_constraints, rejection_sample
from mvsd.sample.metadata import SamplingMetadata
from mvsd.testing import configs
from oracle import rejection as orc
from oracle import topk_topp as otp

pytestmark = pytest.mark.gpu


def _check_rows(x_cpu, out_gpu, ks, ps, label):
    out = out_gpu.cpu().numpy()
    ref = otp.apply_top_k_top_p(torch.from_numpy(x_cpu),
                                None if ks is None else torch.from_numpy(ks),
                                None if ps is None else torch.from_numpy(ps)).numpy()
    flips = 0
    for r in range(x_cpu.shape[0]):
        got, want = np.isfinite(out[r]), np.isfinite(ref[r])
        if np.array_equal(got, want):
            continue
        k = None if ks is None else int(ks[r])
        p = None if ps is None else float(ps[r])
        amb = otp.near_boundary(x_cpu[r], k if (k is not None and 0 < k < x_cpu.shape[1]) else None, p)
        bad = (got != want) & ~amb
        assert not bad.any(), (label, r, np.nonzero(bad)[0][:10], k, p)
        flips += int((got != want).sum())
    kept = np.isfinite(out)
    assert np.array_equal(out[kept], x_cpu[kept])
    print(f"[{label}] rows={x_cpu.shape[0]} boundary flips={flips}", flush=True)


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("mode", ["k", "p", "kp"])
@pytest.mark.parametrize("V", [7, 40, 1001, 4096])
def test_small_rows_match_oracle(device, ties, mode, V):
    g = np.random.default_rng(V + 10 * ties)
    x = g.normal(0, 2, size=(48, V)).astype(np.float32)
    if ties:
        x = np.round(x * 2) / 2
    ks = g.integers(1, V, size=48).astype(np.int64) if "k" in mode else None
    if ks is not None:
        ks[:4] = V        # rows without top-k
    ps = g.uniform(0.05, 0.99, size=48).astype(np.float32) if "p" in mode else None
    if ps is not None:
        ps[4:6] = 1.0     # p = 1 masks only zero-probability entries
        ps[6] = 1e-7      # keeps only the largest
    xg = torch.from_numpy(x).to(device)
    apply_top_k_top_p(xg, None if ks is None else torch.from_numpy(ks).to(device),
                      None if ps is None else torch.from_numpy(ps).to(device))
    _check_rows(x, xg, ks, ps, f"V={V} {mode} ties={ties}")


def test_full_vocab_rows_match_oracle(device):
    V = configs.VOCAB
    g = torch.Generator(device=device).manual_seed(77)
    n = 64
    x = torch.randn((n, V), device=device, generator=g) * 2.0 / 0.8
    ks = torch.full((n,), V, dtype=torch.int64)
    ps = torch.ones(n, dtype=torch.float32)
    ks[:16] = 50
    ks[16:24] = 1
    ps[24:40] = 0.9
    ps[40:48] = 0.5
    ks[48:56] = 1000
    ps[48:56] = 0.8
    x_cpu = x.cpu().numpy()
    apply_top_k_top_p(x, ks.to(device), ps.to(device))
    _check_rows(x_cpu, x, ks.numpy(), ps.numpy(), "full V")


def test_ties_at_the_top_p_crossing_use_index_order(device):
    # 6 equal maxima and a small tail: p chosen so the crossing falls inside the run of ties
    x = np.full((1, 64), -30.0, dtype=np.float32)
    x[0, [3, 9, 20, 33, 41, 60]] = 0.0
    ps = np.array([0.5], dtype=np.float32)
    xg = torch.from_numpy(x).to(device)
    apply_top_k_top_p(xg, None, torch.from_numpy(ps).to(device))
    kept = np.nonzero(np.isfinite(xg.cpu().numpy()[0]))[0].tolist()
    ref = otp.apply_top_k_top_p(torch.from_numpy(x), None, torch.from_numpy(ps)).numpy()
    assert kept == np.nonzero(np.isfinite(ref[0]))[0].tolist() == [33, 41, 60]


def test_c4_constraints_then_verify(device):
    """c4 with its top-k=50 / top-p=0.9 quartiles through apply_sampling_constraints and the
    verify kernel: processed logits match the oracle's masks, and given the processed logits
    the token outputs match the oracle bit for bit."""
    w = configs.ragged_c4(device, B=96)
    sm = SamplingMetadata(temperature=w.temperature, all_greedy=False, all_random=False,
                          top_k=w.top_k, top_p=w.top_p)
    x = w.target_logits.float()
    x_cpu = x.cpu().numpy()
    processed = apply_sampling_constraints(x.clone(), w.cu_num_draft_tokens, sm)
    # oracle masks over the temperature-divided rows
    req = orc.request_of_row(w.num_draft_tokens)
    t = w.temperature.cpu().numpy()[req]
    t = np.where(t == 0, 1.0, t).astype(np.float32)
    xt = (torch.from_numpy(x_cpu) / torch.from_numpy(t).unsqueeze(-1)).numpy()
    ks = w.top_k.cpu().numpy()[req]
    ps = w.top_p.cpu().numpy()[req]
    _check_rows(xt, processed, ks, ps, "c4 processed")
    out = rejection_sample(w.draft_token_ids, w.num_draft_tokens, w.max_spec_len,
                           w.cu_num_draft_tokens, w.draft_probs, processed, w.bonus_token_ids, sm,
                           uniform_probs=w.uniforms, exp_noise=w.exp_noise)
    ref = orc.rejection_sample(w.draft_token_ids.cpu(), w.num_draft_tokens, w.max_spec_len,
                               w.draft_probs.cpu(), processed.cpu(), w.bonus_token_ids.cpu(),
                               temperature=w.temperature.cpu(), all_greedy=False,
                               uniforms=w.uniforms.cpu(), exp_noise=w.exp_noise.cpu(),
                               apply_temperature=False)
    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), w.num_draft_tokens)
    print(f"[c4 top-k/top-p] requests={rep.requests} mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}", flush=True)
    assert not rep.unexplained, rep.unexplained[:5]
