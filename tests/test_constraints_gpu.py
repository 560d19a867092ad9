"""GPU parity of the in-kernel sampling constraints: top-k / top-p applied to the raw verify
rows as per-row thresholds (mvsd_sampling_masks, rejection_sample(apply_top_k_top_p=True)).

Bar:
  * the masks the kernels apply, expanded over the raw rows, equal the masks of the
    processed path (temperature divide, then apply_top_k_top_p on the divided fp32 rows)
    entry for entry, and match oracle/topk_topp.py on the divided rows except top-p
    decisions within 1e-5 of the 1 - p crossing (counted);
  * the verify outputs equal the oracle's rejection sampler run on the rows masked the same
    way, up to the counted flips oracle.compare allows;
  * the corrected division x / T the thresholds rely on equals IEEE division for every
    float x (mvsd_selftest(1))."""

from dataclasses import replace

import numpy as np
import pytest
import torch

from mvsd import _native as nat
from mvsd.sample.metadata import SamplingMetadata
from mvsd.sample.ops.topk_topp_sampler import apply_top_k_top_p
from mvsd.sample.rejection_sampler import (apply_sampling_constraints, rejection_sample,
                                           sampling_masks)
from mvsd.testing import configs
from oracle import rejection as orc
from oracle import topk_topp as otp

pytestmark = pytest.mark.gpu


def _expand(masks: torch.Tensor, x: np.ndarray) -> np.ndarray:
    """Boolean [P, V] masked entries of raw rows x from the [P, 4] row masks."""
    m = masks.cpu().numpy()
    a, b = m[:, 0:1], m[:, 1:2]
    j = np.ascontiguousarray(m[:, 2]).view(np.int32)[:, None]
    idx = np.arange(x.shape[1])[None, :]
    return (x < a) | ((x < b) & (idx <= j))


def _divided(x: np.ndarray, temperature: np.ndarray, req: np.ndarray) -> np.ndarray:
    t = temperature[req]
    t = np.where(t == 0, 1.0, t).astype(np.float32)
    return (torch.from_numpy(x) / torch.from_numpy(t).unsqueeze(-1)).numpy()


def _check_against_oracle(xt, masked, ks, ps, label):
    """masked (bool [P, V]) against the oracle's masks of the divided rows xt."""
    ref = otp.apply_top_k_top_p(torch.from_numpy(xt), torch.from_numpy(ks),
                                torch.from_numpy(ps)).numpy()
    want = ~np.isfinite(ref) & np.isfinite(xt)
    flips = 0
    for r in range(xt.shape[0]):
        if np.array_equal(masked[r], want[r]):
            continue
        k = int(ks[r])
        k = k if 0 < k < xt.shape[1] else None
        amb = otp.near_boundary(xt[r], k, float(ps[r]))
        bad = (masked[r] != want[r]) & ~amb
        assert not bad.any(), (label, r, np.nonzero(bad)[0][:10], ks[r], ps[r])
        flips += int((masked[r] != want[r]).sum())
    print(f"[{label}] rows={xt.shape[0]} boundary flips={flips}", flush=True)


def _metadata(w):
    return SamplingMetadata(temperature=w.temperature, all_greedy=False, all_random=False,
                            top_k=w.top_k, top_p=w.top_p)


def _greedy_rows_unmasked_or_exact(masks, got, want, x, greedy_rows):
    """Greedy rows: no mask unless the row's maximum is tied (then the exact mask), and in
    every case the first unmasked maximum is the processed path's argmax."""
    m = masks.cpu().numpy()
    for r in np.nonzero(greedy_rows)[0]:
        neutral = m[r, 0] == -np.inf and m[r, 1] == -np.inf
        tied = (x[r] == x[r].max()).sum() > 1
        assert (neutral and not got[r].any()) or (tied and np.array_equal(got[r], want[r])), r
        kept = np.where(want[r], -np.inf, x[r])
        assert int(np.argmax(np.where(got[r], -np.inf, x[r]))) == int(np.argmax(kept)), r


@pytest.mark.parametrize("B", [96])
def test_c4_masks_match_processed_path_and_oracle(device, B):
    w = configs.ragged_c4(device, B=B)
    sm = _metadata(w)
    masks = sampling_masks(w.target_logits, w.cu_num_draft_tokens, sm)
    x = w.target_logits.float()
    x_cpu = x.cpu().numpy()
    got = _expand(masks, x_cpu)
    processed = apply_sampling_constraints(x.clone(), w.cu_num_draft_tokens, sm)
    want = ~torch.isfinite(processed).cpu().numpy()
    req = orc.request_of_row(w.num_draft_tokens)
    greedy = w.temperature.cpu().numpy()[req] == 0
    assert greedy.any() and (~greedy).any()
    rnd = ~greedy
    assert np.array_equal(got[rnd], want[rnd]), np.argwhere(got[rnd] != want[rnd])[:10]
    _greedy_rows_unmasked_or_exact(masks, got, want, x_cpu, greedy)
    xt = _divided(x_cpu, w.temperature.cpu().numpy(), req)
    _check_against_oracle(xt[rnd], got[rnd], w.top_k.cpu().numpy()[req][rnd],
                          w.top_p.cpu().numpy()[req][rnd], "c4 in-kernel masks")


@pytest.mark.parametrize("B,V,seed,dtype", [(128, configs.VOCAB, 2024, torch.bfloat16),
                                            (64, configs.VOCAB, 2025, torch.float16),
                                            (4500, 1024, 2027, torch.bfloat16)],
                         ids=["B128", "B64_fp16", "B4500_several_launches"])
def test_c4_in_kernel_constraints_then_verify(device, B, V, seed, dtype):
    """rejection_sample on the raw 2-byte rows with the divide and the constraints in the
    kernels, against the oracle sampler on the same rows masked by the processed path.  Beyond
    4096 requests the constraints kernel masks the whole batch once and several verify launches
    share its masks, plan order and slot arrays."""
    w = configs.ragged_c4(device, B=B, V=V, seed=seed)
    if dtype != w.target_logits.dtype:
        w = replace(w, target_logits=w.target_logits.to(dtype))
    sm = _metadata(w)
    out = rejection_sample(w.draft_token_ids, w.num_draft_tokens, w.max_spec_len,
                           w.cu_num_draft_tokens, w.draft_probs, w.target_logits,
                           w.bonus_token_ids, sm, uniform_probs=w.uniforms,
                           exp_noise=w.exp_noise, apply_temperature=True,
                           apply_top_k_top_p=True)
    processed = apply_sampling_constraints(w.target_logits.float(), w.cu_num_draft_tokens, sm)
    ref = orc.rejection_sample(w.draft_token_ids.cpu(), w.num_draft_tokens, w.max_spec_len,
                               w.draft_probs.cpu(), processed.cpu(), w.bonus_token_ids.cpu(),
                               temperature=w.temperature.cpu(), all_greedy=False,
                               uniforms=w.uniforms.cpu(), exp_noise=w.exp_noise.cpu(),
                               apply_temperature=False)
    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), w.num_draft_tokens)
    print(f"[c4 in-kernel constraints] requests={rep.requests} mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}", flush=True)
    assert not rep.unexplained, rep.unexplained[:5]


def _single_request_rows(device, x: np.ndarray, temps, ks, ps, dtype=torch.float32):
    """One verify row per request: (target, cu, metadata) for rows x [n, V]."""
    n = x.shape[0]
    target = torch.from_numpy(x).to(device=device, dtype=dtype)
    cu = torch.arange(1, n + 1, dtype=torch.int32, device=device)
    sm = SamplingMetadata(temperature=torch.tensor(temps, dtype=torch.float32, device=device),
                          all_greedy=False, all_random=False,
                          top_k=torch.tensor(ks, dtype=torch.int64, device=device),
                          top_p=torch.tensor(ps, dtype=torch.float32, device=device))
    return target, cu, sm


def test_temperature_merging_neighbours(device):
    """Raw values one ulp apart that the divide by T maps to one value: the masks on the raw
    rows treat them as the equal values the processed rows hold (ties by index)."""
    V = 2048
    g = np.random.default_rng(5)
    base = g.normal(0, 2, size=(24, V)).astype(np.float32)
    pairs = g.integers(0, V, size=(24, 400))
    for r in range(24):
        src, dst = pairs[r, :200], pairs[r, 200:]
        base[r, dst] = np.nextafter(base[r, src], np.float32(np.inf))
    temps = [3.0, 0.7, 1.3, 2.9] * 6
    ks = [V, 7, 50, 300, V, 1] * 4
    ps = [0.5, 1.0, 0.9, 1.0, 0.95, 1.0] * 4
    target, cu, sm = _single_request_rows(device, base, temps, ks, ps)
    masks = sampling_masks(target, cu, sm)
    got = _expand(masks, base)
    processed = apply_sampling_constraints(target.clone(), cu, sm)
    want = ~torch.isfinite(processed).cpu().numpy()
    assert np.array_equal(got, want), np.argwhere(got != want)[:10]
    xt = _divided(base, np.array(temps, dtype=np.float32), np.arange(24))
    _check_against_oracle(xt, got, np.array(ks), np.array(ps, dtype=np.float32), "merged")


@pytest.mark.parametrize("case", ["k_above_512", "all_equal_k", "all_equal_p", "p_all"])
def test_fallback_paths(device, case):
    """The bisection fallbacks (k > 512, more tied candidates or bin entries than LDS holds)
    and the every-entry-but-one case, through the in-place op and the row masks."""
    V = 8192
    g = np.random.default_rng(11)
    if case == "k_above_512":
        x = g.normal(0, 2, size=(8, V)).astype(np.float32)
        ks, ps = [600, 1000, 4000, 8000, 513, 2048, 777, 5000], [1.0] * 4 + [0.9, 0.5, 0.99, 0.3]
    elif case == "all_equal_k":
        x = np.zeros((4, V), dtype=np.float32)
        x[1, ::3] = 1.0
        x[2] = np.round(g.normal(0, 1, size=V)).astype(np.float32)
        ks, ps = [50, 5000, 100, 4097], [1.0, 1.0, 0.6, 1.0]
    elif case == "all_equal_p":
        x = np.zeros((4, V), dtype=np.float32)
        x[1, : V // 2] = -0.5
        x[2] = np.round(g.normal(0, 0.2, size=V) * 4) / 4
        x[3, 100:] = -1e-3
        ks, ps = [V, V, V, V], [0.5, 0.3, 0.7, 0.1]
    else:
        x = g.normal(0, 2, size=(4, V)).astype(np.float32)
        x[3, [10, 20, 30]] = x[3].max() + 1.0
        ks, ps = [V, 100, V, V], [1e-9, 1e-9, -0.5, 1e-9]
    temps = [1.0] * x.shape[0]
    ks_np, ps_np = np.array(ks, dtype=np.int64), np.array(ps, dtype=np.float32)
    xg = torch.from_numpy(x).to(device)
    apply_top_k_top_p(xg, torch.from_numpy(ks_np).to(device), torch.from_numpy(ps_np).to(device))
    inplace = ~torch.isfinite(xg).cpu().numpy()
    target, cu, sm = _single_request_rows(device, x, temps, ks, ps)
    got = _expand(sampling_masks(target, cu, sm), x)
    assert np.array_equal(got, inplace)
    _check_against_oracle(x, got, ks_np, ps_np, case)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_rows_with_tied_maxima(device, dtype):
    """Greedy rows whose maximum is tied, under top-p values on both sides of the point where
    the masked prefix reaches the maximum: each mask is neutral (the prefix stops below the
    maximum, so the argmax is unchanged) or the processed path's mask exactly, and the first
    unmasked maximum is the processed path's argmax."""
    V, n = 4096, 24
    g = np.random.default_rng(8)
    x = g.normal(0, 1, size=(n, V)).astype(np.float32)
    for r in range(n):
        ties = int(g.integers(2, 7))
        x[r, g.choice(V, ties, replace=False)] = 9.0 if r % 2 else 4.0
    x = torch.from_numpy(x).to(dtype).float().numpy()  # values the rows hold
    ps = [0.1, 0.3, 0.5, 0.6, 0.9, 1e-7] * 4
    target, cu, sm = _single_request_rows(device, x, [0.0] * n, [V] * n, ps, dtype=dtype)
    masks = sampling_masks(target, cu, sm)
    got = _expand(masks, x)
    processed = apply_sampling_constraints(target.float().clone(), cu, sm)
    want = ~torch.isfinite(processed).cpu().numpy()
    _greedy_rows_unmasked_or_exact(masks, got, want, x, np.ones(n, dtype=bool))
    reach = [r for r in range(n) if want[r][x[r] == x[r].max()].any()]
    assert 0 < len(reach) < n, reach  # both cases occur


def test_greedy_row_argmax_respects_top_p_tie_order(device):
    """A greedy request in a mixed batch is masked too (the reference divides by 1 and masks
    every row): with a tiny top_p only the last of the tied maxima survives, so the greedy
    token is that entry, not the first maximum."""
    V = 4096
    g = np.random.default_rng(3)
    x = g.normal(0, 1, size=(3, V)).astype(np.float32)
    x[0, [5, 10, 700]] = 9.0
    draft_ids = torch.tensor([5, 700, 1], dtype=torch.int32, device=device)
    cu = torch.tensor([1, 3], dtype=torch.int32, device=device)
    target = torch.from_numpy(x).to(device)
    temperature = torch.tensor([0.0, 0.9], dtype=torch.float32, device=device)
    sm = SamplingMetadata(temperature=temperature, all_greedy=False, all_random=False,
                          top_k=torch.tensor([V, 20], dtype=torch.int64, device=device),
                          top_p=torch.tensor([1e-7, 1.0], dtype=torch.float32, device=device))
    draft_probs = torch.softmax(torch.from_numpy(x).to(device) / 0.9, dim=-1)
    uniforms = torch.tensor([0.5, 0.5, 0.5], dtype=torch.float64, device=device)
    noise = torch.empty((2, V), device=device).exponential_()
    bonus = torch.tensor([[1], [2]], dtype=torch.int32, device=device)
    out = rejection_sample(draft_ids, [1, 2], 2, cu, draft_probs, target, bonus, sm,
                           uniform_probs=uniforms, exp_noise=noise, apply_temperature=True,
                           apply_top_k_top_p=True)
    processed = apply_sampling_constraints(target.clone(), cu, sm)
    ref = orc.rejection_sample(draft_ids.cpu(), [1, 2], 2, draft_probs.cpu(), processed.cpu(),
                               bonus.cpu(), temperature=temperature.cpu(), all_greedy=False,
                               uniforms=uniforms.cpu(), exp_noise=noise.cpu(),
                               apply_temperature=False)
    o = out.cpu().numpy()
    assert o[0, 0] == 700, o[0]
    rep = orc.compare(o, ref, draft_ids.cpu(), [1, 2])
    assert not rep.unexplained, rep.unexplained


def test_division_selftest(device):
    failures = torch.zeros(1, dtype=torch.int64, device=device)
    nat.check(nat.lib().mvsd_selftest(1, failures.data_ptr(), nat.stream_of(device)),
              "mvsd_selftest")
    assert int(failures.item()) == 0


def test_masked_call_leaves_workspace_zero(device):
    """A masked call writes row masks into the workspace; the verify kernel zeroes them again,
    so the whole workspace is zero after the call, and a later, smaller unmasked call, whose
    slot arrays overlap the old mask rows, stays exact."""
    from mvsd.sample import rejection_sampler as rs

    w = configs.ragged_c4(device, B=128, seed=2025)
    rejection_sample(w.draft_token_ids, w.num_draft_tokens, w.max_spec_len,
                     w.cu_num_draft_tokens, w.draft_probs, w.target_logits, w.bonus_token_ids,
                     _metadata(w), uniform_probs=w.uniforms, exp_noise=w.exp_noise,
                     apply_temperature=True, apply_top_k_top_p=True)
    torch.cuda.synchronize()
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           nat.stream_of(device))
    ws = rs._WORKSPACES[key].clone()
    nonzero = torch.nonzero(ws).flatten()
    assert nonzero.numel() == 0, f"workspace bytes left non-zero: {nonzero[:8].tolist()}"

    small = configs.random_c2(device, B=64, k=4, seed=2026)
    sm = SamplingMetadata(temperature=small.temperature, all_greedy=False, all_random=True,
                          top_k=None, top_p=None)
    out = rejection_sample(small.draft_token_ids, small.num_draft_tokens, small.max_spec_len,
                           small.cu_num_draft_tokens, small.draft_probs, small.target_logits,
                           small.bonus_token_ids, sm, uniform_probs=small.uniforms,
                           exp_noise=small.exp_noise, apply_temperature=small.apply_temperature)
    ref = orc.rejection_sample(small.draft_token_ids.cpu(), small.num_draft_tokens,
                               small.max_spec_len, small.draft_probs.cpu(),
                               small.target_logits.cpu(), small.bonus_token_ids.cpu(),
                               temperature=small.temperature.cpu(), all_greedy=False,
                               uniforms=small.uniforms.cpu(), exp_noise=small.exp_noise.cpu(),
                               apply_temperature=small.apply_temperature)
    rep = orc.compare(out.cpu().numpy(), ref, small.draft_token_ids.cpu(), small.num_draft_tokens)
    print(f"[after masked call] mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}", flush=True)
    assert not rep.unexplained, rep.unexplained[:5]


@pytest.mark.parametrize("B,k,V", [(16, 3, 32768), (64, 4, 151936)])
def test_masked_chunks_with_zero_maximum(device, B, k, V):
    """Random rows whose only positive entries lie in the first 64 columns; every other entry is
    negative or exactly +0.0, and top-k = 50 masks all of them.  Every chunk of a row past the
    first then has the raw maximum +0.0 and nothing kept, so it publishes the statistics pair
    (+0.0, sum 0).  The call must finish without poisoned rows and give the oracle's tokens on
    the rows masked by the processed path."""
    g = torch.Generator().manual_seed(4400 + B)
    P = B * k
    x = -torch.randn(P, V, generator=g).abs() * 2.0
    x[:, ::3] = 0.0
    x[:, :64] = 1.0 + 2.0 * torch.rand(P, 64, generator=g)
    temps = torch.full((B,), 0.8)
    q = torch.softmax((x / 0.8 + 0.5 * torch.randn(P, V, generator=g)).double(), -1).float()
    head = q[:, :64] / q[:, :64].sum(-1, keepdim=True)
    ids = torch.multinomial(head, 1, generator=g).flatten().to(torch.int32)
    u = torch.rand(P, generator=g, dtype=torch.float64)
    noise = torch.empty(B, V).exponential_(1.0, generator=g)
    bonus = torch.randint(0, V, (B,), generator=g, dtype=torch.int32)
    ks = [k] * B
    cu = torch.tensor(np.cumsum(ks), dtype=torch.int32)
    dev = dict(device=device)
    sm = SamplingMetadata(temperature=temps.to(**dev), all_greedy=False, all_random=True,
                          top_k=torch.full((B,), 50, dtype=torch.int64, **dev), top_p=None)
    out = rejection_sample(ids.to(**dev), ks, k, cu.to(**dev), q.to(**dev), x.to(**dev),
                           bonus.to(**dev), sm, uniform_probs=u.to(**dev),
                           exp_noise=noise.to(**dev), apply_temperature=True,
                           apply_top_k_top_p=True)
    got = out.cpu().numpy()
    assert not (got == nat.POISON).any(), np.flatnonzero((got == nat.POISON).any(axis=1))
    processed = apply_sampling_constraints(x.to(**dev), cu.to(**dev), sm)
    ref = orc.rejection_sample(ids, ks, k, q, processed.cpu(), bonus, temperature=temps,
                               all_greedy=False, uniforms=u, exp_noise=noise,
                               apply_temperature=False)
    rep = orc.compare(got, ref, ids, ks)
    print(f"[zero-max masked chunks B={B} V={V}] mismatched={rep.mismatched} "
          f"accept_flips={rep.accept_flips} recovered_flips={rep.recovered_flips}", flush=True)
    assert not rep.unexplained, rep.unexplained[:5]
    assert (got[:, 0] >= 0).all()
