"""Pinning of the top-k / top-p oracle (oracle/topk_topp.py) against the definition.

The reference's apply_top_k_top_p (minivllm/sample/ops/topk_topp_sampler.py:48-79) has no
known-answer tests of its own; it is torch sort / softmax / cumsum / scatter.  The oracle is
pinned here by a float64 brute force of the definition on small rows (ties included) and by
the properties the definition implies."""

import numpy as np
import pytest
import torch

from oracle import topk_topp as otp


def _rows(seed, n, V, ties):
    g = np.random.default_rng(seed)
    x = g.normal(0, 2, size=(n, V)).astype(np.float32)
    if ties:
        x = np.round(x * 2) / 2           # many exact ties
    return x


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("mode", ["k", "p", "kp"])
def test_oracle_equals_brute_force(ties, mode):
    V = 40
    x = _rows(7 + ties, 64, V, ties)
    g = np.random.default_rng(3)
    ks = g.integers(1, V, size=64) if "k" in mode else None
    ps = g.uniform(0.05, 0.99, size=64).astype(np.float32) if "p" in mode else None
    out = otp.apply_top_k_top_p(torch.from_numpy(x),
                                None if ks is None else torch.from_numpy(ks),
                                None if ps is None else torch.from_numpy(ps)).numpy()
    for r in range(64):
        k = None if ks is None else int(ks[r])
        p = None if ps is None else float(ps[r])
        want = otp.brute_force_mask(x[r], k, p)
        got = np.isfinite(out[r])
        amb = otp.near_boundary(x[r], k, p)
        assert np.array_equal(got[~amb], want[~amb]), (r, k, p)
        assert np.array_equal(out[r][got], x[r][got])


def test_top_k_keeps_ties_and_at_least_k():
    x = np.array([[1.0, 3.0, 3.0, 2.0, 3.0, 0.5]], dtype=np.float32)
    out = otp.apply_top_k_top_p(torch.from_numpy(x), torch.tensor([2]), None).numpy()
    assert np.isfinite(out[0]).tolist() == [False, True, True, False, True, False]


def test_top_p_always_keeps_the_largest():
    x = np.array([[0.0, 1.0, 2.0, 3.0]], dtype=np.float32)
    out = otp.apply_top_k_top_p(torch.from_numpy(x), None, torch.tensor([1e-6])).numpy()
    assert np.isfinite(out[0]).tolist() == [False, False, False, True]


def test_top_p_one_masks_only_zero_probability_entries():
    x = np.array([[0.0, -200.0, 1.0, -1e4]], dtype=np.float32)
    out = otp.apply_top_k_top_p(torch.from_numpy(x), None, torch.tensor([1.0])).numpy()
    assert np.isfinite(out[0]).tolist() == [True, False, True, False]


def test_k_equal_v_is_a_no_op():
    x = _rows(1, 4, 16, False)
    out = otp.apply_top_k_top_p(torch.from_numpy(x), torch.full((4,), 16), None).numpy()
    assert np.array_equal(out, x)
