"""Pins the CPU restatement of the V2 verification (oracle/v2_rejection.py) without the GPU.

* Philox / tl.rand: the Random123 known answers for Philox4x32-10 and the values Triton's
  own interpreter produced (tests/golden/v2_philox.json);
* the chain and the resampling: closed forms in float64 over explicit probabilities on small
  vocabularies (softmax, max(p - q, 0), brute-force Gumbel argmax), and the semantics the
  reference's tests assert (tests/step73/test_v2_rejection_diff.py:318-327, :357-360).
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import v2_rejection as o
from v2_cases import make_case, oracle_args

GOLDEN = Path(__file__).parent / "golden" / "v2_philox.json"


def test_philox_random123_known_answers():
    assert [int(x) for x in o.philox4x32(0, 0, 0, 0, 0, 0)] == [
        0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert [int(x) for x in o.philox4x32(0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF,
                                         0xFFFFFFFF, 0xFFFFFFFF)] == [
        0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert [int(x) for x in o.philox4x32(0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344,
                                         0xA4093822, 0x299F31D0)] == [
        0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_philox_matches_triton_interpreter():
    data = json.loads(GOLDEN.read_text())
    assert len(data["cases"]) == 10
    for c in data["cases"]:
        dt = np.int64 if c["offset_dtype"] == "int64" else np.int32
        off = np.array(c["offsets"], dtype=dt)
        got = np.stack(o.randint4x(np.int64(c["seed"]), off), 1).astype(np.int64)
        assert (got == np.array(c["randint4x"], dtype=np.int64)).all(), c["seed"]
        bits = o.uint_to_uniform_f32(o.randint4x(np.int64(c["seed"]), off)[0]).view(np.int32)
        assert (bits == np.array(c["rand_bits"], dtype=np.int32)).all(), c["seed"]


def test_uniforms_are_in_the_open_interval():
    u = o.tl_rand32(np.int64(7), np.arange(100000, dtype=np.int64))
    assert u.dtype == np.float32 and (u > 0).all() and (u < 1).all()
    assert abs(float(u.mean()) - 0.5) < 0.01
    u64 = o.tl_rand64(np.int64(7), np.arange(100000, dtype=np.int32))
    assert (u64 > 0).all() and (u64 < 1).all()
    # the lowest value is clamped, not zero (gumbel.py:90, :81-82)
    assert o.uint_to_uniform_f32(np.array([0], np.uint32))[0] == 0
    assert o.tl_rand32(np.int64(0), np.array([0], np.int64))[0] >= o.RAND32_MIN


def _softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def test_greedy_semantics():
    V, K = 40, 1
    case = make_case([1, 1, 1], [0.0, 0.0, 0.0], K, V, seed=3, draft_logits=False,
                     greedy_match=0.0)
    t = case["target_logits"].numpy()
    ds = case["draft_sampled"].numpy()
    ds[1] = int(np.argmax(t[0]))            # request 0: draft == argmax -> accepted
    ds[3] = (int(np.argmax(t[2])) + 1) % V  # request 1: mismatch -> argmax written
    ds[5] = -1                               # request 2: invalid -> rejected
    s, n = o.rejection_sample(**oracle_args(case))
    assert n.tolist() == [2, 1, 1]
    assert s[0, :2].tolist() == [int(np.argmax(t[0])), int(np.argmax(t[1]))]
    assert s[1, 0] == int(np.argmax(t[2]))
    assert s[2, 0] == int(np.argmax(t[4]))


def test_random_acceptance_and_residual_closed_form():
    V, K = 64, 3
    temps = [0.7, 1.0, 1.3, 0.9, 0.0, 1.1]
    case = make_case([3, 3, 2, 3, 3, 1], temps, K, V, seed=11, invalid={(3, 1)})
    a = oracle_args(case)
    s, n, margins, gaps = o.rejection_sample(**a, return_margins=True)
    t, dl, ds, cu = a["target_logits"], a["draft_logits"], a["draft_sampled"], a["cu_num_logits"]
    for r in range(len(temps)):
        st = int(a["idx_mapping"][r])
        tt = float(a["temperature"][st])
        start, end = int(cu[r]), int(cu[r + 1])
        if tt == 0.0:
            continue
        acc = 0
        for i in range(end - start - 1):
            d = int(ds[start + i + 1])
            if d < 0:
                break
            p = _softmax64(t[start + i])
            q = _softmax64(dl[st, i].astype(np.float64) / tt)
            u = float(o.tl_rand32(np.int64(a["seed"][st]), np.int64(a["pos"][start + i])))
            if abs(np.log(p[d]) - np.log(u) - np.log(q[d])) < 1e-4:
                pytest.skip("near-boundary draw")
            if not p[d] / q[d] > u:  # log p > log u + log q
                break
            acc += 1
        assert n[r] == acc + 1, r
        assert s[r, :acc].tolist() == [int(x) for x in ds[start + 1:start + 1 + acc]]
        # resampled token: argmax of log(max(p - q, 0)) + Gumbel(u_v), or of the target row
        ri = start + acc
        d = int(ds[ri + 1]) if ri < end - 1 else -1
        p = _softmax64(t[ri])
        if ri < end - 1 and d >= 0:
            q = _softmax64(dl[st, acc].astype(np.float64) / tt)
            with np.errstate(divide="ignore"):
                base = np.log(np.maximum(p - q, 0.0))
        else:
            base = np.log(p)
        gseed = np.int64(o.randint4x(np.int64(a["seed"][st]), np.int64(a["pos"][ri]))[0])
        uu = o.tl_rand32(gseed, np.arange(V, dtype=np.int32)).astype(np.float64)
        score = base - np.log(-np.log1p(-uu))
        top = np.sort(score[np.isfinite(score)])[-2:]
        if top[1] - top[0] < 1e-4:
            continue
        assert s[r, acc] == int(np.argmax(score)), r


def test_one_hot_drafts_and_synthetic_rates():
    V, K = 48, 2
    case = make_case([2, 2, 2], [0.8, 1.0, 0.0], K, V, seed=5, draft_logits=False)
    a = oracle_args(case)
    s, n = o.rejection_sample(**a)
    t, ds, cu = a["target_logits"], a["draft_sampled"], a["cu_num_logits"]
    for r in range(2):
        start = int(cu[r])
        st = int(a["idx_mapping"][r])
        acc = 0
        for i in range(2):
            d = int(ds[start + i + 1])
            u = float(o.tl_rand32(np.int64(a["seed"][st]), np.int64(a["pos"][start + i])))
            if not _softmax64(t[start + i])[d] > u:  # no draft logits: q = 1
                break
            acc += 1
        assert n[r] == acc + 1
        if acc < 2:  # the rejected draft is never resampled
            assert s[r, acc] != int(ds[start + acc + 1])
    rates = np.array([0.9, 0.1], np.float32)
    s2, n2 = o.rejection_sample(**a, synthetic_conditional_rates=rates)
    for r in range(3):
        st = int(a["idx_mapping"][r])
        start = int(cu[r])
        acc = 0
        for i in range(2):
            u = o.tl_rand32(np.int64(a["seed"][st]), np.int64(a["pos"][start + i]))
            if not u < rates[i]:
                break
            acc += 1
        assert n2[r] == acc + 1


def test_planted_mistake_is_caught():
    """A dropped draft term (q ignored) changes decisions the closed form pins."""
    V, K = 64, 3
    case = make_case([3] * 6, [1.0] * 6, K, V, seed=2)
    a = oracle_args(case)
    _, n = o.rejection_sample(**a)
    b = dict(a)
    b["draft_logits"] = None
    _, n_wrong = o.rejection_sample(**b)
    assert (n != n_wrong).any()


def test_flatten_sampled_by_hand():
    """Rows past a request's sampled tokens are 0 (the reference zero-fills first)."""
    sampled = np.array([[5, 6, 7], [8, -1, -1], [9, 10, -1]])
    flat = o.flatten_sampled(sampled, [3, 1, 2], [0, 3, 5, 8], 8)
    assert flat.tolist() == [5, 6, 7, 8, 0, 9, 10, 0]


def test_flip_windows_cover_fp32_evaluation_only():
    """The flip windows the GPU parity tests allow are a few fp32 ulps of each decision's
    magnitudes: one per decided random step, every one far below the 1e-4 a libm-agnostic
    comparison would need, and zero for greedy requests' gaps."""
    case = make_case([4, 4, 0, 3], [0.8, 0.0, 1.0, 1.2], 4, 4096, seed=31)
    es, en, margins, gaps, wins, gap_wins = o.rejection_sample(
        **oracle_args(case), return_margins=True, return_windows=True)
    for r in range(len(en)):
        assert len(wins[r]) == len(margins[r])
        assert all(o.DEVICE_ULPS * o.EPS32 <= w < 1e-4 for w in wins[r])
    assert gap_wins[1] == 0.0 and 0.0 < gap_wins[0] < 1e-4
    assert o.flip_window(1.0) == 8 * 2.0 ** -23
