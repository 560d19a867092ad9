"""GPU parity of the V2 verification kernels (csrc/v2_verify.hip) against the CPU restatement
(oracle/v2_rejection.py) on identical seeded inputs, through the C ABI
(mvsd.worker.gpu.spec_decode.rejection_sample -> mvsd_v2_rejection_sample).

Bar: ``num_sampled`` and every defined entry ``sampled[r, :num_sampled[r]]`` equal the oracle's.
A difference is tolerated only where the oracle's decision is a near-tie that fp32 evaluation
differences (device exp2 / log2 within 3 ulp, other summation orders; numpy on the host) can
flip: an acceptance margin |log p - log u - log q| (standard) or |u - h| (block), or the gap
between the two best Gumbel scores, below 8 fp32 ulps of the magnitudes of the terms that enter
it (oracle.v2_rejection.flip_window).  Such cases are counted and printed; every run so far has
had none.
"""

import numpy as np
import pytest
import torch

from oracle import v2_rejection as o
from v2_cases import make_case, near_tie, oracle_args, repeat_case

pytestmark = pytest.mark.gpu

V = 151936


def _run(case, **kw):
    from mvsd.worker.gpu.spec_decode import rejection_sample
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    if "synthetic_conditional_rates" in kw and kw["synthetic_conditional_rates"] is not None:
        kw["synthetic_conditional_rates"] = kw["synthetic_conditional_rates"].cuda()
    s, n = rejection_sample(**dev, **kw)
    torch.cuda.synchronize()
    return s.cpu().numpy(), n.cpu().numpy()


def _compare(case, name, **kw):
    print(f"[v2 parity] {name}", flush=True)
    s, n = _run(case, **kw)
    okw = dict(kw)
    if okw.get("synthetic_conditional_rates") is not None:
        okw["synthetic_conditional_rates"] = okw["synthetic_conditional_rates"].numpy()
    es, en, margins, gaps, wins, gap_wins = o.rejection_sample(
        **oracle_args(case), **okw, return_margins=True, return_windows=True)
    flips = 0
    for r in range(len(en)):
        same = n[r] == en[r] and (s[r, :en[r]] == es[r, :en[r]]).all()
        if same:
            continue
        near = near_tie(margins[r], wins[r], gaps[r], gap_wins[r])
        assert near, f"{name}: request {r}: got {n[r]} {s[r, :n[r]]}, want {en[r]} {es[r, :en[r]]}"
        flips += 1
    in_window = sum(any(m < w for m, w in zip(margins[r], wins[r])) or gaps[r] < gap_wins[r]
                    for r in range(len(en)))
    print(f"[v2 parity] {name}: {len(en)} requests, {flips} near-tie differences "
          f"({in_window} requests with a decision inside its flip window)", flush=True)
    return s, n, es, en


def test_greedy_full_vocab():
    case = make_case([3, 3, 1, 0, 3, 2], [0.0] * 6, 3, V, seed=1, draft_logits=False,
                     invalid={(4, 1)})
    s, n, es, en = _compare(case, "greedy")
    assert (n == en).all()


@pytest.mark.parametrize("use_fp64", [False, True])
def test_random_with_draft_logits(use_fp64):
    temps = [0.8, 1.0, 0.0, 1.3, 0.5, 0.0, 1.0, 0.9]
    case = make_case([4, 4, 4, 2, 4, 0, 3, 4], temps, 4, V, seed=7, invalid={(6, 2)})
    _compare(case, f"random draft_logits fp64={use_fp64}", use_fp64=use_fp64)


def test_random_one_hot_drafts():
    temps = [0.8, 1.0, 0.0, 1.2, 0.6, 1.0]
    case = make_case([3, 3, 3, 3, 1, 3], temps, 3, V, seed=9, draft_logits=False)
    _compare(case, "random one-hot drafts")


def test_bf16_logits():
    temps = [0.8, 1.0, 0.0, 1.3]
    case = make_case([4, 4, 4, 4], temps, 4, V, seed=13, dtype=torch.bfloat16)
    _compare(case, "bf16 target and draft")


def test_synthetic_rates():
    temps = [0.8, 0.0, 1.0, 0.0]
    case = make_case([3, 3, 3, 3], temps, 3, V, seed=17)
    rates = torch.tensor([0.9, 0.5, 0.2])
    _compare(case, "synthetic", synthetic_conditional_rates=rates)


def test_ragged_batch_many_requests():
    g = np.random.default_rng(21)
    R, K = 48, 5
    nd = [int(x) for x in g.integers(0, K + 1, R)]
    temps = [0.0 if x < 0.4 else float(x) for x in g.uniform(0.0, 1.5, R)]
    case = make_case(nd, temps, K, V, seed=21, states=64)
    _compare(case, "ragged 48 requests")


def test_odd_vocab_and_unaligned_rows():
    Vo = 1000 + 3  # rows not a multiple of 16 bytes: scalar loads
    case = make_case([3, 2, 3], [0.9, 0.0, 1.1], 3, Vo, seed=23)
    _compare(case, "odd vocab")


@pytest.mark.parametrize("use_fp64", [False, True])
def test_block_with_draft_logits(use_fp64):
    temps = [0.8, 1.0, 0.0, 1.3, 0.5, 0.0, 1.0, 0.9]
    case = make_case([4, 4, 4, 2, 4, 0, 3, 4], temps, 4, V, seed=7, invalid={(6, 2)})
    _compare(case, f"block draft_logits fp64={use_fp64}", use_fp64=use_fp64,
             use_block_verification=True)


def test_block_one_hot_drafts():
    temps = [0.8, 1.0, 0.0, 1.2, 0.6, 1.0]
    case = make_case([3, 3, 3, 3, 1, 3], temps, 3, V, seed=9, draft_logits=False,
                     invalid={(5, 2)})
    _compare(case, "block one-hot drafts", use_block_verification=True)


def test_block_bf16_logits():
    temps = [0.8, 1.0, 0.0, 1.3]
    case = make_case([4, 4, 4, 4], temps, 4, V, seed=13, dtype=torch.bfloat16)
    _compare(case, "block bf16 target and draft", use_block_verification=True)


@pytest.mark.parametrize("draft_logits", [True, False])
def test_block_ragged_batch_many_requests(draft_logits):
    g = np.random.default_rng(22)
    R, K = 48, 6
    nd = [int(x) for x in g.integers(0, K + 1, R)]
    temps = [0.0 if x < 0.3 else float(x) for x in g.uniform(0.0, 1.5, R)]
    invalid = {(r, int(g.integers(0, K))) for r in range(0, R, 7)}
    case = make_case(nd, temps, K, V, seed=22, states=64, draft_logits=draft_logits,
                     invalid=invalid)
    _compare(case, f"block ragged 48 requests draft_logits={draft_logits}",
             use_block_verification=True)


def test_block_hand_case_many_seeds():
    """The residual design of tests/step75/test_block_verification.py:80-95 (V = 8, K = 2,
    p_tau < 1 at tau = 1) drawn 512 times: every request matches the oracle, every acceptance
    length occurs, and the block residual differs from the standard one on the same draws."""
    target = [[0.0] * 8, [1.0, 0.5, 0.0, -1.0, 0.0, 0.5, 1.5, 0.0],
              [4.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]]
    draft = [[0.0, 0.6, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
             [0.0, 0.0, 0.0, 2.0, 0.0, 0.0, 0.0, 0.0]]
    case = repeat_case(target, draft, [1, 3], 1.0, 512, seed=75)
    s, n, _, _ = _compare(case, "block hand case x512", use_block_verification=True)
    assert set(n.tolist()) == {1, 2, 3}
    s_std, n_std = _run(case)
    assert (n != n_std).any()


@pytest.mark.parametrize("block", [False, True])
def test_chains_longer_than_a_wavefront(block):
    """K = 100 > 64 steps: the chain decides in pages of one step per lane.  Greedy requests
    whose drafts are all the argmax accept all 100 and cross the page boundary."""
    Vs = 4096 + 3
    temps = [0.0, 0.9, 1.0, 0.0, 0.7]
    case = make_case([100, 100, 70, 65, 100], temps, 100, Vs, seed=41, greedy_match=1.0)
    s, n, es, en = _compare(case, f"K=100 block={block}", use_block_verification=block)
    assert n[0] == 101 and n[3] == 66


@pytest.mark.parametrize("block", [False, True])
def test_batch_many_rows(block):
    """About 1000 logits rows in 240 requests at V = 4096: some greedy, some without drafts,
    some with an invalid draft."""
    g = np.random.default_rng(61 + block)
    R, K = 240, 4
    nd = [int(x) for x in g.integers(0, K + 1, R)]
    temps = [0.0 if x < 0.3 else float(x) for x in g.uniform(0.0, 1.5, R)]
    invalid = {(r, int(g.integers(0, K))) for r in range(0, R, 11)}
    case = make_case(nd, temps, K, 4096, seed=61, states=R + 5, invalid=invalid)
    _compare(case, f"R={R} block={block}", use_block_verification=block)


def test_block_and_standard_differ():
    temps = [0.9] * 16
    case = make_case([4] * 16, temps, 4, 4096, seed=43)
    _, n_blk = _run(case, use_block_verification=True)
    _, n_std = _run(case)
    assert (n_blk != n_std).any()


def test_no_host_synchronisation():
    from mvsd.worker.gpu.spec_decode import rejection_sample
    case = make_case([3, 3], [0.8, 0.0], 3, V, seed=4)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    rejection_sample(**dev)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        rejection_sample(**dev)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()


def test_int64_index_tensors():
    """The dtypes the reference's V2 test passes (tests/step73/test_v2_rejection_diff.py:96-98):
    int64 idx_mapping, expanded_idx_mapping, cu_num_logits and draft_sampled.  Every converted
    index array must stay allocated until the launch, or two of them share one block."""
    temps = [0.8, 1.0, 0.0, 1.3, 0.5, 0.9, 1.1, 0.7]
    case = make_case([4, 4, 4, 2, 4, 3, 4, 4], temps, 4, V, seed=31, states=12)
    for key in ("idx_mapping", "expanded_idx_mapping", "cu_num_logits", "draft_sampled",
                "expanded_local_pos"):
        case[key] = case[key].to(torch.int64)
    _compare(case, "int64 index tensors")


@pytest.mark.parametrize("name", ["draft_sampled", "cu_num_logits", "pos", "idx_mapping",
                                  "expanded_idx_mapping", "expanded_local_pos", "temperature",
                                  "seed", "draft_logits", "synthetic_conditional_rates"])
def test_host_argument_is_refused_before_launch(name):
    """A host tensor for any argument raises before anything is enqueued (the kernels would
    otherwise dereference a host address)."""
    from mvsd.worker.gpu.spec_decode import rejection_sample
    case = make_case([2, 2], [0.8, 0.0], 2, 1024, seed=3)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    kw = {}
    if name == "synthetic_conditional_rates":
        kw[name] = torch.tensor([0.9, 0.5])  # host
    else:
        dev[name] = case[name]  # host copy
    with pytest.raises(NotImplementedError, match="device tensors"):
        rejection_sample(**dev, **kw)


def test_short_synthetic_rates_are_refused():
    from mvsd.worker.gpu.spec_decode import rejection_sample
    case = make_case([3, 3], [0.8, 0.0], 3, 1024, seed=3)
    dev = {k: (v.cuda() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    with pytest.raises(ValueError, match="synthetic_conditional_rates"):
        rejection_sample(**dev, synthetic_conditional_rates=torch.tensor([0.9, 0.5]).cuda())
