"""Host-side checks of the V2 verification boundary that need no GPU: the workspace query
of the C ABI, the wrapper's refusals (minivllm/worker/gpu/spec_decode/
rejection_sampler_utils.py:963-966, :1005-1008), and the V2 RejectionSampler's chunking and
method dispatch (minivllm/worker/gpu/spec_decode/rejection_sampler.py:45-96)."""

import numpy as np
import pytest
import torch

from mvsd import _native as nat
from v2_cases import make_case


def test_workspace_bytes_query():
    lib = nat.lib()
    assert lib.mvsd_v2_workspace_bytes(0, 0, 151936) >= 0
    assert lib.mvsd_v2_workspace_bytes(-1, 4, 151936) == -1
    assert lib.mvsd_v2_workspace_bytes(10, 2, 0) == -1
    small = lib.mvsd_v2_workspace_bytes(1280, 256, 151936)
    # 38 chunks: 6 arrays of 4 B per (row, chunk), 5 per row, 4 per request, 12 B per
    # (request, chunk)
    assert small >= 1280 * 38 * 24 + 1280 * 20 + 256 * 16 + 256 * 38 * 12
    assert small % 256 == 0
    assert lib.mvsd_v2_workspace_bytes(2560, 256, 151936) > small


def test_block_verification_with_synthetic_rates_is_refused():
    """Block verification and synthetic rates are exclusive (:1043-1045); the wrapper asserts
    before any launch, and the C ABI refuses the combination too."""
    from mvsd.worker.gpu.spec_decode import rejection_sample
    case = make_case([1], [1.0], 1, 64, seed=1)
    with pytest.raises(NotImplementedError, match="device tensors"):
        rejection_sample(**case, use_block_verification=True)
    with pytest.raises(AssertionError):
        rejection_sample(**case, synthetic_conditional_rates=torch.ones(1),
                         use_block_verification=True)


def test_host_tensors_are_refused():
    from mvsd.worker.gpu.spec_decode import rejection_sample
    case = make_case([1], [1.0], 1, 64, seed=1)
    with pytest.raises(NotImplementedError, match="device tensors"):
        rejection_sample(**case)


# ------------------------------------------------------------------ chunking (host logic) --

def _cu(rows):
    return np.concatenate(([0], np.cumsum(np.asarray(rows, dtype=np.int64))))


def test_chunk_budget_known_answers():
    """tests/step73/test_v2_verify_chunking.py:43-49: 1 GiB of fp32 rows, at least one."""
    from mvsd.worker.gpu.spec_decode import MAX_CHUNK_BYTES, get_max_chunk_logits
    assert get_max_chunk_logits(151936) == MAX_CHUNK_BYTES // (151936 * 4) == 1766
    assert get_max_chunk_logits(32000) == 8388
    assert get_max_chunk_logits(128256) == 2092
    assert get_max_chunk_logits(MAX_CHUNK_BYTES) == 1


@pytest.mark.parametrize("limit", [5, 6, 7, 11, 64])
def test_chunks_are_maximal_whole_request_runs(limit):
    """Every chunk fits the limit, covers requests in order without gaps, and is maximal:
    adding the next request would exceed the limit (brute force over the batch)."""
    from mvsd.worker.gpu.spec_decode.rejection_sampler import _iter_request_chunks
    rows = [int(x) for x in np.random.default_rng(0).integers(1, 6, 40)]
    cu = _cu(rows)
    chunks = list(_iter_request_chunks(cu, limit))
    assert [i for s, e in chunks for i in range(s, e)] == list(range(len(rows)))
    for s, e in chunks:
        assert cu[e] - cu[s] <= limit
        if e < len(rows):
            assert cu[e + 1] - cu[s] > limit


def test_oversized_request_and_stale_offsets_known_answers():
    """tests/step73/test_v2_verify_chunking.py:74-82 (a request above the limit is a chunk by
    itself) and tests/step75/test_logit_chunks.py:287-300 (fresh vs stale offsets)."""
    from mvsd.worker.gpu.spec_decode.rejection_sampler import _iter_request_chunks
    assert list(_iter_request_chunks(_cu([2, 2, 100, 2, 2]), 10)) == [(0, 2), (2, 3), (3, 5)]
    assert list(_iter_request_chunks(np.array([0, 4, 8, 12]), 8)) == [(0, 2), (2, 3)]
    assert list(_iter_request_chunks(np.array([0, 6, 12, 18]), 8))[0] == (0, 1)
    big = _cu([5] * 512)
    chunks = list(_iter_request_chunks(big, 1766))
    assert len(chunks) == 2 and all(big[e] - big[s] <= 1766 for s, e in chunks)


def test_method_dispatch_at_construction():
    """(rejection_sampler.py:84-96): one switch for block, a conditional-rate table for
    synthetic, neither for standard."""
    from types import SimpleNamespace
    from mvsd.worker.gpu.spec_decode import RejectionSampler
    mk = lambda **kw: SimpleNamespace(num_speculative_tokens=3, **kw)  # noqa: E731
    rs = RejectionSampler(None, mk(rejection_sample_method="standard"), torch.device("cpu"))
    assert not rs.use_block_verification and rs.synthetic_conditional_rates is None
    rs = RejectionSampler(None, mk(rejection_sample_method="block"), torch.device("cpu"))
    assert rs.use_block_verification and rs.synthetic_conditional_rates is None
    rs = RejectionSampler(None, mk(rejection_sample_method="synthetic",
                                   synthetic_acceptance_rates=[0.8, 0.4, 0.2]),
                          torch.device("cpu"))
    assert not rs.use_block_verification
    assert rs.synthetic_conditional_rates.tolist() == pytest.approx([0.8, 0.5, 0.5])
    assert rs.num_speculative_steps == 3
