"""Host-side checks of the V2 verification boundary that need no GPU: the workspace query
of the C ABI and the wrapper's refusals (minivllm/worker/gpu/spec_decode/
rejection_sampler_utils.py:963-966, :1005-1008)."""

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
