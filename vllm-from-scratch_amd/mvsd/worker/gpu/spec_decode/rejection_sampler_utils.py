"""V2 ``rejection_sample`` on the HIP kernels of ``csrc/v2_verify.hip``.

Same name, arguments, dtypes and outputs as the V2 model runner's verification
(minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py:935-1201):

* ``target_logits [num_logits, V]`` (already temperature-scaled), rows of one request
  contiguous, its bonus row last; ``draft_logits [max_num_reqs, K, V]`` pre-temperature, or
  None for one-hot drafts; ``draft_sampled [num_logits]`` where entry ``j + 1`` is the draft
  verified at row ``j``; ``cu_num_logits [num_reqs + 1]`` with a leading 0; ``pos``,
  ``idx_mapping``, ``expanded_idx_mapping``, ``expanded_local_pos``, per-state
  ``temperature`` and ``seed``;
* returns ``(sampled [num_reqs, K + 1] int64, num_sampled [num_reqs] int32)``; entries at or
  past ``num_sampled[r]`` are undefined, as in the reference (``new_empty``, :1118-1121).

Acceptance draws ``u = tl_rand32(seed, pos)`` and the resampling's Gumbel noise
``tl_rand32(tl.randint(seed, pos), vocab index)`` (or the fp64 forms with ``use_fp64``) come
from the same Philox4x32-10 counter stream as Triton's ``tl.randint4x`` / ``tl.rand``
(minivllm/worker/gpu/sample/gumbel.py:72-131), so a draft and its verification can agree on
noise.  Block verification (``use_block_verification=True``, :318-493) is not built and
raises ``NotImplementedError``.  No host synchronisation; every launch is on the current
stream of the target's device.
"""

from __future__ import annotations

import torch

from ...._native import (F32, check, dtype_code, lib, ptr, require_device_tensor,
                         stream_of)

_FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _as(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return t if t.dtype == dtype and t.is_contiguous() else t.to(dtype).contiguous()


def rejection_sample(
    target_logits: torch.Tensor,
    draft_logits: torch.Tensor | None,
    draft_sampled: torch.Tensor,
    cu_num_logits: torch.Tensor,
    pos: torch.Tensor,
    idx_mapping: torch.Tensor,
    expanded_idx_mapping: torch.Tensor,
    expanded_local_pos: torch.Tensor,
    temperature: torch.Tensor,
    seed: torch.Tensor,
    num_speculative_steps: int,
    synthetic_conditional_rates: torch.Tensor | None = None,
    use_fp64: bool = False,
    use_block_verification: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """V2 verification (rejection_sampler_utils.py:935-1201), non-block path."""
    assert target_logits.ndim == 2 and target_logits.stride(-1) == 1
    assert draft_logits is None or (draft_logits.ndim == 3 and draft_logits.stride(-1) == 1)
    if use_block_verification:
        assert synthetic_conditional_rates is None, (
            "Block verification is incompatible with synthetic acceptance rates.")
        raise NotImplementedError(
            "block verification (rejection_sampler_utils.py:318-493) is not built in this "
            "implementation; use use_block_verification=False")
    require_device_tensor(target_logits, "target_logits")
    if target_logits.dtype not in _FLOAT_DTYPES:
        raise TypeError(f"target_logits dtype {target_logits.dtype} is not supported")
    device = target_logits.device
    num_reqs = cu_num_logits.shape[0] - 1
    num_logits, vocab_size = target_logits.shape
    d_stride0 = d_stride1 = 0
    d_code = F32
    if draft_logits is not None:
        require_device_tensor(draft_logits, "draft_logits")
        if draft_logits.dtype not in _FLOAT_DTYPES:
            raise TypeError(f"draft_logits dtype {draft_logits.dtype} is not supported")
        d_stride0, d_stride1 = draft_logits.stride(0), draft_logits.stride(1)
        d_code = dtype_code(draft_logits.dtype)
        # The draft vocabulary may be padded differently (rejection_sampler_utils.py:970-973).
        vocab_size = min(vocab_size, draft_logits.size(-1))
    K = int(num_speculative_steps)
    sampled = draft_sampled.new_empty(num_reqs, K + 1, dtype=torch.int64)
    num_sampled = sampled.new_empty(num_reqs, dtype=torch.int32)
    if num_reqs == 0:
        return sampled, num_sampled
    rates = None
    if synthetic_conditional_rates is not None:
        rates = _as(synthetic_conditional_rates, torch.float32)
    temp = _as(temperature, torch.float32)
    seeds = _as(seed, torch.int64)
    num_states = min(temp.numel(), seeds.numel())
    if draft_logits is not None:
        num_states = min(num_states, draft_logits.shape[0])
    ws_bytes = lib().mvsd_v2_workspace_bytes(num_logits, num_reqs, vocab_size)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    check(lib().mvsd_v2_rejection_sample(
        sampled.data_ptr(), sampled.stride(0), num_sampled.data_ptr(),
        target_logits.data_ptr(), dtype_code(target_logits.dtype), target_logits.stride(0),
        num_logits, ptr(draft_logits), d_code, d_stride0, d_stride1,
        _as(draft_sampled, torch.int32).data_ptr(), _as(cu_num_logits, torch.int32).data_ptr(),
        _as(pos, torch.int64).data_ptr(), _as(idx_mapping, torch.int32).data_ptr(),
        _as(expanded_idx_mapping, torch.int32).data_ptr(),
        _as(expanded_local_pos, torch.int32).data_ptr(), temp.data_ptr(), seeds.data_ptr(),
        num_states, num_reqs, vocab_size, K, ptr(rates), int(bool(use_fp64)),
        workspace.data_ptr(), workspace.numel(), stream_of(device)),
        "mvsd_v2_rejection_sample")
    return sampled, num_sampled
