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
noise.  ``use_block_verification=True`` selects block verification (Sun et al. 2024,
arXiv:2403.10444; :318-493, :608-640, :800-866) for the random requests: the running joint
ratio, the look-ahead residual mass, the last passing position, and the residual
max(p_tau p - q, 0).  No host synchronisation; every launch is on the current stream of the
target's device.
"""

from __future__ import annotations

import torch

from ...._native import (F32, check, dtype_code, lib, ptr, require_device_tensor,
                         stream_of)

_FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _on_device(t: torch.Tensor, name: str, device: torch.device) -> None:
    """Refuse a tensor the kernels cannot address: host memory, or another device."""
    require_device_tensor(t, name)
    if t.device != device:
        raise ValueError(f"{name} is on {t.device} but target_logits is on {device}")


def _as(t: torch.Tensor, dtype: torch.dtype, keep: list) -> torch.Tensor:
    """``t`` as a contiguous ``dtype`` tensor; a converted copy is appended to ``keep`` so that
    it stays allocated until the launch has been enqueued (a temporary freed before the
    launch could hand its memory to the next conversion on the same stream)."""
    if t.dtype == dtype and t.is_contiguous():
        return t
    out = t.to(dtype).contiguous()
    keep.append(out)
    return out


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
    """V2 verification (rejection_sampler_utils.py:935-1201)."""
    assert target_logits.ndim == 2 and target_logits.stride(-1) == 1
    assert draft_logits is None or (draft_logits.ndim == 3 and draft_logits.stride(-1) == 1)
    if use_block_verification:
        assert synthetic_conditional_rates is None, (
            "Block verification is incompatible with synthetic acceptance rates.")
    require_device_tensor(target_logits, "target_logits")
    if target_logits.dtype not in _FLOAT_DTYPES:
        raise TypeError(f"target_logits dtype {target_logits.dtype} is not supported")
    device = target_logits.device
    # Every tensor the kernels read or write must live on the target's device: a host tensor
    # would hand the kernels a host address (the reference's Triton kernels refuse them too).
    named = [("draft_sampled", draft_sampled), ("cu_num_logits", cu_num_logits), ("pos", pos),
             ("idx_mapping", idx_mapping), ("expanded_idx_mapping", expanded_idx_mapping),
             ("expanded_local_pos", expanded_local_pos), ("temperature", temperature),
             ("seed", seed)]
    if draft_logits is not None:
        named.append(("draft_logits", draft_logits))
    if synthetic_conditional_rates is not None:
        named.append(("synthetic_conditional_rates", synthetic_conditional_rates))
    for name, t in named:
        _on_device(t, name, device)
    num_reqs = cu_num_logits.shape[0] - 1
    num_logits, vocab_size = target_logits.shape
    d_stride0 = d_stride1 = 0
    d_code = F32
    if draft_logits is not None:
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
    keep: list[torch.Tensor] = []
    rates = None
    if synthetic_conditional_rates is not None:
        rates = _as(synthetic_conditional_rates, torch.float32, keep)
        if rates.numel() < K:
            raise ValueError(f"synthetic_conditional_rates has {rates.numel()} entries but "
                             f"num_speculative_steps is {K}")
    temp = _as(temperature, torch.float32, keep)
    seeds = _as(seed, torch.int64, keep)
    num_states = min(temp.numel(), seeds.numel())
    if draft_logits is not None:
        num_states = min(num_states, draft_logits.shape[0])
    sampled_i32 = _as(draft_sampled, torch.int32, keep)
    cu = _as(cu_num_logits, torch.int32, keep)
    pos64 = _as(pos, torch.int64, keep)
    idx = _as(idx_mapping, torch.int32, keep)
    eidx = _as(expanded_idx_mapping, torch.int32, keep)
    elpos = _as(expanded_local_pos, torch.int32, keep)
    ws_bytes = lib().mvsd_v2_workspace_bytes(num_logits, num_reqs, vocab_size)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    check(lib().mvsd_v2_rejection_sample(
        sampled.data_ptr(), sampled.stride(0), num_sampled.data_ptr(),
        target_logits.data_ptr(), dtype_code(target_logits.dtype), target_logits.stride(0),
        num_logits, ptr(draft_logits), d_code, d_stride0, d_stride1, sampled_i32.data_ptr(),
        cu.data_ptr(), pos64.data_ptr(), idx.data_ptr(), eidx.data_ptr(), elpos.data_ptr(),
        temp.data_ptr(), seeds.data_ptr(), num_states, num_reqs, vocab_size, K, ptr(rates),
        int(bool(use_fp64)), int(bool(use_block_verification)), workspace.data_ptr(),
        workspace.numel(), stream_of(device)),
        "mvsd_v2_rejection_sample")
    del keep  # the launch is enqueued; stream-ordered frees are safe from here on
    return sampled, num_sampled
