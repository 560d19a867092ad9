"""``get_num_sampled_and_rejected`` of the V2 input batch (minivllm/worker/gpu/
input_batch.py:507-553) on a HIP kernel (csrc/v2_verify.hip, C ABI
``mvsd_v2_num_sampled_and_rejected``).  The V2 runner's ``InputBatch`` itself belongs to the
runner; the verification path reads only the fields its callers pass."""

from __future__ import annotations

import torch

from ..._native import check, lib, require_device_tensor, stream_of


def get_num_sampled_and_rejected(
    num_sampled: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_num_logits: torch.Tensor,
    idx_mapping: torch.Tensor,
    prefill_len: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Zero both counts of a request still prefilling (seq_len < its state's prefill_len);
    else num_rejected = its logits rows - num_sampled.  ``num_sampled`` is updated in place
    and returned with the new ``num_rejected``."""
    device = num_sampled.device
    for name, t in (("num_sampled", num_sampled), ("seq_lens", seq_lens),
                    ("cu_num_logits", cu_num_logits), ("idx_mapping", idx_mapping),
                    ("prefill_len", prefill_len)):
        require_device_tensor(t, name)
    num_reqs = idx_mapping.shape[0]
    keep = []

    def i32(t):
        if t.dtype == torch.int32 and t.is_contiguous():
            return t
        out = t.to(torch.int32).contiguous()
        keep.append(out)
        return out

    ns = i32(num_sampled)
    num_rejected = torch.empty_like(num_sampled)
    nr = num_rejected if num_rejected.dtype == torch.int32 else torch.empty(
        num_rejected.shape, dtype=torch.int32, device=device)
    pl = i32(prefill_len)
    check(lib().mvsd_v2_num_sampled_and_rejected(
        ns.data_ptr(), nr.data_ptr(), i32(seq_lens).data_ptr(), i32(cu_num_logits).data_ptr(),
        i32(idx_mapping).data_ptr(), pl.data_ptr(), num_reqs, pl.numel(), stream_of(device)),
        "mvsd_v2_num_sampled_and_rejected")
    if ns is not num_sampled:
        num_sampled.copy_(ns)
    if nr is not num_rejected:
        num_rejected.copy_(nr)
    del keep
    return num_sampled, num_rejected
