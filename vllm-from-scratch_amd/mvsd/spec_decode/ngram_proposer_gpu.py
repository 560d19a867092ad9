"""Device-resident ngram proposer (drop-in for minivllm/spec_decode/ngram_proposer_gpu.py).

``NgramGPUKernel.forward`` and the match inside ``NgramProposerGPU.propose`` are one HIP
launch (``mvsd_ngram_propose``): one workgroup per request stages the history through LDS,
computes for every window end the common-suffix length with the history's tail, and keeps the
earliest end per n-gram length.  ``propose`` also folds the in-place scatter of this step's
sampled tokens into that launch.  Results are ``drafts [B, k]`` int32 (-1 padded) and
``num_valid [B]`` int32 (leading valid count).

Semantics follow the reference (:56-148, :204-245): largest n in [min_n, max_n] with a match,
earliest window among equals, at least one token after the window, no max_model_len cap.
"""

from __future__ import annotations

import torch

from .. import _native as nat
from ..outputs import DraftTokenIds
from .utils import TargetRows, update_scheduler_for_invalid_drafts  # noqa: F401


def ngram_propose_device(token_ids: torch.Tensor, num_tokens: torch.Tensor, *, min_n: int,
                         max_n: int, k: int, active: torch.Tensor | None = None,
                         new_tokens: torch.Tensor | None = None,
                         new_counts: torch.Tensor | None = None, gate_on_new_counts: bool = False,
                         cap_by_model_len: bool = False, max_model_len: int = 0,
                         ) -> tuple[torch.Tensor, torch.Tensor]:
    """Run ``mvsd_ngram_propose`` on device tensors; returns (drafts, num_valid)."""
    nat.require_device_tensor(token_ids, "token_ids")
    if token_ids.dtype != torch.int32:
        raise TypeError(f"token_ids must be int32, got {token_ids.dtype}")
    if token_ids.ndim != 2 or token_ids.stride(1) != 1:
        raise ValueError("token_ids must be a 2-D row-major tensor")
    device = token_ids.device
    num_reqs = token_ids.shape[0]
    assert num_tokens.shape[0] >= num_reqs
    # one allocation for both outputs: the drafts [num_reqs, k] and the counts after them
    # (as_strided views: cheaper on the host than slicing and reshaping)
    out = torch.empty(num_reqs * (k + 1), dtype=torch.int32, device=device)
    drafts = out.as_strided((num_reqs, k), (k, 1))
    num_valid = out.as_strided((num_reqs,), (1,), num_reqs * k)
    if num_reqs == 0:
        return drafts, num_valid
    lengths = num_tokens if num_tokens.shape[0] == num_reqs else num_tokens[:num_reqs]
    if lengths.dtype != torch.int32 or not lengths.is_contiguous():
        lengths = lengths.to(torch.int32).contiguous()
    act = None
    if active is not None:
        act = active[:num_reqs].to(torch.uint8).contiguous()
    new = counts = None
    new_stride = max_new = 0
    if new_tokens is not None:
        new = new_tokens[:num_reqs]
        if new.dtype != torch.int32 or new.stride(-1) != 1:
            new = new.to(torch.int32).contiguous()
        new_stride, max_new = new.stride(0), new.shape[1]
        counts = new_counts[:num_reqs].to(torch.int32).contiguous()
    status = nat.lib().mvsd_ngram_propose(
        drafts.data_ptr(), num_valid.data_ptr(), token_ids.data_ptr(), token_ids.stride(0),
        token_ids.shape[1], lengths.data_ptr(), None if new is None else new.data_ptr(),
        new_stride, max_new, None if counts is None else counts.data_ptr(),
        None if act is None else act.data_ptr(), int(gate_on_new_counts), num_reqs, min_n, max_n,
        k, int(cap_by_model_len), max_model_len, nat.stream_of(device))
    if status:
        nat.check(status, "mvsd_ngram_propose")
    return drafts, num_valid


class NgramGPUKernel(torch.nn.Module):
    """Match + extract for a batch (reference class of the same name, :32-152)."""

    def __init__(self, vllm_config, prefix: str = "", device: str = "cuda") -> None:
        super().__init__()
        spec_config = vllm_config.speculative_config
        assert spec_config is not None
        assert spec_config.prompt_lookup_min is not None
        assert spec_config.prompt_lookup_max is not None
        self.min_n = spec_config.prompt_lookup_min
        self.max_n = spec_config.prompt_lookup_max
        self.k = spec_config.num_speculative_tokens
        self.max_model_len = vllm_config.model_config.max_model_len
        self.max_num_seqs = vllm_config.scheduler_config.max_num_seqs
        self.device = device

    def forward(self, num_tokens_no_spec: torch.Tensor, token_ids_gpu: torch.Tensor,
                combined_mask: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``(draft_tokens [B, k], num_valid_draft_tokens [B])`` on the device (:130-148)."""
        return ngram_propose_device(token_ids_gpu, num_tokens_no_spec, min_n=self.min_n,
                                    max_n=self.max_n, k=self.k, active=combined_mask)

    def load_model(self, *args, **kwargs):
        pass


class NgramProposerGPU:
    """Reference constructor and methods (:155-340)."""

    def __init__(self, vllm_config, device: torch.device, runner=None) -> None:
        spec_config = vllm_config.speculative_config
        assert spec_config is not None
        assert spec_config.prompt_lookup_min is not None
        assert spec_config.prompt_lookup_max is not None
        self.vllm_config = vllm_config
        self.min_n = spec_config.prompt_lookup_min
        self.max_n = spec_config.prompt_lookup_max
        self.k = spec_config.num_speculative_tokens
        self.max_model_len = vllm_config.model_config.max_model_len
        self.max_num_seqs = vllm_config.scheduler_config.max_num_seqs
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.runner = runner
        self.kernel = NgramGPUKernel(vllm_config=vllm_config, prefix="ngram_gpu_kernel",
                                     device=device)

    def propose(self, num_speculative_tokens: int, num_tokens_no_spec: torch.Tensor,
                token_ids_gpu: torch.Tensor, valid_sampled_token_ids_gpu: torch.Tensor,
                valid_sampled_tokens_count: torch.Tensor,
                ) -> tuple[torch.Tensor, torch.Tensor]:
        """Append this step's tokens to the device history (in place; lengths stay read
        only) and propose from the extended history (:204-245)."""
        assert num_speculative_tokens == self.k
        assert token_ids_gpu.device == self.device
        assert num_tokens_no_spec.device == self.device
        return ngram_propose_device(
            token_ids_gpu, num_tokens_no_spec, min_n=self.min_n, max_n=self.max_n, k=self.k,
            new_tokens=valid_sampled_token_ids_gpu, new_counts=valid_sampled_tokens_count,
            gate_on_new_counts=True)

    def update_token_ids_ngram(self, sampled_token_ids, gpu_input_batch,
                               token_ids_gpu: torch.Tensor, num_tokens_no_spec: torch.Tensor,
                               discard_request_mask: torch.Tensor,
                               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Valid sampled tokens of this step (:247-290) in one ``mvsd_ngram_valid_sampled``
        launch: discarded rows become -1, ids >= vocab do not count, and a row without valid
        tokens takes the history's last token as its next token."""
        num_reqs = gpu_input_batch.num_reqs
        if isinstance(sampled_token_ids, list):
            width = max(max((len(s) for s in sampled_token_ids), default=0), 1)
            padded = [list(s) + [-1] * (width - len(s)) for s in sampled_token_ids]
            sampled_token_ids = torch.tensor(padded, dtype=torch.int32, device=self.device)
        sampled = sampled_token_ids[:num_reqs]
        if sampled.dtype != torch.int32 or sampled.stride(-1) != 1:
            sampled = sampled.to(torch.int32).contiguous()
        nat.require_device_tensor(sampled, "sampled_token_ids")
        tokens = token_ids_gpu if token_ids_gpu.stride(-1) == 1 else token_ids_gpu.contiguous()
        lens = num_tokens_no_spec.to(torch.int32).contiguous()
        discard = discard_request_mask[:num_reqs].to(torch.uint8).contiguous()
        width = sampled.shape[1]
        valid_ids = torch.empty((num_reqs, width), dtype=torch.int32, device=sampled.device)
        counts = torch.empty((num_reqs,), dtype=torch.int32, device=sampled.device)
        next_token_ids = torch.empty((num_reqs,), dtype=torch.int32, device=sampled.device)
        nat.check(nat.lib().mvsd_ngram_valid_sampled(
            next_token_ids.data_ptr(), counts.data_ptr(), valid_ids.data_ptr(),
            valid_ids.stride(0), sampled.data_ptr(), sampled.stride(0), width,
            discard.data_ptr(), tokens.data_ptr(), tokens.stride(0), lens.data_ptr(),
            int(gpu_input_batch.vocab_size), num_reqs, nat.stream_of(sampled.device)),
            "mvsd_ngram_valid_sampled")
        return next_token_ids, counts, valid_ids

    def load_model(self, *args, **kwargs):
        self.kernel.load_model(*args, **kwargs)

    def propose_drafts(self, rows: list[TargetRows], all_token_ids: dict[str, list[int]],
                       input_batch=None, reset_req_ids: set[str] | None = None,
                       sampled_by_row: dict[int, list[int]] | None = None,
                       sample_rows: list[int] | None = None,
                       token_ids_gpu: torch.Tensor | None = None,
                       num_tokens_no_spec_gpu: torch.Tensor | None = None,
                       ) -> DraftTokenIds:
        """Runner entry point (:297-337): one D2H of ``[B, k]`` drafts + ``[B]`` counts."""
        assert token_ids_gpu is not None and num_tokens_no_spec_gpu is not None, (
            "the device ngram proposer needs the runner's history buffers")
        num_reqs = len(rows)
        sampled_by_row = sampled_by_row or {}
        sample_rows = list(range(num_reqs)) if sample_rows is None else list(sample_rows)
        token_ids_gpu = token_ids_gpu[:num_reqs]
        num_tokens_no_spec_gpu = num_tokens_no_spec_gpu[:num_reqs]
        sampled = [list(sampled_by_row.get(row, [])) for row in range(num_reqs)]
        keep = set(sample_rows)
        discard = torch.tensor([row not in keep for row in range(num_reqs)], dtype=torch.bool,
                               device=self.device)
        _next, counts, valid_ids = self.update_token_ids_ngram(
            sampled, input_batch, token_ids_gpu, num_tokens_no_spec_gpu, discard)
        drafts, num_valid = self.propose(self.k, num_tokens_no_spec_gpu, token_ids_gpu,
                                         valid_ids, counts)
        # one device-to-host copy: the drafts with the valid count as an extra column
        host = torch.cat([drafts.to(torch.int64), num_valid.to(torch.int64)[:, None]], dim=1).cpu()
        return DraftTokenIds(req_ids=[t.req_id for t in rows],
                             draft_token_ids=host[:, :-1].tolist(),
                             num_valid_draft_tokens=host[:, -1].tolist())

    def remove_requests(self, req_ids) -> None:
        pass


def update_ngram_gpu_tensors_incremental(input_batch, token_ids_gpu_tensor,
                                         num_tokens_no_spec_gpu, new_req_ids: set[str],
                                         prev_req_id_to_index: dict[str, int] | None,
                                         device) -> None:
    """Keep the device history in step with the batch (:348-416): move reordered rows, copy
    new or resumed requests' histories once, then sync every active row's length."""
    current = input_batch.req_id_to_index
    if not current:
        return
    active = list(current.values())
    active_gpu = torch.tensor(active, dtype=torch.long, device=device)
    if prev_req_id_to_index is not None:
        src, dst = [], []
        for req_id, index in current.items():
            if req_id in new_req_ids:
                continue
            prev = prev_req_id_to_index.get(req_id)
            if prev is not None and prev != index:
                src.append(prev)
                dst.append(index)
        if src:
            s = torch.tensor(src, dtype=torch.long, device=device)
            d = torch.tensor(dst, dtype=torch.long, device=device)
            token_ids_gpu_tensor[d] = token_ids_gpu_tensor[s].clone()
            num_tokens_no_spec_gpu[d] = num_tokens_no_spec_gpu[s].clone()
        copy_ids = [r for r in new_req_ids if r in current]
    else:
        copy_ids = list(current)
    if copy_ids:
        # One host-to-device copy for all of them: the histories padded to the longest, with
        # each row's length as a last column; only the first n entries of a row are written.
        rows = torch.tensor([current[r] for r in copy_ids], dtype=torch.long)
        lens = input_batch.num_tokens_no_spec[rows].to(torch.int64)
        width = min(int(lens.max()), token_ids_gpu_tensor.shape[1])
        if width > 0:
            block = torch.cat([input_batch.token_ids_cpu[rows, :width].to(torch.int64),
                               lens[:, None]], dim=1).to(device)
            rows_gpu = rows.to(device)
            keep = (torch.arange(width, device=device)[None, :] < block[:, -1:])
            current_rows = token_ids_gpu_tensor[rows_gpu, :width]
            token_ids_gpu_tensor[rows_gpu, :width] = torch.where(
                keep, block[:, :width].to(token_ids_gpu_tensor.dtype), current_rows)
    values = input_batch.num_tokens_no_spec[torch.tensor(active, dtype=torch.long)]
    num_tokens_no_spec_gpu.index_copy_(0, active_gpu, values.to(device=device, dtype=torch.int32))
