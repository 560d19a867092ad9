"""The V2 model runner's verification sampler (minivllm/worker/gpu/spec_decode/
rejection_sampler.py:54-337) over the HIP kernels of csrc/v2_verify.hip.

Inputs are the V2 runner's flat layout: ``logits [num_logits, V]`` with each request's rows
contiguous (its K_i verify rows, then its bonus row; ``cu_num_logits`` with a leading 0),
per-state sampling parameters indexed through ``idx_mapping`` / ``expanded_idx_mapping``,
and ``draft_logits [max_num_reqs, K, V]`` indexed by state.  The sampler's
``apply_sampling_params`` (the V2 runner's penalties / temperature / min-p) runs first; the
verification, the logprobs, the flattening of the sampled tokens and the per-request counts
are HIP kernels, with no host synchronisation unless logprobs need the exact row boundaries
of a compacted batch.

The three verification methods are chosen once, at construction (:84-96): "standard"
(Leviathan et al. 2023), "block" (Sun et al. 2024) and "synthetic" (configured conditional
acceptance rates; it does not preserve the target distribution).

Large batches are verified in chunks of whole requests whose fp32 logits stay under 1 GiB
(:49-72, :208-294); a request is never split, and ``draft_logits`` stays global because it is
indexed by state.
"""

from __future__ import annotations

from collections.abc import Iterable, Iterator

import numpy as np
import torch

from ...._native import check, lib, require_device_tensor, stream_of
from ....outputs import LogprobsTensors
from ....spec_decode.utils import unconditional_to_conditional_rates
from ..input_batch import get_num_sampled_and_rejected
from ..sample.logprob import compute_topk_scores
from ..sample.output import SamplerOutput
from ..sample.states import NO_LOGPROBS
from .rejection_sampler_utils import rejection_sample

# Largest fp32 logits buffer one verification chunk may materialise (:45-46).
MAX_CHUNK_BYTES = 2**30
_FP32_BYTES = 4


def get_max_chunk_logits(vocab_size: int) -> int:
    """Logits rows one chunk may hold: as many fp32 rows of ``vocab_size`` as fit in
    MAX_CHUNK_BYTES, and at least one (:49-51)."""
    return max(1, MAX_CHUNK_BYTES // (vocab_size * _FP32_BYTES))


def _iter_request_chunks(cu_num_logits: np.ndarray,
                         max_chunk_logits: int) -> Iterator[tuple[int, int]]:
    """Request ranges [start, end) covering the batch in order, each the longest run from
    ``start`` whose rows fit in ``max_chunk_logits``; a request with more rows than that forms
    a chunk by itself (:54-66)."""
    assert max_chunk_logits > 0
    num_reqs = cu_num_logits.size - 1
    start = 0
    while start < num_reqs:
        limit = int(cu_num_logits[start]) + max_chunk_logits
        # the last request boundary at or below the limit
        end = int(np.searchsorted(cu_num_logits, limit, side="right")) - 1
        end = min(num_reqs, max(end, start + 1))
        yield start, end
        start = end


def flatten_sampled(sampled: torch.Tensor, num_sampled: torch.Tensor,
                    cu_num_logits: torch.Tensor, num_logits: int) -> torch.Tensor:
    """``sampled [num_reqs, K+1]`` laid out over the logits rows (:73-108): row
    ``cu_num_logits[r] + j`` holds ``sampled[r, j]`` for ``j < num_sampled[r]``, 0 elsewhere."""
    device = sampled.device
    for name, t in (("sampled", sampled), ("num_sampled", num_sampled),
                    ("cu_num_logits", cu_num_logits)):
        require_device_tensor(t, name)
    num_reqs = cu_num_logits.shape[0] - 1
    keep = []
    s = sampled if sampled.dtype == torch.int64 and sampled.stride(-1) == 1 else \
        sampled.to(torch.int64).contiguous()
    ns = num_sampled if num_sampled.dtype == torch.int32 else num_sampled.to(torch.int32)
    cu = cu_num_logits if cu_num_logits.dtype == torch.int32 and cu_num_logits.is_contiguous() \
        else cu_num_logits.to(torch.int32).contiguous()
    keep += [s, ns, cu]
    flat = torch.empty(num_logits, dtype=torch.int64, device=device)
    check(lib().mvsd_v2_flatten_sampled(flat.data_ptr(), s.data_ptr(), s.stride(0),
                                        ns.data_ptr(), cu.data_ptr(), num_reqs, num_logits,
                                        stream_of(device)), "mvsd_v2_flatten_sampled")
    del keep
    return flat if sampled.dtype == torch.int64 else flat.to(sampled.dtype)


class RejectionSampler:
    """V2 verification sampler.  ``sampler`` is the V2 runner's sampler: it provides
    ``apply_sampling_params``, ``sampling_states`` (``temperature.gpu``, ``seeds.gpu``,
    ``max_num_logprobs``), ``logprobs_mode``, ``use_fp64_gumbel`` and
    ``req_states.prefill_len.gpu``."""

    def __init__(self, sampler, spec_config, device: torch.device):
        self.sampler = sampler
        self.num_speculative_steps = spec_config.num_speculative_tokens
        method = getattr(spec_config, "rejection_sample_method", "standard")
        self.use_block_verification: bool = method == "block"
        self.synthetic_conditional_rates: torch.Tensor | None = None
        if method == "synthetic":
            rates = spec_config.synthetic_acceptance_rates
            assert rates is not None
            self.synthetic_conditional_rates = torch.tensor(
                unconditional_to_conditional_rates(rates), dtype=torch.float32, device=device)

    def _get_logprobs_tensors(self, sampled, num_sampled, logits, cu_num_logits,
                              cu_num_logits_np, max_num_logprobs) -> LogprobsTensors | None:
        """(:143-168) the top-k logprobs of every logits row, each row scored with the token
        sampled there (0 past a request's sampled tokens)."""
        if max_num_logprobs == NO_LOGPROBS:
            return None
        num_logits = logits.shape[0]
        flat = flatten_sampled(sampled, num_sampled, cu_num_logits, num_logits)
        expanded = num_logits != cu_num_logits.shape[0] - 1
        return compute_topk_scores(
            logits, max_num_logprobs, flat,
            cu_num_logits_np.tolist() if expanded else None,
            logits_mode=self.sampler.logprobs_mode in ("raw_logits", "processed_logits"))

    def _verify(self, logits, draft_logits, draft_sampled, pos, cu_num_logits, idx_mapping,
                idx_mapping_np, expanded_idx_mapping, expanded_local_pos):
        """(:170-206) the sampler's processing of the target logits, then the verification."""
        processed = self.sampler.apply_sampling_params(
            logits, expanded_idx_mapping, idx_mapping, idx_mapping_np, pos, draft_sampled,
            expanded_local_pos)
        states = self.sampler.sampling_states
        sampled, num_sampled = rejection_sample(
            processed, draft_logits, draft_sampled, cu_num_logits, pos, idx_mapping,
            expanded_idx_mapping, expanded_local_pos, states.temperature.gpu, states.seeds.gpu,
            self.num_speculative_steps, self.synthetic_conditional_rates,
            use_fp64=self.sampler.use_fp64_gumbel,
            use_block_verification=self.use_block_verification)
        return processed, sampled, num_sampled

    def _verify_in_chunks(self, logits, input_batch, draft_logits, draft_sampled, pos,
                          max_chunk_logits, max_num_logprobs):
        """(:208-294) verify the batch whole when its rows fit in one chunk, else chunk by
        chunk of whole requests; logprobs are scored per chunk and concatenated with the
        batch-wide row offsets."""
        processed_mode = self.sampler.logprobs_mode in ("processed_logprobs", "processed_logits")
        num_reqs = input_batch.num_reqs
        cu_np = input_batch.cu_num_logits_np
        if max_num_logprobs != NO_LOGPROBS and not getattr(
                input_batch, "cu_num_logits_np_exact", True):
            # The host prefix sums of a compacted batch are an upper bound only; the logprobs'
            # row offsets need the exact ones (one device-to-host copy, only then).
            cu_np = input_batch.cu_num_logits[:num_reqs + 1].to("cpu").numpy()
        if logits.shape[0] <= max_chunk_logits:
            # One chunk.  This also keeps stale host offsets of a compacted batch (always
            # within the limit) from choosing chunk boundaries.
            chunks: Iterable[tuple[int, int]] = ((0, num_reqs),)
        else:
            chunks = _iter_request_chunks(cu_np, max_chunk_logits)

        sampled_parts, count_parts, logprob_parts = [], [], []
        for start, end in chunks:
            lo, hi = int(cu_np[start]), int(cu_np[end])
            chunk_cu_np = cu_np[start:end + 1] - lo
            chunk_cu = input_batch.cu_num_logits[start:end + 1] - lo
            rows = slice(lo, hi)
            processed, sampled, num_sampled = self._verify(
                logits[rows], draft_logits, draft_sampled[rows], pos[rows], chunk_cu,
                input_batch.idx_mapping[start:end], input_batch.idx_mapping_np[start:end],
                input_batch.expanded_idx_mapping[rows], input_batch.expanded_local_pos[rows])
            lp = self._get_logprobs_tensors(
                sampled, num_sampled, processed if processed_mode else logits[rows], chunk_cu,
                chunk_cu_np, max_num_logprobs)
            if lp is not None:
                logprob_parts.append(lp)
            del processed
            sampled_parts.append(sampled)
            count_parts.append(num_sampled)

        if len(sampled_parts) == 1:
            return sampled_parts[0], count_parts[0], (logprob_parts[0] if logprob_parts else None)
        logprobs = None
        if logprob_parts:
            expanded = logits.shape[0] != num_reqs
            logprobs = LogprobsTensors.cat(
                logprob_parts, cu_num_generated_tokens=cu_np.tolist() if expanded else None)
        return torch.cat(sampled_parts), torch.cat(count_parts), logprobs

    def __call__(self, logits: torch.Tensor, input_batch,
                 draft_logits: torch.Tensor | None = None) -> SamplerOutput:
        """(:296-337) verify the batch, then zero the counts of requests still prefilling."""
        draft_sampled = input_batch.input_ids[input_batch.logits_indices]
        pos = input_batch.positions[input_batch.logits_indices]
        max_num_logprobs = self.sampler.sampling_states.max_num_logprobs(
            input_batch.idx_mapping_np)
        sampled, num_sampled, logprobs = self._verify_in_chunks(
            logits, input_batch, draft_logits, draft_sampled, pos,
            get_max_chunk_logits(logits.shape[1]), max_num_logprobs)
        num_sampled, num_rejected = get_num_sampled_and_rejected(
            num_sampled, input_batch.seq_lens, input_batch.cu_num_logits,
            input_batch.idx_mapping, self.sampler.req_states.prefill_len.gpu)
        # NaN counting (VLLM_COMPUTE_NANS_IN_LOGITS, off by default) is not on this path.
        return SamplerOutput(sampled_token_ids=sampled, logprobs_tensors=logprobs,
                             num_nans=None, num_sampled=num_sampled,
                             num_rejected=num_rejected)
