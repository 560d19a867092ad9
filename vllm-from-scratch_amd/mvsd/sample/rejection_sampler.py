"""Speculative-decoding verification on MI355X (drop-in for minivllm/sample/rejection_sampler.py).

Same public names, signatures, dtypes and error behaviour as the reference module:

    RejectionSampler(sampler, spec_config=None, device=None)      (:86-406)
    rejection_sample(draft_token_ids, num_draft_tokens, max_spec_len, cu_num_draft_tokens,
                     draft_probs, target_logits, bonus_token_ids, sampling_metadata,
                     synthetic_mode=False, synthetic_conditional_rates=None)   (:414-534)
    apply_sampling_constraints / expand_batch_to_tokens / generate_uniform_probs /
    sample_recovered_tokens, PLACEHOLDER_TOKEN_ID, GREEDY_TEMPERATURE, MAX_SPEC_LEN

The arithmetic is one persistent HIP launch (``mvsd_rejection_sample`` in include/mvsd.h):
target softmax statistics or greedy argmax over every verify row, the acceptance chain of
each request, and the exponential-race recovered token of the one row each request actually
rejects (the reference scores every row and keeps that one), with bonus emission.  Each target
element is read once, plus the rejected rows' target, draft and noise elements once more.
``RejectionSampler.forward`` also folds the gather of verify rows, the temperature divide and
top-k / top-p into that launch when no logits processor needs the processed logits.

The kernel's cross-workgroup waits are bounded.  If one gives up, the affected requests'
output rows hold INT32_MIN in every entry and ``parse_output``, the path's
only device-to-host copy, raises ``RuntimeError``; the next call is unaffected.

Randomness is drawn by the same seams as the reference, and both stay monkeypatchable:
``generate_uniform_probs`` (fp64 [P]) and the exponential noise of
``sample_recovered_tokens`` (one Exp(1) row per request, drawn by
``generate_exponential_noise``).  Callers may also pass them explicitly
(``uniform_probs=``, ``exp_noise=``).  When a test replaces ``sample_recovered_tokens``
the verify kernel takes its result as the recovered ids, as the reference's random kernel
does.

Differences from the reference, all on inputs the reference does not define:
  * a draft id >= V is rejected (the reference reads out of bounds);
  * acceptance compares the fp32 ratio p/q with the fp64 uniform using IEEE fp32 division
    (the reference's Triton kernel uses its compiler's fp32 divide).
"""

from __future__ import annotations

import functools
from dataclasses import replace
from typing import TYPE_CHECKING

import numpy as np
import torch

from .. import _native as nat
from .metadata import SamplingMetadata
from .ops.topk_topp_sampler import apply_top_k_top_p

if TYPE_CHECKING:
    from ..spec_decode.metadata import SpecDecodeMetadata

PLACEHOLDER_TOKEN_ID = -1
GREEDY_TEMPERATURE = 0
MAX_SPEC_LEN = 128

PROCESSED_LOGPROBS_MODES = ("processed_logits", "processed_logprobs")


class RejectionSampler:
    """Batch verifier with the reference's constructor and call protocol (:86-225).

    ``sampler`` samples the bonus token from each request's bonus row exactly as in the
    reference (:169-181); it is the caller's sampler object.
    """

    def __init__(self, sampler, spec_config=None, device: torch.device | None = None) -> None:
        self.sampler = sampler
        self.logprobs_mode = getattr(sampler, "logprobs_mode", "raw_logprobs")
        self.is_processed_logprobs_mode = self.logprobs_mode in PROCESSED_LOGPROBS_MODES
        self.is_logits_logprobs_mode = self.logprobs_mode in ("raw_logits", "processed_logits")
        method = getattr(spec_config, "rejection_sample_method", "standard")
        self.synthetic_conditional_rates: torch.Tensor | None = None
        if spec_config is not None and method == "synthetic":
            from ..spec_decode.utils import unconditional_to_conditional_rates

            assert spec_config.synthetic_acceptance_rates is not None
            self.synthetic_conditional_rates = torch.tensor(
                unconditional_to_conditional_rates(spec_config.synthetic_acceptance_rates),
                dtype=torch.float32, device=device)
        self.synthetic_mode = self.synthetic_conditional_rates is not None
        if method == "block":
            raise NotImplementedError(
                "rejection_sample_method='block' (block verification) exists only for the V2 "
                "model runner; the V1 rejection sampler implements 'standard' and 'synthetic'")

    def __call__(self, metadata: "SpecDecodeMetadata", draft_probs: torch.Tensor | None,
                 logits: torch.Tensor, sampling_metadata: SamplingMetadata):
        return self.forward(metadata, draft_probs, logits, sampling_metadata)

    def forward(self, metadata: "SpecDecodeMetadata", draft_probs: torch.Tensor | None,
                logits: torch.Tensor, sampling_metadata: SamplingMetadata):
        """``logits`` is the compact ``[P + B, V]`` tensor in metadata row order (:153-225)."""
        from ..outputs import SamplerOutput

        assert metadata.max_spec_len <= MAX_SPEC_LEN
        if len(sampling_metadata.prompt_token_ids) != len(metadata.num_draft_tokens):
            raise ValueError(
                f"sampling metadata has {len(sampling_metadata.prompt_token_ids)} rows but the "
                f"spec metadata has {len(metadata.num_draft_tokens)} requests: they must match "
                "request for request, in the same order")
        max_num_logprobs = sampling_metadata.max_num_logprobs
        if max_num_logprobs == -1:
            # the reference refuses full-vocabulary logprobs on the speculative path too
            # (:257-267): its top-k cannot take -1
            raise NotImplementedError(
                "speculative decoding with logprobs=-1 (the whole vocabulary) is not supported; "
                "request logprobs=k with k >= 1")

        if self._bonus_rows_race_only(sampling_metadata, logits):
            return self._forward_race_only(metadata, draft_probs, logits, sampling_metadata)

        # 1) bonus tokens from the bonus rows with the regular sampler (:169-181); their
        # full-row logits are asked for only when logprobs are (the sampled tokens do not
        # depend on it, and the copy is a [B, V] write)
        bonus_logits = logits[metadata.bonus_logits_indices]
        bonus_out = self.sampler.forward(
            bonus_logits, replace(sampling_metadata, max_num_logprobs=(
                -1 if max_num_logprobs is not None else None)),
            predict_bonus_token=True,
            logprobs_mode_override=("processed_logits" if self.is_processed_logprobs_mode
                                    else "raw_logits"))
        bonus_token_ids = bonus_out.sampled_token_ids

        constrained = (sampling_metadata.top_k is not None
                       or sampling_metadata.top_p is not None)
        needs_processing = (not sampling_metadata.no_penalties
                            or _has_active_min_tokens(sampling_metadata)
                            # a replaced recovered-token seam receives materialised
                            # probabilities, which must carry the constraints
                            or (constrained
                                and sample_recovered_tokens is not _SAMPLE_RECOVERED_TOKENS)
                            # processed logprobs report the processed rows
                            or (max_num_logprobs is not None
                                and self.is_processed_logprobs_mode))
        if not needs_processing:
            # 2+3 fused: gather, fp32 upcast, temperature divide and top-k / top-p happen in
            # the kernels (the constraints become per-row thresholds on the raw rows)
            output_token_ids = rejection_sample(
                metadata.draft_token_ids, metadata.num_draft_tokens, metadata.max_spec_len,
                metadata.cu_num_draft_tokens, draft_probs, logits, bonus_token_ids,
                sampling_metadata, synthetic_mode=self.synthetic_mode,
                synthetic_conditional_rates=self.synthetic_conditional_rates,
                target_rows=metadata.target_logits_indices, apply_temperature=True,
                apply_top_k_top_p=constrained)
            target_logits = None
        else:
            target_logits = logits[metadata.target_logits_indices].to(torch.float32)
            target_logits = self.apply_logits_processors(target_logits, sampling_metadata,
                                                         metadata)
            target_logits = apply_sampling_constraints(
                target_logits, metadata.cu_num_draft_tokens, sampling_metadata)
            output_token_ids = rejection_sample(
                metadata.draft_token_ids, metadata.num_draft_tokens, metadata.max_spec_len,
                metadata.cu_num_draft_tokens, draft_probs, target_logits, bonus_token_ids,
                sampling_metadata, synthetic_mode=self.synthetic_mode,
                synthetic_conditional_rates=self.synthetic_conditional_rates)

        # 4) logprobs of every output position (:212-223); raw modes read the raw verify rows
        logprobs_tensors = None
        if max_num_logprobs is not None:
            bonus_rows = bonus_out.logprobs_tensors.logprobs
            if self.is_processed_logprobs_mode:
                logprobs_tensors = self._get_logprobs_tensors(
                    max_num_logprobs, metadata, logits, target_logits, bonus_rows,
                    output_token_ids)
            else:
                logprobs_tensors = self._get_logprobs_tensors(
                    max_num_logprobs, metadata, logits, None, bonus_rows, output_token_ids)
        return SamplerOutput(sampled_token_ids=output_token_ids,
                             logprobs_tensors=logprobs_tensors)

    def _bonus_rows_race_only(self, sm: SamplingMetadata, logits: torch.Tensor) -> bool:
        """True when the caller's sampler is mvsd.sample.Sampler itself and, for this batch,
        it would only take each bonus row's argmax or exponential race: no logprobs, no
        penalty or active min_tokens, no min_p, top-k or top-p; and the recovered-token seam
        is the module's own."""
        from .sampler import Sampler as DeviceSampler

        return (type(self.sampler) is DeviceSampler and sm.max_num_logprobs is None
                and sm.no_penalties and not _has_active_min_tokens(sm)
                and sm.min_p is None and sm.top_k is None and sm.top_p is None
                and sample_recovered_tokens is _SAMPLE_RECOVERED_TOKENS
                and logits.dtype in (torch.float32, torch.bfloat16, torch.float16)
                and logits.stride(1) == 1)

    def _forward_race_only(self, metadata: "SpecDecodeMetadata",
                           draft_probs: torch.Tensor | None, logits: torch.Tensor,
                           sm: SamplingMetadata):
        """forward when the bonus rows only need the race (``_bonus_rows_race_only``).

        The randomness is drawn exactly as the reference draws it, in its order: the bonus
        rows' Exp(1) noise (Sampler.sample's random_sample, for every row unless the batch is
        all greedy), the uniforms (generate_uniform_probs), the recovered tokens' noise
        (generate_exponential_noise).  Then one race launch reads the bonus rows in place
        (greedy rows: their argmax) and the verify kernel reads the verify rows in place, so
        neither the [B, V] gather of the bonus rows nor its fp32 upcast is written, and the
        race runs between the noise writes and the verification."""
        from ..outputs import SamplerOutput
        from . import sampler as smp

        device = logits.device
        B = len(metadata.num_draft_tokens)
        V = logits.shape[-1]
        num_tokens = int(metadata.draft_token_ids.shape[0])
        all_greedy = bool(sm.all_greedy)
        bonus_noise = uniforms = exp_noise = None
        if not all_greedy:
            bonus_noise = smp.generate_sampler_noise((B, V), sm.generators, device)
        if self.synthetic_mode or not all_greedy:
            uniforms = generate_uniform_probs(num_tokens, metadata.num_draft_tokens,
                                              sm.generators, device)
        if not all_greedy and num_tokens > 0:
            exp_noise = generate_exponential_noise(B, V, metadata.num_draft_tokens,
                                                   sm.generators, device)
        bonus = smp.race_rows(logits, metadata.bonus_logits_indices, bonus_noise,
                              None if all_greedy else sm.temperature)
        output_token_ids = rejection_sample(
            metadata.draft_token_ids, metadata.num_draft_tokens, metadata.max_spec_len,
            metadata.cu_num_draft_tokens, draft_probs, logits, bonus.view(B, 1), sm,
            synthetic_mode=self.synthetic_mode,
            synthetic_conditional_rates=self.synthetic_conditional_rates,
            uniform_probs=uniforms, exp_noise=exp_noise,
            target_rows=metadata.target_logits_indices, apply_temperature=True)
        return SamplerOutput(sampled_token_ids=output_token_ids, logprobs_tensors=None)

    def _get_logprobs_tensors(self, max_num_logprobs: int, metadata: "SpecDecodeMetadata",
                              logits: torch.Tensor, target_logits: torch.Tensor | None,
                              bonus_logits: torch.Tensor,
                              sampled_token_ids: torch.Tensor):
        """Logprobs of every output position ``[B * (max_spec_len + 1)]`` (:229-300).

        Position j of request i reads compact row ``start_i + j`` (clamped): verify row j
        while j < K_i, the bonus row at j = K_i, so accepted, recovered and bonus tokens each
        read their own row and padding positions read rows that parse_output drops with the
        same valid mask.  Verify rows come from ``target_logits`` ([P, V], the processed rows
        in the processed modes) or, when it is None, from ``logits`` at
        ``metadata.target_logits_indices``; the bonus rows from ``bonus_logits`` [B, V].  The
        values are the log-softmax of each row, or the rows themselves in the ``*_logits``
        modes.  One ``mvsd_spec_logprobs`` launch.
        """
        from ..outputs import LogprobsTensors

        if max_num_logprobs == -1:
            raise NotImplementedError(
                "speculative decoding with logprobs=-1 (the whole vocabulary) is not supported")
        device = sampled_token_ids.device
        nat.require_device_tensor(sampled_token_ids, "sampled_token_ids")
        B, W = sampled_token_ids.shape
        V = int(bonus_logits.shape[-1])
        num_tokens = int(metadata.draft_token_ids.shape[0])
        if not 0 <= max_num_logprobs <= V:
            raise ValueError(f"logprobs={max_num_logprobs} outside [0, {V}]")
        keep = []
        rows = None
        if target_logits is None:
            target_logits, rows = logits, _as(metadata.target_logits_indices, torch.int32, device)
        if target_logits.dtype != torch.float32 or target_logits.stride(-1) != 1:
            target_logits = (target_logits if rows is None else target_logits[rows.long()]).float()
            target_logits = target_logits.contiguous()
            rows = None
        bonus = bonus_logits.to(torch.float32)
        if bonus.stride(-1) != 1:
            bonus = bonus.contiguous()
        tokens = _as(sampled_token_ids, torch.int32, device)
        cu = _as(metadata.cu_num_sampled_tokens, torch.int32, device)
        keep += [target_logits, bonus, tokens, cu]
        n_out = max_num_logprobs + 1
        ids = torch.empty((B * W, n_out), dtype=torch.int32, device=device)
        lps = torch.empty((B * W, n_out), dtype=torch.float32, device=device)
        ranks = torch.empty((B * W,), dtype=torch.int32, device=device)
        nat.check(nat.lib().mvsd_spec_logprobs(
            ids.data_ptr(), lps.data_ptr(), ranks.data_ptr(),
            target_logits.data_ptr() if num_tokens else None, target_logits.stride(0),
            None if rows is None else rows.data_ptr(), bonus.data_ptr(), bonus.stride(0),
            cu.data_ptr(), tokens.data_ptr(), tokens.stride(0), B, num_tokens, V, W,
            max_num_logprobs, 1 if self.is_logits_logprobs_mode else 0, nat.stream_of(device)),
            "mvsd_spec_logprobs")
        return LogprobsTensors(ids, lps, ranks)

    def apply_logits_processors(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata,
                                metadata: "SpecDecodeMetadata") -> torch.Tensor:
        """Penalties, then min_tokens, on the fp32 verify rows in place (:338-356).

        Verify row j of request i sees the hypothetical history "committed output + drafts
        [:j]" (:387-406); rows whose history is still shorter than min_tokens get their stop
        tokens masked (the caller's ``Sampler.apply_min_tokens_for_spec_decode``,
        sampler.py:192-228, done here in the same launch).  One ``mvsd_apply_logits_processors``
        launch; the histories are summarised on the host per request (distinct tokens,
        committed counts, prompt flags) and the kernel adds the draft-prefix counts per row.
        """
        num_draft = [int(k) for k in metadata.num_draft_tokens]
        has_penalties = not sampling_metadata.no_penalties
        masks = _min_tokens_rows(sampling_metadata, num_draft)
        if not has_penalties and masks is None:
            return logits
        specs = sampling_metadata.spec_token_ids
        if not specs:
            specs = [[] for _ in num_draft]
        entries = None
        if has_penalties:
            entries = _penalty_entries(sampling_metadata.prompt_token_ids,
                                       sampling_metadata.output_token_ids, specs)
        _launch_logits_processors(
            logits, metadata.cu_num_draft_tokens, num_draft,
            [list(spec)[:k] + [-1] * (k - len(spec)) for spec, k in zip(specs, num_draft)],
            entries, sampling_metadata if has_penalties else None, masks)
        return logits

    @staticmethod
    def apply_penalties(logits: torch.Tensor, sampling_metadata: SamplingMetadata,
                        metadata: "SpecDecodeMetadata",
                        output_token_ids: list[list[int]]) -> torch.Tensor:
        """Penalties of the verify rows with explicit per-row histories (:358-385):
        ``output_token_ids[j]`` is row j's output history, and the prompt is that of row j's
        request.  In place; returns ``logits``."""
        if sampling_metadata.no_penalties:
            return logits
        num_rows = logits.shape[0]
        num_draft = [int(k) for k in metadata.num_draft_tokens]
        prompts = [prompt for prompt, count in zip(sampling_metadata.prompt_token_ids, num_draft)
                   for _ in range(count)]
        cu = metadata.cu_num_draft_tokens
        per_row = replace(
            sampling_metadata,
            presence_penalties=_expand_opt(sampling_metadata.presence_penalties, cu, num_rows),
            frequency_penalties=_expand_opt(sampling_metadata.frequency_penalties, cu, num_rows),
            repetition_penalties=_expand_opt(sampling_metadata.repetition_penalties, cu,
                                             num_rows))
        # every row is a request of its own: one row, no drafts
        rows_cu = torch.arange(1, num_rows + 1, dtype=torch.int32, device=logits.device)
        entries = _penalty_entries(prompts, output_token_ids, [[] for _ in range(num_rows)])
        _launch_logits_processors(logits, rows_cu, [1] * num_rows, [[-1]] * num_rows, entries,
                                  per_row, None)
        return logits

    @staticmethod
    def _combine_outputs_with_spec_tokens(
            output_token_ids: list[list[int]],
            spec_token_ids: list[list[int]] | None = None) -> list[list[int]]:
        """Per-row histories "committed + drafts[:j]", one per draft position; requests
        without drafts give no rows (:387-406)."""
        if spec_token_ids is None:
            return output_token_ids
        result = []
        for out, spec in zip(output_token_ids, spec_token_ids):
            for j in range(len(spec)):
                result.append([*out, *spec[:j]])
        return result

    @staticmethod
    def parse_output(output_token_ids: torch.Tensor, vocab_size: int, discard_req_indices=(),
                     logprobs_tensors=None):
        """``[B, max_spec_len + 1]`` -> ``list[list[int]]``; the path's only D2H (:304-334).

        Logprobs are filtered with the same valid mask, so rejected positions disappear from
        tokens and logprobs together; ``cu_num_generated_tokens`` gives each request's first
        row (before ``discard_req_indices`` is applied, as in the reference)."""
        out = output_token_ids.cpu().numpy()
        if (out == nat.POISON).any():
            bad = np.flatnonzero((out == nat.POISON).any(axis=1)).tolist()
            raise RuntimeError(
                f"verification of requests {bad} gave up waiting for partial results inside the "
                "kernel (output rows poisoned); the call's tokens are unusable, later calls are "
                "not affected")
        valid = (out != PLACEHOLDER_TOKEN_ID) & (out < vocab_size)
        output_logprobs = None
        if logprobs_tensors is not None:
            cu_num_tokens = [0] + valid.sum(axis=1).cumsum().tolist()
            output_logprobs = logprobs_tensors.filter(valid.flatten()).tolists(cu_num_tokens)
        if len(discard_req_indices) > 0:
            valid[list(discard_req_indices)] = False
        return [row[valid[i]].tolist() for i, row in enumerate(out)], output_logprobs


def _penalty_entries(prompts, outputs, specs):
    """Per request: the distinct tokens of prompt, committed output and drafts, each with
    its committed output count and prompt flag, as (ent_off [B+1], ent_tok, ent_info) int32
    arrays with ent_info = count | in_prompt << 31."""
    offs = [0]
    toks: list[np.ndarray] = []
    infos: list[np.ndarray] = []
    for i, spec in enumerate(specs):
        prompt = np.asarray(prompts[i] if i < len(prompts) else [], dtype=np.int64)
        out = np.asarray(outputs[i] if i < len(outputs) else [], dtype=np.int64)
        union = np.unique(np.concatenate([prompt, out, np.asarray(spec, dtype=np.int64)]))
        out_vals, out_counts = np.unique(out, return_counts=True)
        counts = np.zeros(union.shape[0], dtype=np.int64)
        counts[np.searchsorted(union, out_vals)] = out_counts
        in_prompt = np.isin(union, prompt)
        toks.append(union)
        infos.append(counts | (in_prompt.astype(np.int64) << 31))
        offs.append(offs[-1] + union.shape[0])
    tok = np.concatenate(toks) if toks else np.zeros(0, np.int64)
    info = np.concatenate(infos) if infos else np.zeros(0, np.int64)
    return (np.asarray(offs, dtype=np.int32), tok.astype(np.int32),
            info.astype(np.uint32).view(np.int32))


def _min_tokens_rows(sm: SamplingMetadata, num_draft: list[int]):
    """(n_mask [B], stop_off [B+1], stop_tok) for min_tokens (sampler.py:204-228), or None
    when no row is masked: the first clamp(min_tokens - len(output), 0, K_i) rows of request i
    mask its stop tokens."""
    if not sm.min_tokens:
        return None
    n_mask = np.zeros(len(num_draft), dtype=np.int32)
    stop_off = [0]
    stop_tok: list[int] = []
    for i, k in enumerate(num_draft):
        stop_ids = list(sm.stop_token_ids[i]) if i < len(sm.stop_token_ids) else []
        min_tokens = sm.min_tokens[i] if i < len(sm.min_tokens) else 0
        if stop_ids:
            produced = len(sm.output_token_ids[i]) if i < len(sm.output_token_ids) else 0
            n_mask[i] = min(max(min_tokens - produced, 0), k)
            stop_tok.extend(stop_ids)
        stop_off.append(len(stop_tok))
    if not n_mask.any():
        return None
    return n_mask, np.asarray(stop_off, dtype=np.int32), np.asarray(stop_tok, dtype=np.int32)


def _expand_opt(values: torch.Tensor | None, cu: torch.Tensor, num_rows: int):
    return None if values is None else expand_batch_to_tokens(values, cu, num_rows)


def _launch_logits_processors(logits, cu, num_draft, specs, entries, penalties, masks):
    """One mvsd_apply_logits_processors launch on fp32 rows ``logits`` (request-major)."""
    assert logits.ndim == 2 and logits.dtype == torch.float32, "fp32 [P, V] logits expected"
    nat.require_device_tensor(logits, "logits")
    if logits.stride(1) != 1:
        raise ValueError("logits processors need rows with unit stride")
    num_rows, V = logits.shape
    if sum(num_draft) != num_rows:
        raise ValueError(f"{num_rows} verify rows but {sum(num_draft)} draft tokens")
    device = logits.device
    keep = []

    def dev(array, dtype=torch.int32):
        t = torch.as_tensor(np.ascontiguousarray(array)).to(device=device, dtype=dtype)
        keep.append(t)
        return t.data_ptr()

    def dev_opt(values):
        if values is None:
            return None
        t = values.to(device=device, dtype=torch.float32).contiguous()
        keep.append(t)
        return t.data_ptr()

    if entries is not None and entries[1].size == 0:
        entries = None  # no history token anywhere: the penalties are no-ops
    if entries is None and masks is None:
        return
    cu_t = _as(cu, torch.int32, device)
    spec = np.asarray([t for row in specs for t in row], dtype=np.int32)
    ent_off = ent_tok = ent_info = None
    presence = frequency = repetition = None
    if entries is not None:
        ent_off, ent_tok, ent_info = (dev(a) for a in entries)
        presence = dev_opt(penalties.presence_penalties)
        frequency = dev_opt(penalties.frequency_penalties)
        repetition = dev_opt(penalties.repetition_penalties)
    n_mask = stop_off = stop_tok = None
    if masks is not None:
        n_mask, stop_off, stop_tok = (dev(a) for a in masks)
    nat.check(nat.lib().mvsd_apply_logits_processors(
        logits.data_ptr(), logits.stride(0), num_rows, V, len(num_draft), cu_t.data_ptr(),
        dev(spec) if spec.size else None, ent_off, ent_tok, ent_info, presence, frequency,
        repetition, n_mask, stop_off, stop_tok, nat.stream_of(device)),
        "mvsd_apply_logits_processors")


def _has_active_min_tokens(sm: SamplingMetadata) -> bool:
    """True when some row still has to mask stop tokens (min_tokens not yet reached)."""
    for index, min_tokens in enumerate(sm.min_tokens):
        if min_tokens and index < len(sm.stop_token_ids) and sm.stop_token_ids[index]:
            produced = len(sm.output_token_ids[index]) if index < len(sm.output_token_ids) else 0
            if produced < min_tokens:
                return True
    return False


# --------------------------------------------------------------------------- batch entry


def rejection_sample(
    draft_token_ids: torch.Tensor,
    num_draft_tokens: list[int],
    max_spec_len: int,
    cu_num_draft_tokens: torch.Tensor,
    draft_probs: torch.Tensor | None,
    target_logits: torch.Tensor,
    bonus_token_ids: torch.Tensor,
    sampling_metadata: SamplingMetadata,
    synthetic_mode: bool = False,
    synthetic_conditional_rates: torch.Tensor | None = None,
    *,
    uniform_probs: torch.Tensor | None = None,
    exp_noise: torch.Tensor | None = None,
    target_rows: torch.Tensor | None = None,
    apply_temperature: bool = False,
    apply_top_k_top_p: bool = False,
    debug_row_stats: torch.Tensor | None = None,
) -> torch.Tensor:
    """Verify a batch of drafts; returns ``[B, max_spec_len + 1]`` int32, -1 padded.

    Reference signature and semantics (:414-534).  ``target_logits`` is ``[P, V]`` with the
    temperature / top-k / top-p already applied, as in the reference.  Extensions:
      * ``uniform_probs`` [P] fp64 and ``exp_noise`` [B, V] fp32 supply the randomness;
      * ``target_rows`` [P] int32 selects verify row j as ``target_logits[target_rows[j]]``
        (no gather copy), and ``apply_temperature`` divides by the request temperature in the
        kernel (greedy T = 0 -> 1), which together replace the gather + ``div_`` that
        RejectionSampler.forward runs before this function;
      * ``apply_top_k_top_p`` applies ``sampling_metadata.top_k`` / ``top_p`` to the (divided)
        verify rows in the kernels, as ``apply_sampling_constraints`` (:563-571) would;
      * ``debug_row_stats`` (a [P, 3] fp32 device tensor, diagnostics) receives, for each verify
        row of a random request, the kernel's row maximum M, sum S of exp((x - M) / T) and the
        fp32 p[d] its acceptance test compared.
    """
    assert draft_token_ids.ndim == 1
    assert draft_probs is None or draft_probs.ndim == 2
    assert cu_num_draft_tokens.ndim == 1
    assert target_logits.ndim == 2
    nat.require_device_tensor(target_logits, "target_logits")

    batch_size = len(num_draft_tokens)
    num_tokens = draft_token_ids.shape[0]
    vocab_size = target_logits.shape[-1]
    device = target_logits.device
    assert draft_token_ids.is_contiguous()
    assert draft_probs is None or draft_probs.is_contiguous()
    assert bonus_token_ids.is_contiguous()
    if target_rows is None:
        assert target_logits.shape == (num_tokens, vocab_size)
    else:
        assert target_rows.shape == (num_tokens,)
    assert max_spec_len <= MAX_SPEC_LEN
    assert cu_num_draft_tokens.shape[0] == batch_size

    output_token_ids = torch.empty((batch_size, max_spec_len + 1), dtype=torch.int32,
                                   device=device)
    if batch_size == 0:
        return output_token_ids

    all_greedy = bool(sampling_metadata.all_greedy)
    temperature = None
    if not all_greedy:
        temperature = _as(sampling_metadata.temperature, torch.float32, device)

    if uniform_probs is None and (synthetic_mode or not all_greedy):
        uniform_probs = generate_uniform_probs(num_tokens, num_draft_tokens,
                                               sampling_metadata.generators, device)
    top_k = top_p = None
    if apply_top_k_top_p and not all_greedy:
        if sampling_metadata.top_k is not None:
            top_k = _as(sampling_metadata.top_k, torch.int64, device)
            assert top_k.shape == (batch_size,)
        if sampling_metadata.top_p is not None:
            top_p = _as(sampling_metadata.top_p, torch.float32, device)
            assert top_p.shape == (batch_size,)
    recovered_token_ids = None
    if not all_greedy and num_tokens > 0:
        if sample_recovered_tokens is not _SAMPLE_RECOVERED_TOKENS:
            if top_k is not None or top_p is not None:
                raise NotImplementedError(
                    "a replaced sample_recovered_tokens needs processed logits: apply "
                    "apply_sampling_constraints first instead of apply_top_k_top_p=True")
            # a caller replaced the seam: give it materialised probabilities, as the
            # reference does, and use the ids it returns
            target_probs = _softmax_rows(target_logits, target_rows,
                                         _expand_temperature(temperature, cu_num_draft_tokens,
                                                             num_tokens)
                                         if apply_temperature else None)
            recovered_token_ids = sample_recovered_tokens(
                max_spec_len, num_draft_tokens, cu_num_draft_tokens, draft_token_ids,
                draft_probs, target_probs, sampling_metadata, device)
        elif exp_noise is None:
            exp_noise = generate_exponential_noise(batch_size, vocab_size, num_draft_tokens,
                                                   sampling_metadata.generators, device)

    rates = None
    if synthetic_mode:
        assert synthetic_conditional_rates is not None
        rates = _as(synthetic_conditional_rates, torch.float32, device)
        if rates.shape[0] < max_spec_len:
            raise ValueError(f"synthetic_conditional_rates has {rates.shape[0]} entries but "
                             f"max_spec_len is {max_spec_len}")

    draft_ids = _as(draft_token_ids, torch.int32, device)
    cu = _as(cu_num_draft_tokens, torch.int32, device)
    bonus = _as(bonus_token_ids.reshape(-1), torch.int32, device)
    rows = None if target_rows is None else _as(target_rows, torch.int32, device)
    if uniform_probs is not None:
        uniform_probs = _as(uniform_probs, torch.float64, device)
    if recovered_token_ids is not None:
        recovered_token_ids = _as(recovered_token_ids, torch.int32, device)
    if draft_probs is not None:
        nat.require_device_tensor(draft_probs, "draft_probs")
        # the reference's kernels load draft_probs in its own dtype and compute in fp32
        # (:797-806, :882-890); 16-bit probabilities are upcast exactly in the kernel
        if draft_probs.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError(f"draft_probs dtype {draft_probs.dtype} is not supported")
        assert draft_probs.shape == (num_tokens, vocab_size)
    if exp_noise is not None:
        exp_noise = _as(exp_noise, torch.float32, device)
        assert exp_noise.shape == (batch_size, vocab_size) and exp_noise.stride(1) == 1
    if target_logits.stride(1) != 1:
        target_logits = target_logits.contiguous()
    if debug_row_stats is not None:
        nat.require_device_tensor(debug_row_stats, "debug_row_stats")
        if (debug_row_stats.dtype != torch.float32 or tuple(debug_row_stats.shape) != (num_tokens, 3)
                or not debug_row_stats.is_contiguous()):
            raise ValueError("debug_row_stats must be a contiguous [P, 3] float32 tensor")

    dtype = nat.dtype_code(target_logits.dtype)
    handle = nat.lib()
    stream = nat.stream_of(device)
    workspace = _workspace(device, _workspace_bytes(batch_size, num_tokens, vocab_size, dtype,
                                                    max_spec_len), stream)
    args = nat.RejectionArgs(
        output_token_ids=output_token_ids.data_ptr(),
        out_stride=output_token_ids.stride(0),
        target_logits=target_logits.data_ptr(),
        target_dtype=dtype,
        target_stride=target_logits.stride(0),
        target_rows=nat.ptr(rows),
        target_num_rows=target_logits.shape[0],
        draft_probs=nat.ptr(draft_probs),
        draft_dtype=nat.dtype_code(draft_probs.dtype) if draft_probs is not None else nat.F32,
        draft_stride=draft_probs.stride(0) if draft_probs is not None else 0,
        exp_noise=nat.ptr(exp_noise),
        noise_stride=exp_noise.stride(0) if exp_noise is not None else 0,
        uniform_probs=nat.ptr(uniform_probs),
        draft_token_ids=draft_ids.data_ptr(),
        cu_num_draft_tokens=cu.data_ptr(),
        bonus_token_ids=bonus.data_ptr(),
        temperature=nat.ptr(temperature),
        all_greedy=int(all_greedy),
        apply_temperature=int(bool(apply_temperature)),
        recovered_token_ids=nat.ptr(recovered_token_ids),
        synthetic_conditional_rates=nat.ptr(rates),
        batch_size=batch_size,
        num_tokens=num_tokens,
        vocab_size=vocab_size,
        max_spec_len=max_spec_len,
        workspace=workspace.data_ptr(),
        workspace_bytes=workspace.numel(),
        top_k=nat.ptr(top_k),
        top_p=nat.ptr(top_p),
        debug_row_stats=nat.ptr(debug_row_stats),
    )
    nat.check(handle.mvsd_rejection_sample(args, stream), "mvsd_rejection_sample")
    return output_token_ids


def sampling_masks(target_logits: torch.Tensor, cu_num_draft_tokens: torch.Tensor,
                   sampling_metadata: SamplingMetadata, *,
                   target_rows: torch.Tensor | None = None,
                   apply_temperature: bool = True) -> torch.Tensor:
    """The per-row masks ``rejection_sample(..., apply_top_k_top_p=True)`` applies.

    Returns ``[P, 4]`` fp32: row j holds (A, B, J, 0) with J's int32 bits in the third column,
    and entry i of verify row j (raw value x, before the temperature divide) is masked iff
    ``x < A or (x < B and i <= J)`` -- the entries ``apply_sampling_constraints`` (:537-571)
    would set to -inf.  Rows without constraints get (-inf, -inf, -1), and so do the rows of
    greedy requests whose argmax no mask can change: top-k never masks a row's maximum, and
    top-p masks one only when the maximum is tied and the entries below it hold at most 1 - p
    of the mass (such a row gets its full mask)."""
    device = target_logits.device
    nat.require_device_tensor(target_logits, "target_logits")
    if target_logits.stride(1) != 1:
        target_logits = target_logits.contiguous()
    batch_size = cu_num_draft_tokens.shape[0]
    num_tokens = (target_rows.shape[0] if target_rows is not None
                  else target_logits.shape[0])
    all_greedy = bool(sampling_metadata.all_greedy)
    temperature = None if all_greedy else _as(sampling_metadata.temperature, torch.float32, device)
    top_k = (None if sampling_metadata.top_k is None
             else _as(sampling_metadata.top_k, torch.int64, device))
    top_p = (None if sampling_metadata.top_p is None
             else _as(sampling_metadata.top_p, torch.float32, device))
    cu = _as(cu_num_draft_tokens, torch.int32, device)
    rows = None if target_rows is None else _as(target_rows, torch.int32, device)
    masks = torch.empty((num_tokens, 4), dtype=torch.float32, device=device)
    args = nat.RejectionArgs(
        target_logits=target_logits.data_ptr(), target_dtype=nat.dtype_code(target_logits.dtype),
        target_stride=target_logits.stride(0), target_rows=nat.ptr(rows),
        target_num_rows=target_logits.shape[0], cu_num_draft_tokens=cu.data_ptr(),
        temperature=nat.ptr(temperature), all_greedy=int(all_greedy),
        apply_temperature=int(bool(apply_temperature)), batch_size=batch_size,
        num_tokens=num_tokens, vocab_size=target_logits.shape[-1], top_k=nat.ptr(top_k),
        top_p=nat.ptr(top_p))
    nat.check(nat.lib().mvsd_sampling_masks(args, masks.data_ptr(), nat.stream_of(device)),
              "mvsd_sampling_masks")
    return masks


def apply_sampling_constraints(
    logits: torch.Tensor,               # [num_tokens, vocab_size]
    cu_num_draft_tokens: torch.Tensor,  # [batch_size]
    sampling_metadata: SamplingMetadata,
) -> torch.Tensor:
    """Per-row temperature divide (greedy T=0 -> 1) then top-k/top-p, in place (:537-571)."""
    assert logits.ndim == 2
    assert cu_num_draft_tokens.ndim == 1
    if sampling_metadata.all_greedy:
        return logits
    num_tokens = logits.shape[0]
    temperature = expand_batch_to_tokens(sampling_metadata.temperature, cu_num_draft_tokens,
                                         num_tokens, replace_from=GREEDY_TEMPERATURE,
                                         replace_to=1)
    logits.div_(temperature.unsqueeze(-1))
    top_k = None
    if sampling_metadata.top_k is not None:
        top_k = expand_batch_to_tokens(sampling_metadata.top_k, cu_num_draft_tokens, num_tokens)
    top_p = None
    if sampling_metadata.top_p is not None:
        top_p = expand_batch_to_tokens(sampling_metadata.top_p, cu_num_draft_tokens, num_tokens)
    return apply_top_k_top_p(logits, top_k, top_p)


def expand_batch_to_tokens(
    x: torch.Tensor,              # [batch_size]
    cu_num_tokens: torch.Tensor,  # [batch_size]
    num_tokens: int,
    replace_from: int = 0,
    replace_to: int = 0,
) -> torch.Tensor:
    """``[B] -> [num_tokens]``: request i's value repeated over its rows (:574-597)."""
    batch_size = x.shape[0]
    assert cu_num_tokens.shape[0] == batch_size
    expanded = x.new_empty(num_tokens)
    if batch_size == 0:
        return expanded
    nat.require_device_tensor(x, "x")
    src = x.contiguous()
    cu = _as(cu_num_tokens, torch.int32, x.device)
    code = nat.dtype_code(src.dtype)
    nat.check(nat.lib().mvsd_expand_batch_to_tokens(
        expanded.data_ptr(), src.data_ptr(), code, cu.data_ptr(), batch_size, num_tokens,
        float(replace_from), float(replace_to), nat.stream_of(x.device)),
        "mvsd_expand_batch_to_tokens")
    return expanded


def generate_uniform_probs(
    num_tokens: int,
    num_draft_tokens: list[int],
    generators: dict[int, torch.Generator],
    device: torch.device,
) -> torch.Tensor:
    """One fp64 uniform per verify row; seeded requests draw from their own generator and
    requests without drafts consume nothing (:600-624)."""
    uniform_probs = torch.rand((num_tokens,), dtype=torch.float64, device=device)
    start = 0
    for req_idx, n in enumerate(num_draft_tokens):
        if n == 0:
            continue
        generator = generators.get(req_idx)
        if generator is not None:
            uniform_probs[start:start + n].uniform_(generator=generator)
        start += n
    return uniform_probs


def generate_exponential_noise(
    batch_size: int,
    vocab_size: int,
    num_draft_tokens: list[int],
    generators: dict[int, torch.Generator],
    device: torch.device,
) -> torch.Tensor:
    """One Exp(1) row per request, seeded rows from their generator, requests without
    drafts leaving their generator untouched (:646-653)."""
    noise = torch.empty((batch_size, vocab_size), dtype=torch.float32, device=device)
    noise.exponential_()
    for index, generator in generators.items():
        if num_draft_tokens[index] > 0:
            noise[index].exponential_(generator=generator)
    return noise


def sample_recovered_tokens(
    max_spec_len: int,
    num_draft_tokens: list[int],
    cu_num_draft_tokens: torch.Tensor,  # [batch_size]
    draft_token_ids: torch.Tensor,      # [num_tokens]
    draft_probs: torch.Tensor | None,   # [num_tokens, vocab_size]
    target_probs: torch.Tensor,         # [num_tokens, vocab_size]
    sampling_metadata: SamplingMetadata,
    device: torch.device,
    *,
    exp_noise: torch.Tensor | None = None,
) -> torch.Tensor:
    """Recovered ids ``argmax_v max(p - q, 0) * (1 / E[req, v])`` from materialised
    probabilities (:627-670); ``draft_probs=None`` is the point-mass form."""
    batch_size = len(num_draft_tokens)
    vocab_size = target_probs.shape[-1]
    nat.require_device_tensor(target_probs, "target_probs")
    if exp_noise is None:
        exp_noise = generate_exponential_noise(batch_size, vocab_size, num_draft_tokens,
                                               sampling_metadata.generators, device)
    recovered = torch.empty_like(draft_token_ids)
    if draft_token_ids.shape[0] == 0 or max_spec_len == 0:
        return recovered
    out32 = recovered if recovered.dtype == torch.int32 else torch.empty(
        recovered.shape, dtype=torch.int32, device=device)
    cu = _as(cu_num_draft_tokens, torch.int32, device)
    ids = _as(draft_token_ids, torch.int32, device)
    tp = _as(target_probs, torch.float32, device)
    dp = None if draft_probs is None else _as(draft_probs, torch.float32, device)
    noise = _as(exp_noise, torch.float32, device)
    nat.check(nat.lib().mvsd_sample_recovered_tokens(
        out32.data_ptr(), cu.data_ptr(), ids.data_ptr(), nat.ptr(dp),
        dp.stride(0) if dp is not None else 0, tp.data_ptr(), tp.stride(0), noise.data_ptr(),
        noise.stride(0), batch_size, draft_token_ids.shape[0], vocab_size, max_spec_len,
        nat.stream_of(device)), "mvsd_sample_recovered_tokens")
    if out32 is not recovered:
        recovered.copy_(out32)
    return recovered


_SAMPLE_RECOVERED_TOKENS = sample_recovered_tokens


# --------------------------------------------------------------------------- helpers

# One zero-initialised verification workspace per (device, stream).  The kernel leaves it
# zeroed after every call (include/mvsd.h), so it is reused without clearing; it only grows.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


@functools.lru_cache(maxsize=256)
def _workspace_bytes(batch_size: int, num_tokens: int, vocab_size: int, dtype: int,
                     max_spec_len: int) -> int:
    """The verify workspace's size for a call shape (a pure function of these values)."""
    return int(nat.lib().mvsd_rejection_workspace_bytes(batch_size, num_tokens, vocab_size, dtype,
                                                        max_spec_len))


def _workspace(device: torch.device, nbytes: int, stream: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 1 << 16)
        if ws is not None:
            size = max(size, 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        nat.check(nat.lib().mvsd_rejection_workspace_init(ws.data_ptr(), ws.numel(), stream),
                  "mvsd_rejection_workspace_init")
        _WORKSPACES[key] = ws
    return ws


def _as(t: torch.Tensor, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """Contiguous tensor of ``dtype`` on ``device`` (no copy when it already is one)."""
    if t.device != device:
        t = t.to(device)
    if t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _expand_temperature(temperature: torch.Tensor | None, cu: torch.Tensor,
                        num_tokens: int) -> torch.Tensor | None:
    if temperature is None:
        return None
    return expand_batch_to_tokens(temperature, cu, num_tokens, replace_from=GREEDY_TEMPERATURE,
                                  replace_to=1)


def _softmax_rows(logits: torch.Tensor, rows: torch.Tensor | None,
                  row_temperature: torch.Tensor | None) -> torch.Tensor:
    """fp32 probabilities of the verify rows (HIP kernel ``mvsd_softmax_rows``)."""
    src = logits if rows is None else logits[rows.long()]
    src = src.contiguous()
    probs = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    if src.shape[0] == 0:
        return probs
    temp = None if row_temperature is None else _as(row_temperature, torch.float32, src.device)
    nat.check(nat.lib().mvsd_softmax_rows(
        probs.data_ptr(), probs.stride(0), src.data_ptr(), nat.dtype_code(src.dtype),
        src.stride(0), nat.ptr(temp), src.shape[0], src.shape[1], nat.stream_of(src.device)),
        "mvsd_softmax_rows")
    return probs
