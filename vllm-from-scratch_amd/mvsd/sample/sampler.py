"""The regular sampler on MI355X (drop-in for minivllm/sample/sampler.py ``Sampler``).

The rejection sampler takes its bonus tokens from a sampler object (rejection_sampler.py:
169-181); this is one with the reference's names, call protocol and order of operations
(sampler.py:73-120, :243-349):

    logits -> fp32
    -> penalties (bonus rows: history = committed output + all drafts) -> min_tokens
    -> greedy rows: argmax (no temperature)
    -> random rows: / temperature -> min_p -> top-k / top-p -> exponential race
    -> rows with temperature < eps take the greedy result
    -> logprobs of the raw (before any processing) or processed rows on request

Every row operation is a HIP kernel (``mvsd_apply_logits_processors``,
``mvsd_apply_top_k_top_p``, ``mvsd_sampler_rows``, ``mvsd_sampler_race(_rows)``,
``mvsd_spec_logprobs``).  The temperature divide is a tensor divide, as in the reference,
except where nothing reads the divided rows (no min_p, top-k or top-p, and no processed_*
logprobs mode): there one race launch divides each value as it reads it (the same IEEE fp32
quotient) and gives the rows under SAMPLING_EPS their argmax, and the caller's logits are
left undivided.  The race's token is the argmax of softmax(v) / E, evaluated as that of
v log2(e) - log2(E) (the row's max and sum are common to its entries), so only near-ties
within a few fp32 ulps of the keys' magnitudes can differ from the reference's fp32
arithmetic.  The exponential noise is drawn by
``generate_sampler_noise`` in the reference's order (the whole block from the global RNG when
some row has no generator, then each seeded row from its generator), so a given RNG state
gives the same noise; the function is a seam that tests may replace.
"""

from __future__ import annotations

import numpy as np
import torch

from .. import _native as nat
from ..outputs import LogprobsTensors, SamplerOutput
from .metadata import SAMPLING_EPS, SamplingMetadata
from .ops.topk_topp_sampler import apply_top_k_top_p

_ARGMAX, _MIN_P, _LOG_SOFTMAX = 0, 1, 3
_PROCESSED_MODES = ("processed_logits", "processed_logprobs")


def generate_sampler_noise(shape, generators: dict[int, torch.Generator],
                           device: torch.device) -> torch.Tensor:
    """Exp(1) noise of random_sample (ops/topk_topp_sampler.py:82-90)."""
    noise = torch.empty(shape, dtype=torch.float32, device=device)
    if len(generators) != shape[0]:
        noise.exponential_()
    for row, generator in generators.items():
        noise[row].exponential_(generator=generator)
    return noise


def _rows(op, x: torch.Tensor, *, ids=None, out=None, aux=None):
    nat.require_device_tensor(x, "logits")
    assert x.ndim == 2 and x.dtype == torch.float32 and x.stride(1) == 1
    n, V = x.shape
    nat.check(nat.lib().mvsd_sampler_rows(
        op, nat.ptr(ids), nat.ptr(out), 0 if out is None else out.stride(0), x.data_ptr(),
        x.stride(0), nat.ptr(aux), 0 if aux is None or aux.ndim < 2 else aux.stride(0), n, V,
        nat.stream_of(x.device)), "mvsd_sampler_rows")


def random_sample(probs_logits: torch.Tensor, generators: dict[int, torch.Generator],
                  temperature: torch.Tensor | None = None):
    """argmax of softmax(row) / E per row (the exponential race, ops/topk_topp_sampler.py:82-90,
    with the softmax of the processed logits folded in); with ``temperature`` ([N] fp32,
    positive) each row is first divided by its temperature inside the kernel.  One
    ``mvsd_sampler_race`` call."""
    x = probs_logits.contiguous()
    nat.require_device_tensor(x, "logits")
    assert x.ndim == 2 and x.dtype == torch.float32
    n, V = x.shape
    noise = generate_sampler_noise(tuple(x.shape), generators, x.device)
    noise = noise.to(device=x.device, dtype=torch.float32).contiguous()
    ids = torch.empty(n, dtype=torch.int32, device=x.device)
    if temperature is not None:
        temperature = temperature.to(device=x.device, dtype=torch.float32).contiguous()
    lib = nat.lib()
    ws = torch.empty(max(1, lib.mvsd_sampler_race_workspace_bytes(n, V)), dtype=torch.uint8,
                     device=x.device)
    nat.check(lib.mvsd_sampler_race(
        ids.data_ptr(), x.data_ptr(), x.stride(0), noise.data_ptr(), noise.stride(0),
        nat.ptr(temperature), n, V, ws.data_ptr(), ws.numel(), nat.stream_of(x.device)),
        "mvsd_sampler_race")
    return ids.to(torch.int64)


def race_rows(logits: torch.Tensor, row_index: torch.Tensor | None,
              noise: torch.Tensor | None, temperature: torch.Tensor | None,
              greedy_eps: float = SAMPLING_EPS) -> torch.Tensor:
    """Sampled ids (int32 [n]) of the rows ``logits[row_index]`` (fp32, bf16 or fp16, read in
    place) in one ``mvsd_sampler_race_rows`` call: rows whose temperature is below
    ``greedy_eps`` take the argmax of the raw row (greedy_sample), the others the exponential
    race of softmax(row / T) with ``noise`` [n, V]; without noise every row is greedy."""
    nat.require_device_tensor(logits, "logits")
    assert logits.ndim == 2 and logits.stride(1) == 1
    device = logits.device
    rows = None
    n = logits.shape[0]
    if row_index is not None:
        rows = row_index.to(device=device, dtype=torch.int32).contiguous()
        n = rows.shape[0]
    V = logits.shape[1]
    if noise is not None:
        noise = noise.to(device=device, dtype=torch.float32)
        assert noise.shape == (n, V) and noise.stride(1) == 1
    if temperature is not None:
        temperature = temperature.to(device=device, dtype=torch.float32).contiguous()
    ids = torch.empty(n, dtype=torch.int32, device=device)
    lib = nat.lib()
    ws = torch.empty(max(1, lib.mvsd_sampler_race_workspace_bytes(n, V)), dtype=torch.uint8,
                     device=device)
    nat.check(lib.mvsd_sampler_race_rows(
        ids.data_ptr(), logits.data_ptr(), nat.dtype_code(logits.dtype), logits.stride(0),
        nat.ptr(rows), logits.shape[0], nat.ptr(noise), 0 if noise is None else noise.stride(0),
        nat.ptr(temperature), float(greedy_eps), n, V, ws.data_ptr(), ws.numel(),
        nat.stream_of(device)), "mvsd_sampler_race_rows")
    return ids


class TopKTopPSampler:
    """Temperature-scaled logits -> one token per row, with the processed logits or logprobs of
    the ``processed_*`` modes (ops/topk_topp_sampler.py:93-115)."""

    def __init__(self, logprobs_mode: str = "raw_logprobs") -> None:
        self.logprobs_mode = logprobs_mode

    def __call__(self, logits, generators, k, p):
        logits = apply_top_k_top_p(logits, k, p)
        logits_to_return = None
        if self.logprobs_mode == "processed_logits":
            logits_to_return = logits
        elif self.logprobs_mode == "processed_logprobs":
            logits_to_return = Sampler.compute_logprobs(logits)
        return random_sample(logits, generators), logits_to_return


class Sampler:
    def __init__(self, logprobs_mode: str = "raw_logprobs") -> None:
        self.logprobs_mode = logprobs_mode
        self.topk_topp_sampler = TopKTopPSampler(logprobs_mode)

    def forward(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata,
                predict_bonus_token: bool = False,
                logprobs_mode_override: str | None = None) -> SamplerOutput:
        logprobs_mode = logprobs_mode_override or self.logprobs_mode
        assert not (sampling_metadata.all_greedy and sampling_metadata.all_random)
        num_logprobs = sampling_metadata.max_num_logprobs
        raw_logprobs = None
        if num_logprobs is not None:
            if logprobs_mode == "raw_logprobs":
                raw_logprobs = self.compute_logprobs(logits.to(torch.float32))
            elif logprobs_mode == "raw_logits":
                raw_logprobs = (logits.clone() if logits.dtype == torch.float32
                                else logits.to(torch.float32))
        logits = logits.to(torch.float32).contiguous()
        logits = self.apply_logits_processors(logits, sampling_metadata, predict_bonus_token)
        sampled, processed = self.sample(logits, sampling_metadata)
        if processed is not None:
            raw_logprobs = processed
        sampled = sampled.long()
        if num_logprobs is None:
            tensors = None
        elif num_logprobs == -1:
            tensors = LogprobsTensors(torch.empty(0), raw_logprobs, torch.empty(0))
        else:
            tensors = self.gather_logprobs(raw_logprobs, num_logprobs, sampled)
        return SamplerOutput(sampled_token_ids=sampled.to(torch.int32).unsqueeze(dim=1),
                             logprobs_tensors=tensors)

    # -------- logits processors --------

    def apply_logits_processors(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata,
                                predict_bonus_token: bool = False) -> torch.Tensor:
        """Penalties, then min_tokens, in place (sampler.py:122-141); bonus rows
        (``predict_bonus_token``) count every draft in the penalty history."""
        output_token_ids = sampling_metadata.output_token_ids
        if predict_bonus_token and not sampling_metadata.no_penalties:
            output_token_ids = self._combine_outputs_with_spec_tokens(
                output_token_ids, sampling_metadata.spec_token_ids)
        logits = self.apply_penalties(logits, sampling_metadata, output_token_ids)
        return self.apply_min_tokens(logits, sampling_metadata)

    def apply_penalties(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata,
                        output_token_ids: list[list[int]] | None = None) -> torch.Tensor:
        from .rejection_sampler import _launch_logits_processors, _penalty_entries

        if sampling_metadata.no_penalties:
            return logits
        if output_token_ids is None:
            output_token_ids = sampling_metadata.output_token_ids
        n = logits.shape[0]
        cu = torch.arange(1, n + 1, dtype=torch.int32, device=logits.device)
        entries = _penalty_entries(sampling_metadata.prompt_token_ids, output_token_ids,
                                   [[] for _ in range(n)])
        _launch_logits_processors(logits, cu, [1] * n, [[-1]] * n, entries, sampling_metadata,
                                  None)
        return logits

    @staticmethod
    def _combine_outputs_with_spec_tokens(output_token_ids, spec_token_ids=None):
        """Bonus-row histories: committed output + every draft, one row per request
        (sampler.py:159-175)."""
        if spec_token_ids is None:
            return output_token_ids
        return [[*out, *spec] if spec else out
                for out, spec in zip(output_token_ids, spec_token_ids)]

    def apply_min_tokens(self, logits: torch.Tensor,
                         sampling_metadata: SamplingMetadata) -> torch.Tensor:
        """Stop tokens of rows whose committed output is shorter than min_tokens -> -inf
        (sampler.py:177-190)."""
        from .rejection_sampler import _launch_logits_processors

        n = logits.shape[0]
        n_mask = np.zeros(n, dtype=np.int32)
        stop_off, stop_tok = [0], []
        for row, (min_tokens, stop_ids) in enumerate(zip(sampling_metadata.min_tokens,
                                                          sampling_metadata.stop_token_ids)):
            if row < n and stop_ids and len(sampling_metadata.output_token_ids[row]) < min_tokens:
                n_mask[row] = 1
                stop_tok.extend(stop_ids)
            if row < n:
                stop_off.append(len(stop_tok))
        if not n_mask.any():
            return logits
        stop_off += [len(stop_tok)] * (n + 1 - len(stop_off))
        cu = torch.arange(1, n + 1, dtype=torch.int32, device=logits.device)
        _launch_logits_processors(logits, cu, [1] * n, [[-1]] * n, None, None,
                                  (n_mask, np.asarray(stop_off, np.int32),
                                   np.asarray(stop_tok, np.int32)))
        return logits

    def apply_min_tokens_for_spec_decode(self, logits, sampling_metadata, num_draft_tokens):
        """min_tokens on verify rows (sampler.py:192-228): the first clamp(min_tokens -
        len(output), 0, K_i) rows of each request mask its stop tokens."""
        from .rejection_sampler import _launch_logits_processors, _min_tokens_rows

        num_draft = [int(k) for k in num_draft_tokens]
        masks = _min_tokens_rows(sampling_metadata, num_draft)
        if masks is None:
            return logits
        cu = torch.as_tensor(np.cumsum(num_draft), dtype=torch.int32, device=logits.device)
        _launch_logits_processors(logits, cu, num_draft, [[-1] * k for k in num_draft], None,
                                  None, masks)
        return logits

    # -------- sampling --------

    def sample(self, logits: torch.Tensor, sampling_metadata: SamplingMetadata,
               logprobs_mode: str | None = None):
        """(tokens, processed logits / logprobs of the processed_* modes) (sampler.py:243-278)."""
        md = sampling_metadata
        if md.all_greedy:
            # nothing scales or masks an all-greedy batch: the "processed" rows are the rows
            wanted = None
            if md.max_num_logprobs is not None:
                wanted = {"processed_logits": lambda: logits,
                          "processed_logprobs": lambda: self.compute_logprobs(logits)
                          }.get(logprobs_mode or self.logprobs_mode)
            return self.greedy_sample(logits), (wanted() if wanted else None)
        if md.temperature is None:
            raise ValueError("random rows in the batch but no temperature tensor")
        reads_divided_rows = (md.min_p is not None or md.top_k is not None
                              or md.top_p is not None
                              or self.topk_topp_sampler.logprobs_mode in _PROCESSED_MODES)
        if not reads_divided_rows:
            # one race launch: rows under SAMPLING_EPS take their argmax, the others race on
            # fl(x / T) divided as the kernel reads; the caller's rows stay undivided
            noise = generate_sampler_noise(tuple(logits.shape), md.generators, logits.device)
            return race_rows(logits, None, noise, md.temperature).to(torch.int64), None
        # The argmax is taken on the rows as they arrive (penalties applied, no temperature),
        # before the divide below changes them in place.
        argmax_ids = None if md.all_random else self.greedy_sample(logits)
        # rows under SAMPLING_EPS are greedy: their divisor is 1 and their draw is discarded
        greedy_rows = md.temperature < SAMPLING_EPS
        divisor = md.temperature.masked_fill(greedy_rows, 1.0)
        scaled = self.apply_min_p(logits.div_(divisor.unsqueeze(1)), md.min_p)
        drawn, processed = self.topk_topp_sampler(scaled, md.generators, md.top_k, md.top_p)
        if argmax_ids is not None:
            drawn = torch.where(greedy_rows, argmax_ids, drawn)
        return drawn, processed

    @staticmethod
    def apply_min_p(logits: torch.Tensor, min_p: torch.Tensor | None) -> torch.Tensor:
        """Entries whose probability is below max(p) * min_p -> -inf, in place
        (sampler.py:280-293)."""
        if min_p is None:
            return logits
        _rows(_MIN_P, logits, aux=min_p.to(device=logits.device, dtype=torch.float32).contiguous())
        return logits

    @staticmethod
    def greedy_sample(logits: torch.Tensor) -> torch.Tensor:
        x = logits.contiguous()
        ids = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
        _rows(_ARGMAX, x, ids=ids)
        return ids.to(torch.int64)

    # -------- logprobs --------

    @staticmethod
    def compute_logprobs(logits: torch.Tensor) -> torch.Tensor:
        x = logits.to(torch.float32).contiguous()
        out = torch.empty_like(x)
        _rows(_LOG_SOFTMAX, x, out=out)
        return out

    @staticmethod
    def batched_count_greater_than(x: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
        """#{x >= value} per row (sampler.py:318-327): the rank of a token."""
        return (x >= values).sum(-1)

    @staticmethod
    def gather_logprobs(logprobs: torch.Tensor, num_logprobs: int,
                        token_ids: torch.Tensor) -> LogprobsTensors:
        """Sampled token first, then the top ``num_logprobs`` (value, then index), and the
        sampled token's rank (sampler.py:330-349); one ``mvsd_spec_logprobs`` launch with each
        row its own position."""
        assert token_ids.dtype == torch.int64
        x = logprobs.to(torch.float32).contiguous()
        n, V = x.shape
        device = x.device
        ids = torch.empty((n, num_logprobs + 1), dtype=torch.int32, device=device)
        lps = torch.empty((n, num_logprobs + 1), dtype=torch.float32, device=device)
        ranks = torch.empty((n,), dtype=torch.int32, device=device)
        cu = torch.arange(1, n + 1, dtype=torch.int32, device=device)
        tokens = token_ids.to(device=device, dtype=torch.int32).reshape(n, 1).contiguous()
        nat.check(nat.lib().mvsd_spec_logprobs(
            ids.data_ptr(), lps.data_ptr(), ranks.data_ptr(), None, V, None, x.data_ptr(),
            x.stride(0), cu.data_ptr(), tokens.data_ptr(), 1, n, 0, V, 1, num_logprobs, 1,
            nat.stream_of(device)), "mvsd_spec_logprobs")
        return LogprobsTensors(ids, lps, ranks)
