"""Sampling-side verification (drop-in for the in-scope part of minivllm/sample/__init__.py)."""

from .metadata import SAMPLING_EPS, SamplingMetadata
from .ops.topk_topp_sampler import apply_top_k_top_p
from .rejection_sampler import (MAX_SPEC_LEN, PLACEHOLDER_TOKEN_ID, RejectionSampler,
                                apply_sampling_constraints, expand_batch_to_tokens,
                                generate_exponential_noise, generate_uniform_probs,
                                rejection_sample, sample_recovered_tokens, sampling_masks)
from .sampler import Sampler, TopKTopPSampler, generate_sampler_noise, random_sample

__all__ = ["SamplingMetadata", "SAMPLING_EPS", "apply_top_k_top_p", "RejectionSampler",
           "rejection_sample", "sample_recovered_tokens", "apply_sampling_constraints",
           "expand_batch_to_tokens", "generate_uniform_probs", "generate_exponential_noise",
           "sampling_masks", "PLACEHOLDER_TOKEN_ID", "MAX_SPEC_LEN", "Sampler",
           "TopKTopPSampler", "generate_sampler_noise", "random_sample"]
