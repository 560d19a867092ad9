"""V2 speculative-decoding verification (minivllm/worker/gpu/spec_decode)."""

from .rejection_sampler_utils import rejection_sample

__all__ = ["rejection_sample"]
