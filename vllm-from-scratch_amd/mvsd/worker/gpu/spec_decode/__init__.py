"""V2 speculative-decoding verification (minivllm/worker/gpu/spec_decode)."""

from .rejection_sampler import (MAX_CHUNK_BYTES, RejectionSampler, flatten_sampled,
                                get_max_chunk_logits)
from .rejection_sampler_utils import rejection_sample

__all__ = ["MAX_CHUNK_BYTES", "RejectionSampler", "flatten_sampled", "get_max_chunk_logits",
           "rejection_sample"]
