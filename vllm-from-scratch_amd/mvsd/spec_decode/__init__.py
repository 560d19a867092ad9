"""Speculative proposers and step metadata (in-scope part of minivllm/spec_decode/__init__.py)."""

from .metadata import SpecDecodeMetadata
from .metrics import SpecDecodingStats
from .ngram_proposer import NgramProposer
from .ngram_proposer_gpu import NgramGPUKernel, NgramProposerGPU

__all__ = ["SpecDecodeMetadata", "SpecDecodingStats", "NgramProposer", "NgramProposerGPU",
           "NgramGPUKernel"]
