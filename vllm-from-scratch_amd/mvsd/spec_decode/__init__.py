"""Speculative proposers and step metadata (in-scope part of minivllm/spec_decode/__init__.py)."""

from .metadata import SpecDecodeMetadata
from .metrics import SpecDecodingLogging, SpecDecodingStats
from .ngram_proposer import NgramProposer
from .ngram_proposer_gpu import NgramGPUKernel, NgramProposerGPU

__all__ = ["SpecDecodeMetadata", "SpecDecodingLogging", "SpecDecodingStats", "NgramProposer",
           "NgramProposerGPU", "NgramGPUKernel"]
