"""mvsd — MI355X-native speculative-decoding verification.

Drop-in replacements for minivllm's verification path, module for module:

    mvsd.sample.rejection_sampler      <- minivllm/sample/rejection_sampler.py
    mvsd.sample.metadata               <- minivllm/sample/metadata.py
    mvsd.sample.ops.topk_topp_sampler  <- minivllm/sample/ops/topk_topp_sampler.py
    mvsd.spec_decode.metadata          <- minivllm/spec_decode/metadata.py
    mvsd.spec_decode.ngram_proposer    <- minivllm/spec_decode/ngram_proposer.py
    mvsd.spec_decode.ngram_proposer_gpu<- minivllm/spec_decode/ngram_proposer_gpu.py
    mvsd.spec_decode.utils / metrics   <- minivllm/spec_decode/utils.py, metrics.py
    mvsd.outputs                       <- minivllm/outputs.py (SamplerOutput, DraftTokenIds)
    mvsd.testing.spec_metadata         <- minivllm/testing/spec_metadata.py

The arithmetic runs in hand-written HIP kernels for gfx950 (``csrc/``), reached through the C
ABI of ``include/mvsd.h`` (libmvsd.so, loaded with ctypes by ``mvsd._native``).
"""

__version__ = "0.1.0"
