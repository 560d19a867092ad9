"""ctypes binding of libmvsd.so (C ABI in include/mvsd.h).

The library is required: importing a product function without it raises ImportError-like
``RuntimeError`` at first use, and there is no CPU or torch fallback.  Status codes are
turned into ``RuntimeError`` exactly like the reference's ctypes-loaded kernels
(minivllm/layers/ops/rms_norm_cuda.py:95-112,163-188).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from .build import LIB_PATH

# dtype codes (include/mvsd.h)
F32, BF16, F16, F64, I32, I64, U8 = range(7)

# Output entry of a verification whose bounded waits gave up (MVSD_POISON in include/mvsd.h).
POISON = -(2 ** 31)

_TORCH_CODES = {
    torch.float32: F32,
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.float64: F64,
    torch.int32: I32,
    torch.int64: I64,
    torch.uint8: U8,
    torch.bool: U8,
}

c_int, c_int32, c_int64, c_double, c_void_p = (ctypes.c_int, ctypes.c_int32, ctypes.c_int64,
                                              ctypes.c_double, ctypes.c_void_p)
c_float = ctypes.c_float


class RejectionArgs(ctypes.Structure):
    """Mirror of ``mvsd_rejection_args``."""

    _fields_ = [
        ("output_token_ids", c_void_p),
        ("out_stride", c_int64),
        ("target_logits", c_void_p),
        ("target_dtype", c_int),
        ("target_stride", c_int64),
        ("target_rows", c_void_p),
        ("target_num_rows", c_int64),
        ("draft_probs", c_void_p),
        ("draft_dtype", c_int),
        ("draft_stride", c_int64),
        ("exp_noise", c_void_p),
        ("noise_stride", c_int64),
        ("uniform_probs", c_void_p),
        ("draft_token_ids", c_void_p),
        ("cu_num_draft_tokens", c_void_p),
        ("bonus_token_ids", c_void_p),
        ("temperature", c_void_p),
        ("all_greedy", c_int),
        ("apply_temperature", c_int),
        ("recovered_token_ids", c_void_p),
        ("synthetic_conditional_rates", c_void_p),
        ("batch_size", c_int64),
        ("num_tokens", c_int64),
        ("vocab_size", c_int64),
        ("max_spec_len", c_int64),
        ("workspace", c_void_p),
        ("workspace_bytes", c_int64),
        ("top_k", c_void_p),
        ("top_p", c_void_p),
        ("debug_row_stats", c_void_p),
    ]


# name -> (restype, argtypes); every symbol include/mvsd.h declares
SIGNATURES = {
    "mvsd_version": (c_int, []),
    "mvsd_status_string": (ctypes.c_char_p, [c_int]),
    "mvsd_last_hip_error": (c_int, []),
    "mvsd_expand_batch_to_tokens": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int64,
                                            c_double, c_double, c_void_p]),
    "mvsd_rejection_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int, c_int64]),
    "mvsd_rejection_workspace_init": (c_int, [c_void_p, c_int64, c_void_p]),
    "mvsd_set_wait_limit": (c_int, [c_int]),
    "mvsd_rejection_sample": (c_int, [ctypes.POINTER(RejectionArgs), c_void_p]),
    "mvsd_rejection_static_scratch_bytes": (c_int64, []),
    "mvsd_rejection_sample_static": (c_int, [ctypes.POINTER(RejectionArgs), c_void_p]),
    "mvsd_apply_top_k_top_p": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                       c_void_p]),
    "mvsd_selftest": (c_int, [c_int, c_void_p, c_void_p]),
    "mvsd_sampling_masks": (c_int, [ctypes.POINTER(RejectionArgs), c_void_p, c_void_p]),
    "mvsd_softmax_rows": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_int64, c_void_p, c_int64,
                                  c_int64, c_void_p]),
    "mvsd_sample_recovered_tokens": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                             c_void_p, c_int64, c_void_p, c_int64, c_int64,
                                             c_int64, c_int64, c_int64, c_void_p]),
    "mvsd_apply_logits_processors": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64,
                                             c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_void_p]),
    "mvsd_spec_logprobs": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                   c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64,
                                   c_int64, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "mvsd_sampler_rows": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "mvsd_sampler_race_workspace_bytes": (c_int64, [c_int64, c_int64]),
    "mvsd_sampler_race": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                  c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "mvsd_sampler_race_rows": (c_int, [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64,
                                       c_void_p, c_int64, c_void_p, c_float, c_int64, c_int64,
                                       c_void_p, c_int64, c_void_p]),
    "mvsd_ngram_propose": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
                                   c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int,
                                   c_int64, c_int32, c_int32, c_int32, c_int, c_int64,
                                   c_void_p]),
    "mvsd_v2_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "mvsd_v2_rejection_sample": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int, c_int64,
                                         c_int64, c_void_p, c_int, c_int64, c_int64, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int32,
                                         c_void_p, c_int, c_int, c_void_p, c_int64, c_void_p]),
    "mvsd_v2_flatten_sampled": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                        c_int64, c_int64, c_void_p]),
    "mvsd_v2_num_sampled_and_rejected": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_void_p, c_int64, c_int64,
                                                 c_void_p]),
    "mvsd_topk_scores": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                 c_int64, c_int64, c_int64, c_int, c_void_p]),
    "mvsd_ngram_valid_sampled": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                         c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                         c_void_p, c_int64, c_int64, c_void_p]),
}

_lib = None
_lock = threading.Lock()


def library_path() -> Path:
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """Load libmvsd.so once; raise a clear error when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"libmvsd.so is not built ({LIB_PATH}); run `python -m mvsd.build` or "
                    "__graft_entry__.build().  There is no fallback implementation.")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        handle = lib()
        text = handle.mvsd_status_string(status).decode()
        hip = handle.mvsd_last_hip_error()
        extra = f" (hipError {hip})" if status == -4 else ""
        raise RuntimeError(f"{what} failed: {text}{extra}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_CODES[dtype]
    except KeyError as exc:
        raise TypeError(f"unsupported dtype {dtype}") from exc


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's raw handle of a device's current stream (the call its generated kernels use), about
# 25x cheaper than building the torch.cuda.Stream object; the public route where it is absent.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The HIP stream handle of the current stream on `device`."""
    if _raw_stream is not None and torch.cuda.is_initialized():
        index = device.index
        return _raw_stream(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


def require_device_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise NotImplementedError(
            f"{name} is on {t.device}: the verification kernels are HIP kernels and only take "
            "device tensors (the reference likewise refuses CPU tensors, "
            "minivllm/sample/rejection_sampler.py:446-450)")
