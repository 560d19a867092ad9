"""ctypes wrapper of oracle/ngram.c plus a pure-Python brute force for tiny inputs —
TEST INFRASTRUCTURE ONLY (see oracle/ngram.c for what each function restates)."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libmvsd_oracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = ctypes.CDLL(str(LIB))
        i32p = ctypes.POINTER(ctypes.c_int32)
        h.ngram_kmp.argtypes = [i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int64, ctypes.c_int, i32p]
        h.ngram_kmp.restype = ctypes.c_int
        h.ngram_brute_cpu.argtypes = h.ngram_kmp.argtypes
        h.ngram_brute_cpu.restype = ctypes.c_int
        h.ngram_brute_device.argtypes = [i32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, i32p]
        h.ngram_brute_device.restype = ctypes.c_int
        h.ngram_kmp_batch.argtypes = [i32p, ctypes.c_int64, i32p, ctypes.c_int64, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int64, ctypes.c_int, i32p, i32p]
        h.ngram_kmp_batch.restype = None
        h.ngram_brute_device_batch.argtypes = [i32p, ctypes.c_int64, i32p, ctypes.c_int64,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, i32p,
                                               i32p]
        h.ngram_brute_device_batch.restype = None
        _lib = h
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def find_kmp(tokens, min_n: int, max_n: int, max_model_len: int, k: int) -> list[int]:
    """minivllm/spec_decode/ngram_proposer.py:41-99 restated in C."""
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.zeros(max(k, 1), dtype=np.int32)
    n = lib().ngram_kmp(_p(t), len(t), min_n, max_n, max_model_len, k, _p(out))
    return out[:n].tolist()


def find_brute_cpu(tokens, min_n, max_n, max_model_len, k) -> list[int]:
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.zeros(max(k, 1), dtype=np.int32)
    n = lib().ngram_brute_cpu(_p(t), len(t), min_n, max_n, max_model_len, k, _p(out))
    return out[:n].tolist()


def find_brute_device(tokens, min_n, max_n, k) -> tuple[list[int], int]:
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.zeros(k, dtype=np.int32)
    n = lib().ngram_brute_device(_p(t), len(t), min_n, max_n, k, _p(out))
    return out.tolist(), int(n)


def kmp_batch(tokens: np.ndarray, lens: np.ndarray, min_n, max_n, max_model_len, k):
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    ln = np.ascontiguousarray(lens, dtype=np.int32)
    drafts = np.empty((t.shape[0], k), dtype=np.int32)
    counts = np.empty(t.shape[0], dtype=np.int32)
    lib().ngram_kmp_batch(_p(t), t.shape[1], _p(ln), t.shape[0], min_n, max_n, max_model_len, k,
                          _p(drafts), _p(counts))
    return drafts, counts


def brute_device_batch(tokens: np.ndarray, lens: np.ndarray, min_n, max_n, k):
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    ln = np.ascontiguousarray(lens, dtype=np.int32)
    drafts = np.empty((t.shape[0], k), dtype=np.int32)
    counts = np.empty(t.shape[0], dtype=np.int32)
    lib().ngram_brute_device_batch(_p(t), t.shape[1], _p(ln), t.shape[0], min_n, max_n, k,
                                   _p(drafts), _p(counts))
    return drafts, counts


def find_python(tokens, min_n, max_n, k) -> tuple[int, int]:
    """Pure-Python definition for tiny inputs: (earliest start, n) of the longest match."""
    t = list(tokens)
    L = len(t)
    for n in range(max_n, min_n - 1, -1):
        for s in range(0, L - n):
            if t[s:s + n] == t[L - n:]:
                return s, n
    return -1, 0


def valid_sampled_tokens(sampled, discard, token_ids, num_tokens, vocab_size):
    """NgramProposerGPU.update_token_ids_ngram (minivllm/spec_decode/ngram_proposer_gpu.py:
    247-290) in numpy: (next_token_ids, counts, valid_ids).  Discarded rows become -1; the
    count is #{v != -1 and v < vocab_size}; the next token is valid_ids[i, count - 1] when the
    count is positive, else token_ids[i, max(num_tokens[i] - 1, 0)].  Pinned by the
    reference's known answer (tests/step60/test_ngram_gpu_state.py:157-179) and by the
    per-row definition in tests/test_oracle_ngram.py."""
    sampled = np.asarray(sampled, dtype=np.int64)
    valid = sampled.copy()
    valid[np.asarray(discard, dtype=bool)] = -1
    ok = (valid != -1) & (valid < vocab_size)
    counts = ok.sum(axis=1)
    last = np.clip(counts - 1, 0, None)
    selected = valid[np.arange(valid.shape[0]), last] if valid.shape[1] else \
        np.zeros(valid.shape[0], np.int64)
    tokens = np.asarray(token_ids, dtype=np.int64)
    back = np.clip(np.asarray(num_tokens, dtype=np.int64) - 1, 0, None)
    backup = tokens[np.arange(tokens.shape[0]), back]
    nxt = np.where(counts > 0, selected, backup)
    return nxt.astype(np.int32), counts.astype(np.int32), valid.astype(np.int32)
