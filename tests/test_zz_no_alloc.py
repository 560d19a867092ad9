"""mvsd_rejection_sample_static (the verification entry point that allocates nothing: its
scratch is the library's static device array) against mvsd_rejection_sample with a caller
workspace, both called through the C ABI on the same device-resident inputs.

Bar: the token ids are bit-identical (same kernels, same inputs).  Two calls in a row, the
second one smaller, so the static scratch is reused after a larger batch.  The entry point
has no counterpart in the reference.
"""

import ctypes

import numpy as np
import pytest
import torch

from mvsd import _native as nat
from mvsd.testing import configs

V = configs.VOCAB


def _args(w, out, workspace=None):
    """RejectionArgs for workload w (random requests, supplied noise and uniforms, the
    temperature divide in the kernel), writing into `out`."""
    a = nat.RejectionArgs()
    a.output_token_ids = out.data_ptr()
    a.out_stride = out.stride(0)
    a.target_logits = w.target_logits.data_ptr()
    a.target_dtype = nat.dtype_code(w.target_logits.dtype)
    a.target_stride = w.target_logits.stride(0)
    a.target_rows = None if w.target_rows is None else w.target_rows.data_ptr()
    a.target_num_rows = w.target_logits.shape[0]
    a.draft_probs = None if w.draft_probs is None else w.draft_probs.data_ptr()
    a.draft_dtype = nat.F32
    a.draft_stride = 0 if w.draft_probs is None else w.draft_probs.stride(0)
    a.exp_noise = None if w.exp_noise is None else w.exp_noise.data_ptr()
    a.noise_stride = 0 if w.exp_noise is None else w.exp_noise.stride(0)
    a.uniform_probs = None if w.uniforms is None else w.uniforms.data_ptr()
    a.draft_token_ids = w.draft_token_ids.data_ptr()
    a.cu_num_draft_tokens = w.cu_num_draft_tokens.data_ptr()
    a.bonus_token_ids = w.bonus_token_ids.data_ptr()
    a.temperature = None if w.temperature is None else w.temperature.data_ptr()
    a.all_greedy = int(w.all_greedy)
    a.apply_temperature = int(w.apply_temperature)
    a.batch_size = w.batch_size
    a.num_tokens = w.num_tokens
    a.vocab_size = w.vocab_size
    a.max_spec_len = w.max_spec_len
    if w.top_k is not None or w.top_p is not None:
        # sampling constraints in the kernels, after the temperature divide
        a.top_k = None if w.top_k is None else w.top_k.data_ptr()
        a.top_p = None if w.top_p is None else w.top_p.data_ptr()
        a.apply_temperature = 1
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel()
    return a


def _run_both(w, device):
    lib = nat.lib()
    stream = nat.stream_of(device)
    nbytes = lib.mvsd_rejection_workspace_bytes(w.batch_size, w.num_tokens, w.vocab_size,
                                                nat.dtype_code(w.target_logits.dtype),
                                                w.max_spec_len)
    assert 0 < nbytes <= lib.mvsd_rejection_static_scratch_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    nat.check(lib.mvsd_rejection_workspace_init(ws.data_ptr(), ws.numel(), stream),
              "mvsd_rejection_workspace_init")
    width = w.max_spec_len + 1
    ref = torch.full((w.batch_size, width), -7, dtype=torch.int32, device=device)
    got = torch.full((w.batch_size, width), -7, dtype=torch.int32, device=device)
    nat.check(lib.mvsd_rejection_sample(ctypes.byref(_args(w, ref, ws)), stream),
              "mvsd_rejection_sample")
    nat.check(lib.mvsd_rejection_sample_static(ctypes.byref(_args(w, got)), stream),
              "mvsd_rejection_sample_static")
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


@pytest.mark.gpu
def test_static_scratch_matches_workspace_entry(device):
    """Headline-shaped batch, then a smaller mixed one (greedy rows too, target_rows gathers),
    each through both entry points."""
    first = configs.random_c2(device, B=128, k=4, seed=9101)
    second = configs.ragged_c4(device, B=40, seed=9102)
    second = configs.Workload(**{**second.__dict__, "top_k": None, "top_p": None})
    for w in (first, second):
        print(f"[static scratch] {w.name} B={w.batch_size} P={w.num_tokens}", flush=True)
        ref, got = _run_both(w, device)
        assert (ref != -7).all() and (ref != nat.POISON).all()
        assert np.array_equal(ref, got), f"{w.name}: static-scratch entry differs"


@pytest.mark.gpu
def test_static_scratch_repeated_calls(device):
    """Consecutive calls on the shared scratch (it must be left zeroed by each)."""
    a = configs.random_c2(device, B=64, k=4, seed=9103)
    b = configs.greedy_c1(device, B=16, k=3, seed=9104)
    for w in (a, b, a):
        ref, got = _run_both(w, device)
        assert np.array_equal(ref, got), f"{w.name}: static-scratch entry differs"


@pytest.mark.gpu
def test_static_scratch_masked_batch(device):
    """A batch with top-k / top-p (C4-shaped, smaller): the plan, the constraints kernel and
    the masked verify kernel use the static scratch's mask and plan arrays; the tokens are the
    workspace entry's."""
    w = configs.ragged_c4(device, B=96, seed=9103)
    ref, got = _run_both(w, device)
    assert np.array_equal(ref, got), "masked batch: static-scratch entry differs"


def test_static_scratch_refuses_oversized_batches():
    """A batch needing more scratch than the static array holds is refused with
    MVSD_E_SCRATCH before anything is touched (no device needed)."""
    lib = nat.lib()
    cap = lib.mvsd_rejection_static_scratch_bytes()
    assert cap == 16 << 20
    a = nat.RejectionArgs()
    a.batch_size, a.num_tokens, a.vocab_size, a.max_spec_len = 4096, 4096 * 64, V, 64
    a.target_dtype = nat.F32
    assert lib.mvsd_rejection_workspace_bytes(4096, 4096 * 64, V, nat.F32, 64) > cap
    assert lib.mvsd_rejection_sample_static(ctypes.byref(a), None) == -6
    assert b"static scratch" in lib.mvsd_status_string(-6)
