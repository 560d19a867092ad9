"""Host-side logic and the C ABI boundary (no GPU needed).

  * metadata index algebra, parse_output, synthetic-rate conversion, draft trimming and the
    acceptance statistics against the reference's KATs;
  * libmvsd.so loads and exports every function include/mvsd.h declares;
  * the ctypes mirror of mvsd_rejection_args has the C struct's layout (checked against a
    gcc-compiled offsetof probe of the header);
  * the product path refuses CPU tensors and a missing library loudly.
"""

import ctypes
import json
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd import _native as nat
from mvsd.sample.rejection_sampler import (RejectionSampler, expand_batch_to_tokens,
                                           rejection_sample)
from mvsd.sample.metadata import SamplingMetadata
from mvsd.spec_decode.metrics import stats_from_outputs
from mvsd.spec_decode.utils import (unconditional_to_conditional_rates,
                                    update_scheduler_for_invalid_drafts)
from mvsd.testing.spec_metadata import make_metadata

ROOT = Path(__file__).resolve().parents[1]
KATS = json.loads((ROOT / "tests" / "golden" / "reference_kats.json").read_text())
HEADER = ROOT / "include" / "mvsd.h"


@pytest.mark.parametrize("case", KATS["metadata"], ids=lambda c: c["name"])
def test_metadata_kats(case):
    meta = make_metadata(case["drafts"], num_scheduled=case.get("num_scheduled"),
                         input_ids=None if "num_scheduled" not in case else
                         _input_ids(case["drafts"], case["num_scheduled"]))
    for key in ("cu_num_draft_tokens", "cu_num_sampled_tokens", "logits_indices",
                "target_logits_indices", "bonus_logits_indices"):
        assert getattr(meta, key).tolist() == case[key], key
    assert meta.num_draft_tokens == case["num_draft_tokens"]
    assert meta.draft_token_ids.dtype == torch.int32
    assert meta.max_spec_len == max(case["num_draft_tokens"])


def _input_ids(drafts, scheduled):
    ids = []
    for draft, n in zip(drafts, scheduled):
        ids.extend([0] * (n - len(draft)) + list(draft))
    return ids


@pytest.mark.parametrize("case", KATS["parse_output"], ids=lambda c: c["source"])
def test_parse_output_kats(case):
    padded = torch.tensor(case["padded"], dtype=torch.int32)
    out, lp = RejectionSampler.parse_output(padded, case["vocab"],
                                            discard_req_indices=case["discard"])
    assert out == case["expected"] and lp is None


def test_synthetic_rates_kat():
    case = KATS["synthetic_rates"][0]
    assert np.allclose(unconditional_to_conditional_rates(case["rates"]), case["expected"])
    assert unconditional_to_conditional_rates([0.5, 0.0, 0.0]) == [0.5, 0.0, 0.0]


@pytest.mark.parametrize("case", KATS["invalid_draft_trim"], ids=lambda c: c["source"])
def test_invalid_draft_trim_kats(case):
    assert update_scheduler_for_invalid_drafts(case["drafts"], case["valid"]) == case["expected"]


def test_acceptance_stats():
    stats = stats_from_outputs([[1, 2, 3], [4], [5, 6], [7]], [2, 3, 1, 0], 3)
    assert stats.num_drafts == 3
    assert stats.num_draft_tokens == 6
    assert stats.num_accepted_tokens == 2 + 0 + 1
    assert stats.num_accepted_tokens_per_pos == [2, 1, 0]
    assert stats.num_draft_tokens_per_pos == [3, 2, 1]


def test_spec_decoding_logging_aggregates_steps():
    """SpecDecodingLogging (metrics.py:66-146): totals over the observed steps, per-position
    sums over lists of different lengths, rates from the totals, one log line, then a new
    interval; an empty interval reports empty totals without logging; observing copies."""
    from mvsd.spec_decode import SpecDecodingLogging, SpecDecodingStats

    lines = []
    agg = SpecDecodingLogging(log_fn=lambda fmt, *args: lines.append(fmt % args))
    assert agg.log() == {"num_drafts": 0, "num_draft_tokens": 0, "num_accepted_tokens": 0,
                         "accepted_tokens_per_pos": [], "draft_tokens_per_pos": [],
                         "acceptance_rate": None, "mean_acceptance_length": None}
    assert lines == [] and len(agg) == 0
    a = stats_from_outputs([[1, 2, 3], [4], [5, 6]], [2, 3, 1], 3)   # accepted 2, 0, 1
    b = SpecDecodingStats.new(4)
    b.observe_draft(4, 4)
    agg.observe(a)
    agg.observe(b)
    b.observe_draft(4, 1)                  # after observe: not counted
    assert len(agg) == 2
    got = agg.log()
    assert got["num_drafts"] == 4 and got["num_draft_tokens"] == 10
    assert got["num_accepted_tokens"] == 7
    assert got["accepted_tokens_per_pos"] == [3, 2, 1, 1]
    assert got["draft_tokens_per_pos"] == [4, 3, 2, 1]
    assert got["acceptance_rate"] == 0.7
    assert got["mean_acceptance_length"] == 1 + 7 / 4
    assert got["draft_throughput"] > 0 and got["accepted_throughput"] > 0
    assert len(lines) == 1 and "Mean acceptance length: 2.75" in lines[0]
    assert "Accepted: 7 tokens, Drafted: 10 tokens, Avg Draft acceptance rate: 70.0%" in lines[0]
    assert len(agg) == 0 and agg.log()["num_drafts"] == 0


def test_ngram_history_sync_copies_only_each_rows_history():
    """update_ngram_gpu_tensors_incremental (reference ngram_proposer_gpu.py:348-416) on CPU
    tensors: reordered rows move, new requests get their first n tokens in one batched copy,
    entries past n keep what the device buffer held, and every active row's length syncs."""
    from mvsd.spec_decode.ngram_proposer_gpu import update_ngram_gpu_tensors_incremental

    class Batch:
        pass

    batch = Batch()
    batch.token_ids_cpu = torch.tensor([[5, 6, 7, 8, 9], [1, 2, 0, 0, 0], [3, 3, 3, 4, 0]],
                                       dtype=torch.int32)
    batch.num_tokens_no_spec = torch.tensor([4, 2, 3], dtype=torch.int64)
    batch.req_id_to_index = {"a": 0, "b": 1, "c": 2}
    tokens = torch.full((3, 5), -7, dtype=torch.int32)
    lens = torch.zeros(3, dtype=torch.int32)
    update_ngram_gpu_tensors_incremental(batch, tokens, lens, {"a", "b", "c"}, None, "cpu")
    assert tokens.tolist() == [[5, 6, 7, 8, -7], [1, 2, -7, -7, -7], [3, 3, 3, -7, -7]]
    assert lens.tolist() == [4, 2, 3]
    # "c" moves to row 0, "a" to row 2, "d" is new in row 1 with an empty history
    batch.token_ids_cpu[1] = torch.tensor([0, 0, 0, 0, 0], dtype=torch.int32)
    batch.num_tokens_no_spec = torch.tensor([3, 0, 4], dtype=torch.int64)
    batch.req_id_to_index = {"c": 0, "d": 1, "a": 2}
    update_ngram_gpu_tensors_incremental(batch, tokens, lens, {"d"}, {"a": 0, "b": 1, "c": 2},
                                         "cpu")
    assert tokens[0].tolist() == [3, 3, 3, -7, -7] and tokens[2].tolist() == [5, 6, 7, 8, -7]
    assert tokens[1].tolist() == [1, 2, -7, -7, -7]  # nothing to copy for an empty history
    assert lens.tolist() == [3, 0, 4]


def test_block_method_is_refused():
    spec = type("S", (), {"rejection_sample_method": "block"})()
    with pytest.raises(NotImplementedError):
        RejectionSampler(sampler=object(), spec_config=spec)


def header_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(mvsd_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert "mvsd_rejection_sample" in names and "mvsd_ngram_propose" in names
    handle = ctypes.CDLL(str(nat.library_path()))
    for name in names:
        assert hasattr(handle, name), name
    assert set(names) == set(nat.SIGNATURES), "ctypes signatures out of sync with the header"
    assert nat.lib().mvsd_version() == (0 << 16) | (1 << 8)
    assert nat.lib().mvsd_status_string(-3) == b"workspace missing or too small"


def test_ctypes_struct_matches_c_layout(tmp_path):
    fields = [f for f, _ in nat.RejectionArgs._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
           'printf("%zu\\n", sizeof(mvsd_rejection_args));']
    src += [f'printf("%zu\\n", offsetof(mvsd_rejection_args, {f}));' for f in fields]
    src += ["return 0;}"]
    c = tmp_path / "probe.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-o", str(exe), str(c)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(nat.RejectionArgs)
    for f, off in zip(fields, got[1:]):
        assert getattr(nat.RejectionArgs, f).offset == off, f


def test_workspace_query():
    handle = nat.lib()
    small = handle.mvsd_rejection_workspace_bytes(4, 12, 151936, nat.F32, 3)
    big = handle.mvsd_rejection_workspace_bytes(256, 1024, 151936, nat.F32, 4)
    assert 0 < small < big
    assert handle.mvsd_rejection_workspace_bytes(-1, 0, 10, nat.F32, 1) == -1


def test_argument_validation_without_gpu():
    handle = nat.lib()
    args = nat.RejectionArgs()
    args.batch_size = 1
    args.vocab_size = 10
    args.max_spec_len = 200  # > MAX_SPEC_LEN
    assert handle.mvsd_rejection_sample(args, None) == -5
    args.max_spec_len = 1
    assert handle.mvsd_rejection_sample(args, None) == -1  # null output pointer
    assert handle.mvsd_ngram_propose(None, None, None, 0, 0, None, None, 0, 0, None, None, 0,
                                     1, 3, 2, 4, 0, 0, None) == -1  # min_n > max_n
    assert handle.mvsd_ngram_propose(None, None, None, 0, 0, None, None, 0, 0, None, None, 0,
                                     1, 1, 40, 4, 0, 0, None) == -5  # max_n > 32


def test_cpu_tensors_are_refused():
    sm = SamplingMetadata(temperature=None, all_greedy=True, all_random=False, top_k=None,
                          top_p=None)
    with pytest.raises(NotImplementedError):
        rejection_sample(torch.zeros(1, dtype=torch.int32), [1], 1,
                         torch.ones(1, dtype=torch.int32), None, torch.zeros((1, 4)),
                         torch.zeros((1, 1), dtype=torch.int32), sm)
    with pytest.raises(NotImplementedError):
        expand_batch_to_tokens(torch.zeros(2), torch.tensor([1, 2], dtype=torch.int32), 2)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nat, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(nat, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        nat.lib()
