"""GPU parity of the ngram proposers (libmvsd.so, mvsd_ngram_propose) against the reference's
KATs and the C oracle; drafts and valid counts must be bit-exact."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from mvsd.spec_decode.ngram_proposer import NgramProposer
from mvsd.spec_decode.ngram_proposer_gpu import (NgramGPUKernel, NgramProposerGPU,
                                                 ngram_propose_device,
                                                 update_ngram_gpu_tensors_incremental)
from mvsd.spec_decode.utils import TargetRows
from mvsd.testing import configs
from oracle import ngram as ong

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


class Cfg:
    def __init__(self, k=3, min_n=2, max_n=4, max_model_len=64, max_num_seqs=4):
        self.speculative_config = type("SC", (), dict(
            num_speculative_tokens=k, prompt_lookup_min=min_n, prompt_lookup_max=max_n))()
        self.model_config = type("M", (), {"max_model_len": max_model_len})()
        self.scheduler_config = type("S", (), {"max_num_seqs": max_num_seqs})()


class FakeInputBatch:
    def __init__(self, histories, max_model_len, vocab_size=1000, max_num_reqs=None):
        self.max_num_reqs = max_num_reqs or max(len(histories), 1)
        self.vocab_size = vocab_size
        self.token_ids_cpu = torch.zeros((self.max_num_reqs, max_model_len), dtype=torch.int32)
        self.num_tokens_no_spec = torch.zeros(self.max_num_reqs, dtype=torch.int64)
        self.req_ids = []
        self.req_id_to_index = {}
        for i, tokens in enumerate(histories):
            self.set_row(i, tokens, f"r{i}")

    def set_row(self, index, tokens, req_id=None):
        self.token_ids_cpu[index].zero_()
        self.token_ids_cpu[index, :len(tokens)] = torch.tensor(tokens, dtype=torch.int32)
        self.num_tokens_no_spec[index] = len(tokens)
        if req_id is not None:
            while len(self.req_ids) <= index:
                self.req_ids.append(None)
            self.req_ids[index] = req_id
            self.req_id_to_index = {r: i for i, r in enumerate(self.req_ids) if r is not None}

    @property
    def num_reqs(self):
        return sum(1 for r in self.req_ids if r is not None)


def state(histories, max_model_len, device, rows=None):
    rows = rows or len(histories)
    tokens = torch.zeros((rows, max_model_len), dtype=torch.int32, device=device)
    lens = torch.zeros(rows, dtype=torch.int32, device=device)
    for i, h in enumerate(histories):
        tokens[i, :len(h)] = torch.tensor(h, dtype=torch.int32)
        lens[i] = len(h)
    return tokens, lens


@pytest.mark.parametrize("case", KATS["ngram_device"], ids=lambda c: c["source"])
def test_device_kats(case, device):
    kernel = NgramGPUKernel(Cfg(k=case["k"], min_n=case["min_n"], max_n=case["max_n"]))
    tokens, lens = state([case["history"]], 64, device)
    drafts, valid = kernel(lens, tokens, torch.ones(1, dtype=torch.bool, device=device))
    assert drafts[0].tolist() == case["expected"]
    assert int(valid[0]) == case["num_valid"]


def test_scatter_kat_and_read_only_lengths(device):
    case = KATS["ngram_scatter"][0]
    prop = NgramProposerGPU(Cfg(k=case["k"], min_n=case["min_n"], max_n=case["max_n"]), device)
    tokens, lens = state([case["history"]], case["max_model_len"], device)
    before = lens.clone()
    sampled = torch.tensor([case["sampled"]], dtype=torch.int32, device=device)
    counts = torch.tensor([case["count"]], dtype=torch.int32, device=device)
    drafts, valid = prop.propose(case["k"], lens, tokens, sampled, counts)
    n = len(case["history_after_prefix"])
    assert tokens[0, :n].tolist() == case["history_after_prefix"]
    assert tokens[0, n:].abs().sum().item() == 0
    assert torch.equal(lens, before)
    assert drafts[0].tolist() == case["expected"] and int(valid[0]) == case["num_valid"]


def test_temp_length_is_used_for_matching(device):
    prop = NgramProposerGPU(Cfg(k=2, min_n=2, max_n=2), device)
    tokens, lens = state([[3, 4, 3, 4, 3, 4]], 64, device)
    drafts, valid = prop.propose(2, lens, tokens, torch.tensor([[3, 4]], dtype=torch.int32,
                                                               device=device),
                                 torch.tensor([2], dtype=torch.int32, device=device))
    assert drafts[0].tolist() == [3, 4] and int(valid[0]) == 2


def test_fixed_k_is_asserted(device):
    prop = NgramProposerGPU(Cfg(k=3), device)
    tokens, lens = state([[1, 2, 1, 2]], 64, device)
    with pytest.raises(AssertionError):
        prop.propose(2, lens, tokens, torch.tensor([[1]], dtype=torch.int32, device=device),
                     torch.tensor([1], dtype=torch.int32, device=device))


def test_update_token_ids_and_masked_scatter(device):
    """tests/step60/test_ngram_gpu_state.py:157-179"""
    prop = NgramProposerGPU(Cfg(k=2), device)
    batch = FakeInputBatch([[1, 2, 3], [4, 5, 6]], 64, vocab_size=10)
    tokens, lens = state([[1, 2, 3], [4, 5, 6]], 64, device)
    sampled = torch.tensor([[7, 8], [5, 99]], dtype=torch.int32, device=device)
    discard = torch.tensor([True, False], device=device)
    nxt, counts, valid_ids = prop.update_token_ids_ngram(sampled, batch, tokens, lens, discard)
    assert counts.tolist() == [0, 1]
    assert valid_ids[0].tolist() == [-1, -1] and valid_ids[1].tolist() == [5, 99]
    assert nxt.tolist() == [3, 5]
    prop.propose(2, lens[:2], tokens[:2], valid_ids, counts)
    assert tokens[1, :7].tolist() == [4, 5, 6, 5, 0, 0, 0]


@pytest.mark.parametrize("num_reqs,width", [(1, 1), (37, 5), (1024, 8)])
def test_valid_sampled_tokens_match_oracle(device, num_reqs, width):
    """update_token_ids_ngram (one mvsd_ngram_valid_sampled launch) equals oracle/ngram.py's
    restatement: -1 and ids >= vocab anywhere in a row, discarded rows, empty histories, and
    sampled rows given as a list of ragged lists."""
    rng = np.random.default_rng(num_reqs * 10 + width)
    vocab = 50
    histories = [list(rng.integers(0, vocab, int(rng.integers(0, 12)))) for _ in range(num_reqs)]
    batch = FakeInputBatch(histories, 16, vocab_size=vocab)
    tokens, lens = state(histories, 16, device)
    sampled = rng.integers(-1, vocab + 5, (num_reqs, width)).astype(np.int32)
    discard = rng.random(num_reqs) < 0.25
    prop = NgramProposerGPU(Cfg(k=2), device)
    nxt, counts, valid = prop.update_token_ids_ngram(
        torch.from_numpy(sampled).to(device), batch, tokens, lens,
        torch.from_numpy(discard).to(device))
    want = ong.valid_sampled_tokens(sampled, discard, tokens.cpu().numpy(), lens.cpu().numpy(),
                                      vocab)
    assert nxt.cpu().tolist() == want[0].tolist()
    assert counts.cpu().tolist() == want[1].tolist()
    assert valid.cpu().tolist() == want[2].tolist()
    # ragged lists: padded with -1 to the longest row
    ragged = [list(rng.integers(0, vocab, int(rng.integers(0, width + 1)))) for _ in
              range(num_reqs)]
    nxt, counts, valid = prop.update_token_ids_ngram(ragged, batch, tokens, lens,
                                                     torch.from_numpy(discard).to(device))
    w = max(max(len(r) for r in ragged), 1)
    padded = np.array([r + [-1] * (w - len(r)) for r in ragged], dtype=np.int32)
    want = ong.valid_sampled_tokens(padded, discard, tokens.cpu().numpy(), lens.cpu().numpy(),
                                      vocab)
    assert nxt.cpu().tolist() == want[0].tolist()
    assert counts.cpu().tolist() == want[1].tolist()


def test_history_follows_request_ids_across_reorder(device):
    """tests/step60/test_ngram_gpu_state.py:182-225"""
    prop = NgramProposerGPU(Cfg(k=2, min_n=1, max_n=1), device)
    batch = FakeInputBatch([], 64, max_num_reqs=4)
    tokens = torch.zeros((4, 64), dtype=torch.int32, device=device)
    lens = torch.zeros(4, dtype=torch.int32, device=device)

    def rebuild(rows, prev, new_ids):
        batch.req_ids = [r for r, _ in rows]
        batch.req_id_to_index = {r: i for i, (r, _) in enumerate(rows)}
        for i, (r, t) in enumerate(rows):
            batch.set_row(i, t, r)
        update_ngram_gpu_tensors_incremental(batch, tokens, lens, new_ids, prev, device)
        return {r: i for i, (r, _) in enumerate(rows)}

    s = rebuild([("A", [1, 1, 1]), ("B", [2, 2, 2]), ("C", [3, 3, 3])], None, {"A", "B", "C"})
    rebuild([("C", [3, 3, 3]), ("A", [1, 1, 1])], s, set())
    assert tokens[0, :3].tolist() == [3, 3, 3] and tokens[1, :3].tolist() == [1, 1, 1]
    rebuild([("D", [4, 4, 4, 4]), ("C", [3, 3, 3]), ("A", [1, 1, 1])], {"C": 0, "A": 1}, {"D"})
    assert lens[:3].tolist() == [4, 3, 3]
    sampled = torch.tensor([[4, -1], [-1, -1], [-1, -1]], dtype=torch.int32, device=device)
    counts = torch.tensor([1, 0, 0], dtype=torch.int32, device=device)
    drafts, valid = prop.propose(2, lens[:3], tokens[:3], sampled, counts)
    assert drafts[0].tolist() == [4, 4] and int(valid[0]) == 2
    assert int(valid[1]) == 0 and int(valid[2]) == 0


def test_partially_filled_batch_leaves_free_rows(device):
    prop = NgramProposerGPU(Cfg(k=2, min_n=1, max_n=1, max_num_seqs=4), device)
    histories = [[1, 2, 1, 2], [3, 4, 3, 4]]
    batch = FakeInputBatch(histories, 64, max_num_reqs=4)
    tokens, lens = state(histories, 64, device, rows=4)
    free = tokens[2:].clone()
    rows = [TargetRows(f"r{i}", i, 0, 1, 0, len(h), h[-1], True) for i, h in enumerate(histories)]
    out = prop.propose_drafts(rows, {}, input_batch=batch, sampled_by_row={0: [5], 1: [6]},
                              sample_rows=[0, 1], token_ids_gpu=tokens, num_tokens_no_spec_gpu=lens)
    assert out.req_ids == ["r0", "r1"] and len(out.draft_token_ids) == 2
    assert tokens[0, 4].item() == 5 and tokens[1, 4].item() == 6
    assert torch.equal(tokens[2:], free)


@pytest.mark.parametrize("case", KATS["ngram_cpu"], ids=lambda c: c["source"])
def test_host_api_kats(case, device):
    tokens = case["tokens"]
    prop = NgramProposer(Cfg(k=case["k"], min_n=case["min_n"], max_n=case["max_n"],
                             max_model_len=case["max_model_len"], max_num_seqs=1), device)
    buf = np.zeros((1, max(len(tokens), 1)), dtype=np.int32)
    buf[0, :len(tokens)] = tokens
    got = prop.batch_propose(1, [0], np.array([len(tokens)]), buf, case["k"])
    assert got == [case["expected"]]


@pytest.mark.parametrize("case", KATS["ngram_propose"], ids=lambda c: c["source"])
def test_host_api_propose_kats(case, device):
    prop = NgramProposer(Cfg(k=case["k"], min_n=case["min_n"], max_n=case["max_n"],
                             max_model_len=case["max_model_len"], max_num_seqs=4), device)
    batch = FakeInputBatch(case["histories"], case["max_model_len"])
    lens = batch.num_tokens_no_spec.numpy().copy()
    if case["lengths_override"]:
        lens[:] = case["lengths_override"]
    got = prop.propose(case["k"], case["sampled"], lens, batch.token_ids_cpu.numpy())
    assert got == case["expected"]


def test_propose_drafts_protocol(device):
    histories = [[1, 2, 1, 2, 1, 2], [3, 3, 3, 3, 3, 3]]
    all_ids = {f"r{i}": h for i, h in enumerate(histories)}
    prop = NgramProposer(Cfg(k=2, min_n=2, max_n=2), device)
    rows = [TargetRows(f"r{i}", i, 0, 1, 0, len(h), h[-1], True) for i, h in enumerate(histories)]
    out = prop.propose_drafts(rows, all_ids)
    assert out.draft_token_ids == [[1, 2], [3, 3]] and out.num_valid_draft_tokens is None
    short = [TargetRows("r0", 0, 0, 1, 0, 2, 2, True), rows[1]]
    assert prop.propose_drafts(short, all_ids).draft_token_ids[0] == []
    not_ready = [TargetRows("r0", 0, 0, 1, 0, 6, 2, False), rows[1]]
    assert prop.propose_drafts(not_ready, all_ids).draft_token_ids[0] == []
    assert prop.propose_drafts(rows, all_ids, num_speculative_tokens=0).draft_token_ids == [[], []]


@pytest.mark.parametrize("suffix_copies", [False, True], ids=["c3", "c3_suffix_copies"])
def test_c3_full_size_bit_exact(device, suffix_copies):
    """C3 as generated: its copied spans never cover a history's last token, so no suffix
    repeats and every request scans its whole history without a match.  With suffix_copies,
    every other history ends with a copy of an earlier span of 8-64 tokens, so those requests
    find a match of max_n and stop early."""
    tokens = configs.ngram_c3(device, suffix_copies=suffix_copies)
    B, L = tokens.shape
    lens = torch.full((B,), L, dtype=torch.int32, device=device)
    drafts, valid = ngram_propose_device(tokens, lens, min_n=2, max_n=5, k=5)
    exp_d, exp_v = ong.brute_device_batch(tokens.cpu().numpy(), lens.cpu().numpy(), 2, 5, 5)
    assert np.array_equal(drafts.cpu().numpy(), exp_d)
    assert np.array_equal(valid.cpu().numpy(), exp_v)
    print(f"[c3 suffix_copies={suffix_copies}] rows with drafts: {(exp_v > 0).sum()}/{B}",
          flush=True)
    if suffix_copies:
        assert (exp_v[0::2] == 5).all()
    # host API with the max_model_len cap = the reference's CPU KMP, bit-exact
    d2, c2 = ngram_propose_device(tokens, lens, min_n=2, max_n=5, k=5, cap_by_model_len=True,
                                  max_model_len=8192)
    kd, kc = ong.kmp_batch(tokens.cpu().numpy(), lens.cpu().numpy(), 2, 5, 8192, 5)
    assert np.array_equal(c2.cpu().numpy(), kc)
    for r in range(B):
        assert d2[r, :kc[r]].tolist() == kd[r, :kc[r]].tolist()


def test_host_api_c3_twice_with_smaller_batch(device):
    """NgramProposer.propose from pageable numpy histories at the C3 size (ragged lengths,
    some requests inactive) equals the reference CPU KMP; a second, smaller call reuses the
    pinned staging buffers and is exact too."""
    tokens = configs.ngram_c3(device).cpu().numpy()
    B, L = tokens.shape
    rng = np.random.default_rng(5)
    prop = NgramProposer(Cfg(k=5, min_n=2, max_n=5, max_model_len=8192, max_num_seqs=B),
                         device)
    for n, k in ((B, 5), (B // 3, 3)):
        lens = rng.integers(1, L + 1, size=n).astype(np.int32)
        sampled = [[1] if rng.random() < 0.8 else [] for _ in range(n)]
        got = prop.propose(k, sampled, lens, tokens[:n])
        kd, kc = ong.kmp_batch(tokens[:n], lens, 2, 5, 8192, k)
        for r in range(n):
            expect = kd[r, :kc[r]].tolist() if sampled[r] else []
            assert got[r] == expect, (n, r)


@pytest.mark.parametrize("lo,hi,vocab", [(1, 1, 3), (2, 5, 4), (3, 3, 2), (1, 8, 5), (4, 32, 2)])
def test_random_histories_vs_brute_force(device, lo, hi, vocab):
    rng = np.random.default_rng(lo * 100 + hi)
    R, W = 96, 9000
    tokens = rng.integers(0, vocab, size=(R, W)).astype(np.int32)
    lens = rng.integers(0, W + 1, size=R).astype(np.int32)
    lens[:8] = [0, 1, 2, lo, hi, hi + 1, 4096, 4097]
    t = torch.from_numpy(tokens).to(device)
    ln = torch.from_numpy(lens).to(device)
    for k in (1, 5, 17):
        d, v = ngram_propose_device(t, ln, min_n=lo, max_n=hi, k=k)
        ed, ev = ong.brute_device_batch(tokens, lens, lo, hi, k)
        assert np.array_equal(d.cpu().numpy(), ed) and np.array_equal(v.cpu().numpy(), ev)
        d, c = ngram_propose_device(t, ln, min_n=lo, max_n=hi, k=k, cap_by_model_len=True,
                                    max_model_len=W + 3)
        kd, kc = ong.kmp_batch(tokens, lens, lo, hi, W + 3, k)
        assert np.array_equal(c.cpu().numpy(), kc)
        for r in range(R):
            assert d[r, :kc[r]].tolist() == kd[r, :kc[r]].tolist()


def test_unique_tokens_have_no_drafts_and_long_histories_tile(device):
    # no repeats at all -> no drafts; a single early repeat in a 20000-token history is found
    L = 20000
    base = np.arange(L, dtype=np.int32)
    base[100:103] = base[L - 3:]
    t = torch.from_numpy(np.stack([np.arange(L, dtype=np.int32), base])).to(device)
    ln = torch.tensor([L, L], dtype=torch.int32, device=device)
    d, v = ngram_propose_device(t, ln, min_n=2, max_n=3, k=4)
    assert v.tolist() == [0, 4]
    assert d[1].tolist() == [103, 104, 105, 106]
