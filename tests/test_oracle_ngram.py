"""Pin the ngram oracle (oracle/ngram.c) to the reference.

  * the reference's KATs (tests/golden/reference_kats.json, from tests/step60/);
  * the KMP restatement against the brute-force definition on random histories, including
    the 40 random cases the reference generates with default_rng(0) (tests/step60/
    test_ngram.py:54-61), whose expectations the reference took from upstream vLLM;
  * the brute force against a pure-Python definition on tiny inputs.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import ngram

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())

FIXED_CASES = [
    ([1, 2, 3, 1, 2, 9, 1, 2], 2, 2, 4),
    ([1, 2, 3, 4, 1, 2, 3, 4, 1, 2, 3], 3, 3, 2),
    ([5, 5, 5, 5, 5, 5], 2, 5, 3),
    ([7, 8, 9, 1, 2, 3, 7, 8, 9], 3, 5, 2),
    ([7, 8, 9, 1, 2, 3, 7, 8, 9], 5, 6, 2),
    ([1, 2], 5, 5, 3),
    ([1, 2, 3], 1, 3, 4),
    ([9, 9, 9, 1, 9, 9, 9], 3, 3, 4),
    ([4, 1, 2, 3, 4, 1, 2], 1, 1, 3),
]


def reference_random_cases():
    """The same generator calls as tests/step60/test_ngram.py:54-61."""
    rng = np.random.default_rng(0)
    cases = []
    for _ in range(40):
        length = int(rng.integers(1, 40))
        vocab = int(rng.integers(2, 6))
        tokens = rng.integers(0, vocab, size=length).tolist()
        lo, hi = sorted((int(rng.integers(1, 4)), int(rng.integers(1, 6))))
        cases.append((tokens, lo, hi, int(rng.integers(1, 6))))
    return cases


ALL_CASES = FIXED_CASES + reference_random_cases()


@pytest.mark.parametrize("case", KATS["ngram_cpu"], ids=lambda c: c["source"])
def test_kmp_matches_reference_kats(case):
    got = ngram.find_kmp(case["tokens"], case["min_n"], case["max_n"], case["max_model_len"],
                         case["k"])
    assert got == case["expected"]


@pytest.mark.parametrize("case", KATS["ngram_device"], ids=lambda c: c["source"])
def test_device_semantics_kats(case):
    drafts, valid = ngram.find_brute_device(case["history"], case["min_n"], case["max_n"],
                                            case["k"])
    assert drafts == case["expected"] and valid == case["num_valid"]


@pytest.mark.parametrize("tokens,min_n,max_n,k", ALL_CASES)
def test_kmp_equals_brute_force(tokens, min_n, max_n, k):
    for mml in (10 ** 9, len(tokens) + 2, len(tokens)):
        assert (ngram.find_kmp(tokens, min_n, max_n, mml, k)
                == ngram.find_brute_cpu(tokens, min_n, max_n, mml, k)), (tokens, min_n, max_n, mml)


def test_brute_force_matches_python_definition():
    rng = np.random.default_rng(11)
    for _ in range(3000):
        L = int(rng.integers(0, 30))
        tokens = rng.integers(0, 3, size=L).tolist()
        lo = int(rng.integers(1, 4))
        hi = lo + int(rng.integers(0, 4))
        k = int(rng.integers(1, 6))
        s, n = ngram.find_python(tokens, lo, hi, k)
        drafts, valid = ngram.find_brute_device(tokens, lo, hi, k)
        expect = [] if s < 0 else tokens[s + n: s + n + k]
        assert drafts[:len(expect)] == expect and valid == len(expect)
        assert all(d == -1 for d in drafts[len(expect):])


def test_kmp_equals_brute_force_large_random():
    rng = np.random.default_rng(12)
    R, L = 64, 600
    tokens = rng.integers(0, 8, size=(R, L)).astype(np.int32)
    lens = rng.integers(0, L + 1, size=R).astype(np.int32)
    for lo, hi in ((1, 1), (2, 5), (3, 3), (1, 8)):
        d1, c1 = ngram.kmp_batch(tokens, lens, lo, hi, 10 ** 9, 5)
        for r in range(R):
            assert d1[r, :c1[r]].tolist() == ngram.find_brute_cpu(tokens[r, :lens[r]], lo, hi,
                                                                  10 ** 9, 5)


def test_valid_sampled_tokens_reference_kat():
    """tests/step60/test_ngram_gpu_state.py:157-179: row 0 discarded, 99 >= vocab 10 does not
    count, the discarded row falls back to its history's last token."""
    nxt, counts, valid = ngram.valid_sampled_tokens([[7, 8], [5, 99]], [True, False],
                                                    [[1, 2, 3, 0], [4, 5, 6, 0]], [3, 3], 10)
    assert counts.tolist() == [0, 1]
    assert valid.tolist() == [[-1, -1], [5, 99]]
    assert nxt.tolist() == [3, 5]


def test_valid_sampled_tokens_by_definition():
    """Row by row with plain loops: the count skips -1 and ids >= vocab wherever they sit, and
    the next token is the entry at column count - 1 (not the last valid entry)."""
    rng = np.random.default_rng(8)
    sampled = rng.integers(-1, 14, (40, 5))
    discard = rng.random(40) < 0.2
    tokens = rng.integers(0, 10, (40, 9))
    lens = rng.integers(0, 10, 40)
    nxt, counts, valid = ngram.valid_sampled_tokens(sampled, discard, tokens, lens, 10)
    for i in range(40):
        row = [-1] * 5 if discard[i] else list(sampled[i])
        c = sum(1 for v in row if v != -1 and v < 10)
        assert valid[i].tolist() == row and counts[i] == c
        assert nxt[i] == (row[c - 1] if c else tokens[i, max(lens[i] - 1, 0)])
