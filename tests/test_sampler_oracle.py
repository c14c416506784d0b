"""Pins the sampler oracle (oracle_ngram_bans / oracle_sample) before it
checks the GPU sampler.

Known answers: the reference's sampler tests (sampler.rs:617-925), restated
case by case. Independent re-derivation: the ban set computed from the
definition of a repeated n-gram with Python slicing, on random short-vocab
sequences (many repeats), for windows 0 / small / large.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import pyoracle as O

INF = float("inf")


def samp(row, seq, n, w, white=()):
    st, tok, masked = O.sample(np.asarray(row, np.float32), np.asarray(seq, np.uint32), n, w, white)
    assert st == 0
    return tok, masked


def test_argmax_cases():
    assert samp([0.1, -2.0, 3.5, 3.4, 0.0], [], 35, 128)[0] == 2
    assert samp([0.0, 5.0, 1.0, 5.0], [], 0, 0)[0] == 1
    assert samp([math.nan, -INF, 2.0, 1.0], [], 0, 0)[0] == 2
    assert samp([math.nan] * 3, [], 0, 0)[0] == 0
    assert O.sample(np.zeros(0, np.float32), np.zeros(0, np.uint32), 0, 0)[0] == -1


def test_ngram_known_answers():
    assert samp([10.0, 5.0, 5.0], [0, 0], 1, 8)[0] == 1
    assert samp([0.0, 0.0, 0.0, 9.0, 1.0], [7, 3, 7], 2, 16)[0] == 4
    assert samp([9.0, 1.0, 0.0], [5, 0, 5], 2, 0)[0] == 1
    assert samp([3.0, 2.0, 1.0], [0, 1, 2], 1, 8)[0] == 0  # all banned -> lowest -inf index
    assert samp([0.0, 0.0, 9.0, 0.0], [1, 2, 9], 2, 16)[0] == 2
    tok, m = samp([0.0, 0.0, 9.0, 1.0], [0, 2, 0], 2, 16)
    assert tok == 3 and m[2] == -INF and m[3] == 1.0
    assert samp([0.0] * 5 + [9.0], [5, 0, 5], 2, 2)[0] == 5
    assert samp([9.0, 0.0, 0.0], [0, 0, 0], 35, 128)[0] == 0
    _, m = samp([1.0, 2.0, 3.0], [99, 99], 1, 8)
    assert m.tolist() == [1.0, 2.0, 3.0]
    _, m = samp([1.0, 2.0, 3.0], [1, 1], 1, 8, white=[1])
    assert m.tolist() == [1.0, 2.0, 3.0]
    _, m = samp([0.0, 0.0, 0.0], [0, 2, 0], 2, 16)
    assert m.tolist() == [0.0, 0.0, -INF]


def _repeat_35gram_sequence(total_len):
    # sampler.rs:567-582
    prefix = list(range(20, 54))
    seq = prefix + [7] + [99] * (total_len - 69) + prefix
    assert len(seq) == total_len
    return seq


@pytest.mark.parametrize("window,cases", [(128, [(127, 6), (128, 6), (129, 7)]),
                                          (1024, [(1023, 6), (1024, 6), (1025, 7)])])
def test_ngram_35_window_boundaries(window, cases):
    row = np.zeros(128, np.float32)
    row[7], row[6] = 10.0, 9.0
    for total, want in cases:
        assert samp(row, _repeat_35gram_sequence(total), 35, window)[0] == want


def _brute_bans(seq, n, w, vocab, white=()):
    L = len(seq)
    if n == 0 or L < n:
        return set()
    start = 0 if w == 0 else max(0, L - w)
    pre = seq[L - (n - 1):] if n > 1 else []
    out = set()
    for i in range(start, L - n + 1):
        gram = seq[i:i + n]
        if gram[:-1] == pre and gram[-1] not in white and gram[-1] < vocab:
            out.add(gram[-1])
    return out


def test_bans_match_definition_on_random_sequences():
    rng = np.random.default_rng(5)
    for it in range(400):
        vocab = int(rng.integers(2, 9))
        L = int(rng.integers(0, 300))
        seq = rng.integers(0, vocab + 2, L).tolist()  # ids >= vocab exercise the range check
        n = int(rng.integers(0, 6))
        w = int(rng.choice([0, 1, 3, 8, 50, 1000]))
        white = rng.integers(0, vocab, int(rng.integers(0, 3))).tolist()
        got = O.ngram_bans(seq, n, w, vocab, white)
        assert set(got.tolist()) == _brute_bans(seq, n, w, vocab, white), (it, n, w)
        tok, m = samp(rng.standard_normal(vocab).astype(np.float32), seq, n, w, white)
        banned = _brute_bans(seq, n, w, vocab, white)
        assert all(m[b] == -INF for b in banned)
        if len(banned) < vocab:
            assert tok not in banned
