"""Prompt-lookup drafter (E:1624-1628): the oracle against hand-worked cases, an independent
formulation (all windows at once, largest matching start) and the reference's bench prompts."""
import os

import numpy as np
import pytest
from numpy.lib.stride_tricks import sliding_window_view

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "prompts.npz")


def windows_lookup(seq, n, maxlen):
    """every start i <= L-n-1 whose n tokens equal the last n; drafts follow the largest one"""
    seq = np.asarray(seq, np.int64)
    L = seq.size
    if n <= 0 or L <= n:
        return []
    w = sliding_window_view(seq[:L - 1], n)  # starts 0 .. L-1-n
    hits = np.flatnonzero((w == seq[L - n:]).all(axis=1))
    if hits.size == 0:
        return []
    i = int(hits[-1])
    return seq[i + n:min(i + n + maxlen, L)].tolist()


# (seq, n, maxlen, drafts) worked by hand from the rule in E:1626-1627
HAND = [
    ([1, 2, 3, 4, 1, 2, 3, 9, 1, 2], 2, 3, [3, 9, 1]),   # two earlier "1 2": the later one (i=4) wins
    ([1, 2, 3, 4, 1, 2, 3, 9, 1, 2], 3, 3, []),          # "9 1 2" never occurred before
    ([1, 2, 3, 4, 1, 2, 3, 9, 1, 2], 1, 7, [3, 9, 1, 2]),  # last "2" at i=5, copy stops at L
    ([5, 6, 7, 5, 6], 2, 7, [7, 5, 6]),                  # truncated at the end of seq
    ([5, 5, 5], 2, 3, [5]),                              # overlapping occurrence i = 0
    ([5, 5], 2, 3, []),                                  # L <= n
    ([5, 5, 5], 0, 3, []),                               # n = 0: lookup off (NG_N > 0 test)
    ([7, 8, 7, 8], 2, 0, []),                            # maxlen 0
    ([], 1, 3, []),
    ([4, 4, 4, 4, 4], 1, 2, [4]),                        # i = L-2 is the most recent start
]


@pytest.mark.parametrize("case", range(len(HAND)))
def test_hand_cases(orc, case):
    seq, n, ml, want = HAND[case]
    assert windows_lookup(seq, n, ml) == want
    assert orc.prompt_lookup(np.array(seq, np.int32), n, ml).tolist() == want


def test_random_small_alphabet(orc):
    rng = np.random.default_rng(5)
    for trial in range(400):
        L = int(rng.integers(0, 200))
        seq = rng.integers(0, int(rng.integers(2, 6)), L).astype(np.int32)
        n = int(rng.integers(-1, 7))
        ml = int(rng.integers(0, 9))
        assert orc.prompt_lookup(seq, n, ml).tolist() == windows_lookup(seq, n, ml), (trial, L, n, ml)


def test_reference_prompts(orc):
    P = np.load(GOLD)
    hits = 0
    for name in P.files:
        seq = P[name]
        for L in sorted(set(np.linspace(0, seq.size, 40).astype(int).tolist())):
            for n in (1, 2, 3, 4, 8):
                d = orc.prompt_lookup(seq[:L], n, 7)
                assert d.tolist() == windows_lookup(seq[:L], n, 7), (name, L, n)
                hits += d.size > 0
    assert hits > 100  # real text repeats n-grams: the cases exercise the copy, not only misses
