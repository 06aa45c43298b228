"""GPU parity of the prompt-lookup drafter (E:1624-1628) with the history on the device:
every round appends the committed tokens and drafts in one launch; drafts and the stored
history must equal the oracle's on the same sequence."""
import os

import numpy as np
import pytest

from conftest import note

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "prompts.npz")


def rounds(dev, orc, seq0, gen, n, maxlen, rng):
    """feed `gen` in rounds of 1..8 committed tokens; compare each round's drafts"""
    dev.history_set(seq0)
    seq = list(seq0)
    p = 0
    nhit = 0
    while p < len(gen):
        k = int(rng.integers(1, 9))
        app = gen[p:p + k]
        p += len(app)
        seq += list(app)
        got = dev.prompt_lookup(n, maxlen, app)
        want = orc.prompt_lookup(np.array(seq, np.int32), n, maxlen)
        assert got.tolist() == want.tolist(), (len(seq), n, maxlen)
        nhit += got.size > 0
    assert dev.history().tolist() == seq
    return nhit


def test_reference_prompts(orc, dev):
    P = np.load(GOLD)
    rng = np.random.default_rng(3)
    for name in P.files:
        seq = P[name]
        for n in (1, 2, 3, 4):
            note(f"prompt lookup {name} L={seq.size} n={n}")
            cut = seq.size // 2
            rounds(dev, orc, seq[:cut], seq[cut:].tolist(), n, 7, rng)


def test_motif_prompt_6841(orc, dev):
    """the long-prompt workload: a seeded 64-token motif repeated to 6,841 ids plus uniform noise"""
    rng = np.random.default_rng(11)
    motif = rng.integers(0, 262144, 64)
    seq = np.resize(motif, 6841).astype(np.int32)
    noise = rng.random(6841) < 0.05
    seq[noise] = rng.integers(0, 262144, int(noise.sum()))
    gen = np.resize(motif, 300).astype(np.int32)
    for n in (2, 3, 5):
        note(f"prompt lookup motif 6841 n={n}")
        assert rounds(dev, orc, seq, gen.tolist(), n, 7, rng) > 0


def test_random_small_alphabet(orc, dev):
    rng = np.random.default_rng(7)
    for trial in range(60):
        a = int(rng.integers(2, 8))
        L0 = int(rng.integers(0, 3000))
        seq = rng.integers(0, a, L0).astype(np.int32)
        gen = rng.integers(0, a, int(rng.integers(1, 60))).tolist()
        n = int(rng.integers(-1, 9))
        ml = int(rng.integers(0, 17))
        note(f"prompt lookup random trial {trial} L0={L0} n={n} maxlen={ml}")
        rounds(dev, orc, seq, gen, n, ml, rng)


def test_long_ngram_and_growth(orc, dev):
    """n up to 256 (the LDS tail), and a history that outgrows its first allocation"""
    rng = np.random.default_rng(9)
    block = rng.integers(0, 1000, 300).astype(np.int32)
    seq = np.concatenate([block, rng.integers(0, 1000, 5000).astype(np.int32), block[:280]])
    for n in (200, 256):
        note(f"prompt lookup long n-gram n={n}")
        dev.history_set(seq)
        got = dev.prompt_lookup(n, 16)
        want = orc.prompt_lookup(seq, n, 16)
        assert got.tolist() == want.tolist() == block[280:296].tolist()  # i* = 280 - n in the first block
    note("prompt lookup growth past 4096 + 5580 tokens")
    dev.history_set(seq)
    big = rng.integers(0, 50, 20000).tolist()
    full = list(seq)
    for i in range(0, len(big), 16):
        full += big[i:i + 16]
        got = dev.prompt_lookup(3, 5, big[i:i + 16])
        assert got.tolist() == orc.prompt_lookup(np.array(full, np.int32), 3, 5).tolist()
    assert dev.history().tolist() == full


def test_argument_errors(dev):
    dev.history_set(np.arange(10))
    note("prompt lookup argument errors")
    with pytest.raises(RuntimeError):
        dev.prompt_lookup(2, 3, list(range(17)))  # more than 16 appended tokens
    with pytest.raises(RuntimeError):
        dev.prompt_lookup(257, 3)
    with pytest.raises(RuntimeError):
        dev.prompt_lookup(2, 17)
    assert dev.history().tolist() == list(range(10))  # a refused call leaves the history alone
