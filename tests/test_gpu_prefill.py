"""GPU parity of the prefill (E:1594-1599, ENGINE_PREFILL_INT8=1) and of the speculative decode
loop that follows it (prompt lookup E:1624-1628 + verify E:1648-1661), against the oracle:
the last row's final-normed hidden state, every layer's KV rows, the first generated token,
and the committed tokens of every round are bit-identical."""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

# (n, NL, ctx, pfb, pos0): run_mh blocks (< 64), attn_tile blocks, a 4-row split-KV tail (196),
# 1-row exact-float tails on both sides of ATT_PAR (193: split-KV, 65: run_mh), a 2-row run_mh
# tail (34), a prompt past the 512 window (600), a block of 16 and a prompt after earlier context
CASES = [(34, 2, 256, 32, 0), (100, 2, 256, 32, 0), (193, 2, 256, 32, 0), (196, 5, 256, 32, 0),
         (65, 1, 256, 32, 0), (600, 1, 640, 32, 0), (100, 2, 256, 16, 0), (150, 2, 256, 32, 40)]


@pytest.mark.parametrize("n,NL,ctx,pfb,pos0", CASES)
def test_prefill_matches_oracle(orc, g4v, n, NL, ctx, pfb, pos0):
    from oracle import Model
    V, I, seed = 4096, 512, 31
    rng = np.random.default_rng(n + 7 * pos0)
    toks = rng.integers(0, V, n).astype(np.int32)
    note(f"prefill n={n} NL={NL} ctx={ctx} pfb={pfb} pos0={pos0}")
    dev = g4v.Device(0)
    om = Model(orc, seed, V, NL, I, ctx)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        if pos0:
            dev.fake_ctx(pos0, 999)
            om.fake_ctx(pos0, 999)
        g0, hd = dev.prefill(toks, pos0=pos0, pfb=pfb, hidden=True)
        ho = om.prefill(toks, pos0=pos0, pfb=pfb)
        assert same(hd, ho), first_diff(hd, ho)
        for what in ("KC", "VC"):
            a = dev.read(what, np.uint16).reshape(NL, -1, 256)[:, :pos0 + n]
            b = om.get(what, np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)[:, :pos0 + n]
            assert same(a, b), (what, first_diff(a.ravel(), b.ravel()))
        G, _, _ = dev.head_argmax(ho[None, :])
        assert g0 == G[0]
    finally:
        om.close()
        dev.close()


# exact-float prefill (ENGINE_PREFILL_INT8 unset, the engine's default: E:1210, 1363): the same
# block paths with every product in exact float, pfb 1 included
EXACT_CASES = [(100, 2, 256, 32, 0), (196, 3, 256, 32, 0), (193, 2, 256, 32, 0), (70, 1, 128, 1, 0),
               (150, 2, 256, 16, 40)]


@pytest.mark.parametrize("n,NL,ctx,pfb,pos0", EXACT_CASES)
def test_prefill_exact_float_matches_oracle(orc, g4v, n, NL, ctx, pfb, pos0):
    from oracle import Model
    V, I, seed = 4096, 512, 31
    rng = np.random.default_rng(n + 7 * pos0 + pfb)
    toks = rng.integers(0, V, n).astype(np.int32)
    note(f"exact-float prefill n={n} NL={NL} ctx={ctx} pfb={pfb} pos0={pos0}")
    dev = g4v.Device(0)
    om = Model(orc, seed, V, NL, I, ctx)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        dev.set_prefill_int8(False)
        if pos0:
            dev.fake_ctx(pos0, 999)
            om.fake_ctx(pos0, 999)
        g0, hd = dev.prefill(toks, pos0=pos0, pfb=pfb, hidden=True)
        ho = om.prefill(toks, pos0=pos0, pfb=pfb, i8=False)
        assert same(hd, ho), first_diff(hd, ho)
        for what in ("KC", "VC"):
            a = dev.read(what, np.uint16).reshape(NL, -1, 256)[:, :pos0 + n]
            b = om.get(what, np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)[:, :pos0 + n]
            assert same(a, b), (what, first_diff(a.ravel(), b.ravel()))
    finally:
        om.close()
        dev.close()


def test_prefill_then_lookup_decode(orc, g4v):
    """a motif prompt, then rounds of prompt-lookup drafts verified as a chain (E:1617-1661)"""
    from oracle import Model
    V, NL, I, ctx, seed = 4096, 2, 512, 512, 9
    rng = np.random.default_rng(4)
    motif = rng.integers(0, V, 16)
    prompt = np.resize(motif, 120).astype(np.int32)
    note("prefill + 24 lookup/verify rounds")
    dev = g4v.Device(0)
    om = Model(orc, seed, V, NL, I, ctx)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        g0 = dev.prefill(prompt)
        ho = om.prefill(prompt)
        G, _, _ = dev.head_argmax(ho[None, :])
        assert g0 == G[0]
        gen = [g0]
        dev.history_set(np.concatenate([prompt, [g0]]))
        P = len(prompt) - 1
        app = []
        for rnd in range(24):
            drafts = dev.prompt_lookup(3, 3, app)
            seq = np.concatenate([prompt, gen]).astype(np.int32)
            assert drafts.tolist() == orc.prompt_lookup(seq, 3, 3).tolist()
            block = np.array([gen[-1]] + drafts.tolist(), np.int32)
            r = dev.verify(block, len(drafts), 0, P + 1, 8)
            o, _ = om.verify(block, len(drafts), 0, P + 1, 8)
            assert r.nacc == o.nacc and list(r.commit[:r.ncommit]) == list(o.commit[:o.ncommit]), rnd
            app = list(r.commit[:r.ncommit])
            gen += app
            P += r.ncommit
        for what in ("KC", "VC"):
            a = dev.read(what, np.uint16).reshape(NL, -1, 256)[:, :P + 1]
            b = om.get(what, np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)[:, :P + 1]
            assert same(a, b), what
    finally:
        om.close()
        dev.close()


def test_prefill_argument_errors(g4v):
    dev = g4v.Device(0)
    try:
        with pytest.raises(RuntimeError):
            dev.prefill(np.array([1, 2, 3], np.int32))  # no model yet
        dev.model_synth(3, 4096, 1, 512, 128)
        with pytest.raises(RuntimeError):
            dev.prefill(np.arange(200, dtype=np.int32))  # beyond the context capacity
        with pytest.raises(RuntimeError):
            dev.prefill(np.array([1, 2], np.int32), pfb=33)
        with pytest.raises(RuntimeError):
            dev.prefill(np.array([1, 5000], np.int32))  # token outside the vocabulary
    finally:
        dev.close()


def test_prefill_refuses_short_blocks_past_att_par(g4v):
    """blocks before the last of at most 4 rows past position 192 take the split-KV path in the
    reference (E:1305) and one-row blocks its exact-float products (E:311); the prefill runs
    only the last block that way, so such block sizes are refused with a message"""
    dev = g4v.Device(0)
    try:
        dev.model_synth(3, 4096, 1, 512, 512)
        toks = np.arange(1, 301, dtype=np.int32)
        note("prefill pfb 4 / 1 refusals")
        with pytest.raises(RuntimeError, match="pfb < 5"):
            dev.prefill(toks, pfb=4)
        with pytest.raises(RuntimeError, match="pfb 1"):
            dev.prefill(toks[:100], pfb=1)
        dev.prefill(toks[:150], pfb=4)  # every block ends at or before position 192: accepted
    finally:
        dev.close()
