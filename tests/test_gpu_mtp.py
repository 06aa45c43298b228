"""GPU parity of the MTP drafter (draft_step E:1534-1563, chained as E:1631-1646) against the
oracle: every draft, runner-up, score gap and the last hidden state bit for bit, for chains
that start from a given hidden state and from the last verify step's committed state."""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu


def oracle_chain(d, m, tok, h, P, k, T, samepos=False):
    toks, secs, gaps = [], [], []
    for j in range(k):
        tok, h, s, g = d.step(m, tok, h, P + 1 + (0 if samepos else j), P, T)
        toks.append(tok)
        secs.append(s)
        gaps.append(g)
    return toks, secs, np.array(gaps, np.float32), h


# (V, P, T, k): C = V / 128 centroids (32: every centroid is in the top 32; 128 and 2048: a
# real selection), contexts inside and past the 512 window, the reference's 6 splits and 8
CASES = [(4096, 300, 6, 3), (16384, 700, 6, 3), (16384, 40, 8, 2), (16384, 1500, 8, 4), (262144, 900, 6, 3)]


@pytest.mark.parametrize("V,P,T,k", CASES)
def test_draft_chain_matches_oracle(orc, g4v, V, P, T, k):
    from oracle import Drafter, Model
    NL, I, ctx, seed = 15, 512, 2048, 41
    note(f"mtp chain V={V} P={P} T={T} k={k}")
    rng = np.random.default_rng(P)
    dev = g4v.Device(0)
    m = Model(orc, seed, V, NL, I, ctx)
    d = Drafter(orc, seed + 1, V)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        dev.fake_ctx(P + 1, 5150)
        m.fake_ctx(P + 1, 5150)
        dev.drafter_synth(seed + 1)
        h = (rng.standard_normal(1536).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
        tok = int(rng.integers(0, V))
        got = dev.draft_mtp(tok, h, P, k, T)
        want = oracle_chain(d, m, tok, h, P, k, T)
        assert got[0].tolist() == want[0], (got[0], want[0])
        assert got[1].tolist() == want[1], (got[1], want[1])
        assert same(got[2], want[2]), (got[2], want[2])
        assert same(got[3], want[3]), first_diff(got[3], want[3])
    finally:
        d.close()
        m.close()
        dev.close()


@pytest.mark.parametrize("P", [300, 700])
def test_draft_chain_same_position(orc, g4v, P):
    """ENGINE_DRAFT_SAMEPOS (E:1516, 1633): every step at position P + 1 (its RoPE angle and, past
    the 512 window, its window start); then the setting off again gives the P + 1 + j chain"""
    from oracle import Drafter, Model
    V, NL, I, ctx, seed, k, T = 16384, 15, 512, 2048, 45, 4, 6
    note(f"mtp chain same position P={P}")
    rng = np.random.default_rng(P + 1)
    dev = g4v.Device(0)
    m = Model(orc, seed, V, NL, I, ctx)
    d = Drafter(orc, seed + 1, V)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        dev.fake_ctx(P + 1, 5151)
        m.fake_ctx(P + 1, 5151)
        dev.drafter_synth(seed + 1)
        h = (rng.standard_normal(1536).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
        tok = int(rng.integers(0, V))
        for samepos in (True, False):
            dev.set_draft_samepos(samepos)
            got = dev.draft_mtp(tok, h, P, k, T)
            want = oracle_chain(d, m, tok, h, P, k, T, samepos)
            assert got[0].tolist() == want[0] and got[1].tolist() == want[1], (samepos, got[0], want[0])
            assert same(got[2], want[2]) and same(got[3], want[3]), samepos
    finally:
        d.close()
        m.close()
        dev.close()


def test_draft_after_verify(orc, g4v):
    """h = None: the chain starts from the committed hidden state the verify step left on the device"""
    from oracle import Drafter, Model
    V, NL, I, ctx, seed, P = 16384, 15, 512, 1024, 43, 600
    note("mtp chain after a verify step")
    dev = g4v.Device(0)
    m = Model(orc, seed, V, NL, I, ctx)
    d = Drafter(orc, seed + 1, V)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        dev.fake_ctx(P, 77)
        m.fake_ctx(P, 77)
        dev.drafter_synth(seed + 1)
        block = np.array([5, 5, 5, 9], np.int32)
        r = dev.verify(block, 3, 0, P, 8)
        o, ho = m.verify(block, 3, 0, P, 8)
        assert list(r.commit[:r.ncommit]) == list(o.commit[:o.ncommit])
        Pn = P + r.ncommit - 1
        conf = r.commit[r.ncommit - 1]
        got = dev.draft_mtp(conf, None, Pn, 3, 6)
        want = oracle_chain(d, m, conf, ho, Pn, 3, 6)
        assert got[0].tolist() == want[0] and got[1].tolist() == want[1]
        assert same(got[2], want[2]) and same(got[3], want[3])
    finally:
        d.close()
        m.close()
        dev.close()


def test_draft_argument_errors(g4v):
    dev = g4v.Device(0)
    try:
        with pytest.raises(RuntimeError):
            dev.drafter_synth(1)  # no model
        dev.model_synth(3, 4096, 2, 512, 256)
        with pytest.raises(RuntimeError):
            dev.drafter_synth(1)  # fewer than 15 target layers
    finally:
        dev.close()


def test_run_req_loop_matches_oracle(orc, g4v):
    """run_req end to end (E:1594-1661, sibling policy off): prefill, then rounds of prompt-lookup
    drafts or, when the lookup finds none, a 3-step MTP chain, each verified as a chain"""
    from oracle import Drafter, Model
    V, NL, I, ctx, seed = 16384, 15, 512, 1024, 47
    rng = np.random.default_rng(8)
    motif = rng.integers(0, V, 24)
    prompt = np.resize(motif, 200).astype(np.int32)
    noise = rng.random(200) < 0.2
    prompt[noise] = rng.integers(0, V, int(noise.sum()))
    note("run_req loop: prefill 200 + 24 rounds (lookup / MTP)")
    dev = g4v.Device(0)
    m = Model(orc, seed, V, NL, I, ctx)
    d = Drafter(orc, seed + 1, V)
    try:
        dev.model_synth(seed, V, NL, I, ctx)
        dev.drafter_synth(seed + 1)
        g0, hd = dev.prefill(prompt, hidden=True)
        ho = m.prefill(prompt)
        assert same(hd, ho)
        G, _, _ = dev.head_argmax(ho[None, :])
        assert g0 == G[0]
        gen, P, app, h_or, kinds = [g0], len(prompt) - 1, [], ho, set()
        dev.history_set(np.concatenate([prompt, [g0]]))
        for rnd in range(24):
            drafts = dev.prompt_lookup(3, 3, app)
            seq = np.concatenate([prompt, gen]).astype(np.int32)
            assert drafts.tolist() == orc.prompt_lookup(seq, 3, 3).tolist(), rnd
            if drafts.size == 0:
                drafts = dev.draft_mtp(gen[-1], hd if rnd == 0 else None, P, 3, 6)[0]
                want = oracle_chain(d, m, gen[-1], h_or, P, 3, 6)[0]
                assert drafts.tolist() == want, rnd
                kinds.add("mtp")
            else:
                kinds.add("lookup")
            block = np.array([gen[-1]] + drafts.tolist(), np.int32)
            r = dev.verify(block, len(drafts), 0, P + 1, 8)
            o, h_or = m.verify(block, len(drafts), 0, P + 1, 8)
            assert r.nacc == o.nacc and list(r.commit[:r.ncommit]) == list(o.commit[:o.ncommit]), rnd
            app = list(r.commit[:r.ncommit])
            gen += app
            P += r.ncommit
        assert kinds == {"mtp", "lookup"}, kinds  # both drafters took part
        for what in ("KC", "VC"):
            a = dev.read(what, np.uint16).reshape(NL, -1, 256)[:, :P + 1]
            b = m.get(what, np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)[:, :P + 1]
            assert same(a, b), what
    finally:
        d.close()
        m.close()
        dev.close()
