"""The attention path of a decode pass (E:1305 / 1328 / 1337: split-KV for at most 4 rows past
ATT_PAR = 192 keys, attn_tile for 4+ rows past 64, run_mh otherwise): the oracle's verify pass
against the reference's kernels composed the same way (oracle/_ref), token for token and KV byte
for byte."""
import numpy as np
import pytest

from util import first_diff, same

V, NL, I, CTX, NFAKE = 262144, 2, 6144, 1024, 600
# (chain length, pos0): 8 rows tiled; 4 rows below ATT_PAR, tiled; 3 rows, run_mh; 1 row at the
# start of the cache, run_mh; 4 rows past ATT_PAR, split-KV
CASES = [(7, 600), (3, 100), (2, 50), (0, 30), (3, 600)]


@pytest.fixture(scope="module")
def pair(orc, ref):
    from oracle import Model
    om, rm = Model(orc, 9, V, NL, I, CTX), Model(orc, 9, V, NL, I, CTX)
    ref.bind_model(rm)
    yield om, rm
    om.close()
    rm.close()


@pytest.mark.parametrize("na,pos0", CASES)
def test_chain_pass_paths(orc, ref, pair, na, pos0):
    om, rm = pair
    om.fake_ctx(NFAKE, 3)
    rm.fake_ctx(NFAKE, 3)
    toks = np.array([17 + 29 * k for k in range(na + 1)], np.int32)
    o, _ = om.verify(toks, na, 0, pos0)
    r = ref.verify(toks, na, 0, pos0)
    assert (o.nacc, o.ncommit) == (r.nacc, r.ncommit)
    assert list(o.commit[:o.ncommit]) == list(r.commit[:r.ncommit])
    # rows the lazy head evaluates; past the first 4 rows the engine scores its second head group
    # in full (E:1406-1500 per 4-row group), the oracle only along the accepted path
    for i in range(na + 1):
        if o.G[i] >= 0:
            assert o.G[i] == r.G[i], (i, list(o.G), list(r.G))
    for what in ("KC", "VC"):
        a, b = om.get(what, np.uint16, NL * CTX * 256), rm.get(what, np.uint16, NL * CTX * 256)
        assert same(a, b), (what, first_diff(a, b))


@pytest.mark.parametrize("na,pos0", [(7, 600), (6, 100), (5, 30), (7, 20)])
def test_long_chain_accepted(orc, ref, pair, na, pos0):
    """chains of 5 to 7 drafts (ENGINE_NGLEN <= 7, E:1514) taken from the model's greedy tokens,
    accepted in full: 6 to 8 rows through attn_tile or run_mh and both of the engine's 4-row head
    groups"""
    om, rm = pair
    toks = [4242]
    for j in range(na):
        om.fake_ctx(NFAKE, 3)
        o, _ = om.verify(np.array(toks, np.int32), j, 0, pos0)
        toks.append(int(o.G[j]))
    toks = np.array(toks, np.int32)
    om.fake_ctx(NFAKE, 3)
    rm.fake_ctx(NFAKE, 3)
    o, _ = om.verify(toks, na, 0, pos0)
    r = ref.verify(toks, na, 0, pos0)
    assert o.nacc == na and (r.nacc, r.ncommit) == (o.nacc, o.ncommit)
    assert list(o.commit[:o.ncommit]) == list(r.commit[:r.ncommit])
    assert list(o.G[:na + 1]) == list(r.G[:na + 1])
    for what in ("KC", "VC"):
        a, b = om.get(what, np.uint16, NL * CTX * 256), rm.get(what, np.uint16, NL * CTX * 256)
        assert same(a, b), (what, first_diff(a, b))


# the engine's sibling form (E:1634-1655): drafts toks[1..na], sibling row toks[na + 1] at RoPE
# position pos0 + 1.  (na, pos0, allow_b): 3 rows, run_mh; 4 rows below ATT_PAR, run_mh (no
# attn_tile with a sibling); 3 rows past ATT_PAR, split-KV; the tree hit not taken
SIB_CASES = [(1, 100, True), (2, 150, True), (1, 190, True), (1, 100, False)]


@pytest.mark.parametrize("na,pos0,allow_b", SIB_CASES)
def test_sibling_pass_paths(orc, ref, pair, na, pos0, allow_b):
    om, rm = pair
    om.fake_ctx(NFAKE, 3)
    toks = np.array([23 + 31 * k for k in range(na + 2)], np.int32)
    o, _ = om.verify(toks, na, 1, pos0, allow_b=False)  # row 0's token on the same attention path
    toks[na + 1] = o.G[0]  # the sibling holds row 0's greedy token: the tree hit
    if toks[1] == o.G[0]:
        toks[1] += 1
    om.fake_ctx(NFAKE, 3)
    rm.fake_ctx(NFAKE, 3)
    o, _ = om.verify(toks, na, 1, pos0, allow_b=allow_b)
    r = ref.verify(toks, na, 1, pos0, allow_b=allow_b)
    assert o.ncommit == (2 if allow_b else 1) and o.branch == (1 if allow_b else 0)
    assert (o.nacc, o.ncommit, o.branch) == (r.nacc, r.ncommit, r.branch)
    assert list(o.commit[:o.ncommit]) == list(r.commit[:r.ncommit])
    for i in range(na + 2):
        if o.G[i] >= 0:
            assert o.G[i] == r.G[i], (i, list(o.G), list(r.G))
    for what in ("KC", "VC"):
        a, b = om.get(what, np.uint16, NL * CTX * 256), rm.get(what, np.uint16, NL * CTX * 256)
        assert same(a, b), (what, first_diff(a, b))
