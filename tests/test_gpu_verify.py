"""GPU parity of the whole verify pass (synthetic stack, tree drafts, head, acceptance).

The oracle model and the device model are generated from the same seed; the test first
checks that the generated weights are identical, then runs verify passes whose drafts are
chosen to hit every acceptance path: nothing accepted, chain a accepted (fully and
partially) and branch b (the sibling) accepted with KV compaction.
"""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

V, NL, I, CTX, NCTX, SEED = 8192, 3, 6144, 2048, 700, 11


@pytest.fixture(scope="module")
def pair(orc, dev):
    from oracle import Model
    note(f"model synth V={V} NL={NL} ctx={CTX}")
    dev.model_synth(SEED, V, NL, I, CTX)
    dev.fake_ctx(NCTX, 12345)
    om = Model(orc, SEED, V, NL, I, CTX)
    om.fake_ctx(NCTX, 12345)
    yield dev, om
    om.close()


def test_generated_weights_identical(pair):
    dev, om = pair
    for name, dt, cnt in [("E", np.uint16, V * 1536), ("W1_4", np.uint8, I * 768), ("S2_6", np.uint16, 1536 * I // 32),
                          ("N0_4", np.float32, 256), ("N2_1", np.float32, 1536), ("fnorm", np.float32, 1536),
                          ("coef", np.float32, V)]:
        a = dev.read(name, dt)
        b = om.get(name, dt, cnt)
        assert same(a, b), (name, first_diff(a, b))
    assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, NL * CTX * 256))


def _compare(r, o, hid_g=None, hid_o=None):
    assert r.nacc == o.nacc and r.branch == o.branch and r.ncommit == o.ncommit, (r.as_dict(), o.nacc, o.branch)
    assert list(r.commit)[: r.ncommit] == list(o.commit)[: o.ncommit]
    assert list(r.G) == list(o.G), (list(r.G), list(o.G))
    for i in range(8):
        if o.G[i] >= 0:
            assert r.nsurv[i] == o.nsurv[i]
    if hid_g is not None:
        assert same(hid_g, hid_o), first_diff(hid_g, hid_o)


def _both(pair, toks, na, nb, pos0, T=8):
    dev, om = pair
    note(f"verify toks={list(toks)} na={na} nb={nb} pos0={pos0} T={T}")
    r, hg = dev.verify(np.array(toks, np.int32), na, nb, pos0, T, hidden=True)
    o, ho = om.verify(np.array(toks, np.int32), na, nb, pos0, T)
    _compare(r, o, hg, ho)
    return r, o


def test_verify_random_drafts(pair):
    _both(pair, [5, 17, 29, 41], 3, 0, NCTX)
    _both(pair, [5, 17, 29, 41, 53, 65, 77], 3, 3, NCTX)


def test_verify_chain_accepted(pair):
    """drafts equal to the model's own predictions are accepted row by row"""
    toks = [101, 0, 0, 0]
    for depth in range(1, 4):
        _, o = _both(pair, toks, 3, 0, NCTX)
        toks[depth] = o.G[depth - 1]
    r, o = _both(pair, toks, 3, 0, NCTX)
    assert o.nacc == 3


def test_verify_branch_b_accepted(pair):
    """the sibling branch holds the prediction: branch b commits and its KV rows move"""
    _, o = _both(pair, [202, 3, 4, 5, 6, 7, 8], 3, 3, NCTX)
    g0 = o.G[0]
    toks = [202, (g0 + 1) % V, 4, 5, g0, 7, 8]
    r, o = _both(pair, toks, 3, 3, NCTX)
    assert o.branch == 1 and o.nacc >= 1
    dev, om = pair
    assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, NL * CTX * 256))
    assert same(dev.read("VC", np.uint16), om.get("VC", np.uint16, NL * CTX * 256))


def test_graph_replays_match_eager_and_oracle(pair):
    """the captured graph, replayed repeatedly with host work in between, equals eager launches"""
    dev, om = pair
    toks = [77, 1, 2, 3, 4, 5, 6]
    results = []
    for graphs in (False, True):
        dev.set_graphs(graphs)
        for rep in range(4):  # graph mode: eager warm-up, capture, then replays
            note(f"graph={graphs} rep={rep}")
            r, hg = dev.verify(np.array(toks, np.int32), 3, 3, NCTX + 100, 8, hidden=True)
            results.append((r.as_dict(), hg.copy()))
            _ = np.ones(1000).sum()  # host work between replays
    dev.set_graphs(True)
    o, ho = om.verify(np.array(toks, np.int32), 3, 3, NCTX + 100, 8)
    for d, h in results:
        assert d["G"] == list(o.G) and d["nacc"] == o.nacc
        assert same(h, ho)


def test_verify_sequence_of_steps(pair):
    """successive passes commit tokens and advance the position, as run_req does"""
    dev, om = pair
    pos0, conf = NCTX + 40, 300
    for step in range(3):
        toks = [conf, (conf * 7 + 1) % V, (conf * 11 + 2) % V, (conf * 13 + 3) % V]
        r, o = _both(pair, toks, 3, 0, pos0)
        pos0 += r.ncommit
        conf = r.commit[r.ncommit - 1]


@pytest.mark.parametrize("na,nb,pos0", [(3, 3, 700), (3, 0, 740), (7, 0, 760), (1, 0, 100), (5, 0, 60), (0, 0, 720)])
def test_w4a8_verify_passes(orc, g4v, na, nb, pos0):
    """ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8 on (E:1600): passes of two rows or more take
    W4A8 products (lin_multi, E:311) -- the tree and chains past ATT_PAR, a chain of 7 drafts and
    the short passes through the prefill attention kernels -- and a one-row pass stays exact;
    eager and replayed-graph passes equal the oracle's i8 verify pass, drafts the model takes
    included (the accepted rows' heads and the branch-b KV move)"""
    from oracle import Model
    note(f"w4a8 verify na={na} nb={nb} pos0={pos0}")
    dev = g4v.Device(0)
    om = Model(orc, 31, 8192, 3, 6144, 1024)
    try:
        dev.model_synth(31, 8192, 3, 6144, 1024)
        dev.set_prefill_int8(True)
        dev.set_decode_int8(True)
        toks = np.array([40 + 37 * k for k in range(1 + na + nb)], np.int32)
        o0 = None
        for rep in range(3):  # eager, capture, replay (graphs serve split-KV passes)
            dev.fake_ctx(700, 99)
            om.fake_ctx(700, 99)
            if rep == 0:  # drafts the model takes: chain a from its own predictions
                o0, _ = om.verify(toks, na, nb, pos0, 8, i8=True)
                om.fake_ctx(700, 99)
                if na >= 1:
                    toks[1] = o0.G[0]
            r, hg = dev.verify(toks, na, nb, pos0, 8, hidden=True)
            o, ho = om.verify(toks, na, nb, pos0, 8, i8=True)
            _compare(r, o, hg, ho)
            assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, 3 * 1024 * 256)), rep
            assert same(dev.read("VC", np.uint16), om.get("VC", np.uint16, 3 * 1024 * 256)), rep
        if na >= 2 or nb >= 1:  # the W4A8 pass differs from the exact one somewhere
            oe, hoe = om.verify(toks, na, nb, pos0, 8, i8=False)
            assert not same(hoe, ho) or list(oe.G) != list(o.G)
    finally:
        om.close()
        dev.close()


@pytest.mark.parametrize("na,pos0", [(7, 600), (6, 100), (5, 30), (7, 20)])
def test_long_chain_accepted(orc, g4v, na, pos0):
    """chains of 5 to 7 drafts (E:1514 ENGINE_NGLEN <= 7) built from the model's own greedy
    tokens, so that every row is accepted: 6 to 8 rows through attn_tile or run_mh (E:1328-1349),
    the second head pass over up to 7 rows, with the full vocabulary (V = 262,144: the screen
    overflows and the full head scores the rows)"""
    from oracle import Model
    Vb, NLb, Ib, CTXb = 262144, 2, 512, 1024
    note(f"long chain na={na} pos0={pos0} V={Vb}")
    dev = g4v.Device(0)
    om = Model(orc, 31, Vb, NLb, Ib, CTXb)
    try:
        dev.model_synth(31, Vb, NLb, Ib, CTXb)
        toks = [4242]
        for j in range(na):  # extend the chain by the greedy token of its last row
            om.fake_ctx(700, 77)
            o, _ = om.verify(np.array(toks, np.int32), j, 0, pos0, 8)
            assert o.nacc == j
            toks.append(int(o.G[j]))
        toks = np.array(toks, np.int32)
        dev.fake_ctx(700, 77)
        om.fake_ctx(700, 77)
        r, hg = dev.verify(toks, na, 0, pos0, 8, hidden=True)
        o, ho = om.verify(toks, na, 0, pos0, 8)
        _compare(r, o, hg, ho)
        assert r.nacc == na and r.ncommit == na + 1
        note(f"fallback rows {list(r.fallback)}")
        kc, kco = dev.read("KC", np.uint16), om.get("KC", np.uint16, NLb * CTXb * 256)
        vc, vco = dev.read("VC", np.uint16), om.get("VC", np.uint16, NLb * CTXb * 256)
        assert same(kc, kco) and same(vc, vco)
    finally:
        om.close()
        dev.close()


@pytest.mark.parametrize("na,pos0", [(4, 600), (3, 100), (2, 50), (0, 30), (3, 600), (4, 150)])
def test_chain_pass_attention_paths(orc, g4v, na, pos0):
    """decode passes take the engine's attention path (E:1305 / 1328 / 1337): attn_tile for 5 rows
    and for 4 rows below ATT_PAR, run_mh for short passes near the start, split-KV past ATT_PAR;
    the same shape on both sides of the threshold alternates between a captured and an eager pass"""
    from oracle import Model
    note(f"chain pass path na={na} pos0={pos0}")
    dev = g4v.Device(0)
    om = Model(orc, 23, 8192, 3, 6144, 1024)
    try:
        dev.model_synth(23, 8192, 3, 6144, 1024)
        for p in (pos0, 600, pos0):  # the graph of the split shape must not serve the other path
            dev.fake_ctx(700, 4242)
            om.fake_ctx(700, 4242)
            toks = np.array([17 + 29 * k for k in range(na + 1)], np.int32)
            r, hg = dev.verify(toks, na, 0, p, 8, hidden=True)
            o, ho = om.verify(toks, na, 0, p, 8)
            assert r.nacc == o.nacc and list(r.commit[:r.ncommit]) == list(o.commit[:o.ncommit]), p
            assert same(hg, ho), (p, first_diff(hg, ho))
            kc, kco = dev.read("KC", np.uint16), om.get("KC", np.uint16, 3 * 1024 * 256)
            vc, vco = dev.read("VC", np.uint16), om.get("VC", np.uint16, 3 * 1024 * 256)
            assert same(kc, kco) and same(vc, vco), p
    finally:
        om.close()
        dev.close()


@pytest.mark.parametrize("nd,pos0,allow", [(1, 100, True), (2, 150, True), (1, 190, True), (1, 100, False),
                                           (2, 40, True)])
def test_sibling_pass_paths(orc, g4v, nd, pos0, allow):
    """the engine's sibling form (E:1634-1655): run_mh with the sibling's RoPE position and skip
    range below ATT_PAR (no attn_tile even for 4 rows), split-KV past it; the tree hit commits the
    sibling and moves its KV row, and with the hit not allowed only the chain is accepted"""
    from oracle import Model
    note(f"sibling pass nd={nd} pos0={pos0} allow={allow}")
    dev = g4v.Device(0)
    om = Model(orc, 23, 8192, 3, 6144, 1024)
    try:
        dev.model_synth(23, 8192, 3, 6144, 1024)
        dev.fake_ctx(700, 4242)
        om.fake_ctx(700, 4242)
        toks = np.array([19 + 37 * k for k in range(nd + 2)], np.int32)
        o, _ = om.verify(toks, nd, 1, pos0, 8, allow_b=False)  # row 0's token on the same attention path
        toks[nd + 1] = o.G[0]  # the runner-up draft holds row 0's greedy token
        if toks[1] == o.G[0]:
            toks[1] += 1
        for hit_expected in (True, False):
            if not hit_expected:
                toks[nd + 1] = (o.G[0] + 5) % 8192
            dev.fake_ctx(700, 4242)
            om.fake_ctx(700, 4242)
            r, hg = dev.verify_sibling(toks, nd, pos0, 8, allow_hit=allow, hidden=True)
            oo, ho = om.verify(toks, nd, 1, pos0, 8, allow_b=allow)
            assert (r.nacc, r.branch, r.ncommit) == (oo.nacc, oo.branch, oo.ncommit), (hit_expected, r.as_dict())
            assert r.ncommit == (2 if (allow and hit_expected) else 1)
            assert list(r.commit[:r.ncommit]) == list(oo.commit[:oo.ncommit])
            assert same(hg, ho), first_diff(hg, ho)
            kc, kco = dev.read("KC", np.uint16), om.get("KC", np.uint16, 3 * 1024 * 256)
            vc, vco = dev.read("VC", np.uint16), om.get("VC", np.uint16, 3 * 1024 * 256)
            assert same(kc, kco) and same(vc, vco)
    finally:
        om.close()
        dev.close()


def test_verify_argument_errors(g4v):
    """shapes the verify entry points do not serve fail on the host with an error, before any
    launch, and leave the context usable"""
    dev = g4v.Device(0)
    try:
        dev.model_synth(23, 8192, 3, 6144, 1024)
        dev.fake_ctx(700, 4242)
        toks = np.array([5, 6, 7, 8, 9], np.int32)
        for nd in (0, 3):  # the sibling form holds 1 or 2 drafts
            with pytest.raises(RuntimeError):
                dev.verify_sibling(toks, nd, 100, 8)
        with pytest.raises(RuntimeError):  # branch b without a chain
            dev.verify(toks[:2], 0, 1, 100, 8)
        with pytest.raises(RuntimeError):  # past the cache
            dev.verify(toks[:4], 3, 0, 1022, 8)
        long9 = np.arange(9, dtype=np.int32) + 5
        with pytest.raises(RuntimeError):  # a chain of 8 drafts: 9 rows
            dev.verify(long9, 8, 0, 100, 8)
        with pytest.raises(RuntimeError):  # a tree branch of 5 drafts
            dev.verify(long9[:8], 2, 5, 100, 8)
        r = dev.verify_sibling(toks[:3], 1, 100, 8)
        assert r.ncommit >= 1
    finally:
        dev.close()
