"""Full-size verify pass (the benchmark workload): 35 layers, vocabulary 262,144, context 2048,
2 x 3 draft tree; bit-exact against the oracle, including an accepted chain."""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

V, NL, I, CTX, NCTX, SEED = 262144, 35, 6144, 4096, 2048, 1


@pytest.fixture(scope="module")
def full(orc, dev):
    from oracle import Model
    note(f"full model synth V={V} NL={NL}")
    dev.model_synth(SEED, V, NL, I, CTX)
    dev.fake_ctx(NCTX, 12345)
    om = Model(orc, SEED, V, NL, I, CTX)
    om.fake_ctx(NCTX, 12345)
    yield dev, om
    om.close()


def _check(full, toks, na, nb, pos0):
    dev, om = full
    note(f"full verify toks={list(toks)} na={na} nb={nb} pos0={pos0}")
    r, hg = dev.verify(np.array(toks, np.int32), na, nb, pos0, 8, hidden=True)
    o, ho = om.verify(np.array(toks, np.int32), na, nb, pos0, 8)
    assert (r.nacc, r.branch, r.ncommit) == (o.nacc, o.branch, o.ncommit)
    assert list(r.G) == list(o.G) and list(r.commit)[: r.ncommit] == list(o.commit)[: o.ncommit]
    assert same(hg, ho), first_diff(hg, ho)
    return o


def test_full_verify_tree_random_drafts(full):
    _check(full, [11, 1, 2, 3, 4, 5, 6], 3, 3, NCTX)


def test_full_verify_chain_accepted(full):
    toks = [11, 1, 2, 3]
    for d in range(1, 4):
        o = _check(full, toks, 3, 0, NCTX + 1)
        toks[d] = o.G[d - 1]
    o = _check(full, toks, 3, 0, NCTX + 1)
    assert o.nacc == 3


def test_full_kv_cache_identical(full):
    dev, om = full
    assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, NL * CTX * 256))
    assert same(dev.read("VC", np.uint16), om.get("VC", np.uint16, NL * CTX * 256))
