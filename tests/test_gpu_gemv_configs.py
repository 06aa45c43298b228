"""GPU parity of the verify pass under every row-tile GEMV shape (G4V_GEMV_CFG).

The row-tile GEMV takes two launch parameters per product (q/k/v, o, gate/up, down): the
activation rows per block (1..4) and the rows per tile (64 or 32).  They change the block
decomposition only, never the arithmetic, so every shape must reproduce the oracle bit for
bit: greedy tokens, survivor counts, the final hidden state and the new KV rows of all 7 tree
rows (which pass through every layer's q/k/v, o, gate/up and down products).
"""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

V, NL, I, CTX, NCTX, SEED = 8192, 3, 6144, 1024, 500, 23

# "qkv o gate/up down", each "rows,tile"; the default is "2,64 1,64 4,64 1,64"
CONFIGS = ["1,64 1,64 1,64 1,64", "2,32 2,32 2,32 2,32", "3,64 1,32 3,32 2,64", "4,32 2,64 4,64 3,32",
           "4,64 1,64 1,32 4,32"]


@pytest.mark.parametrize("cfg", CONFIGS)
def test_verify_under_gemv_config(orc, g4v, cfg, monkeypatch):
    from oracle import Model
    monkeypatch.setenv("G4V_GEMV_CFG", cfg)
    note(f"gemv config {cfg}: model V={V} NL={NL}")
    dev = g4v.Device(0)
    om = Model(orc, SEED, V, NL, I, CTX)
    try:
        dev.model_synth(SEED, V, NL, I, CTX)
        dev.fake_ctx(NCTX, 12345)
        om.fake_ctx(NCTX, 12345)
        toks = np.array([7, 1234, 88, 4021, 6000, 15, 333], np.int32)
        r, hg = dev.verify(toks, 3, 3, NCTX, 8, hidden=True)
        o, ho = om.verify(toks, 3, 3, NCTX, 8)
        assert r.nacc == o.nacc and r.ncommit == o.ncommit and list(r.G) == list(o.G), (r.as_dict(), list(o.G))
        for i in range(8):
            if o.G[i] >= 0:
                assert r.nsurv[i] == o.nsurv[i]
        assert same(hg, ho), first_diff(hg, ho)
        kc, vc = dev.read("KC", np.uint16), dev.read("VC", np.uint16)
        kco, vco = om.get("KC", np.uint16, NL * CTX * 256), om.get("VC", np.uint16, NL * CTX * 256)
        assert same(kc, kco), first_diff(kc, kco)
        assert same(vc, vco), first_diff(vc, vco)
    finally:
        om.close()
        dev.close()


@pytest.mark.parametrize("cfg", ["2,64 1,64 4,64 1,64", "2,64 1,64 4,64 1,32"])
def test_verify_wide_mlp(orc, g4v, cfg, monkeypatch):
    """a 12288-wide MLP (the Gemma-4-E2B layout's layers 15-34): the down projection at
    K = 12288 on 64- and 32-row tiles reproduces the oracle's hidden state and KV rows"""
    from oracle import Model
    monkeypatch.setenv("G4V_GEMV_CFG", cfg)
    Vw, NLw, Iw = 8192, 2, 12288
    note(f"gemv config {cfg}: model V={Vw} NL={NLw} I={Iw}")
    dev = g4v.Device(0)
    om = Model(orc, SEED, Vw, NLw, Iw, CTX)
    try:
        dev.model_synth(SEED, Vw, NLw, Iw, CTX)
        dev.fake_ctx(NCTX, 12345)
        om.fake_ctx(NCTX, 12345)
        toks = np.array([7, 1234, 88, 4021, 6000, 15, 333], np.int32)
        r, hg = dev.verify(toks, 3, 3, NCTX, 8, hidden=True)
        o, ho = om.verify(toks, 3, 3, NCTX, 8)
        assert r.nacc == o.nacc and r.ncommit == o.ncommit and list(r.G) == list(o.G), (r.as_dict(), list(o.G))
        assert same(hg, ho), first_diff(hg, ho)
        kc, vc = dev.read("KC", np.uint16), dev.read("VC", np.uint16)
        kco, vco = om.get("KC", np.uint16, NLw * CTX * 256), om.get("VC", np.uint16, NLw * CTX * 256)
        assert same(kc, kco), first_diff(kc, kco)
        assert same(vc, vco), first_diff(vc, vco)
    finally:
        om.close()
        dev.close()
