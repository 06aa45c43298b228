"""The caller-weights path of the boundary: a stack assembled with g4v_model_create and the
g4v_model_set_* calls from host arrays (here: the oracle model's own arrays, in the reference's
Q4 byte layout) verifies exactly like the oracle, including a KV cache handed over with
g4v_model_set_kv."""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

V, NL, I, CTX, NCTX, SEED = 4096, 5, 1024, 1024, 300, 21
NS = [2048, 256, 256, 1536, I, I, 1536]
KS = [1536, 1536, 1536, 2048, 1536, 1536, I]


def test_loaded_stack_verifies_like_the_oracle(orc, dev):
    from oracle import Model
    om = Model(orc, SEED, V, NL, I, CTX)
    try:
        om.fake_ctx(NCTX, 777)
        note(f"model_create V={V} NL={NL} I={I}")
        dev.model_create(V, NL, I, CTX)
        with pytest.raises(RuntimeError):  # an incomplete stack is refused, not run
            dev.verify(np.array([1, 2], np.int32), 1, 0, NCTX, 8)
        dev.set_embed(om.get("E", np.uint16, V * 1536))
        for l in range(NL):
            for j in range(7):
                dev.set_matrix(l, j, om.get(f"W{l}_{j}", np.uint8, NS[j] * KS[j] // 2),
                               om.get(f"S{l}_{j}", np.uint16, NS[j] * KS[j] // 32))
            norms = [om.get(f"N{l}_{t}", np.float32, 1536 if t < 4 else 256) for t in range(6)]
            dev.set_norms(l, norms, 0.75, l % 5 != 4)
        dev.set_final_norm(om.get("fnorm", np.float32, 1536))
        kc = om.get("KC", np.uint16, NL * CTX * 256).reshape(NL, CTX, 256)
        vc = om.get("VC", np.uint16, NL * CTX * 256).reshape(NL, CTX, 256)
        for l in range(NL):
            dev.set_kv(l, 0, kc[l, :NCTX], vc[l, :NCTX])
        assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, NL * CTX * 256))
        for toks, na, nb in (([9, 9, 9, 40], 3, 0), ([11, 3, 4, 5, 11, 7, 8], 3, 3), ([6, 1], 1, 0)):
            note(f"loaded-stack verify toks={toks}")
            r, hg = dev.verify(np.array(toks, np.int32), na, nb, NCTX, 8, hidden=True)
            o, ho = om.verify(np.array(toks, np.int32), na, nb, NCTX, 8)
            assert (r.nacc, r.branch, r.ncommit) == (o.nacc, o.branch, o.ncommit)
            assert list(r.G) == list(o.G)
            assert same(hg, ho), first_diff(hg, ho)
        assert same(dev.read("KC", np.uint16), om.get("KC", np.uint16, NL * CTX * 256))
        assert same(dev.read("VC", np.uint16), om.get("VC", np.uint16, NL * CTX * 256))
    finally:
        om.close()
