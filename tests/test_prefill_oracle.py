"""Prefill (E:1594-1599, with ENGINE_PREFILL_INT8=1 and in the default exact float): the
oracle's attention paths and its block composition against the reference's own kernels
(oracle/_ref), and the attention paths against an fp64 softmax."""
import numpy as np
import pytest

from util import first_diff, same

RNG = np.random.default_rng(17)


def kv(npos):
    K = (RNG.standard_normal((npos, 256)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    V = (RNG.standard_normal((npos, 256)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return K, V


def bf(x):
    return (x.astype(np.uint32) << 16).view(np.float32)


def f64_attn(K, V, q, pos, lo):
    out = np.empty_like(q, dtype=np.float64)
    Kf, Vf = bf(K).astype(np.float64), bf(V).astype(np.float64)
    for m in range(q.shape[0]):
        for h in range(8):
            s = Kf[lo[m]:pos[m] + 1] @ q[m, h * 256:(h + 1) * 256].astype(np.float64)
            w = np.exp(s - s.max())
            out[m, h * 256:(h + 1) * 256] = (w / w.sum()) @ Vf[lo[m]:pos[m] + 1]
    return out


@pytest.mark.parametrize("kind,pos0,M,sliding", [("tile", 64, 32, True), ("tile", 700, 32, True),
                                                 ("tile", 700, 25, False), ("tile", 96, 5, False),
                                                 ("mh", 0, 32, True), ("mh", 32, 32, False), ("mh", 0, 3, True)])
def test_attention_paths(orc, kind, pos0, M, sliding):
    K, V = kv(pos0 + M)
    q = RNG.standard_normal((M, 2048)).astype(np.float32) * 0.5
    pos = np.arange(pos0, pos0 + M, dtype=np.int32)
    lo = np.maximum(0, pos - 511) if sliding else np.zeros(M, np.int32)
    got = orc.attn_rows(kind, K, V, q, pos, lo.astype(np.int32))
    ref64 = f64_attn(K, V, q, pos, lo)
    assert np.max(np.abs(got - ref64)) < 2e-2  # bf16-rounded outputs of unit-scale values
    # a row's result does not depend on the rows beside it
    one = orc.attn_rows(kind, K, V, q[-1:], pos[-1:], lo[-1:].astype(np.int32))
    assert same(one[0], got[-1])


@pytest.mark.parametrize("kind,pos0,M,sliding", [("tile", 64, 32, True), ("tile", 700, 32, True),
                                                 ("tile", 700, 25, False), ("tile", 96, 5, False),
                                                 ("mh", 0, 32, True), ("mh", 32, 32, False)])
def test_attention_paths_vs_reference(orc, ref, kind, pos0, M, sliding):
    K, V = kv(pos0 + M)
    q = RNG.standard_normal((M, 2048)).astype(np.float32) * 0.5
    pos = np.arange(pos0, pos0 + M, dtype=np.int32)
    lo = (np.maximum(0, pos - 511) if sliding else np.zeros(M)).astype(np.int32)
    got = orc.attn_rows(kind, K, V, q, pos, lo)
    want = ref.attn_rows(kind, K, V, sliding, q, pos0)
    assert same(got, want), first_diff(got, want)


# (n, NL, ctx): block tails that take every path -- run_mh blocks (positions < 64), attn_tile
# blocks, a 4-row split-KV tail (196), a 1-row float tail (193), a 2-row run_mh tail (34), and a
# prompt past the 512 window (600, one layer)
CASES = [(34, 2, 256), (100, 2, 256), (193, 2, 256), (196, 5, 256), (600, 1, 640)]


@pytest.mark.parametrize("i8", [True, False])
@pytest.mark.parametrize("n,NL,ctx", CASES)
def test_prefill_vs_reference(orc, ref, n, NL, ctx, i8):
    """i8: ENGINE_PREFILL_INT8=1 (W4A8 for blocks of two rows or more); else the engine's
    default, exact float throughout (E:1210, 1363)"""
    from oracle import Model
    V, I, seed = 4096, 512, 31
    toks = RNG.integers(0, V, n).astype(np.int32)
    om, rm = Model(orc, seed, V, NL, I, ctx), Model(orc, seed, V, NL, I, ctx)
    try:
        ho = om.prefill(toks, i8=i8, T=ref.threads)  # the split-KV tail splits over the pool's workers
        ref.bind_model(rm)
        hr = ref.prefill(toks, i8=i8)
        assert same(ho, hr), first_diff(ho, hr)
        for what in ("KC", "VC"):
            a, b = om.get(what, np.uint16, NL * ctx * 256), rm.get(what, np.uint16, NL * ctx * 256)
            assert same(a, b), (what, first_diff(a, b))
    finally:
        om.close()
        rm.close()


def test_prefill_block_size_only_moves_path_boundaries(orc):
    """with W4A8 GEMMs independent of the rows beside them, pfb changes results only through
    the attention path of each block: pfb 16 and 32 give the same KV for the first 64
    positions (run_mh under both) and the same hidden state when every later block tiles"""
    from oracle import Model
    V, NL, I, ctx, seed, n = 4096, 1, 512, 256, 5, 160
    toks = RNG.integers(0, V, n).astype(np.int32)
    a, b = Model(orc, seed, V, NL, I, ctx), Model(orc, seed, V, NL, I, ctx)
    try:
        ha, hb = a.prefill(toks, pfb=32), b.prefill(toks, pfb=16)
        ka, kb = a.get("KC", np.uint16, ctx * 256), b.get("KC", np.uint16, ctx * 256)
        assert same(ka[:64 * 256], kb[:64 * 256])
        assert same(ka, kb)  # one layer: K depends only on the row's own embedding
        assert same(ha, hb)
    finally:
        a.close()
        b.close()
