"""The oracle against the reference's own kernels, live (oracle/_ref/libg4ref.so, built from
the reference sources by oracle/Makefile where they are present; skipped elsewhere).  Fresh
seeds on every shape the fixtures do not hold, compared bit for bit."""
import numpy as np
import pytest

from util import first_diff, same


@pytest.mark.parametrize("M,N,K,seed", [(1, 256, 1536, 101), (2, 160, 2048, 102), (3, 96, 6144, 103),
                                        (4, 64, 1536, 104), (5, 32, 1536, 105), (8, 32, 6144, 106)])
def test_w4g32_w4a8_live(orc, ref, M, N, K, seed):
    W = orc.rand_bytes(orc.stream(seed, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(seed, 2), N * K // 32).reshape(N, K // 32)
    X = orc.normal_f32(orc.stream(seed, 3), M * K, 3.0).reshape(M, K)
    a, b = orc.w4g32(W, S, X), ref.w4g32(W, S, X)
    assert same(a, b), first_diff(a, b)
    y8, q, sx, sm = ref.w4a8(W, S, X)
    qa, sxa, sma = orc.w4a8_quant(X)
    assert same(q, qa) and same(sx, sxa) and same(sm, sma)
    assert same(orc.w4a8(W, S, X), y8)


@pytest.mark.parametrize("ctx,M,T,window,sib,hd", [(1024, 4, 8, True, True, 256), (4097, 3, 16, False, False, 256),
                                                   (64, 1, 8, False, False, 256), (9, 4, 8, False, True, 256),
                                                   (2100, 4, 6, False, True, 512), (700, 1, 8, False, False, 512),
                                                   (33, 2, 6, False, False, 512)])
def test_attention_live(orc, ref, ctx, M, T, window, sib, hd):
    """attn_task + attn_merge (E:743-877, 1019-1059) at head dim 256 and 512 (global layers)"""
    nh = 8
    Kc = orc.normal_bf16(orc.stream(ctx, 11), (ctx + 8) * hd)
    Vc = orc.normal_bf16(orc.stream(ctx, 12), (ctx + 8) * hd)
    q = orc.normal_f32(orc.stream(ctx, 13), M * nh * hd, 1 / 16).reshape(M, nh * hd)
    pos0 = ctx - M
    pos = np.arange(pos0, pos0 + M, dtype=np.int32)
    rp = pos.copy()
    sl, sh = np.ones(M, np.int32), np.zeros(M, np.int32)
    if sib and M > 2:
        rp[-1], sl[-1], sh[-1] = pos0 + 1, pos0 + 1, pos0 + M - 2
    lo = np.array([max(0, r - 511) if window else 0 for r in rp], np.int32)
    kmax = pos0 + M - 1
    kmin = int(min(kmax, lo.min()))
    a, pma, pla = orc.attn(Kc, Vc, hd, nh, q, pos, lo, sl, sh, kmin, kmax, T, parts=True)
    b, pmb, plb = ref.attn(Kc, Vc, hd, nh, q, pos, lo, sl, sh, kmin, kmax, T, parts=True)
    assert same(pma, pmb) and same(pla, plb)
    assert same(a, b), first_diff(a, b)


def test_elementwise_live(orc, ref):
    x = np.concatenate([orc.normal_f32(orc.stream(55, 1), 65536, 20.0),
                        np.linspace(-120, 120, 65536, dtype=np.float32)]).astype(np.float32)
    assert same(orc.exp8(x), ref.vec("ref_exp8", x))
    assert same(orc.gelu8(x), ref.vec("ref_gelu8", x))
    assert same(orc.r16(x[:8192]), ref.vec("ref_rbf8", x[:8192]))
    for L in np.linspace(-35, 35, 141).astype(np.float32):
        assert orc.L.g4o_calc_thr(float(L)) == ref.L.ref_calc_thr(float(L))
