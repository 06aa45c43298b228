"""MTP drafter step (E:1534-1563): the oracle against the reference's own kernels composed as
draft_step composes them (oracle/_ref), on a synthetic drafter over a 15-layer synthetic target."""
import numpy as np
import pytest

from util import first_diff, same

RNG = np.random.default_rng(21)


def bf16_rows(shape, scale=1.0):
    x = (RNG.standard_normal(shape) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("N,K", [(256, 3072), (1024, 256), (2048, 256), (256, 2048), (37, 256)])
def test_b16_gemv_vs_reference(orc, ref, N, K):
    W = bf16_rows((N, K), 0.05)
    x = RNG.standard_normal(K).astype(np.float32)
    y = np.empty(N, np.float32)
    orc.L.g4o_b16_gemv(W, N, K, x, y)
    assert same(y, ref.b16(W, x)), first_diff(y, ref.b16(W, x))


def test_b16_gemv_closed_form(orc):
    W = bf16_rows((64, 512), 0.05)
    x = RNG.standard_normal(512).astype(np.float32)
    y = np.empty(64, np.float32)
    orc.L.g4o_b16_gemv(W, 64, 512, x, y)
    want = ((W.astype(np.uint32) << 16).view(np.float32).astype(np.float64) @ x.astype(np.float64))
    assert np.max(np.abs(y - want)) < 1e-4


def test_drafter_order_is_a_permutation(orc):
    from oracle import Drafter
    d = Drafter(orc, 3, 4096)
    try:
        import ctypes
        order = np.frombuffer((ctypes.c_int64 * 4096).from_address(d.ptr("order")), np.int64)
        assert sorted(order.tolist()) == list(range(4096))
    finally:
        d.close()


@pytest.mark.parametrize("P,T", [(300, 6), (700, 8), (40, 6)])
def test_draft_step_vs_reference(orc, ref, P, T):
    from oracle import Drafter, Model
    V, NL, I, ctx, seed = 4096, 15, 512, 1024, 13
    m = Model(orc, seed, V, NL, I, ctx)
    d = Drafter(orc, seed + 1, V)
    try:
        m.fake_ctx(P + 1, 777)
        ref.bind_model(m)
        ref.bind_drafter(d)
        tok = 123
        h = (RNG.standard_normal(1536).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
        for j in range(3):  # a chain: each step feeds its token and hidden state to the next
            t_o, b_o, s_o, g_o = d.step(m, tok, h, P + 1 + j, P, T)
            t_r, b_r, s_r, g_r = ref.draft_step(tok, h, P + 1 + j, P, T)
            assert (t_o, s_o) == (t_r, s_r) and np.float32(g_o).view(np.uint32) == np.float32(g_r).view(np.uint32), j
            assert same(b_o, b_r), first_diff(b_o, b_r)
            tok, h = t_o, b_o
    finally:
        d.close()
        m.close()
