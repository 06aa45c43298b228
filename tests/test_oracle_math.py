"""The oracle against what the mathematics fixes, independently of its operation order.

These checks complement the bit-exact golden vectors (test_golden.py): each one is chosen so
that a plausible restatement mistake -- a swapped nibble, a dropped -8 offset, a wrong RoPE
pairing, a missing mask term, a loose or wrong screen coefficient, a wrong tie rule, a wrong
acceptance path -- fails it.  fp64 closed forms, round trips, bounds and brute force only.
"""
import math

import numpy as np
import pytest

from util import same

RNG = np.random.default_rng(20261201)


def bf16_to_f64(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def w4_dequant(W, S):
    """int4 G32 matrix to fp64: byte b of a row holds element 2b (low nibble) and 2b+1 (high),
    stored as q + 8; one bf16 scale per 32 elements"""
    N = W.shape[0]
    u = np.empty((N, W.shape[1] * 2), np.int64)
    u[:, 0::2] = W & 15
    u[:, 1::2] = W >> 4
    return (u - 8).astype(np.float64) * np.repeat(bf16_to_f64(S), 32, axis=1)


# ---------------------------------------------------------------------------------------------
# W4G32 / W4A8
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 64, 1536), (4, 96, 1536), (7, 32, 6144)])
def test_w4g32_closed_form_and_row_independence(orc, M, N, K):
    W = orc.rand_bytes(orc.stream(M * 7 + N, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(M * 7 + N, 2), N * K // 32).reshape(N, K // 32)
    X = orc.normal_f32(orc.stream(M * 7 + N, 3), M * K).reshape(M, K)
    Y = orc.w4g32(W, S, X)
    exact = X.astype(np.float64) @ w4_dequant(W, S).T
    scale = np.abs(X.astype(np.float64)) @ np.abs(w4_dequant(W, S)).T
    assert np.all(np.abs(Y - exact) <= 2e-6 * scale + 1e-6)
    for m in range(M):  # a row's result does not depend on the other rows of the pass
        assert same(orc.w4g32(W, S, X[m:m + 1])[0], Y[m])


def test_w4a8_integer_part(orc):
    M, N, K = 3, 64, 1536
    W = orc.rand_bytes(orc.stream(9, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(9, 2), N * K // 32).reshape(N, K // 32)
    X = orc.normal_f32(orc.stream(9, 3), M * K).reshape(M, K)
    q, sx, sm = orc.w4a8_quant(X)
    G = K // 32
    xg = X.reshape(M, G, 32).astype(np.float64)
    assert np.all(np.abs(q) <= 127)
    assert np.allclose(sx, np.abs(xg).max(axis=2) / 127, rtol=1e-6)
    assert np.all(np.abs(q.reshape(M, G, 32) * sx[:, :, None] - xg) <= 0.5 * sx[:, :, None] * (1 + 1e-5))
    assert np.array_equal(sm, q.reshape(M, G, 32).astype(np.int64).sum(axis=2))
    # y = sum_g sw * sx * sum (u - 8) q, the inner sum an exact integer
    u = np.empty((N, K), np.int64)
    u[:, 0::2], u[:, 1::2] = W & 15, W >> 4
    inner = np.einsum("ngk,mgk->mng", (u - 8).reshape(N, G, 32), q.reshape(M, G, 32).astype(np.int64))
    exact = (inner * bf16_to_f64(S)[None] * sx[:, None, :].astype(np.float64)).sum(axis=2)
    Y = orc.w4a8(W, S, X)
    assert np.all(np.abs(Y - exact) <= 1e-5 * np.abs(exact).max() + 1e-6)


# ---------------------------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------------------------
def test_bf16_round_nearest_even(orc):
    bits = np.concatenate([RNG.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32),
                           (RNG.integers(0, 2**16, 2000).astype(np.uint32) << 16) | 0x8000,  # exact ties
                           np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x80000000, 0x00000001], np.uint32)])
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    got = orc.r16(x).astype(np.float64)
    lo = (x.view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    step = ((x.view(np.uint32) & 0xFFFF0000) + 0x10000).view(np.float32).astype(np.float64)
    step = np.where(np.isinf(step), np.sign(step) * 2.0 ** 128, step)  # the value past the largest bf16
    xd = x.astype(np.float64)
    dl, dh = np.abs(xd - lo), np.abs(step - xd)
    even_lo = ((x.view(np.uint32) >> 16) & 1) == 0
    want = np.where(dl < dh, lo, np.where(dh < dl, step, np.where(even_lo, lo, step)))
    want = np.where(np.abs(want) == 2.0 ** 128, np.copysign(np.inf, want), want)  # IEEE overflow
    assert np.array_equal(got, want)


def test_exp8_gelu8_against_fp64(orc):
    x = np.concatenate([np.linspace(-87.0, 88.0, 20001), RNG.normal(0, 5, 4000)]).astype(np.float32)
    e = orc.exp8(x).astype(np.float64)
    assert np.all(np.abs(e - np.exp(x.astype(np.float64))) <= 4e-7 * np.exp(x.astype(np.float64)))
    assert orc.exp8(np.zeros(8, np.float32))[0] == 1.0
    xg = np.linspace(-12, 12, 24001).astype(np.float32)
    xd = xg.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(orc.gelu8(xg) - ref) <= 2e-6 * np.maximum(1, np.abs(xd)))


def test_rmsnorm_and_rope_against_fp64(orc):
    x = orc.normal_f32(orc.stream(3, 7), 1536, 2.0)
    w = (0.5 + RNG.random(1536)).astype(np.float32)
    y = np.empty(1536, np.float32)
    orc.L.g4o_rms(x, w.ctypes.data, 1536, y)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
    assert np.all(np.abs(y - ref) <= 1e-6 * np.abs(ref) + 1e-7)
    for rot, theta in ((1.0, 1e4), (0.25, 1e6)):
        cs = np.empty(700 * 128, np.float32)
        sn = np.empty(700 * 128, np.float32)
        orc.L.g4o_rope_tables(700, 256, theta, rot, cs, sn)
        h = orc.normal_f32(orc.stream(4, 7), 256)
        for p in (0, 1, 333, 699):
            g = h.copy()
            orc.L.g4o_rope(g, np.ascontiguousarray(cs[p * 128:(p + 1) * 128]), np.ascontiguousarray(sn[p * 128:(p + 1) * 128]), 256)
            j = np.arange(128)
            inv = np.where(j < int(256 * rot) // 2, theta ** (-2.0 * j / 256), 0.0)  # NeoX halves
            c, s = np.cos(p * inv), np.sin(p * inv)
            a, b = h[:128].astype(np.float64), h[128:].astype(np.float64)
            want = np.concatenate([a * c - b * s, b * c + a * s])
            assert np.all(np.abs(g - want) <= 1e-5 * (np.abs(a) + np.abs(b)).max())


def test_calc_thr_defining_property(orc):
    Ls = np.sort(np.concatenate([np.linspace(-40, 45, 341), [29.9, 29.99, 30.0, 31.5]])).astype(np.float32)
    prev = -np.inf
    for L in Ls:
        thr = np.float32(orc.L.g4o_calc_thr(float(L)))
        Lr = np.float32(orc.L.g4o_r16(float(L)))
        target = orc.L.g4o_cap(float(Lr))
        z = np.float32(thr + np.float32(0.25))
        assert orc.L.g4o_cap(orc.L.g4o_r16(float(z))) == target  # z keeps L's capped value
        assert z <= Lr
        for zz in np.linspace(float(Lr) - 64, float(z) - 1e-3 * max(1.0, abs(float(z))), 400).astype(np.float32):
            assert orc.L.g4o_cap(orc.L.g4o_r16(float(zz))) != target  # ... and is the smallest such z
        assert thr >= prev  # monotone in L
        prev = thr


# ---------------------------------------------------------------------------------------------
# split-KV attention
# ---------------------------------------------------------------------------------------------
def _attn_case(orc, ctx, M, seed):
    hd, nh = 256, 8
    Kc = orc.normal_bf16(orc.stream(seed, 1), ctx * hd)
    Vc = orc.normal_bf16(orc.stream(seed, 2), ctx * hd)
    q = orc.normal_f32(orc.stream(seed, 3), M * nh * hd, 1 / 16).reshape(M, nh * hd)
    return Kc, Vc, q


def _allowed(p, pos, lo, sl, sh):
    return lo <= p <= pos and not (sl <= p <= sh)


@pytest.mark.parametrize("window,sib", [(False, False), (True, False), (False, True)])
def test_attention_brute_force_fp64(orc, window, sib):
    ctx, M, hd, nh = 900, 4, 256, 8
    Kc, Vc, q = _attn_case(orc, ctx, M, 13)
    pos0 = ctx - M
    pos = np.arange(pos0, pos0 + M, dtype=np.int32)
    rp = pos.copy()
    sl, sh = np.ones(M, np.int32), np.zeros(M, np.int32)
    if sib:
        rp[-1], sl[-1], sh[-1] = pos0 + 1, pos0 + 1, pos0 + M - 2
    lo = np.array([max(0, r - 511) if window else 0 for r in rp], np.int32)
    kmax = pos0 + M - 1
    kmin = int(lo.min())
    out, pm, pl = orc.attn(Kc, Vc, hd, nh, q, pos, lo, sl, sh, kmin, kmax, 8, parts=True)
    K64 = bf16_to_f64(Kc).reshape(ctx, hd)
    V64 = bf16_to_f64(Vc).reshape(ctx, hd)
    for m in range(M):
        ps = [p for p in range(ctx) if _allowed(p, pos[m], lo[m], sl[m], sh[m])]
        for h in range(nh):
            s = K64[ps] @ q[m, h * hd:(h + 1) * hd].astype(np.float64)  # no 1/sqrt(d) scale
            w = np.exp(s - s.max())
            o = (w / w.sum()) @ V64[ps]
            got = out[m, h * hd:(h + 1) * hd]
            assert np.all(np.abs(got - o) <= 2.0 ** -8 * np.abs(o) + 1e-6), (m, h)
            # the per-split partials satisfy the log-sum-exp merge identity
            mx = pm[:, m, h].astype(np.float64)
            live = pl[:, m, h] > 0
            lsum = (pl[live, m, h] * np.exp(mx[live] - mx[live].max())).sum()
            assert abs(lsum - np.exp(s - mx[live].max()).sum()) <= 1e-5 * lsum


def test_attention_masks_and_split_count(orc):
    """positions outside [lo, pos] or inside the skip range cannot influence the output: giving
    them huge values leaves every bit unchanged; the split count moves results by at most one
    bf16 step"""
    ctx, M, hd, nh = 700, 4, 256, 8
    Kc, Vc, q = _attn_case(orc, ctx, M, 17)
    pos0 = ctx - M - 20  # positions beyond kmax exist in the cache
    pos = np.arange(pos0, pos0 + M, dtype=np.int32)
    lo = np.array([max(0, p - 511) for p in pos], np.int32)
    sl = np.array([1, 1, pos0 + 1, pos0 + 1], np.int32)
    sh = np.array([0, 0, pos0 + 1, pos0 + 2], np.int32)
    args = (hd, nh, q, pos, lo, sl, sh, int(lo.min()), pos0 + M - 1)
    base = orc.attn(Kc, Vc, *args, 8)
    Vb = Vc.reshape(ctx, hd).copy()
    big = np.uint16(0x4700)  # bf16 32768
    for p in range(ctx):
        if not any(_allowed(p, pos[m], lo[m], sl[m], sh[m]) for m in range(M)):
            Vb[p] = big
    assert same(orc.attn(Kc, Vb.ravel(), *args, 8), base)
    for m in range(M):  # row-wise: a position masked for row m only
        for p in (lo[m] - 1, pos[m] + 1, sl[m] if sl[m] <= sh[m] else None):
            if p is None or p < 0 or p >= ctx or _allowed(p, pos[m], lo[m], sl[m], sh[m]):
                continue
            Vr = Vc.reshape(ctx, hd).copy()
            Vr[p] = big
            assert same(orc.attn(Kc, Vr.ravel(), *args, 8)[m], base[m])
    for T in (1, 3, 16):
        o = orc.attn(Kc, Vc, *args, T)
        assert np.all(np.abs(o - base) <= 2.0 ** -7 * np.abs(base) + 1e-7)


# ---------------------------------------------------------------------------------------------
# exp3 head, screen soundness, tie rule
# ---------------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def small_head(orc):
    V, K = 4096, 1536
    E = orc.normal_bf16(orc.stream(23, 1), V * K, 0.02)
    return V, K, E, orc.exp3_pack(E, V, K), orc.screen_build(E, V, K)


def test_exp3_round_trip(orc, small_head):
    """decoding the packed head returns every bf16 weight exactly (one-hot activations)"""
    V, K, E, P, _ = small_head
    Ef = bf16_to_f64(E).reshape(V, K)
    cols = list(range(0, 32)) + list(RNG.choice(K, 64, replace=False))
    for c0 in range(0, len(cols), 4):
        X = np.zeros((4, K), np.float32)
        cc = cols[c0:c0 + 4]
        for i, c in enumerate(cc):
            X[i, c] = 1.0
        Y = orc.exp3_gemm(P, X)
        for i, c in enumerate(cc):
            assert np.array_equal(Y[i].astype(np.float64), Ef[:, c]), c


def test_exp3_codebook_is_most_frequent(orc, small_head):
    V, K, E, P, _ = small_head
    ex = (E >> 7) & 0xFF
    counts = np.bincount(ex, minlength=256)
    order = sorted(range(256), key=lambda e: (-counts[e], e))  # stable: ties by exponent
    assert list(P["cb"]) == order[:8]


def test_screen_bound_is_sound_and_tight(orc, small_head):
    """|exact logit - screen logit| <= coef * |h| on every row (Cauchy-Schwarz on the int4
    residual), with equality approached when h is the residual itself"""
    V, K, E, P, (Wq, Sq, coef) = small_head
    Ef = bf16_to_f64(E).reshape(V, K)
    Vq = w4_dequant(Wq.reshape(V, K // 2), Sq.reshape(V, K // 32))
    for seed in range(3):
        h = orc.r16(orc.normal_f32(orc.stream(29, seed), K))
        hn = math.sqrt(float((h.astype(np.float64) ** 2).sum()))
        s = orc.w4g32(Wq.reshape(V, K // 2), Sq.reshape(V, K // 32), h[None])[0].astype(np.float64)
        t = Ef @ h.astype(np.float64)
        assert np.all(np.abs(t - s) <= coef.astype(np.float64) * hn * (1 + 1e-5) + 1e-6)
    for n in (0, 1234, V - 1):
        r = (Ef[n] - Vq[n]).astype(np.float32)
        s = orc.w4g32(Wq.reshape(V, K // 2)[n:n + 1], Sq.reshape(V, K // 32)[n:n + 1], r[None])[0, 0]
        gap = abs(float(Ef[n] @ r.astype(np.float64)) - float(s))
        bound = float(coef[n]) * math.sqrt(float((r.astype(np.float64) ** 2).sum()))
        assert 0.99 * bound <= gap <= bound * (1 + 1e-5)
    # scales are bf16(amax / 7) and every in-range weight rounds to its nearest level
    sc = bf16_to_f64(Sq).reshape(V, K // 32)
    amax = np.abs(Ef).reshape(V, K // 32, 32).max(axis=2)
    assert np.array_equal(sc, bf16_to_f64(np.array([orc.L.g4o_f2bf(float(np.float32(a / 7))) for a in amax.ravel()],
                                                  np.uint16)).reshape(V, K // 32))
    inr = np.abs(Ef / np.repeat(np.where(sc > 0, sc, 1), 32, axis=1)) <= 7.5
    assert np.all(np.abs(Ef - Vq)[inr] <= 0.5 * np.repeat(sc, 32, axis=1)[inr] * (1 + 1e-6))


def _full_head_greedy(orc, P, h):
    """lowest index i with v_i >= max - 2 and cap(v_i) == cap(max) over all r16 logits"""
    lg = orc.r16(orc.exp3_gemm(P, h[None])[0])
    mx = lg.max()
    cm = orc.L.g4o_cap(float(mx))
    for i in np.flatnonzero(lg >= mx - 2):
        if orc.L.g4o_cap(float(lg[i])) == cm:
            return int(i), lg
    raise AssertionError("no candidate")


def test_screened_greedy_equals_full_head(orc, small_head):
    V, K, E, P, scr = small_head
    Ef = bf16_to_f64(E).reshape(V, K)
    rows = [orc.r16(orc.normal_f32(orc.stream(31, s), K)) for s in range(3)]
    for n in (7, 2048, 4095):  # aligned rows: the screen prunes to a handful of survivors
        rows.append(orc.r16((Ef[n] * 60 + RNG.normal(0, 0.3, K)).astype(np.float32)))
    for h in rows:
        info, surv, sval = orc.head_row(h, scr, P, seeds=[1, 2, 3], limit=30000)
        g, lg = _full_head_greedy(orc, P, h)
        assert info.G == g
        if not info.fallback:
            assert g in set(surv.tolist())
            assert same(sval, lg[surv])


# ---------------------------------------------------------------------------------------------
# greedy longest-prefix acceptance over the draft tree
# ---------------------------------------------------------------------------------------------
def brute_accept(toks, G, na, nb):
    """enumerate every path of the tree (row 0, then a prefix of chain a or of branch b) and
    keep the longest one whose every token is the greedy token of its predecessor"""
    best = ([0], 0)
    for br, rows in ((0, list(range(1, na + 1))), (1, list(range(na + 1, na + nb + 1)))):
        for k in range(1, len(rows) + 1):
            path = [0] + rows[:k]
            if all(G[path[i - 1]] >= 0 and toks[path[i]] == G[path[i - 1]] for i in range(1, len(path))):
                if len(path) > len(best[0]):
                    best = (path, br)
    path, br = best
    return len(path) - 1, (br if len(path) > 1 else 0), [G[r] for r in path]


def test_acceptance_brute_force(orc):
    from oracle import Model
    V, NL = 2048, 1
    m = Model(orc, 3, V, NL, 512, 256)
    try:
        m.fake_ctx(100, 7)
        cases = []
        for trial in range(24):
            na, nb = [(3, 3), (3, 0), (2, 2), (1, 1), (3, 1)][trial % 5]
            c = int(RNG.integers(0, V))
            # this stack's greedy token of a row is mostly the row's own token, so runs of c
            # are accepted; random cut points exercise every prefix length and both branches
            toks = [c] + [c if RNG.random() < 0.7 else int(RNG.integers(0, V)) for _ in range(na + nb)]
            cases.append((toks, na, nb))
        for toks, na, nb in cases:
            m.fake_ctx(100, 7)
            o, _ = m.verify(np.array(toks, np.int32), na, nb, 100, 8)
            G = list(o.G)
            nacc, br, commit = brute_accept(toks, G, na, nb)
            assert (o.nacc, o.branch, o.ncommit) == (nacc, br, nacc + 1), (toks, G)
            assert list(o.commit)[:o.ncommit] == commit
    finally:
        m.close()
