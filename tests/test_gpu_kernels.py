"""GPU parity of the individual verify-path kernels against the oracle (bit-exact).

Each case builds seeded inputs with the oracle's generators, runs the gfx950 kernel
through the C ABI and compares every output bit with the oracle, which is itself pinned
to the reference's own kernels (test_oracle_ref.py) and to the committed fixtures.
"""
import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu


def _w4(orc, seed, N, K):
    W = orc.rand_bytes(orc.stream(seed, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(seed, 2), N * K // 32).reshape(N, K // 32)
    return W, S


# (M, N, K): the verify shapes (q 2048, k/v 256, o K=2048, gate/up 6144, fused 12288, down K=6144)
GEMV_CASES = [(1, 1536, 1536), (2, 6144, 1536), (4, 1536, 6144), (8, 1536, 1536), (7, 2048, 1536),
              (3, 256, 2048), (4, 12288, 1536), (5, 512, 6144), (6, 1536, 2048), (8, 6144, 1536)]


@pytest.mark.parametrize("M,N,K", GEMV_CASES)
def test_w4g32_bit_exact(orc, dev, M, N, K):
    seed = 1000 * M + N + K
    W, S = _w4(orc, seed, N, K)
    X = orc.normal_f32(orc.stream(seed, 3), M * K).reshape(M, K)
    note(f"w4g32 M={M} N={N} K={K} seed={seed}")
    mat = dev.w4_upload(W, S)
    y = dev.w4g32(mat, X)
    yo = orc.w4g32(W, S, X)
    assert same(y, yo), first_diff(y, yo)


@pytest.mark.parametrize("M,Ns", [(7, (2048, 256, 256)), (1, (1536,)), (4, (512, 1536))])
def test_w4g32_multi_matches_single(orc, dev, M, Ns):
    """lin_multi's phase (E:310-317): the matrices of one launch give each matrix's own product"""
    K = 1536
    X = orc.normal_f32(orc.stream(900 + M, 3), M * K).reshape(M, K)
    WS = [_w4(orc, 900 + j, N, K) for j, N in enumerate(Ns)]
    mats = [dev.w4_upload(W, S) for W, S in WS]
    note(f"w4g32 multi M={M} N={Ns}")
    for (W, S), y in zip(WS, dev.w4g32_multi(mats, X)):
        yo = orc.w4g32(W, S, X)
        assert same(y, yo), first_diff(y, yo)
    with pytest.raises(RuntimeError):  # different K
        W2, S2 = _w4(orc, 999, 256, 2048)
        dev.w4g32_multi([mats[0], dev.w4_upload(W2, S2)], X)


def test_w4g32_bf16_inputs_and_repeat(orc, dev):
    """bf16-valued activations (the o/down inputs) and a second call on the same handle"""
    W, S = _w4(orc, 77, 1536, 2048)
    mat = dev.w4_upload(W, S)
    for M in (4, 1):
        X = orc.normal_bf16(orc.stream(77, M), M * 2048).astype(np.uint32) << 16
        X = X.view(np.float32).reshape(M, 2048)
        note(f"w4g32 bf16 inputs M={M}")
        assert same(dev.w4g32(mat, X), orc.w4g32(W, S, X))


def _norm_expected(orc, W, S, mode, o, xin, w1, w2, scalar):
    """the residual / RMS block between sub-blocks (E:1358-1361 mode 1, E:1375-1404 mode 2) and
    the product it feeds, composed from the oracle's rms and r16 (both pinned by golden vectors)"""
    M, H = o.shape
    xa = np.empty((M, H), np.float32)
    x1 = np.empty((M, H), np.float32)
    tmp = np.empty(H, np.float32)
    for i in range(M):
        oi = orc.r16(o[i])
        orc.L.g4o_rms(oi, w1.ctypes.data, H, tmp)
        x = orc.r16(xin[i] + orc.r16(tmp))
        if mode == 2:
            x = orc.r16(x * np.float32(scalar))
        orc.L.g4o_rms(np.ascontiguousarray(x), w2.ctypes.data, H, tmp)
        xa[i] = orc.r16(tmp) if mode == 1 else tmp
        x1[i] = x
    return orc.w4g32(W, S, xa), x1


def _norm_inputs(orc, kind, M, seed):
    """o, xin rows: 'normal' (one sum per lane in any order is exact), 'wide' (every lane needs
    the ordered chain: magnitudes from 2^-60 to 2^20), 'mixed' (a few lanes of each row wide),
    'edge' (a zero row, a one-element row, fp32 subnormals)"""
    H = 1536
    rng = np.random.default_rng(seed)
    o = orc.normal_f32(orc.stream(seed, 5), M * H).reshape(M, H)
    xin = orc.r16(orc.normal_f32(orc.stream(seed, 6), M * H).reshape(M, H) * 2)
    if kind == "wide":
        o = o * np.exp2(rng.integers(-60, 21, (M, H))).astype(np.float32)
        xin = orc.r16(xin * np.exp2(rng.integers(-60, 21, (M, H))).astype(np.float32))
    elif kind == "mixed":
        for i in range(M):
            j = rng.choice(H, 6, replace=False)
            o[i, j] *= np.float32(2.0 ** -40)
            xin[i, j] = orc.r16(xin[i, j] * np.float32(2.0 ** -45))
    elif kind == "edge":
        o[0] = 0
        if M > 1:
            o[1] = 0
            o[1, 17] = 3.0
        if M > 2:
            o[2, ::3] = np.float32(1e-40)
            xin[2, ::5] = 0
    return np.ascontiguousarray(o, np.float32), np.ascontiguousarray(xin, np.float32)


@pytest.mark.parametrize("mode,kind,M,rpb,tr", [
    (1, "normal", 7, 4, 64), (2, "normal", 7, 2, 64), (1, "wide", 7, 4, 64), (2, "wide", 7, 2, 64),
    (1, "mixed", 8, 3, 64), (2, "mixed", 5, 1, 64), (1, "edge", 3, 2, 32), (2, "edge", 7, 4, 32),
    (2, "wide", 1, 1, 32), (1, "mixed", 7, 4, 32)])
def test_norm_gemm_bit_exact(orc, dev, mode, kind, M, rpb, tr):
    """the norm prologue of the row-tile GEMV (both RMS factors, residual, layer scalar) against
    the oracle's composition, for sums that any order gives exactly and sums that need the
    reference's order"""
    seed = 500 + 10 * mode + M + rpb
    W, S = _w4(orc, seed, 256, 1536)
    o, xin = _norm_inputs(orc, kind, M, seed)
    w1 = orc.r16(0.5 + orc.normal_f32(orc.stream(seed, 7), 1536) ** 2 / 4)
    w2 = orc.r16(0.5 + orc.normal_f32(orc.stream(seed, 8), 1536) ** 2 / 4)
    note(f"norm gemm mode={mode} kind={kind} M={M} rows/block={rpb} tile={tr}")
    mat = dev.w4_upload(W, S)
    y, x1 = dev.w4g32_norm(mat, mode, o, xin, w1, w2, 0.75, rpb, tr)
    ye, x1e = _norm_expected(orc, W, S, mode, o, xin, w1, w2, 0.75)
    assert same(x1, x1e), first_diff(x1, x1e)
    assert same(y, ye), first_diff(y, ye)


def _attn_case(orc, ctx, M, T, window, tree, seed, hd=256):
    nh = 8
    Kc = orc.normal_bf16(orc.stream(seed, 1), (ctx + 8) * hd)
    Vc = orc.normal_bf16(orc.stream(seed, 2), (ctx + 8) * hd)
    q = orc.normal_f32(orc.stream(seed, 3), M * nh * hd, 1 / 16).reshape(M, nh * hd)
    pos0 = ctx
    pos = np.array([pos0 + m for m in range(M)], np.int32)
    rope = pos.copy()
    sl = np.ones(M, np.int32)
    sh = np.zeros(M, np.int32)
    if tree:  # rows na+1.. form branch b: RoPE by depth, skip chain a's slots
        na = (M - 1) // 2 + (M - 1) % 2
        for r in range(na + 1, M):
            rope[r] = pos0 + (r - na)
            sl[r] = pos0 + 1
            sh[r] = pos0 + na
    lo = np.array([max(0, rp - 511) if window else 0 for rp in rope], np.int32)
    kmax = pos0 + M - 1
    kmin = min(kmax, int(lo.min()))
    return Kc, Vc, hd, nh, q, pos, lo, sl, sh, kmin, kmax, T


ATTN_CASES = [(512, 4, 8, False, False), (2048, 4, 8, False, False), (6841, 4, 8, False, False),
              (2048, 4, 8, True, False), (6841, 4, 8, True, False), (2048, 7, 8, False, True),
              (2048, 7, 8, True, True), (300, 2, 6, False, False), (1000, 8, 16, True, True),
              (64, 1, 8, False, False)]


@pytest.mark.parametrize("ctx,M,T,window,tree", ATTN_CASES)
def test_attn_splitkv_bit_exact(orc, dev, ctx, M, T, window, tree):
    args = _attn_case(orc, ctx, M, T, window, tree, seed=ctx * 31 + M)
    note(f"attn ctx={ctx} M={M} T={T} window={window} tree={tree}")
    out = dev.attn(*args)
    ref = orc.attn(*args)
    assert same(out, ref), first_diff(out, ref)


@pytest.mark.parametrize("ctx,M,T,tree", [(700, 1, 8, False), (2048, 4, 6, False), (6841, 4, 8, False),
                                          (2048, 7, 8, True), (40, 3, 6, False), (1000, 8, 16, True)])
def test_attn_splitkv_hd512_bit_exact(orc, dev, ctx, M, T, tree):
    """the 512-wide global layers of the Gemma-4-E2B layout (E:1225): the same split geometry,
    chains over 32 steps"""
    args = _attn_case(orc, ctx, M, T, False, tree, seed=ctx * 17 + M, hd=512)
    note(f"attn hd=512 ctx={ctx} M={M} T={T} tree={tree}")
    out = dev.attn(*args)
    ref = orc.attn(*args)
    assert same(out, ref), first_diff(out, ref)


def _head_inputs(orc, V, seed):
    E = orc.normal_bf16(orc.stream(seed, 1), V * 1536, 0.02)
    P = orc.exp3_pack(E, V, 1536)
    scr = orc.screen_build(E, V, 1536)
    return E, P, scr


def _rows(orc, E, seed, kind, M):
    K = 1536
    if kind == "random":
        return orc.r16(orc.normal_f32(orc.stream(seed, 9), M * K)).reshape(M, K)
    # aligned with a few rows at varied strengths so the screen keeps tens of candidates
    rows = []
    for m in range(M):
        base = orc.bf2f(E[(777 + 13 * m) * K:(778 + 13 * m) * K]).astype(np.float32)
        noise = orc.normal_f32(orc.stream(seed, 20 + m), K, 1.0)
        rows.append(orc.r16(base * (12.0 + 8.0 * m) + noise))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("V,kind,M", [(16384, "random", 1), (16384, "aligned", 3), (32768, "aligned", 4),
                                      (16384, "random", 4)])
def test_head_argmax_bit_exact(orc, dev, V, kind, M):
    seed = V + M
    E, P, scr = _head_inputs(orc, V, seed)
    h = _rows(orc, E, seed, kind, M)
    note(f"head V={V} kind={kind} M={M}")
    dev.head_build(E, V)
    G, ns, fb = dev.head_argmax(h)
    for m in range(M):
        info, surv, sval = orc.head_row(h[m], scr, P, limit=30000, cap=30000)
        assert G[m] == info.G, (m, G[m], info.G)
        assert ns[m] == info.nsurv, (m, ns[m], info.nsurv)
        assert bool(fb[m]) == (info.nsurv > 30000)
        if info.nsurv <= 30000:
            idx, val, n = dev.head_survivors(m)
            assert n == info.nsurv
            assert same(idx, surv) and same(val, sval)


def test_head_full_vocab(orc, dev):
    """262,144-row head: random rows fall back to the full head, aligned rows are screened"""
    V = 262144
    E, P, scr = _head_inputs(orc, V, 5)
    h = np.concatenate([_rows(orc, E, 5, "random", 2), _rows(orc, E, 5, "aligned", 2)])
    note("head V=262144 random x2 + aligned x2")
    dev.head_build(E, V)
    G, ns, fb = dev.head_argmax(h)
    for m in range(4):
        info, surv, sval = orc.head_row(h[m], scr, P)
        assert G[m] == info.G and ns[m] == info.nsurv, (m, G[m], info.G, ns[m], info.nsurv)
    assert fb[0] == 1 and fb[1] == 1 and fb[2] == 0 and fb[3] == 0


def test_head_exp3_form(orc, dev):
    """the exp3 form the full head streams (x3sm / x3ix, laid out in the fma-lane order of the
    decoded head) carries exactly the oracle's X3 packing (X3:25-43): the codebook, every weight's
    sign|mantissa byte and codebook index (the nearest entry for an exception); and decoding it
    by the documented byte rule gives the decoded head weight for weight"""
    V, K = 16384, 1536
    E, P, _ = _head_inputs(orc, V, 31)
    note("exp3 form V=16384")
    dev.head_build(E, V)
    cb = dev.read("cb", np.uint8)
    assert same(cb, P["cb"])
    sm = dev.read("x3sm", np.uint32).reshape(V, 24, 8, 2)
    ix = dev.read("x3ix", np.uint32).reshape(V, 24, 8)
    dec = dev.read("dec", np.uint16).reshape(V, 24, 8, 8)
    # oracle X3 data: per (row, group) 32 sign|mantissa bytes then three 4-byte index bit planes
    data = P["data"].reshape(V, K // 32, 44)
    smo = data[:, :, :32]
    planes = data[:, :, 32:].copy().view(np.uint32).reshape(V, K // 32, 3)
    # entry (p, j), weight k: group 2p + k // 4, position [j, 16 + j, 8 + j, 24 + j][k % 4]
    j = np.arange(8)
    for k in range(8):
        g = 2 * np.arange(24)[:, None] + k // 4
        pos = np.array([0, 16, 8, 24])[k % 4] + j[None, :]
        want_sm = smo[:, g, pos]
        bits = (planes[:, g, :] >> pos[None, :, :, None].astype(np.uint32)) & 1
        want_ix = bits[..., 0] | (bits[..., 1] << 1) | (bits[..., 2] << 2)
        got_sm = (sm[..., k & 1] >> (8 * (k >> 1))) & 0xFF
        got_ix = (ix >> (8 * (k >> 1) + 4 * (k & 1))) & 0xF
        assert same(got_sm.astype(np.uint8), want_sm), k
        assert same(got_ix, want_ix.astype(np.uint32)), k
        bf = ((got_sm & 0x80) << 8) | (cb[got_ix].astype(np.uint32) << 7) | (got_sm & 0x7F)
        assert same(bf.astype(np.uint16), dec[..., k]), k
    assert P["ptr"][-1] > 0  # the fixture holds exceptions (nearest-entry indices are exercised)


def test_hbm_stream_probe(dev):
    """the device bandwidth probe (bench/stream_bw.cpp:10-19 method): a 2 GiB buffer, far past the
    last-level cache, read and copied at a rate between 1 TB/s and the 8 TB/s HBM peak"""
    note("hbm stream probe 2 GiB")
    rd = dev.hbm_stream(2 << 30, 5)
    cp = dev.hbm_stream(1 << 30, 5, copy=True)
    assert 1000.0 < rd < 8000.0, rd
    assert 1000.0 < cp < 8000.0, cp
    with pytest.raises(RuntimeError):
        dev.hbm_stream(1000, 1)


def test_head_build_vs_reference_engine(orc, dev):
    """the device's screen build (int4 bytes, bf16 scales, coefficients of all 262,144 rows)
    against the screen the reference engine's own main() builds (E:1235-1244;
    tests/golden/screen_build.npz from tests/golden/make_screen_build.py) on the seed-1
    embedding with rows of exact nearbyintf ties, near-ties, clamp ends and zero groups"""
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from golden_cases import HEAD_V, crc, screen_build_embedding
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "screen_build.npz"))
    E = screen_build_embedding(orc)
    assert crc(E) == int(g["crc_E"][0])
    note("head build V=262144 on the reference-engine fixture embedding")
    dev.head_build(E, HEAD_V)
    Wq = dev.read("Wq", np.uint8).reshape(HEAD_V, 768)
    Sq = dev.read("Sq", np.uint16).reshape(HEAD_V, 48)
    coef = dev.read("coef", np.float32)
    rows = g["rows"]
    assert same(Wq[rows], g["Wq_rows"]), first_diff(Wq[rows], g["Wq_rows"])
    assert same(Sq[rows], g["Sq_rows"]) and same(coef[rows], g["coef_rows"])
    assert crc(Wq) == int(g["crc_Wq"][0]) and crc(Sq) == int(g["crc_Sq"][0]) and crc(coef) == int(g["crc_coef"][0])
