"""Case list and seeded input construction shared by make_golden.py (which writes the
fixtures from the reference's kernels) and tests/test_golden.py (which checks the oracle
against them).  Inputs are rebuilt from seeds with the oracle's counter generator; the
fixtures store a CRC-32 of each input so both sides provably saw the same bytes."""
import zlib

import numpy as np

# (M, N, K, seed): verify-pass row counts 1..8, the q/k/v/o/gate/up shapes at K=1536, down K=6144
W4_CASES = [(1, 64, 1536, 1), (2, 96, 1536, 2), (3, 128, 1536, 3), (4, 256, 1536, 4), (5, 64, 6144, 5),
            (7, 64, 2048, 6), (8, 192, 1536, 7), (6, 32, 6144, 8)]
VEC_SEED = 31
CTHR_L = np.array([-50.0, -2.0, -0.3, 0.0, 0.1, 1.3, 2.718, 5.5, 9.9, 12.0, 17.0, 21.25, 25.0, 28.0, 29.5, 29.97,
                   30.0, 33.0, 40.0, 1e4], np.float32)
# (ctx, M, T, window, sibling row): the 4-row verify attention at 512/2048/6841, sliding-window
# 512, a sibling row with its skip range, a 6-way split and 2 rows (the reference's
# attention holds at most 4 rows, E:739)
ATTN_CASES = [(512, 4, 8, False, False), (2048, 4, 8, False, False), (700, 3, 8, True, False),
              (300, 4, 8, False, True), (6841, 4, 8, True, False), (200, 2, 6, False, False),
              (2048, 4, 8, True, True)]
GATEUP_CASE = (3, 256, 1536)
EXP3_CASE = (512, 1536, 42)
HEAD_V = 262144
SCREEN_SEED = 77
# synthetic stack (seed, V, layers, FFN, KV capacity, fake context length)
VERIFY_MODEL = (5, 262144, 2, 6144, 1024, 600)
# (chain length na, sibling length nb, pos0, draft kind)
VERIFY_CASES = [(3, 0, 600, "random"), (3, 3, 600, "random"), (3, 0, 600, "chain"), (3, 3, 600, "branch_b"),
                (1, 1, 610, "random")]


def crc(a):
    return zlib.crc32(np.ascontiguousarray(a).view(np.uint8).tobytes()) & 0xFFFFFFFF


def w4_inputs(o, M, N, K, seed):
    W = o.rand_bytes(o.stream(seed, 1), N * K // 2).reshape(N, K // 2)
    S = o.scales(o.stream(seed, 2), N * K // 32).reshape(N, K // 32)
    X = o.normal_f32(o.stream(seed, 3), M * K).reshape(M, K)
    return W, S, X


def vec_inputs(o):
    x = np.concatenate([o.normal_f32(o.stream(VEC_SEED, 1), 8192, 8.0),
                        o.normal_f32(o.stream(VEC_SEED, 2), 4096, 40.0),
                        np.linspace(-100, 100, 4096, dtype=np.float32)]).astype(np.float32)
    w = o.normal_f32(o.stream(VEC_SEED, 3), 1536, 0.5)
    cs = np.empty(64 * 128, np.float32)
    sn = np.empty(64 * 128, np.float32)
    o.L.g4o_rope_tables(64, 256, 1e4, 1.0, cs, sn)
    return x, w, cs, sn


def attn_inputs(o, ctx, M, T, window, sib):
    hd, nh = 256, 8
    Kc = o.normal_bf16(o.stream(ctx, 1), (ctx + 8) * hd)
    Vc = o.normal_bf16(o.stream(ctx, 2), (ctx + 8) * hd)
    q = o.normal_f32(o.stream(ctx + 100 * M, 3), M * nh * hd, 1 / 16).reshape(M, nh * hd)
    pos0 = ctx - M
    pos = np.array([pos0 + m for m in range(M)], np.int32)
    rope = pos.copy()
    sl = np.ones(M, np.int32)
    sh = np.zeros(M, np.int32)
    if sib:  # the last row is a depth-1 sibling: RoPE at pos0+1, skipping the chain rows
        rope[M - 1] = pos0 + 1
        sl[M - 1] = pos0 + 1
        sh[M - 1] = pos0 + M - 2
    lo = np.array([max(0, rp - 511) if window else 0 for rp in rope], np.int32)
    kmax = pos0 + M - 1
    return dict(K=Kc, V=Vc, q=q, pos=pos, lo=lo, sl=sl, sh=sh, kmin=int(min(kmax, lo.min())), kmax=kmax)


def gateup_inputs(o):
    M, I, K = GATEUP_CASE
    Wg = o.rand_bytes(o.stream(5, 11), I * K // 2).reshape(I, K // 2)
    Sg = o.scales(o.stream(6, 11), I * K // 32).reshape(I, K // 32)
    Wu = o.rand_bytes(o.stream(7, 11), I * K // 2).reshape(I, K // 2)
    Su = o.scales(o.stream(8, 11), I * K // 32).reshape(I, K // 32)
    X = o.r16(o.normal_f32(o.stream(9, 11), M * K)).reshape(M, K)
    return Wg, Sg, Wu, Su, X


def exp3_inputs(o):
    N, K, seed = EXP3_CASE
    E = o.normal_bf16(o.stream(seed, 1), N * K, 0.02)
    h = o.r16(o.normal_f32(o.stream(seed, 2), 4 * K)).reshape(4, K)
    return E, h


def screen_h(o, E):
    """rows 0-1: random (the screen keeps most of the vocabulary); rows 2-3: aligned with
    vocabulary rows 777 and 200001 so the screen prunes to a handful of survivors"""
    K = 1536
    rows = [o.r16(o.normal_f32(o.stream(SCREEN_SEED, 10 + m), K)) for m in range(2)]
    for m, n in ((2, 777), (3, 200001)):
        base = o.bf2f(E[n * K:(n + 1) * K]).astype(np.float32)
        rows.append(o.r16(base * 60 + o.normal_f32(o.stream(SCREEN_SEED, 10 + m), K, 0.3)))
    return np.stack(rows).astype(np.float32)


# ---- screen build run by the reference engine's own main() (E:1235-1244) ----
# embedding: the synthetic stack's E at seed 1 (V = 262,144, the bench workload's), with the rows
# of SCREEN_TIE_ROWS replaced by screen_tie_rows(): groups whose weights sit exactly on
# half-integer multiples of the group scale (nearbyintf's ties go to even), one bf16 step either
# side of such ties, groups at the clamp ends, zero groups and negative zeros.
SCREEN_BUILD_SEED = 1
SCREEN_TIE_ROWS = [17 + 10007 * i for i in range(24)]


def screen_tie_rows():
    """{row: 1536 bf16 bits}; every group g has amax = 7 * sc with sc a bf16 power of two or
    1.5 times one, so f2bf(amax / 7) == sc exactly and (k + 1/2) * sc divides to an exact tie"""
    rows = {}
    for r, n in enumerate(SCREEN_TIE_ROWS):
        vals = np.zeros(1536, np.float32)
        for g in range(48):
            kind = (r + g) % 6
            e = -12 + (r * 7 + g * 5) % 9                      # scale exponents 2^-12 .. 2^-4
            sc = np.float32(2.0 ** e) * (np.float32(1.5) if (g + r) % 2 else np.float32(1.0))
            w = np.zeros(32, np.float32)
            sign = np.float32(1.0 if (r + g) % 3 else -1.0)
            w[0] = sign * np.float32(7.0) * sc                 # the group's amax
            ks = np.arange(-7, 7, dtype=np.float32)            # ties (k + 1/2) sc, |.| <= 6.5 sc
            if kind == 0:                                      # ties only
                w[1:] = [(ks[i % 14] + np.float32(0.5)) * sc for i in range(31)]
            elif kind == 1:                                    # ties and exact multiples
                w[1:] = [(ks[i % 14] + np.float32(0.5 * (i % 2))) * sc for i in range(31)]
            elif kind == 2:                                    # one bf16 step above / below a tie
                for i in range(1, 32):
                    t = (ks[i % 14] + np.float32(0.5)) * sc
                    tb = np.float32(t).view(np.uint32)
                    step = np.uint32(1 << 16) if i % 2 else np.uint32(0)
                    if t != 0 and i % 4 >= 2:
                        tb = np.uint32(tb - (1 << 16)) if i % 2 else np.uint32(tb + (1 << 16))
                    else:
                        tb = np.uint32(tb + step)
                    w[i] = np.uint32(tb).view(np.float32)
            elif kind == 3:                                    # the clamp ends: -7 sc .. 7 sc, -6.5, 6.5
                w[1:] = [(-7.0, 7.0, -6.5, 6.5, -0.5, 0.5)[i % 6] * sc for i in range(31)]
            elif kind == 4:                                    # zero group (sc = 0), negative zeros
                w[:] = 0.0
                w[1::2] = -0.0
            else:                                              # ties at +-1/2, +-3/2 only
                w[1:] = [(-1.5, -0.5, 0.5, 1.5)[i % 4] * sc for i in range(31)]
            vals[g * 32:(g + 1) * 32] = w
        bits = (vals.view(np.uint32) >> 16).astype(np.uint16)
        assert np.all((vals.view(np.uint32) & 0xFFFF) == 0)
        rows[n] = bits
    return rows


def screen_build_embedding(o):
    """the 262,144 x 1536 bf16 embedding the reference engine builds its screen from"""
    from oracle import Model
    m = Model(o, SCREEN_BUILD_SEED, HEAD_V, 1, 512, 16)
    E = m.get("E", np.uint16, HEAD_V * 1536)
    m.close()
    for n, bits in screen_tie_rows().items():
        E[n * 1536:(n + 1) * 1536] = bits
    return E


# rows of the reference's screen kept verbatim in the fixture besides the tie rows
SCREEN_SAMPLE_ROWS = [0, 1, 777, 4095, 65536, 131071, 200001, 262143]


# ---- the long-prompt workload at its full size (bench.py --workload long_prompt) ----
LONG_PROMPT = dict(seed=1, V=262144, NL=35, I=6144, ctx=8192, dseed=2, rounds=256, ngram=3, nglen=3, k=3, dsplit=6,
                   nsplit=8)
