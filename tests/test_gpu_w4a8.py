"""GPU parity of the W4A8 path (w4a8::quant + w4a8::tile through i8_task) — bit-exact.

Three anchors:
- the golden vectors written from the reference's own AVX2 kernels (tests/golden/w4.npz);
- the oracle on fresh seeded shapes: the verify row counts M = 1..8 (ENGINE_DECODE_INT8 decode)
  and the prefill block sizes (M = 17, 64, 200) that take more than one MFMA row tile;
- the full prefill shape M = 6841 through rows the oracle recomputes on their own (every row
  of W4A8 depends only on its own activations, so any subset of rows is a complete check).
"""
import os
import sys

import numpy as np
import pytest

from conftest import note
from util import first_diff, same

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from golden_cases import W4_CASES, crc, w4_inputs  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("i", range(len(W4_CASES)))
def test_w4a8_golden(orc, dev, i):
    g = np.load(os.path.join(HERE, "golden", "w4.npz"), allow_pickle=False)
    M, N, K, seed = W4_CASES[i]
    W, S, X = w4_inputs(orc, M, N, K, seed)
    assert list(g[f"in_crc_{i}"]) == [crc(W), crc(S), crc(X)]
    note(f"w4a8 golden case {i}: M={M} N={N} K={K}")
    q, sx, sm = dev.w4a8_quant(X)
    assert same(q, g[f"w4a8_q_{i}"]) and same(sx, g[f"w4a8_sx_{i}"]) and same(sm, g[f"w4a8_sum_{i}"])
    y = dev.w4a8(dev.w4_upload(W, S), X)
    assert same(y, g[f"w4a8_{i}"]), first_diff(y, g[f"w4a8_{i}"])


# (M, N, K): decode rows 1..8 on the verify shapes, then prefill row blocks
A8_CASES = [(1, 1536, 1536), (2, 6144, 1536), (4, 1536, 6144), (8, 12288, 1536), (3, 256, 2048),
            (7, 2048, 1536), (17, 1536, 1536), (64, 2048, 1536), (200, 1536, 2048),
            # decode kernel: a full and a partial phase of 64 groups, six phases at M = 8; and
            # the 16-row tile kernel at M = 12
            (5, 512, 2560), (8, 256, 12288), (12, 512, 2560)]


@pytest.mark.parametrize("M,N,K", A8_CASES)
def test_w4a8_bit_exact(orc, dev, M, N, K):
    seed = 7000 + 10 * M + N + K
    W = orc.rand_bytes(orc.stream(seed, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(seed, 2), N * K // 32).reshape(N, K // 32)
    X = orc.normal_f32(orc.stream(seed, 3), M * K).reshape(M, K)
    note(f"w4a8 M={M} N={N} K={K} seed={seed}")
    y = dev.w4a8(dev.w4_upload(W, S), X)
    yo = orc.w4a8(W, S, X)
    assert same(y, yo), first_diff(y, yo)


def test_w4a8_quant_edges(orc, dev):
    """zero groups (sx = 0, inv = 0), exact half-way products (RNE), bf16-valued rows, a
    single large outlier per group and negative-only groups"""
    K = 1536
    rows = []
    z = np.zeros(K, np.float32)
    z[32:64] = orc.normal_f32(orc.stream(5, 1), 32)  # group 0 all zero, group 1 random
    rows.append(z)
    h = np.tile(np.array([127.0, 0.5, 1.5, -2.5, 3.5, -0.5, 63.5, -126.5], np.float32), K // 8)
    rows.append(h)  # amax 127 -> inv 1: every .5 is a tie
    b = orc.normal_bf16(orc.stream(5, 2), K).astype(np.uint32) << 16
    rows.append(b.view(np.float32))
    o = orc.normal_f32(orc.stream(5, 3), K, 0.01)
    o[::32] = 50.0
    rows.append(o)
    rows.append(-np.abs(orc.normal_f32(orc.stream(5, 4), K)))
    X = np.stack(rows).astype(np.float32)
    note("w4a8 quant edge rows")
    q, sx, sm = dev.w4a8_quant(X)
    qo, sxo, smo = orc.w4a8_quant(X)
    assert same(q, qo) and same(sx, sxo) and same(sm, smo)
    W = orc.rand_bytes(orc.stream(5, 5), 256 * K // 2).reshape(256, K // 2)
    S = orc.scales(orc.stream(5, 6), 256 * K // 32).reshape(256, K // 32)
    y = dev.w4a8(dev.w4_upload(W, S), X)
    assert same(y, orc.w4a8(W, S, X))


def test_w4a8_prefill_6841(orc, dev):
    """the long-prompt prefill GEMM in one launch (M = 6841, K = 1536 -> N = 1536); rows
    checked against the oracle: first, last, tile edges and seeded picks"""
    M, N, K, seed = 6841, 1536, 1536, 4242
    W = orc.rand_bytes(orc.stream(seed, 1), N * K // 2).reshape(N, K // 2)
    S = orc.scales(orc.stream(seed, 2), N * K // 32).reshape(N, K // 32)
    X = orc.normal_f32(orc.stream(seed, 3), M * K).reshape(M, K)
    note(f"w4a8 prefill M={M} N={N} K={K}")
    y = dev.w4a8(dev.w4_upload(W, S), X)
    rows = sorted(set([0, 1, 15, 16, 63, 64, 65, 6783, 6784, 6839, 6840] +
                      list(orc.ints(orc.stream(seed, 4), 21, 0, M - 1))))
    yo = orc.w4a8(W, S, X[rows])
    assert same(y[rows], yo), first_diff(y[rows], yo)
    assert np.all(np.isfinite(y))
