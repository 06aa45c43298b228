"""GPU parity of the allocation-free split-KV attention entry point (g4v_attn_splitkv_noalloc)
against g4v_attn_splitkv and the oracle's split-KV attention (E:743-877, E:1019-1059) on the same
inputs: device buffers in and out, scratch in the library's file-scope device array, two calls in
a row with the second on a smaller input (the scratch keeps the first call's contents), bit for
bit."""
import ctypes as C

import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu


class _Hip:
    """device buffers for the test through the HIP runtime the library itself links"""

    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        self.bufs = []

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = C.c_void_p()
        assert self.L.hipMalloc(C.byref(p), C.c_size_t(max(a.nbytes, 16))) == 0
        self.bufs.append(p)
        assert self.L.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) == 0  # host to device
        return p.value

    def get(self, ptr, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.L.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(out.nbytes), 2) == 0
        return out

    def free(self):
        for p in self.bufs:
            self.L.hipFree(p)
        self.bufs = []


def _case(orc, npos, M, T, window, seed):
    hd, nh = 256, 8
    Kc = orc.normal_bf16(orc.stream(seed, 1), npos * hd)
    Vc = orc.normal_bf16(orc.stream(seed, 2), npos * hd)
    q = orc.normal_f32(orc.stream(seed, 3), M * nh * hd, 1 / 16).reshape(M, nh * hd)
    pos0 = npos - M
    pos = np.array([pos0 + m for m in range(M)], np.int32)
    lo = np.array([max(0, p - 511) if window else 0 for p in pos], np.int32)
    sl, sh = np.ones(M, np.int32), np.zeros(M, np.int32)
    kmax = pos0 + M - 1
    return Kc, Vc, q, pos, lo, sl, sh, int(min(kmax, lo.min())), kmax, T


def test_noalloc_matches_attn_splitkv(orc, dev):
    hip = _Hip()
    try:
        for npos, M, T, window, seed in ((3000, 7, 8, False, 5), (900, 3, 6, True, 6)):
            note(f"attn noalloc npos={npos} M={M} T={T} window={window}")
            Kc, Vc, q, pos, lo, sl, sh, kmin, kmax, T = _case(orc, npos, M, T, window, seed)
            want = dev.attn(Kc, Vc, 256, 8, q, pos, lo, sl, sh, kmin, kmax, T)
            od = hip.put(np.full((M, 2048), np.nan, np.float32))
            dev.attn_noalloc(hip.put(Kc), hip.put(Vc), npos, hip.put(q), M, pos, lo, sl, sh, kmin, kmax, T, od)
            got = hip.get(od, (M, 2048), np.float32)
            assert same(got, want), first_diff(got, want)
            ref = orc.attn(Kc, Vc, 256, 8, q, pos, lo, sl, sh, kmin, kmax, T)
            assert same(got, ref), first_diff(got, ref)
    finally:
        hip.free()


def test_noalloc_rejects_beyond_scratch(orc, dev):
    """more positions than the scratch holds: a clear error, nothing launched"""
    hip = _Hip()
    try:
        kd = hip.put(np.zeros(4097 * 256, np.uint16))
        qd = hip.put(np.zeros((1, 2048), np.float32))
        z = np.zeros(1, np.int32)
        with pytest.raises(RuntimeError, match="4096 positions"):
            dev.attn_noalloc(kd, kd, 4097, qd, 1, z + 4096, z, z + 1, z, 0, 4096, 8, qd)
    finally:
        hip.free()
