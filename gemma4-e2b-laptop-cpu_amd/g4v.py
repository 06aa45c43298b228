"""ctypes binding of libg4v.so (include/g4v.h): the gfx950 speculative-verify path.

Mirrors the reference engine's kernel-call surface (engine/gemma4_engine.cpp and the
w4g32 / w4a8 / bf16_exp3_head headers) one entry point per reference function; arrays are
numpy, all device memory is owned by the library.  There is no CPU fallback: loading fails
loudly when libg4v.so is missing.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libg4v.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_vp = C.c_void_p
_i = C.c_int

# every symbol include/g4v.h declares, with its ctypes signature
SIGNATURES = {
    "g4v_create": (_i, [_i, C.POINTER(_vp)]),
    "g4v_destroy": (None, [_vp]),
    "g4v_error": (C.c_char_p, [_vp]),
    "g4v_device_info": (_i, [_vp, C.c_char_p, _i, C.POINTER(_i), C.POINTER(_i)]),
    "g4v_w4_upload": (_i, [_vp, _u8p, _u16p, _i, _i]),
    "g4v_w4g32_gemm": (_i, [_vp, _i, _f32p, _i, _f32p]),
    "g4v_w4g32_bench": (_i, [_vp, _i, _i, _i, C.POINTER(C.c_float)]),
    "g4v_model_create_gemma": (_i, [_vp, _i, _i32p, _i]),
    "g4v_model_synth_gemma": (_i, [_vp, C.c_uint64, _i, _i32p, _i]),
    "g4v_model_set_norms_gemma": (_i, [_vp, _i, C.POINTER(C.c_void_p), C.c_float]),
    "g4v_model_set_ple": (_i, [_vp, _u8p, _u16p, _f32p]),
    "g4v_model_set_ple_rows": (_i, [_vp, _i, _i, _u16p]),
    "g4v_w4g32_gemm_multi": (_i, [_vp, _i, _i32p, _f32p, _i, C.POINTER(C.c_void_p)]),
    "g4v_w4g32_norm_gemm": (_i, [_vp, _i, _i, _f32p, _f32p, _f32p, _f32p, C.c_float, _i, _i, _i, _f32p, _f32p]),
    "g4v_w4a8_quant": (_i, [_vp, _f32p, _i, _i, _vp, _f32p, _i32p]),
    "g4v_w4a8_gemm": (_i, [_vp, _i, _f32p, _i, _f32p]),
    "g4v_w4a8_bench": (_i, [_vp, _i, _i, _i, C.POINTER(C.c_float)]),
    "g4v_w4g32_time": (_i, [_vp, _i, _i32p, _i, _i, _i, C.POINTER(C.c_float)]),
    "g4v_attn_time": (_i, [_vp, _i, _i, _i, _i, _i, _i, C.POINTER(C.c_float)]),
    "g4v_head_time": (_i, [_vp, _f32p, _i, _i, C.POINTER(C.c_float), _i32p, _i32p]),
    "g4v_attn_splitkv": (_i, [_vp, _u16p, _u16p, _i, _i, _i, _i, _f32p, _i32p, _i32p, _i32p, _i32p,
                              _i, _i, _i, _f32p]),
    "g4v_attn_splitkv_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _i32p, _i32p, _i32p, _i32p,
                                      _i, _i, _i, _vp]),
    "g4v_head_build": (_i, [_vp, _u16p, _i]),
    "g4v_head_argmax": (_i, [_vp, _f32p, _i, _i32p, _i32p, _i32p]),
    "g4v_head_survivors": (_i, [_vp, _i, _i32p, _f32p, _i, C.POINTER(_i)]),
    "g4v_model_synth": (_i, [_vp, C.c_uint64, _i, _i, _i, _i]),
    "g4v_model_create": (_i, [_vp, _i, _i, _i, _i]),
    "g4v_model_set_embed": (_i, [_vp, _u16p]),
    "g4v_model_set_matrix": (_i, [_vp, _i, _i, _u8p, _u16p]),
    "g4v_model_set_norms": (_i, [_vp, _i, C.POINTER(_vp), C.c_float, _i]),
    "g4v_model_set_final_norm": (_i, [_vp, _f32p]),
    "g4v_model_set_kv": (_i, [_vp, _i, _i, _i, _u16p, _u16p]),
    "g4v_model_fake_ctx": (_i, [_vp, _i, C.c_uint64]),
    "g4v_model_read": (_i, [_vp, C.c_char_p, _vp, C.c_size_t, C.POINTER(C.c_size_t)]),
    "g4v_verify_step": (_i, [_vp, _i32p, _i, _i, _i, _i, _vp, _vp]),
    "g4v_verify_sibling": (_i, [_vp, _i32p, _i, _i, _i, _i, _vp, _vp]),
    "g4v_profile": (_i, [_vp, C.c_uint]),
    "g4v_profile_read": (_i, [_vp, _vp, _vp, _vp, _i]),
    "g4v_prefill_head_stats": (_i, [_vp, _i32p, _i32p]),
    "g4v_hbm_stream": (_i, [_vp, C.c_size_t, _i, _i, _vp]),
    "g4v_sync": (_i, [_vp]),
    "g4v_set_graphs": (_i, [_vp, _i]),
    "g4v_set_prefill_int8": (_i, [_vp, _i]),
    "g4v_set_decode_int8": (_i, [_vp, _i]),
    "g4v_set_draft_samepos": (_i, [_vp, _i]),
    "g4v_prefill": (_i, [_vp, _i32p, _i, _i, _i, _i, C.POINTER(_i), _vp]),
    "g4v_drafter_synth": (_i, [_vp, C.c_uint64]),
    "g4v_drafter_load": (_i, [_vp, _vp]),
    "g4v_draft_mtp": (_i, [_vp, _i, _vp, _i, _i, _i, _i32p, _vp, _vp, _vp]),
    "g4v_slots_init": (_i, [_vp, _i, _i]),
    "g4v_slot_begin": (_i, [_vp, _i32p, _i, C.POINTER(_i), C.POINTER(_i)]),
    "g4v_slot_end": (_i, [_vp, _i32p, _i, _vp, _i, _i]),
    "g4v_history_set": (_i, [_vp, _i32p, _i]),
    "g4v_prompt_lookup": (_i, [_vp, _i32p, _i, _i, _i, _i32p, C.POINTER(_i)]),
    "g4v_history_read": (_i, [_vp, _vp, _i, C.POINTER(_i)]),
    "g4v_expf_selftest": (C.c_longlong, [C.c_uint32, C.c_uint32, C.c_uint32]),
}

# kernel classes of g4v_profile (include/g4v.h)
PROF_TAGS = ["gemv_qkv", "gemv_o", "gemv_gateup", "gemv_down", "attn", "rows", "head_screen", "head_select",
             "head_rescore", "head_full", "head_tie", "accept", "head_pass2"]


class DrafterTensors(C.Structure):
    """g4v_drafter_tensors (include/g4v.h)"""
    _fields_ = [(n, _vp) for n in ("pre", "post", "cent", "emb", "norm", "order")] + \
               [(n, _vp * 4) for n in ("q", "o", "gate", "up", "down")] + \
               [("nv", (_vp * 5) * 4), ("scalar", C.c_uint16 * 4), ("C", C.c_int32), ("hd", C.c_int32 * 4)]


class VerifyResult(C.Structure):
    _fields_ = [("nacc", _i), ("branch", _i), ("ncommit", _i), ("commit", _i * 8), ("G", _i * 8),
                ("fallback", _i * 8), ("nsurv", _i * 8)]

    def as_dict(self):
        return dict(nacc=self.nacc, branch=self.branch, ncommit=self.ncommit,
                    commit=list(self.commit)[: self.ncommit], G=list(self.G),
                    fallback=list(self.fallback), nsurv=list(self.nsurv))


_LIB = None


def load(path=LIB_PATH):
    """Load libg4v.so (raises when it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() (make -C {HERE})")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class Device:
    """One library context on one HIP device (the engine's Pool + buffers, on the GPU)."""

    def __init__(self, device=0):
        self.L = load()
        h = _vp()
        rc = self.L.g4v_create(device, C.byref(h))
        if rc != 0:
            raise RuntimeError(f"g4v_create failed ({rc})")
        self.h = h

    def close(self):
        if self.h:
            self.L.g4v_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.L.g4v_error(self.h).decode()} ({rc})")

    def info(self):
        name = C.create_string_buffer(256)
        cus, lds = _i(), _i()
        self._ok(self.L.g4v_device_info(self.h, name, 256, C.byref(cus), C.byref(lds)), "device_info")
        return dict(name=name.value.decode(), cus=cus.value, lds_per_block=lds.value)

    # ---- W4G32 (Q4 + gemm_rows_tile) ----
    def w4_upload(self, W, S):
        W = _c(W, np.uint8)
        S = _c(S, np.uint16)
        N = W.shape[0]
        K = W.shape[1] * 2
        h = self.L.g4v_w4_upload(self.h, W, S, N, K)
        if h < 0:
            self._ok(h, "w4_upload")
        return h, N, K

    def w4g32(self, mat, X):
        h, N, K = mat
        X = _c(X, np.float32)
        M = X.shape[0]
        assert X.shape[1] == K
        Y = np.empty((M, N), np.float32)
        self._ok(self.L.g4v_w4g32_gemm(self.h, h, X, M, Y), "w4g32_gemm")
        return Y

    def w4g32_norm(self, mat, mode, o, xin, w1, w2, scalar, rows_per_block=2, tile_rows=64):
        h, N, K = mat
        o, xin = _c(o, np.float32), _c(xin, np.float32)
        M = o.shape[0]
        Y = np.empty((M, N), np.float32)
        X1 = np.empty((M, K), np.float32)
        self._ok(self.L.g4v_w4g32_norm_gemm(self.h, h, mode, o, xin, _c(w1, np.float32), _c(w2, np.float32),
                                            scalar, M, rows_per_block, tile_rows, Y, X1), "w4g32_norm_gemm")
        return Y, X1

    def w4g32_multi(self, mats, X):
        X = _c(X, np.float32)
        M = X.shape[0]
        hs = np.array([m[0] for m in mats], np.int32)
        Ys = [np.empty((M, m[1]), np.float32) for m in mats]
        ptrs = (C.c_void_p * len(mats))(*[y.ctypes.data for y in Ys])
        self._ok(self.L.g4v_w4g32_gemm_multi(self.h, len(mats), hs, X, M, ptrs), "w4g32_gemm_multi")
        return Ys

    def w4g32_bench(self, mat, M, iters=100):
        us = C.c_float()
        self._ok(self.L.g4v_w4g32_bench(self.h, mat[0], M, iters, C.byref(us)), "w4g32_bench")
        return us.value

    # ---- W4A8 (w4a8::quant + w4a8::tile through i8_task) ----
    def w4a8_quant(self, X):
        X = _c(X, np.float32)
        M, K = X.shape
        q = np.empty((M, K), np.int8)
        sx = np.empty((M, K // 32), np.float32)
        sm = np.empty((M, K // 32), np.int32)
        self._ok(self.L.g4v_w4a8_quant(self.h, X, M, K, q.ctypes.data, sx, sm), "w4a8_quant")
        return q, sx, sm

    def w4a8(self, mat, X):
        h, N, K = mat
        X = _c(X, np.float32)
        M = X.shape[0]
        assert X.shape[1] == K
        Y = np.empty((M, N), np.float32)
        self._ok(self.L.g4v_w4a8_gemm(self.h, h, X, M, Y), "w4a8_gemm")
        return Y

    def w4g32_time(self, mats, M, iters=50, cold=False, w4a8=False):
        """device us per launch of the row-tile GEMV (w4a8: the W4A8 product) over the matrices
        `mats` (handles) on M rows"""
        us = C.c_float()
        h = np.array([m[0] for m in mats], np.int32)
        fl = (1 if cold else 0) | (2 if w4a8 else 0)
        self._ok(self.L.g4v_w4g32_time(self.h, len(mats), h, M, iters, fl, C.byref(us)), "w4g32_time")
        return us.value

    def attn_time(self, npos, M, T=8, window=False, iters=50, cold=False):
        """device us per split-KV attention (split + merge) of M rows at the end of npos positions"""
        us = C.c_float()
        self._ok(self.L.g4v_attn_time(self.h, npos, M, T, 1 if window else 0, iters, 1 if cold else 0, C.byref(us)),
                 "attn_time")
        return us.value

    def head_time(self, h, iters=20, cold=False):
        """(device us per head pass of row h, its survivors, whether it fell back to the full head)"""
        us = C.c_float()
        ns = np.zeros(1, np.int32)
        fb = np.zeros(1, np.int32)
        self._ok(self.L.g4v_head_time(self.h, _c(h, np.float32), iters, 1 if cold else 0, C.byref(us), ns, fb),
                 "head_time")
        return us.value, int(ns[0]), bool(fb[0])

    def w4a8_bench(self, mat, M, iters=100):
        us = C.c_float()
        self._ok(self.L.g4v_w4a8_bench(self.h, mat[0], M, iters, C.byref(us)), "w4a8_bench")
        return us.value

    # ---- split-KV attention ----
    def attn(self, Kc, Vc, hd, nh, q, pos, lo, skip_lo, skip_hi, kmin, kmax, T):
        Kc = _c(Kc, np.uint16)
        Vc = _c(Vc, np.uint16)
        q = _c(q, np.float32)
        M = q.shape[0]
        npos = Kc.size // hd
        out = np.empty((M, nh * hd), np.float32)
        self._ok(self.L.g4v_attn_splitkv(self.h, Kc, Vc, npos, hd, nh, M, q, _c(pos, np.int32), _c(lo, np.int32),
                                         _c(skip_lo, np.int32), _c(skip_hi, np.int32), kmin, kmax, T, out),
                 "attn_splitkv")
        return out

    def attn_noalloc(self, Kd, Vd, npos, q_d, M, pos, lo, skip_lo, skip_hi, kmin, kmax, T, out_d):
        """g4v_attn_splitkv_noalloc on device pointers (Kd, Vd, q_d, out_d: integers)"""
        self._ok(self.L.g4v_attn_splitkv_noalloc(self.h, Kd, Vd, npos, 256, 8, M, q_d, _c(pos, np.int32),
                                                 _c(lo, np.int32), _c(skip_lo, np.int32), _c(skip_hi, np.int32),
                                                 kmin, kmax, T, out_d), "attn_splitkv_noalloc")

    # ---- head ----
    def head_build(self, E, V):
        self._ok(self.L.g4v_head_build(self.h, _c(E, np.uint16), V), "head_build")

    def head_argmax(self, h):
        h = _c(h, np.float32).reshape(-1, 1536)
        M = h.shape[0]
        G = np.empty(M, np.int32)
        ns = np.empty(M, np.int32)
        fb = np.empty(M, np.int32)
        self._ok(self.L.g4v_head_argmax(self.h, h, M, G, ns, fb), "head_argmax")
        return G, ns, fb

    def head_survivors(self, m, cap=30000):
        idx = np.empty(cap, np.int32)
        val = np.empty(cap, np.float32)
        n = _i()
        self._ok(self.L.g4v_head_survivors(self.h, m, idx, val, cap, C.byref(n)), "head_survivors")
        k = min(n.value, cap)
        return idx[:k].copy(), val[:k].copy(), n.value

    # ---- model + verify ----
    def model_synth(self, seed, V, NL, I=6144, ctxcap=4096):
        self._ok(self.L.g4v_model_synth(self.h, seed, V, NL, I, ctxcap), "model_synth")

    def model_create(self, V, NL, I=6144, ctxcap=4096):
        """an empty stack; fill it with set_embed / set_matrix / set_norms / set_final_norm"""
        self._ok(self.L.g4v_model_create(self.h, V, NL, I, ctxcap), "model_create")

    def set_embed(self, E):
        self._ok(self.L.g4v_model_set_embed(self.h, _c(E, np.uint16)), "model_set_embed")

    def set_matrix(self, layer, j, w, s):
        self._ok(self.L.g4v_model_set_matrix(self.h, layer, j, _c(w, np.uint8), _c(s, np.uint16)),
                 "model_set_matrix")

    def set_norms(self, layer, norms, scalar, sliding):
        """norms: in_ln, post_attn, pre_ff, post_ff [1536] and q_norm, k_norm [256]"""
        arrs = [_c(v, np.float32) for v in norms]
        ptrs = (_vp * 6)(*[a.ctypes.data for a in arrs])
        self._ok(self.L.g4v_model_set_norms(self.h, layer, ptrs, scalar, 1 if sliding else 0), "model_set_norms")

    def model_create_gemma(self, V, mlp, ctxcap=4096):
        self._ok(self.L.g4v_model_create_gemma(self.h, V, _c(mlp, np.int32), ctxcap), "model_create_gemma")

    def model_synth_gemma(self, seed, V, mlp, ctxcap=4096):
        """the Gemma-4-E2B layout with device-generated weights"""
        self._ok(self.L.g4v_model_synth_gemma(self.h, seed, V, _c(mlp, np.int32), ctxcap), "model_synth_gemma")

    def set_norms_gemma(self, layer, norms, scalar):
        """norms: 7 float vectors (k_norm None past layer 14)"""
        keep = [None if v is None else _c(v, np.float32) for v in norms]
        arr = (C.c_void_p * 7)(*[None if v is None else v.ctypes.data for v in keep])
        self._ok(self.L.g4v_model_set_norms_gemma(self.h, layer, arr, scalar), "model_set_norms_gemma")

    def set_ple(self, w, s, plnorm):
        self._ok(self.L.g4v_model_set_ple(self.h, _c(w, np.uint8), _c(s, np.uint16), _c(plnorm, np.float32)),
                 "model_set_ple")

    def set_ple_rows(self, tok0, rows):
        rows = _c(rows, np.uint16)
        self._ok(self.L.g4v_model_set_ple_rows(self.h, tok0, rows.shape[0], rows), "model_set_ple_rows")

    def set_final_norm(self, w):
        self._ok(self.L.g4v_model_set_final_norm(self.h, _c(w, np.float32)), "model_set_final_norm")

    def set_kv(self, layer, pos0, K, V):
        K, V = _c(K, np.uint16), _c(V, np.uint16)
        self._ok(self.L.g4v_model_set_kv(self.h, layer, pos0, K.size // 256, K, V), "model_set_kv")

    def fake_ctx(self, n, seed=12345):
        self._ok(self.L.g4v_model_fake_ctx(self.h, n, seed), "model_fake_ctx")

    def read(self, what, dtype):
        nb = C.c_size_t()
        self._ok(self.L.g4v_model_read(self.h, what.encode(), None, 0, C.byref(nb)), f"model_read {what}")
        out = np.empty(nb.value // np.dtype(dtype).itemsize, dtype)
        self._ok(self.L.g4v_model_read(self.h, what.encode(), out.ctypes.data, out.nbytes, C.byref(nb)),
                 f"model_read {what}")
        return out

    # ---- prefill ----
    def prefill(self, toks, pos0=0, pfb=32, nsplit=8, hidden=False):
        """prompt pass; returns the first generated token (and the last row's hidden state)"""
        toks = _c(toks, np.int32)
        g0 = _i()
        hid = np.empty(1536, np.float32)
        self._ok(self.L.g4v_prefill(self.h, toks, toks.size, pos0, pfb, nsplit, C.byref(g0), hid.ctypes.data),
                 "prefill")
        return (g0.value, hid) if hidden else g0.value

    # ---- MTP drafter ----
    def drafter_synth(self, seed):
        self._ok(self.L.g4v_drafter_synth(self.h, seed), "drafter_synth")

    def drafter_load(self, t):
        """t: dict of the drafter checkpoint's arrays (DrafterTensors names; per-layer lists)"""
        keep = []

        def p(a, dt):
            a = np.ascontiguousarray(a, dt)
            keep.append(a)
            return a.ctypes.data

        dt = DrafterTensors()
        for n in ("pre", "post", "cent", "emb", "norm"):
            setattr(dt, n, p(t[n], np.uint16))
        dt.order = p(t["order"], np.int64)
        for n in ("q", "o", "gate", "up", "down"):
            arr = getattr(dt, n)
            for l in range(4):
                arr[l] = p(t[n][l], np.uint16)
        for l in range(4):
            for k in range(5):
                dt.nv[l][k] = p(t["nv"][l][k], np.uint16)
            dt.scalar[l] = int(t["scalar"][l])
            dt.hd[l] = int(t["hd"][l])
        dt.C = int(t["C"])
        self._ok(self.L.g4v_drafter_load(self.h, C.addressof(dt)), "drafter_load")

    def draft_mtp(self, tok, h, P, k, nsplit=6):
        """k chained draft steps; h = None takes the last verify step's hidden state.
        Returns (drafts, runners-up, gaps, last hidden state)"""
        d = np.empty(k, np.int32)
        sec = np.empty(k, np.int32)
        gap = np.empty(k, np.float32)
        hid = np.empty(1536, np.float32)
        hp = None if h is None else _c(h, np.float32)
        self._ok(self.L.g4v_draft_mtp(self.h, tok, None if hp is None else hp.ctypes.data, P, k, nsplit, d,
                                      sec.ctypes.data, gap.ctypes.data, hid.ctypes.data), "draft_mtp")
        return d, sec, gap, hid

    # ---- prefix cache ----
    def slots_init(self, nslot, min_reuse=32):
        self._ok(self.L.g4v_slots_init(self.h, nslot, min_reuse), "slots_init")

    def slot_begin(self, toks):
        """(start, slot used) for a request with prompt toks"""
        toks = _c(toks, np.int32)
        st, used = _i(), _i()
        self._ok(self.L.g4v_slot_begin(self.h, toks, toks.size, C.byref(st), C.byref(used)), "slot_begin")
        return st.value, used.value

    def slot_end(self, toks, gen, P):
        toks = _c(toks, np.int32)
        gen = _c(np.asarray(gen, np.int32).reshape(-1), np.int32)
        self._ok(self.L.g4v_slot_end(self.h, toks, toks.size, gen.ctypes.data if gen.size else None, gen.size, P),
                 "slot_end")

    # ---- prompt-lookup drafter ----
    def history_set(self, toks):
        toks = _c(toks, np.int32)
        self._ok(self.L.g4v_history_set(self.h, toks if toks.size else np.zeros(1, np.int32), toks.size),
                 "history_set")

    def prompt_lookup(self, n, maxlen, append=()):
        """append the committed tokens, then the prompt-lookup drafts (int32 array)"""
        app = _c(np.asarray(append, np.int32).reshape(-1), np.int32)
        out = np.zeros(max(maxlen, 1), np.int32)
        nd = _i()
        self._ok(self.L.g4v_prompt_lookup(self.h, app if app.size else np.zeros(1, np.int32), app.size, n,
                                          maxlen, out, C.byref(nd)), "prompt_lookup")
        return out[:nd.value].copy()

    def history(self):
        L = _i()
        self._ok(self.L.g4v_history_read(self.h, None, 0, C.byref(L)), "history_read")
        out = np.empty(max(L.value, 1), np.int32)
        self._ok(self.L.g4v_history_read(self.h, out.ctypes.data, out.size, C.byref(L)), "history_read")
        return out[:L.value]

    def sync(self):
        self._ok(self.L.g4v_sync(self.h), "sync")

    def hbm_stream(self, nbytes, passes=10, copy=False):
        """device read (or copy: read + write bytes) bandwidth in GB/s over a buffer of nbytes"""
        g = C.c_double()
        self._ok(self.L.g4v_hbm_stream(self.h, nbytes, passes, 1 if copy else 0, C.byref(g)), "hbm_stream")
        return g.value

    def set_graphs(self, on):
        self._ok(self.L.g4v_set_graphs(self.h, 1 if on else 0), "set_graphs")

    def set_prefill_int8(self, on):
        self._ok(self.L.g4v_set_prefill_int8(self.h, 1 if on else 0), "set_prefill_int8")

    def set_decode_int8(self, on):
        """ENGINE_DECODE_INT8 (E:1600): W4A8 verify passes of two rows or more while prefill int8 is on"""
        self._ok(self.L.g4v_set_decode_int8(self.h, 1 if on else 0), "set_decode_int8")

    def set_draft_samepos(self, on):
        """ENGINE_DRAFT_SAMEPOS (E:1516, 1633): every draft step of a chain at position P + 1"""
        self._ok(self.L.g4v_set_draft_samepos(self.h, 1 if on else 0), "set_draft_samepos")

    def profile(self, tags=None):
        """start per-kernel-class event timing for `tags` (names of PROF_TAGS; None = all)"""
        mask = 0
        for i, t in enumerate(PROF_TAGS):
            if tags is None or t in tags:
                mask |= 1 << i
        self._ok(self.L.g4v_profile(self.h, mask), "profile")

    def profile_read(self):
        n = len(PROF_TAGS)
        ms = np.zeros(n, np.float64)
        by = np.zeros(n, np.float64)
        cnt = np.zeros(n, np.int64)
        self.L.g4v_profile_read(self.h, ms.ctypes.data, by.ctypes.data, cnt.ctypes.data, n)
        return {t: dict(ms=float(ms[i]), bytes=float(by[i]), launches=int(cnt[i])) for i, t in enumerate(PROF_TAGS)}

    def prefill_head_stats(self):
        """(screen survivors, fallback) of the last prefill's head row"""
        ns = np.zeros(1, np.int32)
        fb = np.zeros(1, np.int32)
        self._ok(self.L.g4v_prefill_head_stats(self.h, ns, fb), "prefill_head_stats")
        return int(ns[0]), bool(fb[0])

    def verify(self, toks, na, nb, pos0, T=8, hidden=False):
        r = VerifyResult()
        hid = np.empty(1536, np.float32) if hidden else None
        self._ok(self.L.g4v_verify_step(self.h, _c(toks, np.int32), na, nb, pos0, T, C.addressof(r),
                                        None if hid is None else hid.ctypes.data), "verify_step")
        return (r, hid) if hidden else r

    def verify_sibling(self, toks, nd, pos0, T=8, allow_hit=True, hidden=False):
        """the engine's pass with drafts toks[1..nd] and the sibling row toks[nd + 1]"""
        r = VerifyResult()
        hid = np.empty(1536, np.float32) if hidden else None
        self._ok(self.L.g4v_verify_sibling(self.h, _c(toks, np.int32), nd, pos0, T, 1 if allow_hit else 0,
                                           C.addressof(r), None if hid is None else hid.ctypes.data),
                 "verify_sibling")
        return (r, hid) if hidden else r
