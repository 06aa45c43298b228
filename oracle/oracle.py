"""ctypes bindings for the C oracle (liboracle.so) and the reference harness (_ref/libg4ref.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker (or the timed CPU baseline).  The product never imports it.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_ORACLE = os.path.join(HERE, "liboracle.so")
LIB_REF = os.path.join(HERE, "_ref", "libg4ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_vp = C.c_void_p
_i, _i64, _u64, _f, _d = C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_double


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class HeadInfo(C.Structure):
    _fields_ = [("G", _i), ("fallback", _i), ("ref_overflow", _i), ("nsurv", _i),
                ("Lmax", _f), ("thr", _f), ("vmax", _f)]


class VerifyOut(C.Structure):
    _fields_ = [("nacc", _i), ("branch", _i), ("ncommit", _i), ("commit", _i * 8), ("G", _i * 8),
                ("fallback", _i * 8), ("nsurv", _i * 8)]


class Oracle:
    """The C restatement of the reference's verify path (see g4_oracle.h)."""

    def __init__(self, path=LIB_ORACLE):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        L = self.L = C.CDLL(path)
        sig = {
            "g4o_f2bf": (C.c_uint16, [_f]), "g4o_bf2f": (_f, [C.c_uint16]), "g4o_r16": (_f, [_f]),
            "g4o_exp8": (_f, [_f]), "g4o_gelu8": (_f, [_f]), "g4o_sumsq": (_d, [_f32p, _i]),
            "g4o_rms_inv": (_f, [_f32p, _i]), "g4o_rms": (None, [_f32p, _vp, _i, _f32p]),
            "g4o_rms_r16_inplace": (None, [_f32p, _vp, _i]),
            "g4o_rope": (None, [_f32p, _f32p, _f32p, _i]),
            "g4o_rope_tables": (None, [_i, _i, _d, _d, _f32p, _f32p]),
            "g4o_cap": (_f, [_f]), "g4o_calc_thr": (_f, [_f]),
            "g4o_vec_exp8": (None, [_f32p, _i, _f32p]), "g4o_vec_gelu8": (None, [_f32p, _i, _f32p]),
            "g4o_prep_x": (None, [_f32p, _i, _f32p, _f32p, _f32p]),
            "g4o_w4g32_gemm": (None, [_u8p, _u16p, _f32p, _i, _i, _i, _f32p]),
            "g4o_w4a8_quant": (None, [_f32p, _i, _i, _i8p, _f32p, _i32p]),
            "g4o_w4a8_gemm": (None, [_u8p, _u16p, _f32p, _i, _i, _i, _f32p]),
            "g4o_prompt_lookup": (_i, [_i32p, _i, _i, _i, _i32p]),
            "g4o_exp3_codebook": (None, [_u16p, _i64, _u8p]),
            "g4o_exp3_count": (_i64, [_u16p, _i, _i, _u8p, _i64p]),
            "g4o_exp3_pack": (None, [_u16p, _i, _i, _u8p, _u8p, _i64p, _u16p, _f32p]),
            "g4o_exp3_gemm": (None, [_u8p, _u8p, _i64p, _u16p, _f32p, _i, _i, _f32p, _i, _f32p]),
            "g4o_screen_build": (None, [_u16p, _i, _i, _u8p, _u16p, _f32p]),
            "g4o_head_row": (None, [_f32p, _i, _i, _u8p, _u16p, _f32p, _u8p, _u8p, _i64p, _u16p,
                                    _f32p, _vp, _i, _i, _i32p, _f32p, _i, C.POINTER(HeadInfo)]),
            "g4o_attn_splitkv": (None, [_u16p, _u16p, _i, _i, _i, _f32p, _i, _i32p, _i32p, _i32p,
                                        _i32p, _i, _i, _i, _f32p, _i, _vp, _vp]),
            "g4o_model_new": (_vp, [_u64, _i, _i, _i, _i]), "g4o_model_free": (None, [_vp]),
            "g4o_model_fake_ctx": (None, [_vp, _i, _u64]),
            "g4o_model_bytes": (_i, [_vp, C.c_char_p, _vp, _i64]),
            "g4o_model_ptr": (_vp, [_vp, C.c_char_p]),
            "g4o_verify": (None, [_vp, _i32p, _i, _i, _i, _i, C.POINTER(VerifyOut), _vp]),
            "g4o_verify_ex": (None, [_vp, _i32p, _i, _i, _i, _i, _i, C.POINTER(VerifyOut), _vp]),
            "g4o_verify_i8": (None, [_vp, _i32p, _i, _i, _i, _i, _i, _i, C.POINTER(VerifyOut), _vp]),
            "g4o_forward_fill": (None, [_vp, _i32p, _i, _i, _i]),
            "g4o_prefill": (None, [_vp, _i32p, _i, _i, _i, _i, _vp]),
            "g4o_prefill_ex": (None, [_vp, _i32p, _i, _i, _i, _i, _i, _vp]),
            "g4o_model_head": (_i, [_vp, _f32p, _i32p, _i]),
            "g4o_drafter_new": (_vp, [C.c_uint64, _i]), "g4o_drafter_free": (None, [_vp]),
            "g4o_drafter_ptr": (_vp, [_vp, C.c_char_p]),
            "g4o_b16_gemv": (None, [_u16p, _i, _i, _f32p, _f32p]),
            "g4o_draft_step": (_i, [_vp, _vp, _i, _f32p, _i, _i, _i, _f32p, C.POINTER(_i), C.POINTER(_f)]),
            "g4o_attn_tile": (None, [_u16p, _u16p, _i, _i, _i, _f32p, _i, _i32p, _i32p, _f32p, _i]),
            "g4o_attn_mh": (None, [_u16p, _u16p, _i, _i, _i, _f32p, _i, _i32p, _i32p, C.c_void_p, C.c_void_p, _f32p,
                                   _i]),
            "g4o_stream": (_u64, [_u64, _u64]),
            "g4o_gen_normal_f32": (None, [_u64, _i64, _f, _f32p]),
            "g4o_gen_normal_bf16": (None, [_u64, _i64, _f, _u16p]),
            "g4o_gen_bytes": (None, [_u64, _i64, _u8p]),
            "g4o_gen_scales": (None, [_u64, _i64, _f, _f, _u16p]),
            "g4o_gen_ints": (None, [_u64, _i64, C.c_int32, C.c_int32, _i32p]),
            "g4h_read_gbs": (_d, [_i32p, _i, C.c_size_t, _i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args

    def host_read_gbs(self, cpus, nbytes=1 << 30, passes=6):
        """host read bandwidth with one pinned thread per CPU in `cpus` (host_stream.c)"""
        return self.L.g4h_read_gbs(np.ascontiguousarray(cpus, np.int32), len(cpus), nbytes, passes)

    # ---- generators ----
    def stream(self, seed, tag):
        return self.L.g4o_stream(seed, tag)

    def normal_f32(self, seed, n, scale=1.0):
        out = np.empty(n, np.float32)
        self.L.g4o_gen_normal_f32(seed, n, scale, out)
        return out

    def normal_bf16(self, seed, n, scale=1.0):
        out = np.empty(n, np.uint16)
        self.L.g4o_gen_normal_bf16(seed, n, scale, out)
        return out

    def rand_bytes(self, seed, n):
        out = np.empty(n, np.uint8)
        self.L.g4o_gen_bytes(seed, n, out)
        return out

    def scales(self, seed, n, lo=0.005, span=0.015):
        out = np.empty(n, np.uint16)
        self.L.g4o_gen_scales(seed, n, lo, span, out)
        return out

    def ints(self, seed, n, lo, hi):
        out = np.empty(n, np.int32)
        self.L.g4o_gen_ints(seed, n, lo, hi, out)
        return out

    # ---- numerics ----
    def bf2f(self, b):
        return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)

    def r16(self, x):
        return np.array([self.L.g4o_r16(float(v)) for v in np.ravel(x)], np.float32).reshape(np.shape(x))

    def exp8(self, x):
        x = _c(x, np.float32)
        y = np.empty_like(x)
        self.L.g4o_vec_exp8(x, x.size, y)
        return y

    def gelu8(self, x):
        x = _c(x, np.float32)
        y = np.empty_like(x)
        self.L.g4o_vec_gelu8(x, x.size, y)
        return y

    def w4g32(self, W, S, X):
        X = _c(X, np.float32)
        M, K = X.shape
        N = W.shape[0]
        Y = np.empty((M, N), np.float32)
        self.L.g4o_w4g32_gemm(_c(W, np.uint8), _c(S, np.uint16), X, M, N, K, Y)
        return Y

    def w4a8(self, W, S, X):
        X = _c(X, np.float32)
        M, K = X.shape
        N = W.shape[0]
        Y = np.empty((M, N), np.float32)
        self.L.g4o_w4a8_gemm(_c(W, np.uint8), _c(S, np.uint16), X, M, N, K, Y)
        return Y

    def w4a8_quant(self, X):
        X = _c(X, np.float32)
        M, K = X.shape
        q = np.empty((M, K), np.int8)
        sx = np.empty((M, K // 32), np.float32)
        sm = np.empty((M, K // 32), np.int32)
        self.L.g4o_w4a8_quant(X, M, K, q, sx, sm)
        return q, sx, sm

    def prompt_lookup(self, seq, n, maxlen):
        seq = _c(seq, np.int32)
        out = np.zeros(max(maxlen, 1), np.int32)
        nd = self.L.g4o_prompt_lookup(seq, len(seq), n, maxlen, out)
        return out[:nd]

    def exp3_pack(self, E, N, K):
        E = _c(E, np.uint16)
        cb = np.empty(8, np.uint8)
        self.L.g4o_exp3_codebook(E, N * K, cb)
        ptr = np.empty(N + 1, np.int64)
        ne = self.L.g4o_exp3_count(E, N, K, cb, ptr)
        data = np.empty(N * (K // 32) * 44, np.uint8)
        col = np.empty(max(ne, 1), np.uint16)
        dl = np.empty(max(ne, 1), np.float32)
        self.L.g4o_exp3_pack(E, N, K, cb, data, ptr, col, dl)
        return dict(cb=cb, data=data, ptr=ptr, col=col, delta=dl, N=N, K=K)

    def exp3_gemm(self, P, X):
        X = _c(X, np.float32)
        M = X.shape[0]
        Y = np.empty((M, P["N"]), np.float32)
        self.L.g4o_exp3_gemm(P["data"], P["cb"], P["ptr"], P["col"], P["delta"], P["N"], P["K"], X, M, Y)
        return Y

    def screen_build(self, E, N, K):
        Wq = np.empty(N * K // 2, np.uint8)
        Sq = np.empty(N * K // 32, np.uint16)
        coef = np.empty(N, np.float32)
        self.L.g4o_screen_build(_c(E, np.uint16), N, K, Wq, Sq, coef)
        return Wq, Sq, coef

    def head_row(self, h, scr, P, seeds=None, limit=30000, cap=30000):
        Wq, Sq, coef = scr
        V = coef.size
        K = P["K"]
        surv = np.zeros(cap, np.int32)
        sval = np.zeros(cap, np.float32)
        info = HeadInfo()
        sd = None if seeds is None else _c(seeds, np.int32)
        self.L.g4o_head_row(_c(h, np.float32), V, K, Wq, Sq, coef, P["data"], P["cb"], P["ptr"],
                            P["col"], P["delta"], None if sd is None else sd.ctypes.data,
                            0 if sd is None else sd.size, limit, surv, sval, cap, C.byref(info))
        n = min(info.nsurv, cap)
        return info, surv[:n].copy(), sval[:n].copy()

    def attn_rows(self, kind, Kc, Vc, q, pos, lo, skip=None):
        """prefill attention of rows q [M][2048] at pos[m] over [lo[m], pos[m]]: kind 'tile' or 'mh';
        skip (mh only): (skip_lo, skip_hi) per row, positions the row ignores"""
        q = _c(q, np.float32)
        M = q.shape[0]
        out = np.empty((M, 2048), np.float32)
        args = (_c(Kc, np.uint16), _c(Vc, np.uint16), 256, 8, M, q, 2048, _c(pos, np.int32), _c(lo, np.int32))
        if kind == "tile":
            self.L.g4o_attn_tile(*args, out, 2048)
        else:
            sl = None if skip is None else _c(skip[0], np.int32)
            sh = None if skip is None else _c(skip[1], np.int32)
            self.L.g4o_attn_mh(*args, None if sl is None else sl.ctypes.data, None if sh is None else sh.ctypes.data,
                               out, 2048)
        return out

    def attn(self, Kc, Vc, hd, nh, q, pos, lo, skip_lo, skip_hi, kmin, kmax, T, parts=False):
        q = _c(q, np.float32)
        M = q.shape[0]
        out = np.empty((M, nh * hd), np.float32)
        pm = np.empty((T, M, nh), np.float32) if parts else None
        pl = np.empty((T, M, nh), np.float32) if parts else None
        self.L.g4o_attn_splitkv(_c(Kc, np.uint16), _c(Vc, np.uint16), hd, nh, M, q, nh * hd,
                                _c(pos, np.int32), _c(lo, np.int32), _c(skip_lo, np.int32),
                                _c(skip_hi, np.int32), kmin, kmax, T, out, nh * hd,
                                None if pm is None else pm.ctypes.data,
                                None if pl is None else pl.ctypes.data)
        return (out, pm, pl) if parts else out


class Model:
    """Oracle synthetic decoder stack (g4_oracle_model.c)."""

    def __init__(self, orc, seed, V, NL, I=6144, ctx=4096):
        self.o, self.V, self.NL, self.I, self.ctx = orc, V, NL, I, ctx
        self.h = orc.L.g4o_model_new(seed, V, NL, I, ctx)

    def close(self):
        if self.h:
            self.o.L.g4o_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def fake_ctx(self, n, seed=12345):
        self.o.L.g4o_model_fake_ctx(self.h, n, seed)

    def get(self, what, dtype, count):
        out = np.empty(count, dtype)
        rc = self.o.L.g4o_model_bytes(self.h, what.encode(), out.ctypes.data, out.nbytes)
        if rc != 0:
            raise KeyError(what)
        return out

    def prefill(self, toks, pos0=0, pfb=32, T=8, i8=True):
        """prefill toks at pos0.. (W4A8 linear layers for blocks of two rows or more; i8 False:
        exact float throughout); returns the last row's final-normed hidden"""
        toks = _c(toks, np.int32)
        hid = np.empty(1536, np.float32)
        self.o.L.g4o_prefill_ex(self.h, toks, toks.size, pos0, pfb, T, 1 if i8 else 0, hid.ctypes.data)
        return hid

    def head(self, h, seeds=()):
        """greedy token of one final-normed row"""
        sd = np.asarray(list(seeds)[:8] or [0], np.int32)
        return self.o.L.g4o_model_head(self.h, _c(h, np.float32), sd, len(list(seeds)[:8]))

    def verify(self, toks, na, nb, pos0, T=8, allow_b=True, i8=False):
        """one verify pass (tree of na chain rows and nb branch rows); allow_b False: branch b is
        never committed (the engine's sibling row when the tree hit is not taken); i8: W4A8 linear
        layers for passes of two rows or more (G_I8_ACTIVE in the decode, E:311, E:1600)"""
        out = VerifyOut()
        hid = np.empty(1536, np.float32)
        self.o.L.g4o_verify_i8(self.h, _c(toks, np.int32), na, nb, pos0, T, 1 if allow_b else 0, 1 if i8 else 0,
                               C.byref(out), hid.ctypes.data)
        return out, hid


class Drafter:
    """Oracle synthetic MTP drafter (g4_oracle_draft.c) on a target Model."""

    def __init__(self, orc, seed, V):
        self.o, self.V, self.C = orc, V, V // 128
        self.h = orc.L.g4o_drafter_new(seed, V)

    def close(self):
        if self.h:
            self.o.L.g4o_drafter_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def ptr(self, what):
        return self.o.L.g4o_drafter_ptr(self.h, what.encode())

    def step(self, model, tok, h, pos, P, T=6):
        """one draft step: (token, b_out [1536], second-best token, gap)"""
        b = np.empty(1536, np.float32)
        sec, gap = _i(), _f()
        t = self.o.L.g4o_draft_step(model.h, self.h, tok, _c(h, np.float32), pos, P, T, b, C.byref(sec), C.byref(gap))
        return t, b, sec.value, gap.value


class RefLayer(C.Structure):
    _fields_ = [("W", _vp * 7), ("S", _vp * 7), ("nv", _vp * 6), ("scalar", _f), ("sliding", _i)]


class RefModel(C.Structure):
    _fields_ = [("V", _i), ("NL", _i), ("I", _i), ("ctx", _i), ("E", _vp), ("fnorm", _vp), ("KC", _vp), ("VC", _vp),
                ("cs", _vp * 2), ("sn", _vp * 2), ("L", RefLayer * 64)]


class RefDrafter(C.Structure):
    _fields_ = [("pre", _vp), ("post", _vp), ("cent", _vp), ("emb", _vp), ("q", _vp * 4), ("o", _vp * 4),
                ("gate", _vp * 4), ("up", _vp * 4), ("down", _vp * 4), ("nv", (_vp * 5) * 4), ("dnorm", _vp),
                ("order", _vp), ("C", _i)]


class RefOut(C.Structure):
    _fields_ = [("nacc", _i), ("branch", _i), ("ncommit", _i), ("commit", _i * 8), ("G", _i * 8),
                ("fallback", _i * 8), ("nsurv", _i * 8)]


class Ref:
    """The reference engine's own kernels (oracle/_ref/libg4ref.so) on its worker pool."""

    def __init__(self, path=LIB_REF, threads=1, cpus=None):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.L = C.CDLL(path)
        sig = {
            "ref_start": (_i, [_i]), "ref_threads": (_i, []), "ref_start_cpus": (_i, [_i32p, _i]),
            "ref_w4g32": (None, [_u8p, _u16p, _f32p, _i, _i, _i, _f32p]),
            "ref_w4a8": (None, [_u8p, _u16p, _f32p, _i, _i, _i, _f32p, _i8p, _f32p, _i32p]),
            "ref_exp8": (None, [_f32p, _i, _f32p]), "ref_gelu8": (None, [_f32p, _i, _f32p]),
            "ref_rbf8": (None, [_f32p, _i, _f32p]), "ref_f2bf": (None, [_f32p, _i, _u16p]),
            "ref_ss": (_d, [_f32p, _i]), "ref_rms": (None, [_f32p, _vp, _i, _f32p]),
            "ref_rms_r16_inplace": (None, [_f32p, _vp, _i]),
            "ref_rms_prep_x": (None, [_f32p, _f32p, _i, _vp, _f32p, _f32p, _f32p, _i]),
            "ref_add_res_prep_x": (None, [_f32p, _f32p, _i, _f32p, _f32p, _f32p]),
            "ref_add_res_inplace": (None, [_f32p, _f32p, _i]),
            "ref_rope": (None, [_f32p, _f32p, _f32p, _i]),
            "ref_prep_x": (None, [_f32p, _i, _f32p, _f32p, _f32p]),
            "ref_calc_thr": (_f, [_f]),
            "ref_gate_up": (None, [_u8p, _u16p, _u8p, _u16p, _i, _i, _f32p, _i, _f32p, _f32p,
                                   _f32p, _f32p, _f32p]),
            "ref_attn": (_i, [_u16p, _u16p, _i, _i, _i, _f32p, _i, _i32p, _i32p, _i32p, _i32p,
                                _i, _i, _i, _f32p, _i, _vp, _vp, _vp, _vp, _vp]),
            "ref_screen": (_i, [_u8p, _u16p, _f32p, _f32p, _i, _f32p, _i32p, _i32p, _f32p,
                                _f32p, _i32p]),
            "ref_exp3_pack": (_i64, [_u16p, _i, _i, _u8p]),
            "ref_exp3_get": (None, [_u8p, _i64p, _u16p, _f32p]),
            "ref_resc": (_f, [_f32p, _i32p, _i, _f32p]),
            "ref_head": (None, [_f32p, _i, _f32p]),
            "ref_head_setup": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i]),
            "ref_verify": (_i, [C.POINTER(RefModel), _i32p, _i, _i, _i, C.POINTER(RefOut)]),
            "ref_verify_ex": (_i, [C.POINTER(RefModel), _i32p, _i, _i, _i, _i, C.POINTER(RefOut)]),
            "ref_last_hidden": (None, [_f32p]),
            "ref_attn_tile": (None, [_u16p, _u16p, _i, _f32p, _i, _i, _f32p]),
            "ref_attn_mh": (None, [_u16p, _u16p, _i, _f32p, _i, _i, _f32p]),
            "ref_prefill": (_i, [C.POINTER(RefModel), _i32p, _i, _i, _i, _vp]),
            "ref_prefill_ex": (_i, [C.POINTER(RefModel), _i32p, _i, _i, _i, _i, _vp]),
            "ref_pack_reset": (None, []),
            "ref_b16": (None, [_u16p, _i, _i, _f32p, _f32p]),
            "ref_draft_step": (_i, [C.POINTER(RefModel), C.POINTER(RefDrafter), _i, _f32p, _i, _i, _i, _f32p,
                                    C.POINTER(_i), C.POINTER(_f)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if cpus is not None:
            self.threads = L.ref_start_cpus(np.ascontiguousarray(cpus, np.int32), len(cpus))
        else:
            self.threads = L.ref_start(threads)
        self.model = None

    def bind_model(self, model):
        """run ref_verify on the oracle model's own arrays (no copies of the layer weights)"""
        o, h = model.o, model.h
        ptr = lambda w: o.L.g4o_model_ptr(h, w.encode())
        self.L.ref_pack_reset()  # W4A8 repacks are keyed by weight address
        rm = RefModel()
        rm.V, rm.NL, rm.I, rm.ctx = model.V, model.NL, model.I, model.ctx
        rm.E, rm.fnorm, rm.KC, rm.VC = ptr("E"), ptr("fnorm"), ptr("KC"), ptr("VC")
        rm.cs[0], rm.cs[1], rm.sn[0], rm.sn[1] = ptr("cs0"), ptr("cs1"), ptr("sn0"), ptr("sn1")
        for l in range(model.NL):
            for j in range(7):
                rm.L[l].W[j] = ptr(f"W{l}_{j}")
                rm.L[l].S[j] = ptr(f"S{l}_{j}")
            for t in range(6):
                rm.L[l].nv[t] = ptr(f"N{l}_{t}")
            rm.L[l].scalar = 0.75
            rm.L[l].sliding = 1 if l % 5 != 4 else 0
        self.L.ref_head_setup(ptr("Wq"), ptr("Sq"), ptr("coef"), ptr("x3"), ptr("cb"), ptr("xptr"), ptr("xcol"),
                              ptr("xdel"), model.V)
        self.model = rm

    def bind_drafter(self, dr):
        rd = RefDrafter()
        for f in ("pre", "post", "cent", "emb", "order"):
            setattr(rd, f, dr.ptr(f))
        rd.dnorm = dr.ptr("dnorm")
        for l in range(4):
            rd.q[l], rd.o[l], rd.gate[l], rd.up[l], rd.down[l] = (dr.ptr(f"L{l}_{t}") for t in range(5))
            for t in range(5):
                rd.nv[l][t] = dr.ptr(f"L{l}_{10 + t}")
        rd.C = dr.C
        self.drafter = rd

    def draft_step(self, tok, h, pos, P, T=6):
        b = np.empty(1536, np.float32)
        sec, gap = _i(), _f()
        t = self.L.ref_draft_step(C.byref(self.model), C.byref(self.drafter), tok, _c(h, np.float32), pos, P, T, b,
                                  C.byref(sec), C.byref(gap))
        if t < 0:
            raise ValueError("ref_draft_step: needs 1 <= T <= 16 and a target of at least 15 layers")
        return t, b, sec.value, gap.value

    def b16(self, W, x):
        W = _c(W, np.uint16)
        y = np.empty(W.shape[0], np.float32)
        self.L.ref_b16(W, W.shape[0], W.shape[1], _c(x, np.float32), y)
        return y

    def attn_rows(self, kind, Kc, Vc, sliding, q, pos0):
        """attn_tile / run_mh of rows q [M][2048] at pos0 .. pos0+M-1 (causal, window 512 if sliding)"""
        q = _c(q, np.float32)
        out = np.empty((q.shape[0], 2048), np.float32)
        fn = self.L.ref_attn_tile if kind == "tile" else self.L.ref_attn_mh
        fn(_c(Kc, np.uint16), _c(Vc, np.uint16), 1 if sliding else 0, q, pos0, q.shape[0], out)
        return out

    def prefill(self, toks, pos0=0, pfb=32, i8=True):
        hid = np.empty(1536, np.float32)
        toks = _c(toks, np.int32)
        rc = self.L.ref_prefill_ex(C.byref(self.model), toks, toks.size, pos0, pfb, 1 if i8 else 0, hid.ctypes.data)
        if rc != 0:
            raise ValueError("ref_prefill: pfb must be 1..32")
        return hid

    def verify(self, toks, na, nb, pos0, allow_b=True):
        out = RefOut()
        rc = self.L.ref_verify_ex(C.byref(self.model), _c(toks, np.int32), na, nb, pos0, 1 if allow_b else 0,
                                  C.byref(out))
        if rc != 0:
            raise RuntimeError("ref_verify needs V = 262144 and at most 8 rows")
        return out

    def last_hidden(self):
        """the final-normed hidden state of the last verify pass's last committed row"""
        h = np.empty(1536, np.float32)
        self.L.ref_last_hidden(h)
        return h

    def w4g32(self, W, S, X):
        X = _c(X, np.float32)
        M, K = X.shape
        N = W.shape[0]
        Y = np.empty((M, N), np.float32)
        self.L.ref_w4g32(_c(W, np.uint8), _c(S, np.uint16), X, M, N, K, Y)
        return Y

    def w4a8(self, W, S, X):
        X = _c(X, np.float32)
        M, K = X.shape
        N = W.shape[0]
        Y = np.empty((M, N), np.float32)
        q = np.empty((M, K), np.int8)
        sx = np.empty((M, K // 32), np.float32)
        sm = np.empty((M, K // 32), np.int32)
        self.L.ref_w4a8(_c(W, np.uint8), _c(S, np.uint16), X, M, N, K, Y, q, sx, sm)
        return Y, q, sx, sm

    def vec(self, name, x):
        x = _c(x, np.float32)
        y = np.empty_like(x)
        getattr(self.L, name)(x, x.size, y)
        return y

    def exp3_pack(self, E, N, K, cb):
        ne = self.L.ref_exp3_pack(_c(E, np.uint16), N, K, _c(cb, np.uint8))
        data = np.empty(N * (K // 32) * 44, np.uint8)
        ptr = np.empty(N + 1, np.int64)
        col = np.empty(max(ne, 1), np.uint16)
        dl = np.empty(max(ne, 1), np.float32)
        self.L.ref_exp3_get(data, ptr, col, dl)
        return dict(cb=np.array(cb, np.uint8), data=data, ptr=ptr, col=col[:ne], delta=dl[:ne], N=N, K=K)

    def attn(self, Kc, Vc, hd, nh, q, pos, lo, skip_lo, skip_hi, kmin, kmax, T, prep=False, parts=False):
        q = _c(q, np.float32)
        M = q.shape[0]
        K = nh * hd
        out = np.empty((M, K), np.float32)
        xe = np.empty((M, K // 2), np.float32) if prep else None
        xo = np.empty((M, K // 2), np.float32) if prep else None
        gs = np.empty((M, K // 32), np.float32) if prep else None
        pm = np.empty((T, M, nh), np.float32) if parts else None
        pl = np.empty((T, M, nh), np.float32) if parts else None
        ptr = lambda a: None if a is None else a.ctypes.data
        rc = self.L.ref_attn(_c(Kc, np.uint16), _c(Vc, np.uint16), hd, nh, M, q, K, _c(pos, np.int32),
                             _c(lo, np.int32), _c(skip_lo, np.int32), _c(skip_hi, np.int32), kmin, kmax,
                             T, out, K, ptr(xe), ptr(xo), ptr(gs), ptr(pm), ptr(pl))
        if rc != 0:
            raise ValueError("ref_attn: outside the reference's capacity (M <= 4, T <= 16, hd <= 512)")
        res = [out]
        if prep:
            res += [xe, xo, gs]
        if parts:
            res += [pm, pl]
        return res[0] if len(res) == 1 else tuple(res)


def ref_available():
    return os.path.exists(LIB_REF)
