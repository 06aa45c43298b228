"""Write the golden vectors of the verify path from the reference's own kernels.

Inputs come from the seeded counter generator (oracle/g4_rng.h: splitmix64 hash, Irwin-Hall
normals); a CRC-32 of every generated input is stored beside the outputs so a drift of the
generator shows up as a fixture mismatch rather than as a silent change of the case.  Every
output is produced by oracle/_ref/libg4ref.so, i.e. by the functions of
engine/gemma4_engine.cpp, engine/w4g32_avx2.h, engine/w4a8_avx2.h and engine/bf16_exp3_head.h
compiled from the reference's sources with its own build flags (build.sh:5, -march pinned
to x86-64-v3).  The fixtures are data only (numpy .npz, no pickles) and the script is the
only thing that needs the reference; tests read the .npz files.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py
"""
import json
import os
import platform
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from golden_cases import (ATTN_CASES, CTHR_L, EXP3_CASE, GATEUP_CASE, HEAD_V, SCREEN_SEED,  # noqa: E402
                          VERIFY_CASES, VERIFY_MODEL, W4_CASES, attn_inputs, crc, exp3_inputs, gateup_inputs,
                          screen_h, vec_inputs, w4_inputs)
from oracle import Model, Oracle, Ref, ref_available  # noqa: E402


def save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"{name}.npz: {os.path.getsize(path)} bytes", flush=True)


def versions():
    glibc = subprocess.run(["ldd", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    gcc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    return {"glibc": glibc, "gcc": gcc, "machine": platform.machine(),
            "flags": "-O3 -march=x86-64-v3 -mtune=generic -std=c++20 -fopenmp (reference build.sh:5, ISA pinned)"}


def main():
    if not ref_available():
        sys.exit("oracle/_ref/libg4ref.so is not built: the golden vectors come from the reference's kernels")
    o = Oracle()
    # 8 workers: the verify pass splits attention over the pool (E:1290), and the engine runs 8
    # of them past 1,024 tokens; every other wrapper is worker-count independent or runs one
    r = Ref(threads=8)
    if r.threads != 8:
        sys.exit(f"the reference pool started {r.threads} workers; the verify fixtures need 8")

    # ---- W4G32 / W4A8 skinny GEMM (w4g32_avx2.h:64-96, w4a8_avx2.h:20-61) ----
    out = {}
    for i, (M, N, K, seed) in enumerate(W4_CASES):
        W, S, X = w4_inputs(o, M, N, K, seed)
        out[f"in_crc_{i}"] = np.array([crc(W), crc(S), crc(X)], np.uint32)
        out[f"w4g32_{i}"] = r.w4g32(W, S, X)
        y, q, sx, sm = r.w4a8(W, S, X)
        out[f"w4a8_{i}"], out[f"w4a8_q_{i}"], out[f"w4a8_sx_{i}"], out[f"w4a8_sum_{i}"] = y, q, sx, sm
    save("w4", **out)

    # ---- elementwise: exp8, gelu8, rbf8, f2bf, ss, rms, rope, calc_thr (E:33-60, 318-404, 445-448) ----
    x, w, cs, sn = vec_inputs(o)
    out = {"in_crc": np.array([crc(x), crc(w), crc(cs), crc(sn)], np.uint32),
           "exp8": r.vec("ref_exp8", x), "gelu8": r.vec("ref_gelu8", x), "rbf8": r.vec("ref_rbf8", x)}
    bf = np.empty(x.size, np.uint16)
    r.L.ref_f2bf(np.ascontiguousarray(x), x.size, bf)
    out["f2bf"] = bf
    rows = x[: 4 * 1536].reshape(4, 1536).copy()
    out["ss"] = np.array([r.L.ref_ss(np.ascontiguousarray(rows[m]), 1536) for m in range(4)], np.float64)
    rms = np.empty((4, 1536), np.float32)
    for m in range(4):
        y = np.empty(1536, np.float32)
        r.L.ref_rms(np.ascontiguousarray(rows[m]), w.ctypes.data, 1536, y)
        rms[m] = y
    out["rms"] = rms
    head = rows[:, :256].copy()
    for m in range(4):
        hm = np.ascontiguousarray(head[m])
        r.L.ref_rms_r16_inplace(hm, w.ctypes.data, 256)
        head[m] = hm
    out["rms_r16_head"] = head
    rope = np.empty((3, 256), np.float32)
    for i, p in enumerate([0, 5, 63]):
        h = rows[0, :256].copy()
        r.L.ref_rope(h, np.ascontiguousarray(cs[p * 128:(p + 1) * 128]), np.ascontiguousarray(sn[p * 128:(p + 1) * 128]), 256)
        rope[i] = h
    out["rope"] = rope
    out["cthr_L"] = CTHR_L
    out["cthr"] = np.array([r.L.ref_calc_thr(float(v)) for v in CTHR_L], np.float32)
    save("vec", **out)

    # ---- split-KV attention + LSE merge + prep of the o_proj input (E:739-877, 1019-1059) ----
    out = {}
    for i, case in enumerate(ATTN_CASES):
        a = attn_inputs(o, *case)
        out[f"in_crc_{i}"] = np.array([crc(a["K"]), crc(a["V"]), crc(a["q"])], np.uint32)
        res, xe, xo, gs, pm, pl = r.attn(a["K"], a["V"], 256, 8, a["q"], a["pos"], a["lo"], a["sl"], a["sh"],
                                         a["kmin"], a["kmax"], case[2], prep=True, parts=True)
        out[f"out_{i}"], out[f"pm_{i}"], out[f"pl_{i}"] = res, pm, pl
        out[f"gs_{i}"] = gs
    save("attn", **out)

    # ---- fused gate/up + gelu + down-input prep (E:256-302) ----
    M, I, K = GATEUP_CASE
    Wg, Sg, Wu, Su, X = gateup_inputs(o)
    gb = np.empty((M, I), np.float32); ub = np.empty((M, I), np.float32)
    xe = np.empty((M, I // 2), np.float32); xo = np.empty((M, I // 2), np.float32); gs = np.empty((M, I // 32), np.float32)
    r.L.ref_gate_up(Wg, Sg, Wu, Su, I, K, X, M, gb, ub, xe, xo, gs)
    save("gateup", in_crc=np.array([crc(Wg), crc(Sg), crc(Wu), crc(Su), crc(X)], np.uint32),
         gate=gb, up=ub, act_even=xe, act_odd=xo, act_gsum=gs)

    # ---- exp3 head: codebook, pack, full head, rescore (bf16_exp3_head.h; E:539-579, 1232-1234) ----
    N, K, seed = EXP3_CASE
    E, h = exp3_inputs(o)
    P = o.exp3_pack(E, N, K)  # codebook only; the packing itself comes from the reference below
    Q = r.exp3_pack(E, N, K, P["cb"])
    Y = np.empty((4, N), np.float32)
    r.L.ref_head(np.ascontiguousarray(h), 4, Y)
    idx = np.arange(0, N, 7, dtype=np.int32)
    fv = np.empty(idx.size, np.float32)
    mx = r.L.ref_resc(np.ascontiguousarray(h[1]), idx, idx.size, fv)
    save("exp3", in_crc=np.array([crc(E), crc(h)], np.uint32), cb=Q["cb"], ptr=Q["ptr"], col=Q["col"],
         delta=Q["delta"], data_crc=np.array([crc(Q["data"])], np.uint32), logits=Y, resc_idx=idx, resc=fv,
         resc_max=np.array([mx], np.float32))

    # ---- head screen scan at V = 262144 (E:449-538), one worker: the survivor set ----
    E = o.normal_bf16(o.stream(SCREEN_SEED, 1), HEAD_V * 1536, 0.02)
    scr = o.screen_build(E, HEAD_V, 1536)
    hh = screen_h(o, E)
    seedL = np.full(4, -1e30, np.float32)
    cap = 16384
    cnt = np.zeros(4, np.int32); idx = np.zeros(4 * cap, np.int32); uu = np.zeros(4 * cap, np.float32)
    tmax = np.zeros(4, np.float32); ovf = np.zeros(4, np.int32)
    r.L.ref_screen(scr[0], scr[1], scr[2], np.ascontiguousarray(hh), 4, seedL, cnt, idx, uu, tmax, ovf)
    out = {"in_crc": np.array([crc(E), crc(hh), crc(scr[0]), crc(scr[1]), crc(scr[2])], np.uint32),
           "tmax": tmax, "overflow": ovf}
    for m in range(4):
        thr = r.L.ref_calc_thr(float(tmax[m]))
        ri, ru = idx[m * cap:m * cap + cnt[m]], uu[m * cap:m * cap + cnt[m]]
        keep = ru >= thr
        out[f"surv_{m}"] = ri[keep].astype(np.int32)
        out[f"surv_u_{m}"] = ru[keep].astype(np.float32)
        out[f"thr_{m}"] = np.array([thr], np.float32)
    save("screen", **out)
    del E, scr

    # ---- whole verify pass of the synthetic stack through the reference's kernels ----
    seed, V, NL, I, ctx, nfake = VERIFY_MODEL
    m = Model(o, seed, V, NL, I, ctx)
    r.bind_model(m)
    m.fake_ctx(nfake, 12345)
    out = {"weights_crc": np.array([crc(m.get("E", np.uint16, V * 1536)), crc(m.get("W1_4", np.uint8, I * 768)),
                                    crc(m.get("KC", np.uint16, NL * ctx * 256)),
                                    crc(m.get("coef", np.float32, V))], np.uint32)}

    def ref_verify(toks, na, nb, pos0):
        m.fake_ctx(nfake, 12345)  # every case starts from the same cache
        return r.verify(np.asarray(toks, np.int32), na, nb, pos0)

    for i, (na, nb, pos0, kind) in enumerate(VERIFY_CASES):
        M = 1 + na + nb
        toks = [5 + 12 * k for k in range(M)]
        if kind == "chain":  # drafts equal to the stack's own greedy tokens: all accepted
            toks = [101] + [0] * na
            for depth in range(1, na + 1):
                toks[depth] = ref_verify(toks, na, 0, pos0).G[depth - 1]
        elif kind == "branch_b":  # the sibling holds the greedy token: branch b commits
            g0 = ref_verify([202, 3, 4, 5, 6, 7, 8], na, nb, pos0).G[0]
            toks = [202, (g0 + 1) % V, 4, 5, g0, 7, 8]
        ro = ref_verify(toks, na, nb, pos0)
        out[f"toks_{i}"] = np.asarray(toks, np.int32)
        out[f"res_{i}"] = np.array([ro.nacc, ro.branch, ro.ncommit] + list(ro.commit) + list(ro.G) +
                                   list(ro.fallback) + list(ro.nsurv), np.int32)
        out[f"kv_crc_{i}"] = np.array([crc(m.get("KC", np.uint16, NL * ctx * 256)),
                                       crc(m.get("VC", np.uint16, NL * ctx * 256))], np.uint32)
        print(f"verify case {i} {kind}: toks={toks} nacc={ro.nacc} branch={ro.branch} G={list(ro.G)}", flush=True)
    m.close()
    save("verify", **out)

    with open(os.path.join(HERE, "versions.json"), "w") as f:
        json.dump(versions(), f, indent=1)


if __name__ == "__main__":
    main()
