"""A synthetic checkpoint of the Gemma-4-E2B layer layout and the reference's run_req over it.

The checkpoint is what the reference engine's main() loads (engine/gemma4_engine.cpp:1214-1232):
model.safetensors plus a tensor index (name, dtype, byte offset, byte count, shape), with
35 layers of head_dim 256 (l % 5 != 4) or 512, k/v projections in layers 0..14 only, per-layer
MLP widths, the per-layer-input tensors and a vocabulary of 262,144.  Every tensor is drawn from
the oracle's generators (oracle/g4_rng.h) by seed; the embedding is the synthetic model's
(seed EMBED_SEED, so the oracle's head matches it), and the per-layer embedding table has rows
only for the ids in PLE_IDS (a sparse region of the file, zero elsewhere).

run_req_k0 restates run_req (E:1584-1661) with ENGINE_K=0: the prompt in blocks of 32 rows,
then one-row decode passes (E:1615), greedy tokens from the certified head, over the oracle.
"""
import ctypes as C
import os

import numpy as np

H, NL, PD, V = 1536, 35, 256, 262144
EMBED_SEED, WEIGHT_SEED = 5, 77
MLP = [512 if l < 15 else 1024 for l in range(NL)]  # the checkpoint's 6144 / 12288, scaled down
PLE_IDS = list(range(2, 2050, 7))  # ids whose per-layer embedding rows are nonzero


def layer_hd(l):
    return 256 if l % 5 != 4 else 512


def tensor_list():
    """(name, kind, shape) in file order; kind 'q4' (int4 matrix [N, K] as weight_packed I32
    [N, K/8] + weight_scale BF16 [N, K/32]) or 'vec' (bf16)"""
    out = []
    for l in range(NL):
        p = f"layers.{l}."
        hd, ff = layer_hd(l), MLP[l]
        out.append((p + "self_attn.q_proj", "q4", (8 * hd, H)))
        if l < 15:
            out.append((p + "self_attn.k_proj", "q4", (hd, H)))
            out.append((p + "self_attn.v_proj", "q4", (hd, H)))
            out.append((p + "self_attn.k_norm.weight", "vec", (hd,)))
        out.append((p + "self_attn.o_proj", "q4", (H, 8 * hd)))
        out.append((p + "mlp.gate_proj", "q4", (ff, H)))
        out.append((p + "mlp.up_proj", "q4", (ff, H)))
        out.append((p + "mlp.down_proj", "q4", (H, ff)))
        out.append((p + "per_layer_input_gate", "q4", (PD, H)))
        out.append((p + "per_layer_projection", "q4", (H, PD)))
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm", "post_per_layer_input_norm"):
            out.append((p + n + ".weight", "vec", (H,)))
        out.append((p + "self_attn.q_norm.weight", "vec", (hd,)))
        out.append((p + "layer_scalar", "vec", (1,)))
    out.append(("per_layer_model_projection", "q4", (NL * PD, H)))
    out.append(("per_layer_projection_norm.weight", "vec", (PD,)))
    out.append(("norm.weight", "vec", (H,)))
    return out


def gen_tensor(orc, idx, name, kind, shape):
    """the tensor's bytes from the oracle's generators, stream (WEIGHT_SEED, 100 + idx)"""
    st = lambda t: orc.stream(WEIGHT_SEED, 100 + 4 * idx + t)
    if kind == "q4":
        N, K = shape
        w = orc.rand_bytes(st(0), N * K // 2).reshape(N, K // 2)
        s = orc.scales(st(1), N * K // 32, 0.004, 0.012).reshape(N, K // 32)
        return w, s
    n = shape[0]
    if name.endswith("layer_scalar"):
        return np.array([0x3F40], np.uint16)  # bf16 0.75
    u = (orc.normal_f32(st(0), n) + 8.0) / 8.0  # about 1 +- 0.125
    if ".q_norm" in name or ".k_norm" in name:
        u = u * 0.25
    return (orc.r16(u).view(np.uint32) >> 16).astype(np.uint16)


def write_checkpoint(orc, d):
    """write model.safetensors (raw tensor bytes; the engine reads the index offsets only) and
    index.tsv into d; returns the embedding (uint16 [V][H])"""
    from oracle import Model
    m = Model(orc, EMBED_SEED, V, 1, 256, 64)  # the synthetic embedding (and its head) of EMBED_SEED
    E = m.get("E", np.uint16, V * H).reshape(V, H)
    m.close()
    rows, off = [], 0
    path = os.path.join(d, "model.safetensors")
    with open(path, "wb") as f:
        def put(name, dt, arr, shape):
            nonlocal off
            b = np.ascontiguousarray(arr).tobytes()
            f.write(b)
            rows.append((name, dt, off, len(b), ",".join(map(str, shape))))
            off += len(b)
            pad = (-off) % 64
            f.write(b"\0" * pad)
            off += pad

        put("embed_tokens.weight", "BF16", E, (V, H))
        for i, (name, kind, shape) in enumerate(tensor_list()):
            t = gen_tensor(orc, i, name, kind, shape)
            if kind == "q4":
                put(name + ".weight_packed", "I32", t[0], (shape[0], shape[1] // 8))
                put(name + ".weight_scale", "BF16", t[1], (shape[0], shape[1] // 32))
            else:
                put(name, "BF16", t, shape)
        # the per-layer embedding table last: rows of PLE_IDS written, the rest left as holes
        ple_off = off
        for tok in PLE_IDS:
            f.seek(ple_off + tok * NL * PD * 2)
            f.write(ple_rows(orc, [tok]).tobytes())
        f.truncate(ple_off + V * NL * PD * 2)
        rows.append(("embed_tokens_per_layer.weight", "BF16", ple_off, V * NL * PD * 2, f"{V},{NL * PD}"))
    with open(os.path.join(d, "index.tsv"), "w") as f:
        for name, dt, o, nb, shape in rows:
            f.write(f"model.language_model.{name}\t{dt}\t{o}\t{nb}\t{shape}\n")
    return E


def ple_rows(orc, toks):
    """the per-layer embedding rows of the listed ids (bf16 [n][35 * 256])"""
    out = np.empty((len(toks), NL * PD), np.uint16)
    for i, t in enumerate(toks):
        out[i] = orc.normal_bf16(orc.stream(WEIGHT_SEED, 50000 + t), NL * PD, 0.5)
    return out


class Q4(C.Structure):
    _fields_ = [("w", C.c_void_p), ("s", C.c_void_p), ("N", C.c_int32), ("K", C.c_int32)]


class GLayer(C.Structure):
    _fields_ = [(n, Q4) for n in ("q", "k", "v", "o", "gate", "up", "down", "pg", "pp")] + \
               [(n, C.c_void_p) for n in ("in_ln", "post_attn", "pre_ff", "post_ff", "post_ple", "qn", "kn")] + \
               [("scalar", C.c_uint16)]


class GemmaIn(C.Structure):
    _fields_ = [("L", GLayer * NL), ("plproj", Q4), ("plnorm", C.c_void_p), ("fnorm", C.c_void_p), ("E", C.c_void_p),
                ("V", C.c_int32), ("nple", C.c_int32), ("ple_ids", C.c_void_p), ("ple_rows", C.c_void_p)]


class GemmaOracle:
    """the oracle's Gemma-layout forward over a checkpoint directory (tensors mapped in place)
    and the head of the synthetic model with the same embedding"""

    def __init__(self, orc, d, ctx=1024, i8=False):
        from oracle import Model
        L = orc.L
        L.g4o_gemma_new.restype = C.c_void_p
        L.g4o_gemma_new.argtypes = [C.POINTER(GemmaIn), C.c_int]
        L.g4o_gemma_free.argtypes = [C.c_void_p]
        L.g4o_gemma_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                        C.c_int]
        L.g4o_gemma_set_i8.argtypes = [C.c_void_p, C.c_int]
        L.g4o_gemma_cache.restype = C.c_void_p
        L.g4o_gemma_cache.argtypes = [C.c_void_p, C.c_int, C.c_int]
        self.orc, self.ctx = orc, ctx
        self.raw = np.memmap(os.path.join(d, "model.safetensors"), np.uint8, "r")
        idx = {}
        for line in open(os.path.join(d, "index.tsv")):
            n, dt, o, nb, sh = line.rstrip("\n").split("\t")
            idx[n.replace("model.language_model.", "")] = (int(o), int(nb), tuple(int(x) for x in sh.split(",")))
        ptr = lambda n: self.raw.ctypes.data + idx[n][0]

        def q4(n):
            N, K8 = idx[n + ".weight_packed"][2]
            return Q4(ptr(n + ".weight_packed"), ptr(n + ".weight_scale"), N, K8 * 8)

        gi = GemmaIn()
        for l in range(NL):
            p = f"layers.{l}."
            A = gi.L[l]
            A.q = q4(p + "self_attn.q_proj")
            if l < 15:
                A.k, A.v = q4(p + "self_attn.k_proj"), q4(p + "self_attn.v_proj")
                A.kn = ptr(p + "self_attn.k_norm.weight")
            A.o, A.gate, A.up, A.down = (q4(p + "self_attn.o_proj"), q4(p + "mlp.gate_proj"), q4(p + "mlp.up_proj"),
                                         q4(p + "mlp.down_proj"))
            A.pg, A.pp = q4(p + "per_layer_input_gate"), q4(p + "per_layer_projection")
            A.in_ln, A.post_attn = ptr(p + "input_layernorm.weight"), ptr(p + "post_attention_layernorm.weight")
            A.pre_ff, A.post_ff = ptr(p + "pre_feedforward_layernorm.weight"), ptr(p + "post_feedforward_layernorm.weight")
            A.post_ple, A.qn = ptr(p + "post_per_layer_input_norm.weight"), ptr(p + "self_attn.q_norm.weight")
            A.scalar = int(self.raw[idx[p + "layer_scalar"][0]:idx[p + "layer_scalar"][0] + 2].view(np.uint16)[0])
        gi.plproj = q4("per_layer_model_projection")
        gi.plnorm, gi.fnorm, gi.E = ptr("per_layer_projection_norm.weight"), ptr("norm.weight"), ptr("embed_tokens.weight")
        gi.V = V
        self.ple_ids = np.array(PLE_IDS, np.int32)
        self.ple = ple_rows(orc, PLE_IDS)
        gi.nple, gi.ple_ids, gi.ple_rows = len(PLE_IDS), self.ple_ids.ctypes.data, self.ple.ctypes.data
        self.gi = gi
        self.h = L.g4o_gemma_new(C.byref(gi), ctx)
        L.g4o_gemma_set_i8(self.h, 1 if i8 else 0)  # ENGINE_PREFILL_INT8=1: W4A8 blocks of >= 2 rows
        self.head = Model(orc, EMBED_SEED, V, 1, 256, 64)

    def close(self):
        if self.h:
            self.orc.L.g4o_gemma_free(self.h)
            self.h = None
            self.head.close()

    def forward(self, toks, pos0, T, hf, sibling=-1):
        toks = np.ascontiguousarray(toks, np.int32)
        M = len(toks)
        hb = np.zeros((M, H), np.float32)
        self.orc.L.g4o_gemma_forward(self.h, toks.ctypes.data, M, pos0, T, sibling, hb.ctypes.data, hf)
        return hb

    def greedy(self, h, seeds):
        return self.head.head(h, list(seeds)[:8])

    def cache(self, l, v):
        hd = layer_hd(l)
        p = self.orc.L.g4o_gemma_cache(self.h, l, v)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (self.ctx * hd,)).copy()


def run_req_k0(go, prompt, nnew, T, pfb=32):
    """run_req (E:1584-1661) with ENGINE_K=0 on an empty cache: FIRST and the GEN tokens"""
    n = len(prompt)
    G = None
    for b in range(0, n, pfb):  # E:1594-1599 (the last block's last row feeds the head)
        blk = prompt[b:b + pfb]
        last = b + len(blk) == n
        hb = go.forward(blk, b, T, len(blk) - 1 if last else len(blk))
        if last:
            G = go.greedy(hb[len(blk) - 1], blk)
    gen = [G]
    is_stop = lambda t: t in (106, 1)
    for i in range(1, nnew):  # E:1615
        if is_stop(gen[-1]):
            break
        hb = go.forward([gen[-1]], n + i - 1, T, 0)
        gen.append(go.greedy(hb[0], [gen[-1]]))
    gen = gen[:nnew]
    for i, g in enumerate(gen):
        if is_stop(g):
            return gen[:i + 1]
    return gen
