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

write_drafter writes a drafter checkpoint in the form main() loads with ENGINE_K > 0 (E:1519-1528:
bf16 tensors, 4 layers of hidden 256 with 4 query heads, head dim 256 in layers 0..2 and 512 in
layer 3, FFN 2048, 2048 centroids of 128 tokens).  Its weights are drawn so that its drafts are
often right on this target: the pre-projection reads only the token's embedding (the hidden-state
half is zero; A ternary), so the residual stream starts at u_tok ~ A e_tok; the layers add small
contributions (post-attention / post-FFN norm weights near 0.03); the tokens are ordered into
clusters by 11 balanced sign splits of u_t along random directions, each centroid being the sum
of its signed directions, and each token's drafter embedding is u_t / |u_t| scaled by 0.12-0.2.
The drafter then mostly proposes its input token again (the target's continuations repeat
tokens here), with score gaps around the sibling thresholds of E:1639-1641.
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


DRAFTER_SEED = 88
DR_H, DR_F, DR_C = 256, 2048, 2048


def bf16_of(x):
    """round-to-nearest-even bf16 bits of finite float32 values"""
    u = np.array(x, np.float32).view(np.uint32)
    r = (u >> 16) & 1
    u += 0x7FFF
    u += r
    u >>= 16
    return u.astype(np.uint16)


def fake_ctx_rows(n, seed=12345):
    """E:1249-1250 ENGINE_FAKE_CTX: owner layer l < 15 gets n positions of bf16 K and V rows from
    one LCG (rs = rs * 1664525 + 1013904223 mod 2^32, value ((rs >> 9) % 2001 - 1000) / 700 in
    float32), element i = p * hd + e drawing K then V, the layers in order.  Returns [(K, V)] of
    [n][hd] uint16 per layer.  The sequence is formed in closed form: rs_k = a^k rs_0 + c (1 + a +
    ... + a^(k-1)) in wrapping uint32 arithmetic."""
    a, c = np.uint32(1664525), np.uint32(1013904223)
    counts = [2 * n * layer_hd(l) for l in range(15)]
    N = sum(counts)
    with np.errstate(over="ignore"):
        A = np.cumprod(np.full(N, a, np.uint32), dtype=np.uint32)          # a^k, k = 1..N
        Sg = np.cumsum(np.concatenate([np.ones(1, np.uint32), A[:-1]]), dtype=np.uint32)  # 1 + ... + a^(k-1)
        rs = A * np.uint32(seed) + c * Sg
    vals = ((rs >> 9).astype(np.int64) % 2001 - 1000).astype(np.float32) / np.float32(700.0)
    out, o = [], 0
    for l in range(15):
        hd = layer_hd(l)
        v = bf16_of(vals[o:o + counts[l]]).reshape(n, hd, 2)
        out.append((np.ascontiguousarray(v[:, :, 0]), np.ascontiguousarray(v[:, :, 1])))
        o += counts[l]
    return out


def drafter_tensors(orc, E):
    """(name, dtype, array, shape) of the drafter checkpoint (E:1523-1528) for the target embedding E"""
    st = lambda tag: orc.stream(DRAFTER_SEED, tag)
    nrm = lambda tag, n, s=1.0: orc.normal_f32(st(tag), n, s)
    # A and R ternary: every sum below is exact in float64 (bf16 inputs), so the clustering does
    # not depend on the summation order of the machine's BLAS
    A = orc.ints(st(1), DR_H * H, -1, 1).reshape(DR_H, H).astype(np.float64)
    U = np.empty((V, DR_H), np.float64)
    buf = np.empty((16384, H), np.uint32)  # one slice of the embedding widened at a time
    for r0 in range(0, V, 16384):
        buf[:] = E[r0:r0 + 16384]
        buf <<= 16
        U[r0:r0 + 16384] = buf.view(np.float32).astype(np.float64) @ A.T
    R = orc.ints(st(2), 11 * DR_H, -1, 1).reshape(11, DR_H).astype(np.float64)
    groups = [np.arange(V)]
    for i in range(11):  # balanced median splits: cluster index bits, level 0 the most significant
        nxt = []
        for g in groups:
            o = g[np.argsort(U[g] @ R[i], kind="stable")]
            nxt += [o[:len(o) // 2], o[len(o) // 2:]]
        groups = nxt
    order = np.concatenate(groups).astype(np.int64)
    bits = ((np.arange(DR_C)[:, None] >> (10 - np.arange(11))[None, :]) & 1) * 2.0 - 1.0
    cent = (bits @ R).astype(np.float32) * np.float32(0.05)
    un = U / np.sqrt((U * U).sum(axis=1, keepdims=True))
    sc = 0.12 + 0.08 * (orc.normal_f32(st(3), V) % 1.0)
    emb = (un * sc[:, None]).astype(np.float32)
    out = []
    pre = np.zeros((DR_H, 2 * H), np.float32)
    pre[:, :H] = A * 2.0 ** -5
    out.append(("pre_projection.weight", "BF16", bf16_of(pre), (DR_H, 2 * H)))
    for l in range(4):
        hd = 256 if l < 3 else 512
        p = f"model.layers.{l}."
        t0 = 100 + 20 * l
        out.append((p + "self_attn.q_proj.weight", "BF16", bf16_of(nrm(t0, 4 * hd * DR_H, 0.06)), (4 * hd, DR_H)))
        out.append((p + "self_attn.o_proj.weight", "BF16", bf16_of(nrm(t0 + 1, DR_H * 4 * hd, 0.03)), (DR_H, 4 * hd)))
        out.append((p + "mlp.gate_proj.weight", "BF16", bf16_of(nrm(t0 + 2, DR_F * DR_H, 0.06)), (DR_F, DR_H)))
        out.append((p + "mlp.up_proj.weight", "BF16", bf16_of(nrm(t0 + 3, DR_F * DR_H, 0.06)), (DR_F, DR_H)))
        out.append((p + "mlp.down_proj.weight", "BF16", bf16_of(nrm(t0 + 4, DR_H * DR_F, 0.02)), (DR_H, DR_F)))
        u = lambda tag, n, b, w: bf16_of(b + w * (orc.normal_f32(st(tag), n) % 1.0))
        out.append((p + "input_layernorm.weight", "BF16", u(t0 + 5, DR_H, 0.5, 1.0), (DR_H,)))
        out.append((p + "post_attention_layernorm.weight", "BF16", u(t0 + 6, DR_H, 0.02, 0.02), (DR_H,)))
        out.append((p + "pre_feedforward_layernorm.weight", "BF16", u(t0 + 7, DR_H, 0.5, 1.0), (DR_H,)))
        out.append((p + "post_feedforward_layernorm.weight", "BF16", u(t0 + 8, DR_H, 0.02, 0.02), (DR_H,)))
        out.append((p + "self_attn.q_norm.weight", "BF16", u(t0 + 9, hd, 0.2, 0.1), (hd,)))
        out.append((p + "layer_scalar", "BF16", np.array([[0x3F80, 0x3F40, 0x3F80, 0x3F60][l]], np.uint16), (1,)))
    out.append(("post_projection.weight", "BF16", bf16_of(nrm(4, H * DR_H, 0.06)), (H, DR_H)))
    out.append(("masked_embedding.centroids.weight", "BF16", bf16_of(cent), (DR_C, DR_H)))
    out.append(("model.norm.weight", "BF16", bf16_of(0.9 + 0.2 * (orc.normal_f32(st(5), DR_H) % 1.0)), (DR_H,)))
    out.append(("model.embed_tokens.weight", "BF16", bf16_of(emb), (V, DR_H)))
    out.append(("masked_embedding.token_ordering", "I64", order, (V,)))
    return out


def write_drafter(orc, d, E):
    """the drafter checkpoint: d/drafter/model.safetensors and d/drafter_index.tsv (the
    ENGINE_DRAFTER_DIR / ENGINE_DRAFTER_INDEX of E:1519)"""
    os.makedirs(os.path.join(d, "drafter"), exist_ok=True)
    rows, off = [], 0
    with open(os.path.join(d, "drafter", "model.safetensors"), "wb") as f:
        for name, dt, arr, shape in drafter_tensors(orc, E):
            b = np.ascontiguousarray(arr).tobytes()
            f.write(b)
            rows.append((name, dt, off, len(b), ",".join(map(str, shape))))
            off += len(b)
            pad = (-off) % 64
            f.write(b"\0" * pad)
            off += pad
    with open(os.path.join(d, "drafter_index.tsv"), "w") as f:
        for name, dt, o, nb, shape in rows:
            f.write(f"{name}\t{dt}\t{o}\t{nb}\t{shape}\n")


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
        L.g4o_gemma_kv_move.argtypes = [C.c_void_p, C.c_int, C.c_int]
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

    def set_i8(self, on):
        """W4A8 products for passes of two rows or more from now on (ENGINE_PREFILL_INT8 blocks)"""
        self.orc.L.g4o_gemma_set_i8(self.h, 1 if on else 0)

    def kv_move(self, src, dst):
        """E:1651: the KV rows of slot src copied to slot dst in every owner cache"""
        self.orc.L.g4o_gemma_kv_move(self.h, src, dst)

    def forward(self, toks, pos0, T, hf, sibling=-1):
        toks = np.ascontiguousarray(toks, np.int32)
        M = len(toks)
        hb = np.zeros((M, H), np.float32)
        self.orc.L.g4o_gemma_forward(self.h, toks.ctypes.data, M, pos0, T, sibling, hb.ctypes.data, hf)
        return hb

    def greedy(self, h, seeds):
        return self.head.head(h, list(seeds)[:8])

    def fake_ctx(self, n, seed=12345):
        """E:1249-1250: the first n positions of the owner caches from the LCG (fake_ctx_rows)"""
        for l, (K, V) in enumerate(fake_ctx_rows(n, seed)):
            hd = layer_hd(l)
            for v, rows in ((0, K), (1, V)):
                p = self.orc.L.g4o_gemma_cache(self.h, l, v)
                dst = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (self.ctx * hd,))
                dst[:n * hd] = rows.reshape(-1)

    def cache(self, l, v):
        hd = layer_hd(l)
        p = self.orc.L.g4o_gemma_cache(self.h, l, v)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (self.ctx * hd,)).copy()


class DrafterIn(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("pre", "post", "cent", "emb", "dnorm", "order")] + \
               [(n, C.c_void_p * 4) for n in ("q", "o", "gate", "up", "down")] + \
               [("nv", (C.c_void_p * 5) * 4), ("scalar", C.c_uint16 * 4), ("V", C.c_int32), ("C", C.c_int32),
                ("hd", C.c_int32 * 4)]


class GemmaDrafter:
    """the oracle's drafter over a drafter checkpoint (write_drafter's files, tensors mapped in place)"""

    def __init__(self, orc, d):
        L = orc.L
        L.g4o_drafter_load.restype = C.c_void_p
        L.g4o_drafter_load.argtypes = [C.POINTER(DrafterIn)]
        L.g4o_drafter_free.argtypes = [C.c_void_p]
        L.g4o_gemma_draft_step.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                           C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_float)]
        self.orc = orc
        self.raw = np.memmap(os.path.join(d, "drafter", "model.safetensors"), np.uint8, "r")
        idx = {}
        for line in open(os.path.join(d, "drafter_index.tsv")):
            n, dt, o, nb, sh = line.rstrip("\n").split("\t")
            idx[n] = (int(o), int(nb), tuple(int(x) for x in sh.split(",")))
        ptr = lambda n: self.raw.ctypes.data + idx[n][0]
        di = DrafterIn()
        di.pre, di.post = ptr("pre_projection.weight"), ptr("post_projection.weight")
        di.cent, di.emb = ptr("masked_embedding.centroids.weight"), ptr("model.embed_tokens.weight")
        di.dnorm, di.order = ptr("model.norm.weight"), ptr("masked_embedding.token_ordering")
        for l in range(4):
            p = f"model.layers.{l}."
            di.q[l], di.o[l] = ptr(p + "self_attn.q_proj.weight"), ptr(p + "self_attn.o_proj.weight")
            di.gate[l], di.up[l] = ptr(p + "mlp.gate_proj.weight"), ptr(p + "mlp.up_proj.weight")
            di.down[l] = ptr(p + "mlp.down_proj.weight")
            for t, n in enumerate(("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                                   "post_feedforward_layernorm", "self_attn.q_norm")):
                di.nv[l][t] = ptr(p + n + ".weight")
            o = idx[p + "layer_scalar"][0]
            di.scalar[l] = int(self.raw[o:o + 2].view(np.uint16)[0])
            di.hd[l] = idx[p + "self_attn.q_proj.weight"][2][0] // 4
        di.V, di.C = idx["model.embed_tokens.weight"][2][0], idx["masked_embedding.centroids.weight"][2][0]
        self.di = di
        self.h = L.g4o_drafter_load(C.byref(di))

    def close(self):
        if self.h:
            self.orc.L.g4o_drafter_free(self.h)
            self.h = None

    def step(self, go, tok, h, pos, P, T):
        """one draft step on the Gemma oracle go: (token, next hidden, runner-up, gap)"""
        b = np.empty(H, np.float32)
        sec, gap = C.c_int(), C.c_float()
        hh = np.ascontiguousarray(h, np.float32)
        t = self.orc.L.g4o_gemma_draft_step(go.h, self.h, tok, hh.ctypes.data, pos, P, T, b.ctypes.data,
                                            C.byref(sec), C.byref(gap))
        return t, b, sec.value, gap.value


class GemmaTarget:
    """the Gemma oracle and its drafter as a run_req target (tests/protocol.py)"""

    def __init__(self, go, dr=None):
        self.go, self.dr = go, dr

    def prefill(self, toks, pos0, T, i8):
        n = len(toks)
        self.go.set_i8(i8)
        try:
            for b in range(0, n, 32):  # E:1594-1599
                blk = toks[b:b + 32]
                last = b + len(blk) == n
                hb = self.go.forward(blk, pos0 + b, T, len(blk) - 1 if last else len(blk))
        finally:
            self.go.set_i8(False)
        return hb[len(blk) - 1]

    def head(self, h, seeds):
        return self.go.greedy(h, seeds)

    def verify(self, block, nd, nb, pos0, T, allow_b):
        """fwd of the block (E:1649), the lazy head (E:1475-1488) and acceptance (E:1650-1660)"""
        from types import SimpleNamespace
        block = [int(t) for t in block]
        sib = nd + 1 if nb else -1
        hb = self.go.forward(block, pos0, T, 0, sibling=sib)
        G0 = self.head(hb[0], block)
        if sib > 0 and allow_b and block[1] != G0 and block[sib] == G0:  # the sibling row holds row 0's token
            Gs = self.head(hb[sib], block)
            self.go.kv_move(pos0 + sib, pos0 + 1)
            return SimpleNamespace(nacc=1, branch=1, commit=[G0, Gs], G0=G0), hb[sib]
        G = [G0]
        while len(G) - 1 < nd and block[len(G)] == G[-1]:
            G.append(self.head(hb[len(G)], block))
        return SimpleNamespace(nacc=len(G) - 1, branch=0, commit=G, G0=G0), hb[len(G) - 1]

    def draft(self, tok, h, pos, P, T):
        return self.dr.step(self.go, tok, h, pos, P, T)

    def fake_ctx(self, n):
        self.go.fake_ctx(n)


def run_req_k0(go, prompt, nnew, T, pfb=32, rows=None):
    """run_req (E:1584-1661) with ENGINE_K=0 on an empty cache: FIRST and the GEN tokens; rows
    (a list) receives the final-normed hidden row of every head evaluation in order"""
    n = len(prompt)
    G = None
    for b in range(0, n, pfb):  # E:1594-1599 (the last block's last row feeds the head)
        blk = prompt[b:b + pfb]
        last = b + len(blk) == n
        hb = go.forward(blk, b, T, len(blk) - 1 if last else len(blk))
        if last:
            G = go.greedy(hb[len(blk) - 1], blk)
            if rows is not None:
                rows.append(hb[len(blk) - 1].copy())
    gen = [G]
    is_stop = lambda t: t in (106, 1)
    for i in range(1, nnew):  # E:1615
        if is_stop(gen[-1]):
            break
        hb = go.forward([gen[-1]], n + i - 1, T, 0)
        gen.append(go.greedy(hb[0], [gen[-1]]))
        if rows is not None:
            rows.append(hb[0].copy())
    gen = gen[:nnew]
    for i, g in enumerate(gen):
        if is_stop(g):
            return gen[:i + 1]
    return gen


def gap_line(orc, P, h, chosen):
    """E:1497 the engine's debug line of one head row: the full head's r16 logits (exp3 form, as
    head_task computes them), the largest t1 at its first index id1, the largest of the others t2 at
    its first index id2, printed as "GAP %.4f %.4f id1=%d id2=%d chosen=%d" with t1 - t2 in float"""
    lg = orc.r16(orc.exp3_gemm(P, np.asarray(h, np.float32)[None])[0])
    i1 = int(np.argmax(lg))
    rest = lg.copy()
    rest[i1] = -np.inf
    i2 = int(np.argmax(rest))
    t1, t2 = np.float32(lg[i1]), np.float32(lg[i2])
    return "GAP %.4f %.4f id1=%d id2=%d chosen=%d" % (float(t1), float(np.float32(t1 - t2)), i1, i2, chosen)
