"""The engine front-end (gemma4-e2b-laptop-cpu_amd/g4v_engine): the reference engine's line
protocol (E:1681-1689) over the library, driven as the reference's server drives it.  Every
request's FIRST / TOK / GEN lines are checked against run_req (E:1584-1679) restated over the
oracle: prefix reuse, prefill, prompt-lookup or MTP drafts, the sibling row (ENGINE_SIB_GAP 1,
and the tree mode of BENCH_MODE k 1), chain or sibling verify."""
import os
import subprocess
from types import SimpleNamespace

import numpy as np
import pytest

from conftest import PKG, note
from protocol import RunReq

pytestmark = pytest.mark.gpu

SEED, V, NL, I, CTX, T = 71, 16384, 15, 512, 1024, 6
ENV = dict(ENGINE_SERVE="1", ENGINE_STREAM="1", ENGINE_NGRAM="3", ENGINE_NGLEN="3", ENGINE_K="3",
           ENGINE_CTX=str(CTX), ENGINE_CPUS="0,2,4,6,8,10")


class SynthTarget:
    """the synthetic stack and drafter of the oracle as a run_req target (tests/protocol.py)"""

    def __init__(self, orc, dec_i8=False):
        from oracle import Drafter, Model
        self.m = Model(orc, SEED, V, NL, I, CTX)
        self.d = Drafter(orc, SEED + 1, V)
        self.dec_i8 = dec_i8  # G_I8_ACTIVE in the decode (E:1600): W4A8 passes of two rows or more

    def prefill(self, toks, pos0, T, i8):
        return self.m.prefill(toks, pos0=pos0, T=T, i8=i8)

    def head(self, h, seeds):
        return self.m.head(h, seeds)

    def verify(self, block, nd, nb, pos0, T, allow_b):
        o, hid = self.m.verify(block, nd, nb, pos0, T, allow_b=allow_b, i8=self.dec_i8)
        return SimpleNamespace(nacc=o.nacc, branch=o.branch, commit=list(o.commit)[:o.ncommit], G0=o.G[0]), hid

    def draft(self, tok, h, pos, P, T):
        return self.d.step(self.m, tok, h, pos, P, T)

    def close(self):
        self.d.close()
        self.m.close()


class OracleEngine(RunReq):
    """run_req over the oracle's synthetic stack with prompt lookup (ENGINE_NGRAM=3)"""

    def __init__(self, orc, t0=T, adaptive=False, draft_same=True, cut=192, i8=False, nglen=3, dec_i8=False):
        self.target = SynthTarget(orc, dec_i8)
        super().__init__(orc, self.target, t0=t0, adaptive=adaptive, draft_same=draft_same, cut=cut, i8=i8, ngram=3,
                         nglen=nglen)

    def close(self):
        self.target.close()


def run_protocol(orc, requests, tree_from, env_extra, **engine):
    """send the requests (prompt, nnew, k_draft, tree) to the engine, "BENCH_MODE 2 1" before
    request tree_from, and check every line against OracleEngine(orc, **engine)"""
    exe = os.path.join(PKG, "g4v_engine")
    if not os.path.exists(exe):
        pytest.fail("g4v_engine not built (make -C gemma4-e2b-laptop-cpu_amd)")
    env = dict(os.environ, **dict(ENV, **env_extra))
    lines = ""
    for i, (p, nn, _, _) in enumerate(requests):
        if i == tree_from:
            lines += "BENCH_MODE 2 1\n"
        lines += f"{nn} {' '.join(map(str, p))}\n"
    proc = subprocess.run([exe, f"synth:{SEED}:{V}:{NL}:{I}", "-", "-", "0"], input=lines, env=env,
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out = proc.stdout.splitlines()
    oe = OracleEngine(orc, **engine)
    try:
        it = iter(out)
        sib_rounds = hits = 0
        per_req = []
        for k, (prompt, nn, kd, tree) in enumerate(requests):
            if k == tree_from:
                assert next(it) == "MODE k=2 tree=1"
            g0, gen, start = oe.run_req(prompt, nn, kd, tree)
            sib_rounds += oe.sib_rounds
            hits += oe.hits
            per_req.append((oe.sib_rounds, oe.hits))
            first = next(it)
            assert first == f"FIRST {g0}", (k, first, g0)
            streamed = []
            line = next(it)
            while line.startswith("TOK"):
                streamed += [int(x) for x in line.split()[1:]]
                line = next(it)
            assert line.startswith("GEN:"), line
            got = [int(x) for x in line.split()[1:]]
            assert got == gen, (k, got, gen)
            assert [g0] + streamed == gen, (k, streamed)
            timing = next(it)
            assert timing.startswith("TIMING") and f"reused={start} " in timing, (k, timing)
        # E:1673 per request: the sibling rows proposed (TREE attempts) and committed (hits)
        rank1 = [ln for ln in proc.stderr.splitlines() if ln.startswith("RANK1")]
        assert len(rank1) == len(requests), proc.stderr[-1000:]
        for k, ln in enumerate(rank1):
            assert f"TREE attempts={per_req[k][0]} hits={per_req[k][1]}" in ln, (k, ln, per_req[k])
        note(f"sibling rounds {sib_rounds}, tree hits {hits}, split counts {sorted(oe.splits_seen)}")
        return sib_rounds, oe.splits_seen
    finally:
        oe.close()


def test_engine_protocol_matches_oracle(orc):
    rng = np.random.default_rng(5)
    motif = rng.integers(0, V, 16).tolist()
    a = (motif * 8)[:100]
    b = rng.integers(0, V, 40).tolist()
    c = rng.integers(0, V, 30).tolist()
    requests = [(a, 20, 3, False), (b, 10, 3, False), (a, 15, 3, False), (a + [5, 6, 7], 8, 3, False),
                (c, 24, 3, False), (b + [9], 16, 2, True), (c + [4], 12, 2, True)]
    note("engine protocol: 7 requests over a 15-layer synthetic stack")
    sib_rounds, _ = run_protocol(orc, requests, 5, {})
    assert sib_rounds > 0


@pytest.mark.parametrize("cpus,extra", [
    (8, {}),  # the first prompt splits 8 ways, every later pass 6 (the drafter's set_active persists)
    (8, dict(ENGINE_ADAPTIVE_THREADS="1")),  # 6 / 8 either side of position 192, per pass
    (8, dict(ENGINE_ADAPTIVE_THREADS="1", ENGINE_DRAFT_SAME="0", ENGINE_THREAD_CUTOFF="150")),
    (4, dict(ENGINE_ADAPTIVE_THREADS="1")),  # set_active clamps to the pool
])
def test_engine_split_counts_follow_pool(orc, cpus, extra):
    """the split-KV count of every pass follows the reference pool's active workers"""
    rng = np.random.default_rng(11)
    a = rng.integers(0, V, 176).tolist()
    b = rng.integers(0, V, 230).tolist()
    requests = [(a, 40, 3, False), (b, 12, 3, False), (a + [7], 10, 3, False)]
    note(f"engine split counts: {cpus} CPUs, {extra}")
    env = dict(extra, ENGINE_CPUS=",".join(str(2 * i) for i in range(cpus)))
    _, seen = run_protocol(orc, requests, len(requests), env, t0=cpus,
                           adaptive="ENGINE_ADAPTIVE_THREADS" in extra,
                           draft_same=extra.get("ENGINE_DRAFT_SAME") != "0",
                           cut=int(extra.get("ENGINE_THREAD_CUTOFF", 192)))
    assert seen == ({4} if cpus == 4 else {6, 8}), seen


@pytest.mark.parametrize("nglen", [5, 7])
def test_engine_long_lookup_chains(orc, nglen):
    """ENGINE_NGLEN up to 7 (E:1514): prompt-lookup chains of up to 7 drafts verified in one pass"""
    rng = np.random.default_rng(13)
    motif = rng.integers(0, V, 24).tolist()
    requests = [((motif * 9)[:200], 30, 3, False), ((motif * 3)[:50] + [11, 12], 20, 3, False)]
    note(f"engine lookup chains, ENGINE_NGLEN={nglen}")
    run_protocol(orc, requests, len(requests), dict(ENGINE_NGLEN=str(nglen)), nglen=nglen)


def test_engine_prefill_int8(orc):
    """ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8=0: W4A8 prompt blocks, exact-float decode
    (E:1210, 1596, 1600); with the decode's W4A8 left on (its default, the server's mode) the
    verify passes of two rows or more multiply W4A8 too, drafting and the tree mode included.
    Settings the engine does not restate end it with exit status 2."""
    rng = np.random.default_rng(12)
    requests = [(rng.integers(0, V, 70).tolist(), 12, 3, False), (rng.integers(0, V, 33).tolist(), 8, 3, False)]
    run_protocol(orc, requests, len(requests), dict(ENGINE_PREFILL_INT8="1", ENGINE_DECODE_INT8="0"), i8=True)
    requests = [(rng.integers(0, V, 70).tolist(), 16, 3, False), (rng.integers(0, V, 40).tolist(), 12, 3, False),
                (rng.integers(0, V, 50).tolist(), 12, 2, True)]
    run_protocol(orc, requests, 2, dict(ENGINE_PREFILL_INT8="1"), i8=True, dec_i8=True)
    exe = os.path.join(PKG, "g4v_engine")
    for extra in (dict(ENGINE_ATT_PAR="128"), dict(ENGINE_SPLITKV="0")):
        proc = subprocess.run([exe, f"synth:{SEED}:{V}:{NL}:{I}", "-", "-", "0"], input="4 1 2 3\n",
                              env=dict(os.environ, **dict(ENV, **extra)), capture_output=True, text=True, timeout=120)
        assert proc.returncode == 2 and "g4v_engine:" in proc.stderr, (extra, proc.returncode, proc.stderr[-500:])


def write_checkpoint(om, d, V, NL, I):
    """the oracle's stack as a safetensors checkpoint with the engine's tensor index beside it
    (name, dtype, absolute byte offset, byte count, shape: the format the engine reads, E:1218-1222)"""
    import json
    H = 1536
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj"]
    Ns, Ks = [2048, 256, 256, H, I, I, H], [H, H, H, 2048, H, H, I]
    norms = ["input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm",
             "self_attn.q_norm", "self_attn.k_norm"]
    bf = lambda f: (np.ascontiguousarray(f, np.float32).view(np.uint32) >> 16).astype(np.uint16)  # exact: bf16 values
    tensors = [("embed_tokens.weight", "BF16", [V, H], om.get("E", np.uint16, V * H)),
               ("norm.weight", "BF16", [H], bf(om.get("fnorm", np.float32, H)))]
    for l in range(NL):
        p = f"layers.{l}."
        for j in range(7):
            w = om.get(f"W{l}_{j}", np.uint8, Ns[j] * Ks[j] // 2)
            s = om.get(f"S{l}_{j}", np.uint16, Ns[j] * Ks[j] // 32)
            tensors.append((p + names[j] + ".weight_packed", "I32", [Ns[j], Ks[j] // 8], w))
            tensors.append((p + names[j] + ".weight_scale", "BF16", [Ns[j], Ks[j] // 32], s))
        for t, nm in enumerate(norms):
            n = H if t < 4 else 256
            tensors.append((p + nm + ".weight", "BF16", [n], bf(om.get(f"N{l}_{t}", np.float32, n))))
        tensors.append((p + "layer_scalar", "BF16", [1], bf(np.array([0.75], np.float32))))
    header, off = {}, 0
    for name, dt, shape, arr in tensors:
        header["model.language_model." + name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + arr.nbytes]}
        off += arr.nbytes
    hb = json.dumps(header).encode()
    hb += b" " * (-len(hb) % 8)
    with open(os.path.join(d, "model.safetensors"), "wb") as f:
        f.write(np.uint64(len(hb)).tobytes())
        f.write(hb)
        for _, _, _, arr in tensors:
            f.write(np.ascontiguousarray(arr).tobytes())
    with open(os.path.join(d, "index.tsv"), "w") as f:
        for name, v in header.items():
            a, b = v["data_offsets"]
            f.write(f"{name}\t{v['dtype']}\t{8 + len(hb) + a}\t{b - a}\t{','.join(map(str, v['shape']))}\n")


def test_engine_loads_checkpoint(orc, tmp_path):
    """the engine on a checkpoint of the synthetic stack (model.safetensors + tensor index)
    answers exactly as on the stack generated in place: the loader maps every tensor"""
    from oracle import Model
    exe = os.path.join(PKG, "g4v_engine")
    NLc = 15
    om = Model(orc, SEED, V, NLc, I, CTX)
    try:
        write_checkpoint(om, str(tmp_path), V, NLc, I)
    finally:
        om.close()
    rng = np.random.default_rng(9)
    motif = rng.integers(0, V, 12).tolist()
    requests = [((motif * 6)[:60], 16), (rng.integers(0, V, 25).tolist(), 12)]
    lines = "".join(f"{nn} {' '.join(map(str, p))}\n" for p, nn in requests)
    env = dict(os.environ, **ENV, ENGINE_DRAFTER_SEED=str(SEED + 1))
    outs = []
    for model, index in ((f"synth:{SEED}:{V}:{NLc}:{I}", "-"), (str(tmp_path), str(tmp_path / "index.tsv"))):
        note(f"engine on {model}")
        proc = subprocess.run([exe, model, index, "-", "0"], input=lines, env=env, capture_output=True, text=True,
                              timeout=240)
        assert proc.returncode == 0, proc.stderr[-2000:]
        outs.append([ln for ln in proc.stdout.splitlines() if not ln.startswith("TIMING")])
    assert outs[0] == outs[1]
    assert sum(ln.startswith("GEN:") for ln in outs[1]) == len(requests)
    # a layer without its own k/v projections (the KV-shared layers of Gemma-4-E2B) is refused
    with open(tmp_path / "index.tsv") as f:
        kept = [ln for ln in f if ".layers.1.self_attn.k_proj." not in ln]
    with open(tmp_path / "shared.tsv", "w") as f:
        f.writelines(kept)
    proc = subprocess.run([exe, str(tmp_path), str(tmp_path / "shared.tsv"), "-", "0"], input=lines, env=env,
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 2 and "KV-shared" in proc.stderr, (proc.returncode, proc.stderr[-500:])
