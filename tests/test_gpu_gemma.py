"""The Gemma-4-E2B layer layout on the device (g4v_model_create_gemma): head_dim 256 / 512
layers, KV sharing past layer 14, per-layer MLP widths and the per-layer-input branch, on the
synthetic checkpoint of tests/golden/gemma_layout.py uploaded through the C ABI.

  * run_req with ENGINE_K=0 (prefill in blocks of 32, then one-row decode passes, 6 splits)
    gives the FIRST / GEN tokens the reference engine's own main() gave on the same checkpoint
    (tests/golden/gemma_layout.npz), with exact float prompt blocks and with W4A8 ones
    (ENGINE_PREFILL_INT8=1, g4v_set_prefill_int8);
  * a prompt's final-normed state and every owner cache equal the oracle's (bit for bit), in
    both prefill modes;
  * a chain pass of greedy drafts and the sibling form commit what the oracle's rows give, in
    exact float and with W4A8 verify passes (ENGINE_DECODE_INT8, g4v_set_decode_int8);
  * g4v_engine's drafting sessions, the server's environment (W4A8 prompt and verify) among them,
    print what the reference engine printed."""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import note
from util import first_diff, same

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import gemma_layout as gl  # noqa: E402

pytestmark = pytest.mark.gpu
FX = os.path.join(HERE, "golden", "gemma_layout.npz")


def upload(dev, d, ctx):
    """the checkpoint in d onto the device, tensor by tensor as the engine's loader would"""
    raw = np.memmap(os.path.join(d, "model.safetensors"), np.uint8, "r")
    idx = {}
    for line in open(os.path.join(d, "index.tsv")):
        n, dt, o, nb, sh = line.rstrip("\n").split("\t")
        idx[n.replace("model.language_model.", "")] = (int(o), int(nb), tuple(int(x) for x in sh.split(",")))
    get = lambda n, dt=np.uint8: np.asarray(raw[idx[n][0]:idx[n][0] + idx[n][1]]).view(dt)
    bfv = lambda n: (get(n, np.uint16).astype(np.uint32) << 16).view(np.float32)
    dev.model_create_gemma(gl.V, gl.MLP, ctx)
    dev.set_embed(get("embed_tokens.weight", np.uint16))
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj", "per_layer_input_gate", "per_layer_projection"]
    for l in range(gl.NL):
        p = f"layers.{l}."
        for j, nm in enumerate(names):
            if j in (1, 2) and l >= 15:
                continue
            N, K8 = idx[p + nm + ".weight_packed"][2]
            dev.set_matrix(l, j, get(p + nm + ".weight_packed").reshape(N, K8 * 4),
                           get(p + nm + ".weight_scale", np.uint16))
        nv = [bfv(p + n + ".weight") for n in ("input_layernorm", "post_attention_layernorm",
                                                "pre_feedforward_layernorm", "post_feedforward_layernorm",
                                                "post_per_layer_input_norm", "self_attn.q_norm")]
        nv.append(bfv(p + "self_attn.k_norm.weight") if l < 15 else None)
        dev.set_norms_gemma(l, nv, float(bfv(p + "layer_scalar")[0]))
    N, K8 = idx["per_layer_model_projection.weight_packed"][2]
    dev.set_ple(get("per_layer_model_projection.weight_packed").reshape(N, K8 * 4),
                get("per_layer_model_projection.weight_scale", np.uint16), bfv("per_layer_projection_norm.weight"))
    ple = np.asarray(raw[idx["embed_tokens_per_layer.weight"][0]:]).view(np.uint16)
    for t in gl.PLE_IDS:
        dev.set_ple_rows(t, ple[t * gl.NL * gl.PD:(t + 1) * gl.NL * gl.PD].reshape(1, -1))
    dev.set_final_norm(bfv("norm.weight"))


@pytest.fixture(scope="module")
def gemma(orc, g4v, gemma_ckpt):
    d = gemma_ckpt
    fx = np.load(FX)
    ctx = int(fx["ctx"][0])
    dev = g4v.Device(0)
    note("uploading it")
    upload(dev, d, ctx)
    dev.set_prefill_int8(False)  # exact float prompt blocks unless a test asks for W4A8
    yield dev, d, fx, ctx
    dev.close()


def device_run_req_k0(dev, prompt, nnew, T):
    """run_req (E:1584-1661) with ENGINE_K=0 over the library: prefill, then one-row passes"""
    n = len(prompt)
    gen = [int(dev.prefill(np.array(prompt, np.int32), 0, 32, T))]
    for i in range(1, nnew):
        if gen[-1] in (106, 1):
            break
        r = dev.verify(np.array([gen[-1]], np.int32), 0, 0, n + i - 1, T)
        gen.append(int(r.commit[0]))
    gen = gen[:nnew]
    for i, g in enumerate(gen):
        if g in (106, 1):
            return gen[:i + 1]
    return gen


@pytest.mark.parametrize("i8", [False, True])
@pytest.mark.parametrize("i", [0, 1, 2])
def test_gemma_tokens_match_reference_engine(gemma, i, i8):
    dev, d, fx, ctx = gemma
    sfx = "_i8" if i8 else ""
    prompts = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])
    want = np.split(fx["gens" + sfx], np.cumsum(fx["gen_lens" + sfx])[:-1])[i]
    note(f"gemma run_req prompt {i} ({len(prompts[i])} tokens), int8 prefill {i8}")
    dev.set_prefill_int8(i8)
    try:
        got = device_run_req_k0(dev, [int(t) for t in prompts[i]], int(fx["nnew"][0]), int(fx["cpus"][0]))
    finally:
        dev.set_prefill_int8(False)
    assert got[0] == int(fx["first" + sfx][i])
    assert got == [int(t) for t in want], (got, list(want))


@pytest.mark.parametrize("i8", [False, True])
def test_gemma_prefill_state_and_caches(orc, gemma, i8):
    dev, d, fx, ctx = gemma
    prompt = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])[2]  # 196 tokens: split-KV tail
    go = gl.GemmaOracle(orc, d, ctx, i8=i8)
    dev.set_prefill_int8(i8)
    try:
        note(f"gemma prefill of 196 tokens against the oracle, int8 {i8}")
        hd_ = None
        for b in range(0, len(prompt), 32):
            blk = [int(t) for t in prompt[b:b + 32]]
            last = b + len(blk) == len(prompt)
            hb = go.forward(blk, b, 6, len(blk) - 1 if last else len(blk))
            if last:
                hd_ = hb[len(blk) - 1]
        g0, h = dev.prefill(np.array(prompt, np.int32), 0, 32, 6, hidden=True)
        assert same(h, hd_), first_diff(h, hd_)
        n = len(prompt)
        for l in range(15):
            hdl = gl.layer_hd(l)
            for v, nm in ((0, "GK"), (1, "GV")):
                a = dev.read(f"{nm}{l}", np.uint16)[:n * hdl]
                b = go.cache(l, v)[:n * hdl]
                assert same(a, b), (nm, l, first_diff(a, b))
    finally:
        dev.set_prefill_int8(False)
        go.close()


@pytest.mark.parametrize("kind,pos0,i8", [("chain", 210, False), ("chain", 40, False), ("sibling", 150, False),
                                          ("sibling", 240, False), ("chain", 210, True), ("chain", 40, True),
                                          ("sibling", 240, True), ("chain7", 210, True), ("chain7", 210, False),
                                          ("chain0", 210, False), ("chain0", 40, False)])
def test_gemma_multirow_passes(orc, gemma, kind, pos0, i8):
    """a chain of 3 greedy drafts (split-KV past 192 keys, run_mh below), of 7 (attn_tile), a one-row
    pass (no drafts) and the sibling form (nd 2 + the runner-up at RoPE position pos0 + 1, E:1634-1655) after a prefill,
    against the oracle's rows: committed tokens and the committed row's state.  i8:
    ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8 on (E:1600), W4A8 prompt blocks and verify
    passes on both sides"""
    dev, d, fx, ctx = gemma
    prompt = [int(t) for t in np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])[2]][:pos0]
    while len(prompt) < pos0:
        prompt = prompt + prompt[:pos0 - len(prompt)]
    go = gl.GemmaOracle(orc, d, ctx, i8=i8)
    dev.set_prefill_int8(i8)
    dev.set_decode_int8(i8)
    try:
        for b in range(0, pos0, 32):
            blk = prompt[b:b + 32]
            hb = go.forward(blk, b, 6, len(blk) - 1 if b + len(blk) == pos0 else len(blk))
        g0 = go.greedy(hb[len(blk) - 1], blk)
        dev.prefill(np.array(prompt, np.int32), 0, 32, 6)
        # greedy chain from the oracle (one-row passes on a copy of the state would move its cache,
        # so the chain is taken as the model's own continuation of a fresh forward per step)
        if kind.startswith("chain"):
            nd = {"chain7": 7, "chain0": 0}.get(kind, 3)
            toks = [g0]
            for j in range(nd):
                hh = go.forward(toks[:j + 1], pos0, 6, 0)
                toks.append(go.greedy(hh[j], toks[:j + 1]))
            hh = go.forward(toks, pos0, 6, 0)
            G = [go.greedy(hh[m], toks) for m in range(nd + 1)]
            r, h = dev.verify(np.array(toks, np.int32), nd, 0, pos0, 6, hidden=True)
            note(f"chain of {nd} at {pos0}: oracle G {G}, device commit {list(r.commit[:r.ncommit])}")
            assert r.nacc == nd and list(r.commit[:nd + 1]) == G
            assert same(h, hh[nd]), first_diff(h, hh[nd])
        else:
            # row 0's greedy token does not depend on the later rows' tokens: take it from a
            # first pass, then put it into the sibling row and a different token into draft 1
            toks = [g0, 11, 7, 13]
            G0 = go.greedy(go.forward(toks, pos0, 6, 0, sibling=3)[0], toks)
            toks = [g0, G0 + 1, 7, G0]
            hs = go.forward(toks, pos0, 6, 0, sibling=3)
            assert go.greedy(hs[0], toks) == G0
            G3 = go.greedy(hs[3], toks)
            r, h = dev.verify_sibling(np.array(toks, np.int32), 2, pos0, 6, True, hidden=True)
            note(f"sibling at {pos0}: oracle G0 {G0} G3 {G3}, device {r.as_dict()}")
            assert (r.nacc, r.branch, r.ncommit) == (1, 1, 2) and list(r.commit[:2]) == [G0, G3]
            assert same(h, hs[3]), first_diff(h, hs[3])
            for l in range(15):  # the sibling's rows moved into place (E:1651)
                hdl = gl.layer_hd(l)
                for v, nm in ((0, "GK"), (1, "GV")):
                    a = dev.read(f"{nm}{l}", np.uint16)[(pos0 + 1) * hdl:(pos0 + 2) * hdl]
                    b = go.cache(l, v)[(pos0 + 3) * hdl:(pos0 + 4) * hdl]
                    assert same(a, b), (nm, l)
    finally:
        dev.set_prefill_int8(False)
        dev.set_decode_int8(False)
        go.close()


@pytest.mark.parametrize("i8", [False, True])
def test_gemma_engine_matches_reference_engine(gemma, i8):
    """g4v_engine on the checkpoint directory and its index, as main() is run (E:1211-1231), in
    serve mode over the three prompts: FIRST / GEN lines equal the reference engine's"""
    dev, d, fx, ctx = gemma
    exe = os.path.join(os.path.dirname(HERE), "gemma4-e2b-laptop-cpu_amd", "g4v_engine")
    sfx = "_i8" if i8 else ""
    prompts = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])
    gens = np.split(fx["gens" + sfx], np.cumsum(fx["gen_lens" + sfx])[:-1])
    nnew = int(fx["nnew"][0])
    env = dict(os.environ, ENGINE_SERVE="1", ENGINE_K="0", ENGINE_CTX=str(ctx), ENGINE_DECODE_INT8="0",
               ENGINE_CPUS=",".join(str(c) for c in range(int(fx["cpus"][0]))))
    for k in ("ENGINE_PREFILL_INT8", "ENGINE_ADAPTIVE_THREADS", "ENGINE_NGRAM", "ENGINE_STREAM"):
        env.pop(k, None)
    if i8:
        env["ENGINE_PREFILL_INT8"] = "1"
    lines = "".join(f"{nnew} {' '.join(map(str, p))}\n" for p in prompts)
    note(f"g4v_engine on the Gemma-layout checkpoint, int8 prefill {i8}")
    proc = subprocess.run([exe, d, os.path.join(d, "index.tsv"), "-", "0"], input=lines, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    firsts = [int(ln.split()[1]) for ln in proc.stdout.splitlines() if ln.startswith("FIRST")]
    got = [[int(x) for x in ln.split()[1:]] for ln in proc.stdout.splitlines() if ln.startswith("GEN:")]
    assert firsts == [int(t) for t in fx["first" + sfx]]
    assert got == [[int(t) for t in g] for g in gens], (got, gens)


def test_gemma_engine_stage_lines(gemma, tmp_path):
    """g4v_engine's observability lines on the 196-token prompt, plain decode (ENGINE_K=0):
    SCREEN (E:1690) counts every head call -- the warm-up pass, the prompt's last row and one row
    per decode step -- as a screened row or a fallback; DECODE_STAGE (E:1672) one forward per
    decode step, with split-KV attention time (positions past 192) and no drafter time; STAGES
    (E:1691) every forward call (the warm-up, 7 prompt blocks of 32, the decode steps).  The
    tokens equal the reference engine's."""
    dev, d, fx, ctx = gemma
    exe = os.path.join(os.path.dirname(HERE), "gemma4-e2b-laptop-cpu_amd", "g4v_engine")
    prompt = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])[2]
    want = [int(t) for t in np.split(fx["gens"], np.cumsum(fx["gen_lens"])[:-1])[2]]
    nnew = int(fx["nnew"][0])
    pf = tmp_path / "prompt.ids"
    pf.write_text(" ".join(str(int(t)) for t in prompt) + "\n")
    env = dict(os.environ, ENGINE_K="0", ENGINE_CTX=str(ctx), ENGINE_DECODE_INT8="0", ENGINE_HEAD_SCREEN="1",
               ENGINE_DECODE_STAGE="1", ENGINE_STAGE_PROF="1",
               ENGINE_CPUS=",".join(str(c) for c in range(int(fx["cpus"][0]))))
    for k in ("ENGINE_PREFILL_INT8", "ENGINE_ADAPTIVE_THREADS", "ENGINE_NGRAM", "ENGINE_STREAM", "ENGINE_SERVE"):
        env.pop(k, None)
    note(f"g4v_engine stage lines, prompt of {len(prompt)} tokens, {nnew} new")
    proc = subprocess.run([exe, d, os.path.join(d, "index.tsv"), str(pf), str(nnew)], env=env, capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    gen = [[int(x) for x in ln.split()[1:]] for ln in proc.stdout.splitlines() if ln.startswith("GEN:")]
    assert gen == [want]
    steps = len(want) - 1
    lines = {ln.split()[0]: ln for ln in proc.stderr.splitlines() if ln.split()}
    assert {"DECODE_STAGE", "STAGES"} <= set(lines), proc.stderr[-3000:]
    # the same head calls through the library, counted by the reference's rule (E:1472, 1489): a
    # row's survivors until the call's first row that overflows the screen, which counts one
    # fallback; the line is printed only when some row was screened (E:1690)
    T = int(fx["cpus"][0])
    cnt = dict(rows=0, surv=0, max=0, fb=0)

    def count(G, ns, fbk):
        for g, n, f in zip(G, ns, fbk):
            if g < 0:
                continue
            if f:
                cnt["fb"] += 1
                return
            cnt["rows"] += 1
            cnt["surv"] += n
            cnt["max"] = max(cnt["max"], n)

    dev.prefill(np.array([2], np.int32), 0, 32, T)  # the warm-up pass (E:1578)
    ns, f = dev.prefill_head_stats()
    count([0], [ns], [f])
    toks = [int(dev.prefill(np.array(prompt, np.int32), 0, 32, T))]
    ns, f = dev.prefill_head_stats()
    count([0], [ns], [f])
    for i in range(1, len(want)):
        r = dev.verify(np.array([toks[-1]], np.int32), 0, 0, len(prompt) + i - 1, T)
        toks.append(int(r.commit[0]))
        count(list(r.G), list(r.nsurv), list(r.fallback))
    assert toks == want
    assert cnt["rows"] + cnt["fb"] == steps + 2
    if cnt["rows"]:
        scr = re.match(r"SCREEN rows=(\d+) survivors mean=([0-9.]+) max=(\d+) fallbacks=(\d+)$", lines["SCREEN"])
        assert (int(scr[1]), int(scr[3]), int(scr[4])) == (cnt["rows"], cnt["max"], cnt["fb"]), lines["SCREEN"]
        assert abs(float(scr[2]) - cnt["surv"] / cnt["rows"]) <= 0.051, lines["SCREEN"]
    else:
        assert "SCREEN" not in lines, lines["SCREEN"]
    ds = re.match(r"DECODE_STAGE forwards=(\d+) layers_ms=([0-9.]+) split_att_ms=([0-9.]+) head_ms=([0-9.]+) "
                  r"draft_ms=([0-9.]+) total_ms=([0-9.]+)$", lines["DECODE_STAGE"])
    fwd, lay, att, head, dr, tot = int(ds[1]), *(float(ds[i]) for i in range(2, 7))
    assert fwd == steps, lines["DECODE_STAGE"]
    assert 0 < att < lay and head > 0 and dr == 0, lines["DECODE_STAGE"]
    assert lay + head <= tot + 1.0, lines["DECODE_STAGE"]
    st = re.match(r"STAGES total over (\d+) fwd calls \(ms\): layers (\d+) \(of which split-KV attention (\d+)\) \| "
                  r"head (\d+) \| drafter (\d+)$", lines["STAGES"])
    assert int(st[1]) == 1 + (len(prompt) + 31) // 32 + steps, lines["STAGES"]
    assert int(st[5]) == 0, lines["STAGES"]


def drafter_arrays(d):
    """the drafter checkpoint of gemma_layout.write_drafter as Device.drafter_load's dict"""
    raw = np.memmap(os.path.join(d, "drafter", "model.safetensors"), np.uint8, "r")
    idx = {}
    for line in open(os.path.join(d, "drafter_index.tsv")):
        n, dt, o, nb, sh = line.rstrip("\n").split("\t")
        idx[n] = (int(o), int(nb), tuple(int(x) for x in sh.split(",")))
    get = lambda n, dt=np.uint16: np.asarray(raw[idx[n][0]:idx[n][0] + idx[n][1]]).view(dt)
    t = dict(pre=get("pre_projection.weight"), post=get("post_projection.weight"),
             cent=get("masked_embedding.centroids.weight"), emb=get("model.embed_tokens.weight"),
             norm=get("model.norm.weight"), order=get("masked_embedding.token_ordering", np.int64),
             C=idx["masked_embedding.centroids.weight"][2][0])
    for n, key in (("q", "self_attn.q_proj"), ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"),
                   ("up", "mlp.up_proj"), ("down", "mlp.down_proj")):
        t[n] = [get(f"model.layers.{l}.{key}.weight") for l in range(4)]
    t["nv"] = [[get(f"model.layers.{l}.{k}.weight") for k in ("input_layernorm", "post_attention_layernorm",
                                                                "pre_feedforward_layernorm",
                                                                "post_feedforward_layernorm", "self_attn.q_norm")]
               for l in range(4)]
    t["scalar"] = [int(get(f"model.layers.{l}.layer_scalar")[0]) for l in range(4)]
    t["hd"] = [idx[f"model.layers.{l}.self_attn.q_proj.weight"][2][0] // 4 for l in range(4)]
    return t


@pytest.mark.parametrize("P", [60, 195, 300])
def test_gemma_drafter_chain(orc, gemma, P):
    """the drafter checkpoint on the device (g4v_drafter_load: layer 3 of head dim 512 over the
    layout's owner cache 14, layers 0..2 over cache 13): a 3-step chain after a prefill of P + 1
    tokens equals the oracle's draft steps (tokens, runners-up, gaps, last hidden state)"""
    dev, d, fx, ctx = gemma
    prompt = [int(t) for t in np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])[2]]
    while len(prompt) < P + 1:
        prompt = prompt + prompt[:P + 1 - len(prompt)]
    prompt = prompt[:P + 1]
    dev.drafter_load(drafter_arrays(d))
    go = gl.GemmaOracle(orc, d, ctx)
    dr = gl.GemmaDrafter(orc, d)
    try:
        note(f"gemma drafter chain after {P + 1} prompt tokens")
        h = gl.GemmaTarget(go).prefill(np.array(prompt, np.int32), 0, 6, False)
        g0, hd_ = dev.prefill(np.array(prompt, np.int32), 0, 32, 6, hidden=True)
        assert same(hd_, h)
        tok, hh, want = g0, h, []
        for j in range(3):
            tok, hh, sec, gap = dr.step(go, tok, hh, P + 1 + j, P, 6)
            want.append((tok, sec, gap))
        drafts, secs, gaps, hid = dev.draft_mtp(g0, h, P, 3, 6)
        note(f"oracle {want}, device {list(drafts)} {list(secs)} {list(gaps)}")
        assert [int(x) for x in drafts] == [w[0] for w in want]
        assert [int(x) for x in secs] == [w[1] for w in want]
        assert same(np.array(gaps, np.float32), np.array([w[2] for w in want], np.float32))
        assert same(hid, hh), first_diff(hid, hh)
    finally:
        dr.close()
        go.close()


# the drafting sessions of tests/golden/make_gemma_layout.py
# k3_i8: the server's environment, W4A8 prompt blocks and verify passes (E:1600)
DRAFT_MODES = {"k3": dict(ENGINE_K="3"), "tree": dict(ENGINE_K="2", ENGINE_TREE="1"),
               "ng": dict(ENGINE_K="3", ENGINE_NGRAM="2", ENGINE_NGLEN="5"),
               "k3_i8": dict(ENGINE_K="3", ENGINE_PREFILL_INT8="1", ENGINE_DECODE_INT8="1"),
               "k3_same": dict(ENGINE_K="3", ENGINE_DRAFT_SAMEPOS="1"),  # E:1516, 1633
               "fake": dict(ENGINE_K="3", ENGINE_FAKE_CTX="300")}         # E:1211, 1249-1250


@pytest.mark.parametrize("mode", list(DRAFT_MODES))
def test_gemma_engine_drafting_matches_reference_engine(gemma, mode):
    """g4v_engine with the drafter checkpoint (ENGINE_DRAFTER_DIR / ENGINE_DRAFTER_INDEX) in serve
    mode: FIRST / GEN lines and the RANK1 / TREE counts equal the reference engine's session"""
    dev, d, fx, ctx = gemma
    exe = os.path.join(os.path.dirname(HERE), "gemma4-e2b-laptop-cpu_amd", "g4v_engine")
    prompts = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])
    gens = np.split(fx["gens_" + mode], np.cumsum(fx["gen_lens_" + mode])[:-1])
    nnew = int(fx["nnew_d"][0])
    env = dict(os.environ, ENGINE_SERVE="1", ENGINE_CTX=str(ctx), ENGINE_DECODE_INT8="0",
               ENGINE_CPUS=",".join(str(c) for c in range(int(fx["cpus"][0]))),
               ENGINE_DRAFTER_DIR=os.path.join(d, "drafter"), ENGINE_DRAFTER_INDEX=os.path.join(d, "drafter_index.tsv"))
    for k in ("ENGINE_PREFILL_INT8", "ENGINE_ADAPTIVE_THREADS", "ENGINE_NGRAM", "ENGINE_NGLEN", "ENGINE_STREAM",
              "ENGINE_TREE", "ENGINE_SIB_GAP", "ENGINE_SIB_LONG", "ENGINE_POLICY", "ENGINE_DRAFT_SAMEPOS",
              "ENGINE_FAKE_CTX", "ENGINE_TAU", "ENGINE_NO_TILED", "ENGINE_SLOTS"):
        env.pop(k, None)
    env.update(DRAFT_MODES[mode])
    lines = "".join(f"{nnew} {' '.join(map(str, p))}\n" for p in prompts)
    note(f"g4v_engine drafting session {mode} on the Gemma-layout checkpoint")
    proc = subprocess.run([exe, d, os.path.join(d, "index.tsv"), "-", "0"], input=lines, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    firsts = [int(ln.split()[1]) for ln in proc.stdout.splitlines() if ln.startswith("FIRST")]
    got = [[int(x) for x in ln.split()[1:]] for ln in proc.stdout.splitlines() if ln.startswith("GEN:")]
    rank1 = [[int(w.split("=")[1]) for w in ln.split() if "=" in w] for ln in proc.stderr.splitlines()
             if ln.startswith("RANK1")]
    assert firsts == [int(t) for t in fx["first_" + mode]]
    assert got == [[int(t) for t in g] for g in gens], (got, gens)
    assert rank1 == [[int(v) for v in r] for r in fx["rank1_" + mode]], rank1


def test_gemma_engine_needs_drafter_files(gemma):
    """ENGINE_K > 0 without the drafter checkpoint ends with a message, as main() needs it (E:1519)"""
    dev, d, fx, ctx = gemma
    exe = os.path.join(os.path.dirname(HERE), "gemma4-e2b-laptop-cpu_amd", "g4v_engine")
    env = dict(os.environ, ENGINE_K="3", ENGINE_CTX=str(ctx), ENGINE_DRAFTER_DIR=os.path.join(d, "none"),
               ENGINE_DRAFTER_INDEX=os.path.join(d, "none.tsv"))
    pf = os.path.join(d, "p.ids")
    with open(pf, "w") as f:
        f.write("5 6 7\n")
    proc = subprocess.run([exe, d, os.path.join(d, "index.tsv"), pf, "4"], env=env, capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 2 and "none.tsv" in proc.stderr, (proc.returncode, proc.stderr[-500:])


def test_gemma_synth_layout(g4v):
    """g4v_model_synth_gemma (the benchmark's Gemma-4-E2B workload, weights generated on the
    device) runs prefill, decode and chain passes; two contexts from one seed agree bit for bit"""
    outs = []
    for _ in range(2):
        dev = g4v.Device(0)
        try:
            dev.model_synth_gemma(17, 16384, [512] * 15 + [1024] * 20, 1024)
            toks = (np.arange(300, dtype=np.int32) * 37) % 16384
            g0, h = dev.prefill(toks, 0, 32, 6, hidden=True)
            r1, h1 = dev.verify(np.array([g0], np.int32), 0, 0, 300, 6, hidden=True)
            r4, h4 = dev.verify(np.array([g0, 5, 6, 7], np.int32), 3, 0, 300, 6, hidden=True)
            outs.append((g0, h, r1.commit[0], h1, r4.as_dict(), h4))
        finally:
            dev.close()
    a, b = outs
    assert a[0] == b[0] and a[2] == b[2] and a[4] == b[4]
    assert same(a[1], b[1]) and same(a[3], b[3]) and same(a[5], b[5])
    assert a[4]["G"][0] == a[2]  # row 0 of the chain pass is the decode pass's row


def test_gemma_split_limit_binds_split_blocks_only(g4v):
    """the per-split limit of the split buffer binds only passes that take the split-KV path (at
    most 4 rows past ATT_PAR, E:1305): a 3,000-token prompt in blocks of 32 (attn_tile, E:1328)
    runs with one split and gives the state six splits give; a 1-row pass there with one split is
    refused, and runs with six"""
    V, n = 16384, 3000
    toks = (np.arange(n, dtype=np.int32) * 101 + 7) % V
    outs = []
    for ns in (1, 6):
        dev = g4v.Device(0)
        try:
            dev.model_synth_gemma(23, V, [512] * 15 + [1024] * 20, 4096)
            note(f"gemma prefill n={n} pfb=32 nsplit={ns}")
            g0, h = dev.prefill(toks, 0, 32, ns, hidden=True)
            if ns == 1:
                with pytest.raises(RuntimeError, match="context too long for nsplit"):
                    dev.verify(np.array([g0], np.int32), 0, 0, n, 1)
            r1 = dev.verify(np.array([g0], np.int32), 0, 0, n, 6)
            outs.append((g0, h, r1.commit[0]))
        finally:
            dev.close()
    assert outs[0][0] == outs[1][0] and outs[0][2] == outs[1][2]
    assert same(outs[0][1], outs[1][1])
