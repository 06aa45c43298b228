"""The oracle's Gemma-4-E2B layer layout (oracle/g4_oracle_gemma.c: head_dim 256 / 512 layers,
KV sharing past layer 14, per-layer MLP widths, per-layer inputs, partial RoPE) against the
reference engine's main() run unchanged on the same synthetic checkpoint
(tests/golden/make_gemma_layout.py, oracle/_ref/gemma4_engine): FIRST and GEN tokens of three
prompts whose prefill blocks and decode passes take run_mh, attn_tile and split-KV (6 splits),
with exact float prompt blocks and with W4A8 ones (ENGINE_PREFILL_INT8=1).

With the drafter checkpoint of gemma_layout.write_drafter, run_req restated over the oracle
(tests/protocol.py: MTP drafts with the sibling row, tree mode, prompt lookup) reproduces the
reference engine's drafting sessions: FIRST / GEN lines and the RANK1 / TREE counts (E:1673).

The fixture pins bit-level arithmetic through the tokens: planting either of two mistakes in
the oracle -- 8 attention splits for 6, or the per-layer embedding rows dropped -- changes the
tokens of the 196-token prompt."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import gemma_layout as gl  # noqa: E402
from protocol import RunReq  # noqa: E402

# the drafting sessions of tests/golden/make_gemma_layout.py: (k, tree, ngram, nglen)
# mode -> (ENGINE_K, ENGINE_TREE, ENGINE_NGRAM, ENGINE_NGLEN, ENGINE_DRAFT_SAMEPOS, ENGINE_FAKE_CTX)
MODES = {"k3": (3, False, 0, 3, False, 0), "tree": (2, True, 0, 3, False, 0), "ng": (3, False, 2, 5, False, 0),
         "k3_same": (3, False, 0, 3, True, 0), "fake": (3, False, 0, 3, False, 300)}

FX = os.path.join(HERE, "golden", "gemma_layout.npz")
# the sessions of a setting (same-position drafts, the fake context) and the logit lines are pinned
# on the first prompt (40 tokens: run_mh in prefill and decode, both head dims); G4V_ORACLE_ALL=1
# checks every prompt
ALL = os.environ.get("G4V_ORACLE_ALL") == "1"
ONE_PROMPT = {"k3_same", "fake"}


@pytest.fixture(scope="module")
def ckpt(orc, gemma_ckpt):
    d = gemma_ckpt
    fx = np.load(FX)
    prompts = np.split(fx["prompts"], np.cumsum(fx["prompt_lens"])[:-1])
    gens = np.split(fx["gens"], np.cumsum(fx["gen_lens"])[:-1])
    return d, fx, prompts, gens


@pytest.mark.parametrize("i,i8", [(0, False), (1, False), (2, False), (2, True)])
def test_gemma_layout_matches_reference_engine(orc, ckpt, i, i8):
    d, fx, prompts, gens = ckpt
    sfx = "_i8" if i8 else ""
    want = np.split(fx["gens" + sfx], np.cumsum(fx["gen_lens" + sfx])[:-1])[i]
    go = gl.GemmaOracle(orc, d, int(fx["ctx"][0]), i8=i8)
    try:
        gen = gl.run_req_k0(go, [int(t) for t in prompts[i]], int(fx["nnew"][0]), int(fx["cpus"][0]))
    finally:
        go.close()
    assert gen[0] == int(fx["first" + sfx][i])
    assert gen == [int(t) for t in want], (gen, list(want))


def test_gemma_head_logits_match_reference_engine(orc, ckpt):
    """the logits, not only the tokens: the reference engine run unchanged with its full head and
    ENGINE_DEBUG_GAP=1 prints, for every head row (the warm-up pass at position 0, then the
    prompt's last row and each decode row), the two largest r16 logits and their ids (E:1497).
    The oracle's hidden states through its full exp3 head reproduce every line: run_mh in the
    40-token prompt's prefill and decode (head dim 256 and, in the global layers, 512), attn_tile
    and split-KV in the others, and the RoPE tables of both layer types"""
    d, fx, prompts, gens = ckpt
    from oracle import Model
    m = Model(orc, gl.EMBED_SEED, gl.V, 1, 256, 64)
    E = m.get("E", np.uint16, gl.V * gl.H).reshape(gl.V, gl.H)
    m.close()
    P = orc.exp3_pack(E, gl.V, gl.H)
    T, nnew = int(fx["cpus"][0]), int(fx["nnew"][0])
    for i, p in enumerate(prompts if ALL else prompts[:1]):
        want = [str(x) for x in fx[f"gap_{i}"]]
        go = gl.GemmaOracle(orc, d, int(fx["ctx"][0]))
        try:
            hw = go.forward([2], 0, T, 0)[0]  # E:1578 the warm-up pass
            rows = [hw]
            chosen = [go.greedy(hw, [2])]
            gen = gl.run_req_k0(go, [int(t) for t in p], nnew, T, rows=rows)
        finally:
            go.close()
        chosen += gen
        got = [gl.gap_line(orc, P, h, c) for h, c in zip(rows, chosen)]
        assert got == want, (i, [(a, b) for a, b in zip(got, want) if a != b][:3])


def test_gemma_fixture_detects_planted_mistakes(orc, ckpt):
    d, fx, prompts, gens = ckpt
    want = [int(t) for t in gens[2]]
    go = gl.GemmaOracle(orc, d, int(fx["ctx"][0]))
    try:  # 8 splits where the engine ran 6
        assert gl.run_req_k0(go, [int(t) for t in prompts[2]], int(fx["nnew"][0]), 8) != want
    finally:
        go.close()
    ids = gl.PLE_IDS
    gl.PLE_IDS = [1]  # the per-layer embedding rows dropped
    try:
        go = gl.GemmaOracle(orc, d, int(fx["ctx"][0]))
        try:
            assert gl.run_req_k0(go, [int(t) for t in prompts[2]], int(fx["nnew"][0]), int(fx["cpus"][0])) != want
        finally:
            go.close()
    finally:
        gl.PLE_IDS = ids


@pytest.mark.parametrize("mode", list(MODES))
def test_gemma_drafting_matches_reference_engine(orc, ckpt, mode):
    d, fx, prompts, gens = ckpt
    k, tree, ngram, nglen, samepos, fake_n = MODES[mode]
    want = np.split(fx["gens_" + mode], np.cumsum(fx["gen_lens_" + mode])[:-1])
    go = gl.GemmaOracle(orc, d, int(fx["ctx"][0]))
    dr = gl.GemmaDrafter(orc, d)
    try:
        rr = RunReq(orc, gl.GemmaTarget(go, dr), t0=int(fx["cpus"][0]), ngram=ngram, nglen=nglen, samepos=samepos,
                    fake_n=fake_n)
        for i, p in enumerate(prompts if ALL or mode not in ONE_PROMPT else prompts[:1]):
            g0, gen, start = rr.run_req([int(t) for t in p], int(fx["nnew_d"][0]), k, tree)
            assert start == 0 and g0 == int(fx["first_" + mode][i])
            assert gen == [int(t) for t in want[i]], (mode, i, gen, list(want[i]))
            assert rr.rank1() == [int(v) for v in fx["rank1_" + mode][i]], (mode, i, rr.rank1())
    finally:
        dr.close()
        go.close()
