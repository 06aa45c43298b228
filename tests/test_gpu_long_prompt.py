"""The long-prompt workload at its full size on the GPU against the fixture written from the
reference's kernels (tests/golden/make_long_prompt.py): the 6,841-token motif prompt prefilled
through the 35-layer stack at V = 262,144 (W4A8 linear layers, E:1594-1599), then 256 rounds of
run_req's loop (E:1617-1661) with prompt-lookup drafts or 3-step MTP chains, each verified as a
chain.  Bit-exact: the last prompt row's final-normed hidden state, the first token, every
round's drafts and committed tokens, and the key / value rows of every layer after the last
round (CRC-32 per layer)."""
import os
import sys
import zlib

import numpy as np
import pytest

from conftest import note
from util import first_diff, same

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from golden_cases import LONG_PROMPT  # noqa: E402


def test_long_prompt_matches_reference(g4v):
    g = np.load(os.path.join(HERE, "golden", "long_prompt.npz"), allow_pickle=False)
    L = LONG_PROMPT
    prompt = g["prompt"]
    note(f"long prompt: prefill {prompt.size} tokens, {L['rounds']} rounds, NL={L['NL']} V={L['V']}")
    dev = g4v.Device(0)
    try:
        dev.model_synth(L["seed"], L["V"], L["NL"], L["I"], L["ctx"])
        dev.drafter_synth(L["dseed"])
        g0, h0 = dev.prefill(prompt, hidden=True)
        assert same(h0, g["h0"]), first_diff(h0, g["h0"])
        assert g0 == int(g["g0"][0])
        dev.history_set(np.concatenate([prompt, [g0]]))
        gen, P, app = [g0], prompt.size - 1, []
        dptr, cptr = g["dptr"], g["cptr"]
        for rnd in range(L["rounds"]):
            want_d = g["drafts"][dptr[rnd]:dptr[rnd + 1]].tolist()
            d = dev.prompt_lookup(L["ngram"], L["nglen"], app)
            kind = 0
            if d.size == 0:
                d = dev.draft_mtp(gen[-1], h0 if rnd == 0 else None, P, L["k"], L["dsplit"])[0]
                kind = 1
            assert kind == int(g["kinds"][rnd]) and d.tolist() == want_d, (rnd, kind, d.tolist(), want_d)
            r = dev.verify(np.array([gen[-1]] + d.tolist(), np.int32), len(d), 0, P + 1, L["nsplit"])
            app = list(r.commit[:r.ncommit])
            assert app == g["commits"][cptr[rnd]:cptr[rnd + 1]].tolist(), (rnd, app)
            gen += app
            P += r.ncommit
        assert P == int(g["P"][0])
        kc = dev.read("KC", np.uint16).reshape(L["NL"], -1, 256)
        vc = dev.read("VC", np.uint16).reshape(L["NL"], -1, 256)
        for l in range(L["NL"]):
            got = [zlib.crc32(np.ascontiguousarray(kc[l, :P + 1]).tobytes()) & 0xFFFFFFFF,
                   zlib.crc32(np.ascontiguousarray(vc[l, :P + 1]).tobytes()) & 0xFFFFFFFF]
            assert got == g["kv_crc"][l].tolist(), l
    finally:
        dev.close()
