"""GPU check of the multi-slot prefix cache (run_req, E:1568-1593, E:1671): the slot each request
runs on, the reused prefix, and the KV cache of every conversation across slot switches, against
the oracle running each conversation on a model of its own."""
import numpy as np
import pytest

from conftest import note
from util import same

pytestmark = pytest.mark.gpu

V, NL, I, CTX, SEED = 4096, 2, 512, 512, 61


class SlotPolicy:
    """E:1579-1593 restated on token lists (the expected start / slot of every request)"""

    def __init__(self, nslot, min_reuse):
        self.stored = [dict(keys=[], kv_len=0, stamp=0) for _ in range(nslot - 1)]
        self.act = dict(keys=[], kv_len=0, stamp=0)
        self.tick, self.min_reuse = 0, min_reuse

    @staticmethod
    def lcp(keys, kv_len, toks):
        m = 0
        while m < kv_len and m < len(toks) and keys[m] == toks[m]:
            m += 1
        return m

    def begin(self, toks):
        common, used = self.lcp(self.act["keys"], self.act["kv_len"], toks), 0
        self.tick += 1
        if self.stored:
            best, bc = -1, common
            for i, s in enumerate(self.stored):
                m = self.lcp(s["keys"], s["kv_len"], toks)
                if m > bc:
                    best, bc = i, m
            if best >= 0:
                self.act["stamp"] = self.tick
                self.act, self.stored[best] = self.stored[best], self.act
                used, common = best + 1, bc
            elif bc < self.min_reuse:
                v = min(range(len(self.stored)), key=lambda i: (self.stored[i]["stamp"], i))
                self.act["stamp"] = self.tick
                self.act, self.stored[v] = self.stored[v], self.act
                self.act = dict(keys=[], kv_len=0, stamp=self.act["stamp"])
                common, used = 0, v + 1
            self.act["stamp"] = self.tick
        return min(common, len(toks) - 1), used

    def end(self, toks, gen, P):
        keys = list(toks) + [g for i, g in enumerate(gen) if i <= P - len(toks)]
        self.act["keys"], self.act["kv_len"] = keys, min(P + 1, len(keys))


def test_prefix_cache_across_conversations(orc, g4v):
    from oracle import Model
    rng = np.random.default_rng(2)
    dev = g4v.Device(0)
    models = {}
    try:
        dev.model_synth(SEED, V, NL, I, CTX)
        dev.slots_init(3, 8)
        pol = SlotPolicy(3, 8)
        convs = {"a": rng.integers(0, V, 60).tolist(), "b": rng.integers(0, V, 45).tolist(),
                 "c": rng.integers(0, V, 30).tolist()}
        state = {}  # conversation -> tokens so far (prompt + committed)
        # requests: new a, new b, a continued, new c (evicts the LRU), b continued, a continued
        for step, name in enumerate(["a", "b", "a", "c", "b", "a"]):
            if name not in state:
                prompt = convs[name]
                models[name] = Model(orc, SEED, V, NL, I, CTX)
            else:
                prompt = state[name] + rng.integers(0, V, 7).tolist()
            note(f"prefix cache request {step}: conversation {name}, {len(prompt)} tokens")
            start, used = dev.slot_begin(np.array(prompt, np.int32))
            assert (start, used) == pol.begin(prompt), step
            if name in state:
                assert start > 0  # the conversation's own KV came back
            m = models[name]
            g0, hd = dev.prefill(np.array(prompt[start:], np.int32), pos0=start, hidden=True)
            ho = m.prefill(np.array(prompt[start:], np.int32), pos0=start)
            assert same(hd, ho), step
            gen, P = [g0], len(prompt) - 1
            for _ in range(3):  # plain decode rounds (no drafts)
                r = dev.verify(np.array([gen[-1]], np.int32), 0, 0, P + 1, 8)
                o, _ = m.verify(np.array([gen[-1]], np.int32), 0, 0, P + 1, 8)
                assert list(r.commit[:r.ncommit]) == list(o.commit[:o.ncommit]), step
                gen += list(r.commit[:r.ncommit])
                P += r.ncommit
            dev.slot_end(np.array(prompt, np.int32), gen, P)
            pol.end(prompt, gen, P)
            state[name] = prompt + gen[:P - len(prompt) + 1]
            for what in ("KC", "VC"):
                a = dev.read(what, np.uint16).reshape(NL, -1, 256)[:, :P + 1]
                b = m.get(what, np.uint16, NL * CTX * 256).reshape(NL, CTX, 256)[:, :P + 1]
                assert same(a, b), (step, what)
    finally:
        for m in models.values():
            m.close()
        dev.close()
