"""The engine front-end (gemma4-e2b-laptop-cpu_amd/g4v_engine): the reference engine's line
protocol (E:1681-1689) over the library, driven as the reference's server drives it.  Every
request's FIRST / TOK / GEN lines are checked against run_req (E:1584-1679, sibling row off)
restated over the oracle: prefix reuse, prefill, prompt-lookup or MTP drafts, chain verify."""
import os
import subprocess

import numpy as np
import pytest

from conftest import PKG, note

pytestmark = pytest.mark.gpu

SEED, V, NL, I, CTX, T = 71, 16384, 15, 512, 1024, 6
ENV = dict(ENGINE_SERVE="1", ENGINE_STREAM="1", ENGINE_NGRAM="3", ENGINE_NGLEN="3", ENGINE_K="3",
           ENGINE_CTX=str(CTX), ENGINE_CPUS="0,2,4,6,8,10")


def is_stop(t):
    return t in (106, 1)


class OracleEngine:
    """run_req over the oracle with one active cache (ENGINE_SLOTS=1)"""

    def __init__(self, orc):
        from oracle import Drafter, Model
        self.orc = orc
        self.m = Model(orc, SEED, V, NL, I, CTX)
        self.d = Drafter(orc, SEED + 1, V)
        self.keys, self.kv_len = [], 0
        self.m.prefill(np.array([2], np.int32), T=T)  # E:1578 warm-up at position 0

    def close(self):
        self.d.close()
        self.m.close()

    def run_req(self, prompt, nnew):
        n = len(prompt)
        common = 0
        while common < self.kv_len and common < n and self.keys[common] == prompt[common]:
            common += 1
        start = min(common, n - 1)
        h = self.m.prefill(np.array(prompt[start:], np.int32), pos0=start, T=T)
        g0 = self.m.head(h, prompt[start:][-8:])
        gen, P, stopped, toks_out = [g0], n - 1, is_stop(g0), []
        hprev = h
        while len(gen) < nnew and not stopped:
            seq = np.array(prompt + gen, np.int32)
            drafts = self.orc.prompt_lookup(seq, 3, 3).tolist()
            if not drafts:
                tok, hh = gen[-1], hprev
                for j in range(3):
                    tok, hh, _, _ = self.d.step(self.m, tok, hh, P + 1 + j, P, T)
                    drafts.append(tok)
            block = np.array([gen[-1]] + drafts, np.int32)
            o, hprev = self.m.verify(block, len(drafts), 0, P + 1, T)
            for i in range(o.nacc + 1):
                gen.append(o.commit[i])
                if is_stop(o.commit[i]):
                    stopped = True
                    break
            P += o.nacc + 1
        self.keys = list(prompt) + [g for i, g in enumerate(gen) if i <= P - n]
        self.kv_len = min(P + 1, len(self.keys))
        gen = gen[:nnew]
        for i, g in enumerate(gen):
            if is_stop(g):
                gen = gen[:i + 1]
                break
        return g0, gen, start


def test_engine_protocol_matches_oracle(orc):
    exe = os.path.join(PKG, "g4v_engine")
    if not os.path.exists(exe):
        pytest.fail("g4v_engine not built (make -C gemma4-e2b-laptop-cpu_amd)")
    rng = np.random.default_rng(5)
    motif = rng.integers(0, V, 16).tolist()
    a = (motif * 8)[:100]
    b = rng.integers(0, V, 40).tolist()
    requests = [(a, 20), (b, 10), (a, 15), (a + [5, 6, 7], 8)]
    note("engine protocol: 4 requests over a 15-layer synthetic stack")
    env = dict(os.environ, **ENV)
    lines = "".join(f"{nn} {' '.join(map(str, p))}\n" for p, nn in requests)
    proc = subprocess.run([exe, f"synth:{SEED}:{V}:{NL}:{I}", "-", "-", "0"], input=lines, env=env,
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out = proc.stdout.splitlines()
    oe = OracleEngine(orc)
    try:
        it = iter(out)
        for k, (prompt, nn) in enumerate(requests):
            g0, gen, start = oe.run_req(prompt, nn)
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
    finally:
        oe.close()
