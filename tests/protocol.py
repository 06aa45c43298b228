"""run_req (E:1584-1679) of the reference engine restated over an oracle target: the test-side
mirror of the engine's request loop, used to check the engine front-end (g4v_engine) and, on
the Gemma-4-E2B layout, pinned against the reference engine's own output.

A target provides
  prefill(toks, pos0, T, i8) -> the final-normed state of the last prompt row (E:1594-1599)
  head(h, seeds)            -> the greedy token of a final-normed row (E:1406-1502)
  verify(block, nd, nb, pos0, T, allow_b) -> (result, hidden): one pass over the confirmed token,
      nd chain drafts and nb (0 / 1) sibling rows; result.nacc, .branch, .commit, .G0, and the
      committed row's final-normed state (E:1647-1661)
  draft(tok, h, pos, P, T)  -> (token, next hidden, runner-up, gap) (draft_step, E:1534-1563)
  fake_ctx(n)               -> (ENGINE_FAKE_CTX only) the caches' first n positions from the LCG
                               (E:1249-1250)
"""
import numpy as np


def is_stop(t):
    return t in (106, 1)  # E:1609


class RunReq:
    """run_req with one active cache (ENGINE_SLOTS=1).  Attention splits over the pool's active
    workers (E:1327, 1544): t0 = the ENGINE_CPUS count, set_active clamps to [1, t0] (E:110-112),
    draft steps set 6 (8 past the cutoff with ENGINE_ADAPTIVE_THREADS and ENGINE_DRAFT_SAME,
    E:1535), forward passes set 6 / 8 only with ENGINE_ADAPTIVE_THREADS (E:1257), and the count
    persists.  i8: ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8=0.  ngram / nglen: ENGINE_NGRAM
    (0: no prompt lookup) and ENGINE_NGLEN; sib_long: ENGINE_SIB_LONG.  r1 holds the process's
    RANK1 counts (E:1655: rounds with MTP drafts, top-1 hits, runner-up-only hits); sib_rounds and
    hits the last request's TREE attempts and hits (E:1583, 1648-1650).  samepos: ENGINE_DRAFT_SAMEPOS
    (every draft step at position P + 1, E:1633); fake_n: ENGINE_FAKE_CTX (the caches' first fake_n
    positions from the LCG before the warm-up, every request at fake_n + its positions, no prefix
    reuse: E:1249-1250, 1599, 1615-1617, 1675)."""

    def __init__(self, orc, target, t0=6, adaptive=False, draft_same=True, cut=192, i8=False, ngram=3, nglen=3,
                 sib_long=False, samepos=False, fake_n=0):
        self.orc, self.t = orc, target
        self.t0, self.active, self.adaptive, self.draft_same, self.cut, self.i8 = t0, t0, adaptive, draft_same, cut, i8
        self.ngram, self.nglen, self.sib_long = ngram, nglen, sib_long
        self.samepos, self.fake_n = samepos, fake_n
        if fake_n:
            target.fake_ctx(fake_n)
        self.keys, self.kv_len = [], 0
        self.splits_seen = set()
        self.r1 = [0, 0, 0]
        self.sib_rounds = self.hits = 0
        self.prefill(np.array([2], np.int32), 0)  # E:1578 warm-up at position 0

    def set_active(self, a):
        self.active = self.t0 if a < 1 else min(a, self.t0)
        self.splits_seen.add(self.active)
        return self.active

    def fwd_splits(self, pos0, M):
        if self.adaptive:
            self.set_active(8 if pos0 + M > self.cut else 6)
        self.splits_seen.add(self.active)
        return self.active

    def prefill(self, toks, pos0):
        for b in range(0, len(toks), 32):
            self.fwd_splits(pos0 + b, min(32, len(toks) - b))
        return self.t.prefill(np.asarray(toks, np.int32), pos0, self.active, self.i8)

    def run_req(self, prompt, nnew, k_draft=3, tree=False):
        """(FIRST token, GEN tokens, reused prefix length) of one request"""
        n = len(prompt)
        common = 0
        while common < self.kv_len and common < n and self.keys[common] == prompt[common]:
            common += 1
        start = min(common, n - 1)
        F = self.fake_n
        h = self.prefill(prompt[start:], F + start)
        g0 = self.t.head(h, prompt[start:][-8:])
        gen, P, stopped = [g0], F + n - 1, is_stop(g0)
        hprev, state, rounds, self.sib_rounds, self.hits = h, 1, 0, 0, 0
        if k_draft == 0:  # E:1615: one-row passes
            for i in range(1, nnew):
                if stopped:
                    break
                o, _ = self.t.verify(np.array([gen[-1]], np.int32), 0, 0, F + n + i - 1,
                                     self.fwd_splits(F + n + i - 1, 1))
                gen.append(o.commit[0])
                stopped = is_stop(gen[-1])
            P = F + n + max(0, nnew - 1) - 1
        while k_draft > 0 and len(gen) < nnew and not stopped:  # E:1617-1661
            k = min(k_draft, 3)
            if tree:
                k = min(k, 2)
            drafts = []
            if self.ngram > 0:  # E:1624-1628
                seq = np.array(prompt + gen, np.int32)
                drafts = self.orc.prompt_lookup(seq, self.ngram, self.nglen).tolist()
            used_ng, sec1, gap1, use_sib = bool(drafts), -1, -1.0, False
            if not used_ng:  # E:1632-1645
                tok, hh = gen[-1], hprev
                for j in range(k):
                    ts = self.set_active(8 if self.draft_same and self.adaptive and P + 1 > self.cut else 6)
                    tok, hh, sec, gap = self.t.draft(tok, hh, P + 1 + (0 if self.samepos else j), P, ts)
                    if j == 0:
                        sec1, gap1 = sec, gap
                        allow = rounds >= 1 and state < 2 and k >= 2 and sec1 >= 0 and sec1 != tok
                        if P + 1 + k > 192:
                            cond = self.sib_long and (gap1 <= 0.85 or 1.65 <= gap1 <= 2.55)
                        else:
                            cond = gap1 <= (2.55 if (rounds <= 3 or state == 1) else 1.80)
                        if allow and cond:
                            drafts.append(tok)
                            use_sib = True
                            break
                    drafts.append(tok)
            nd = len(drafts)
            sib = nd + 1 if ((tree or use_sib) and not used_ng and nd >= 1 and sec1 >= 0 and sec1 != drafts[0]) else -1
            block = np.array([gen[-1]] + drafts + ([sec1] if sib > 0 else []), np.int32)
            if sib > 0:
                self.sib_rounds += 1
                allow_hit = tree or (P + 1 + sib <= 192 and gap1 >= 0.25)
                o, hprev = self.t.verify(block, nd, 1, P + 1, self.fwd_splits(P + 1, len(block)), allow_hit)
            else:
                o, hprev = self.t.verify(block, nd, 0, P + 1, self.fwd_splits(P + 1, len(block)), True)
            rounds += 1
            if o.branch == 1:  # E:1650-1653
                self.hits += 1
                gen.append(o.commit[0])
                if not is_stop(o.commit[0]) and len(gen) < nnew:
                    gen.append(o.commit[1])
                stopped = is_stop(gen[-1])
                P += 2
                state = 1
                continue
            if not used_ng and nd >= 1:  # E:1655
                self.r1[0] += 1
                if drafts[0] == o.G0:
                    self.r1[1] += 1
                elif sec1 == o.G0:
                    self.r1[2] += 1
            state = 0 if o.nacc == 0 else (2 if (not use_sib and o.nacc == nd) else 1)
            for i in range(o.nacc + 1):
                gen.append(o.commit[i])
                if is_stop(o.commit[i]):
                    stopped = True
                    break
            P += o.nacc + 1
        self.keys = list(prompt) + [g for i, g in enumerate(gen) if i <= P - F - n]
        self.kv_len = 0 if F else min(P + 1, len(self.keys))
        gen = gen[:nnew]
        for i, g in enumerate(gen):
            if is_stop(g):
                gen = gen[:i + 1]
                break
        return g0, gen, start

    def rank1(self):
        """the RANK1 line's counts after the last request: rounds, top1, top2_only, attempts, hits"""
        return [self.r1[0], self.r1[1], self.r1[2], self.sib_rounds, self.hits]
