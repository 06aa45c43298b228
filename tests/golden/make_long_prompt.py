"""Write the long-prompt fixture (the bench's long-prompt workload at its full size) from the
reference's own kernels.

Workload: the synthetic 35-layer stack (seed 1, V = 262,144, FFN 6144, cache of 8192 positions)
and the synthetic MTP drafter (seed 2); the 6,841-token prompt of bench.long_prompt_tokens() (a
seeded 64-token motif repeated, 5% uniform noise tokens); the prefill in blocks of 32 (W4A8 linear
layers, the engine's attention path per block, E:1594-1599 with ENGINE_PREFILL_INT8=1); then 256
rounds of run_req's loop (E:1617-1661): prompt-lookup drafts (n-gram 3, up to 3, E:1624-1628), or
when the lookup finds none a 3-step MTP chain (draft_step E:1534-1563, 6 splits) from the last
committed hidden state, each verified as a chain with 8 splits.

Every forward runs in oracle/_ref/libg4ref.so (the reference's kernels composed as fwd /
draft_step compose them; tests/test_prefill_oracle.py, test_draft_oracle.py and
test_oracle_vs_ref.py pin that composition against the C oracle bit for bit); the lookup is the
oracle's (pinned by tests/test_prompt_lookup.py).  Stored: the prompt, the last prompt row's
final-normed hidden state, the first token, every round's drafts, draft kind and committed
tokens, and a CRC-32 of every layer's key and value rows 0 .. P after the last round.

Run from the repository root after `make -C oracle` (about 5 minutes on 8 cores):
    python tests/golden/make_long_prompt.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from golden_cases import LONG_PROMPT, crc  # noqa: E402
from oracle import Drafter, Model, Oracle, Ref, ref_available  # noqa: E402


def main():
    if not ref_available():
        sys.exit("oracle/_ref/libg4ref.so is not built: the long-prompt fixture comes from the reference's kernels")
    import bench
    seed, V, NL, I, ctx, dseed = (LONG_PROMPT[k] for k in ("seed", "V", "NL", "I", "ctx", "dseed"))
    rounds, ngram, nglen, k, dsplit = (LONG_PROMPT[k] for k in ("rounds", "ngram", "nglen", "k", "dsplit"))
    prompt = bench.long_prompt_tokens()
    o = Oracle()
    m = Model(o, seed, V, NL, I, ctx)
    d = Drafter(o, dseed, V)
    r = Ref(threads=8)
    if r.threads != 8:
        sys.exit(f"the reference pool started {r.threads} workers; the verify passes need 8")
    r.bind_model(m)
    r.bind_drafter(d)
    t0 = time.time()
    h0 = r.prefill(prompt)
    g0 = m.head(h0)
    print(f"prefill {len(prompt)} tokens: {time.time() - t0:.1f} s, first token {g0}", flush=True)
    gen, P, h = [g0], len(prompt) - 1, h0
    drafts, kinds, commits = [], [], []
    for rnd in range(rounds):
        seq = np.concatenate([prompt, gen]).astype(np.int32)
        dr = o.prompt_lookup(seq, ngram, nglen).tolist()
        kind = 0
        if not dr:  # the MTP chain (E:1631-1646, sibling policy off)
            tok, hc = gen[-1], h
            for j in range(k):
                tok, hc, _, _ = r.draft_step(tok, hc, P + 1 + j, P, dsplit)
                dr.append(tok)
            kind = 1
        block = np.array([gen[-1]] + dr, np.int32)
        out = r.verify(block, len(dr), 0, P + 1)
        com = list(out.commit[:out.ncommit])
        h = r.last_hidden()
        drafts.append(dr)
        kinds.append(kind)
        commits.append(com)
        gen += com
        P += out.ncommit
        if rnd % 32 == 31:
            print(f"round {rnd + 1}: P {P}, {time.time() - t0:.1f} s", flush=True)
    KC = m.get("KC", np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)
    VC = m.get("VC", np.uint16, NL * ctx * 256).reshape(NL, ctx, 256)
    kv_crc = np.array([[crc(KC[l, :P + 1]), crc(VC[l, :P + 1])] for l in range(NL)], np.uint32)
    dptr = np.cumsum([0] + [len(x) for x in drafts]).astype(np.int32)
    cptr = np.cumsum([0] + [len(x) for x in commits]).astype(np.int32)
    path = os.path.join(HERE, "long_prompt.npz")
    np.savez_compressed(path, prompt=prompt.astype(np.int32), h0=h0, g0=np.array([g0], np.int32),
                        drafts=np.array(sum(drafts, []), np.int32), dptr=dptr, kinds=np.array(kinds, np.int8),
                        commits=np.array(sum(commits, []), np.int32), cptr=cptr, P=np.array([P], np.int32),
                        kv_crc=kv_crc)
    acc = sum(len(c) - 1 for c in commits)
    print(f"long_prompt.npz: {os.path.getsize(path)} bytes; {rounds} rounds, {len(gen) - 1} tokens committed after "
          f"the first, {acc} drafts accepted, {sum(kinds)} MTP rounds, P = {P}", flush=True)
    d.close()
    m.close()


if __name__ == "__main__":
    main()
