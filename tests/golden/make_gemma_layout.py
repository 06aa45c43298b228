"""Write the Gemma-layout fixture from the reference engine run unchanged.

oracle/_ref/gemma4_engine is engine/gemma4_engine.cpp compiled by `make -C oracle` from its own
source.  It runs here on the synthetic checkpoint of gemma_layout.write_checkpoint (35 layers of
head_dim 256 / 512, KV sharing, per-layer inputs, V = 262,144), ENGINE_DECODE_INT8=0,
ENGINE_K=0 (prefill, then one-row decode passes), the certified head (ENGINE_HEAD_SCREEN=1) and
ENGINE_CPUS of 6 CPUs (6 attention splits), twice: exact float prefill (ENGINE_PREFILL_INT8
unset: first, gens) and W4A8 prefill blocks (ENGINE_PREFILL_INT8=1: first_i8, gens_i8).  Each
prompt of cases() is one engine run; its FIRST and GEN lines are stored.

Then, with the drafter checkpoint of gemma_layout.write_drafter (ENGINE_DRAFTER_DIR /
ENGINE_DRAFTER_INDEX), three serve-mode sessions (ENGINE_SERVE=1, the three prompts in order,
NNEW_D tokens each) in the drafting modes of DRAFT_MODES: per request the FIRST and GEN lines
and the stderr line "RANK1 rounds= top1= top2_only= TREE attempts= hits=" (E:1673; the RANK1
counts run over the session) are stored as first_<mode>, gens_<mode>, gen_lens_<mode>,
rank1_<mode> [3][5].  Mode k3_i8 is the server's environment (E:1600): W4A8 prompt blocks
(ENGINE_PREFILL_INT8=1) and W4A8 verify passes of two rows or more (ENGINE_DECODE_INT8 on).
Mode k3_same runs every draft step at position P + 1 (ENGINE_DRAFT_SAMEPOS=1, E:1633); mode fake
starts from a fake context of FAKE_N positions (ENGINE_FAKE_CTX, E:1211, 1249-1250: the caches'
first positions from the engine's LCG, every request after them, no prefix reuse).

`--modes m1,m2` runs only those drafting sessions and adds their arrays to the fixture already
written (the checkpoint is rebuilt from the same seeds).

`--gap` (also part of a full run) runs each prompt once more with the full head and its debug
line (ENGINE_HEAD_SCREEN unset, ENGINE_DEBUG_GAP=1, ENGINE_K=0, exact float prefill): per head
row the engine prints "GAP t1 t1-t2 id1= id2= chosen=" (E:1497), the row's two largest r16
logits and their ids, so the logits of run_mh (hd 256 and 512, the 40-token prompt) and of the
RoPE tables are pinned at the printed resolution, not only through tokens.  Stored as gap_<i>.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_gemma_layout.py
"""
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

import gemma_layout as gl  # noqa: E402
from golden_cases import crc  # noqa: E402
from oracle import Oracle  # noqa: E402

EXE = os.path.join(ROOT, "oracle", "_ref", "gemma4_engine")
CPUS, NNEW, CTX = 6, 12, 1024
NNEW_D = 24
FAKE_N = 300
# name -> engine settings of a drafting session (SIB_GAP 1, the default, lets the sibling row in)
DRAFT_MODES = {"k3": dict(ENGINE_K="3"), "tree": dict(ENGINE_K="2", ENGINE_TREE="1"),
               "ng": dict(ENGINE_K="3", ENGINE_NGRAM="2", ENGINE_NGLEN="5"),
               "k3_i8": dict(ENGINE_K="3", ENGINE_PREFILL_INT8="1", ENGINE_DECODE_INT8="1"),
               "k3_same": dict(ENGINE_K="3", ENGINE_DRAFT_SAMEPOS="1"),
               "fake": dict(ENGINE_K="3", ENGINE_FAKE_CTX=str(FAKE_N))}


def base_env():
    env = dict(os.environ, ENGINE_CPUS=",".join(str(c) for c in range(CPUS)), ENGINE_HEAD_SCREEN="1",
               ENGINE_DECODE_INT8="0", ENGINE_CTX=str(CTX))
    for k in ("ENGINE_PREFILL_INT8", "ENGINE_SERVE", "ENGINE_STREAM", "ENGINE_ADAPTIVE_THREADS", "ENGINE_K",
              "ENGINE_TREE", "ENGINE_NGRAM", "ENGINE_NGLEN", "ENGINE_SIB_GAP", "ENGINE_SIB_LONG", "ENGINE_POLICY",
              "ENGINE_TAU", "ENGINE_DRAFT_SAMEPOS", "ENGINE_SLOTS", "ENGINE_FAKE_CTX", "ENGINE_NO_TILED"):
        env.pop(k, None)
    return env


def parse_rank1(line):
    """RANK1 rounds=a top1=b top2_only=c TREE attempts=d hits=e -> [a, b, c, d, e]"""
    return [int(w.split("=")[1]) for w in line.split() if "=" in w]


def cases(orc):
    """prompts whose last prefill block takes each attention path (E:1305-1337): 40 tokens (run_mh,
    then run_mh decode), 100 (attn_tile tail), 196 (a 4-row split-KV tail, then split-KV decode);
    half their tokens have per-layer embedding rows"""
    out = []
    for n, seed in ((40, 1), (100, 2), (196, 3)):
        t = orc.ints(orc.stream(gl.WEIGHT_SEED, 90000 + seed), n, 2, gl.V)
        pick = orc.ints(orc.stream(gl.WEIGHT_SEED, 91000 + seed), n, 0, len(gl.PLE_IDS))
        t[::2] = np.array(gl.PLE_IDS, np.int32)[pick[::2]]
        out.append(t.astype(np.int32))
    return out


def main():
    if not os.path.exists(EXE):
        sys.exit("oracle/_ref/gemma4_engine is not built (make -C oracle with the reference sources)")
    only = sys.argv[sys.argv.index("--modes") + 1].split(",") if "--modes" in sys.argv else None
    gap_only = "--gap" in sys.argv
    if gap_only:
        only = ["(none)"]
    orc = Oracle()
    prompts = cases(orc)
    out = {}
    path = os.path.join(HERE, "gemma_layout.npz")
    if only:
        with np.load(path) as f:
            out = {k: f[k] for k in f.files}
        if not np.array_equal(out["prompts"], np.concatenate(prompts)):
            sys.exit("the fixture's prompts differ from cases(): regenerate it whole")
    with tempfile.TemporaryDirectory() as d:
        gl.write_checkpoint(orc, d)
        for sfx, i8 in (("", False), ("_i8", True)) if not only else ():
            env = dict(base_env(), ENGINE_K="0")
            if i8:
                env["ENGINE_PREFILL_INT8"] = "1"
            firsts, gens = [], []
            for i, p in enumerate(prompts):
                pf = os.path.join(d, f"prompt{i}.txt")
                with open(pf, "w") as f:
                    f.write(" ".join(map(str, p)) + "\n")
                r = subprocess.run([EXE, d, os.path.join(d, "index.tsv"), pf, str(NNEW)], env=env,
                                   capture_output=True, text=True, timeout=1800)
                if r.returncode != 0:
                    sys.exit(f"engine failed ({r.returncode}): {r.stderr[-2000:]}")
                lines = r.stdout.splitlines()
                first = int([ln for ln in lines if ln.startswith("FIRST")][0].split()[1])
                gen = [int(x) for x in [ln for ln in lines if ln.startswith("GEN:")][0].split()[1:]]
                print(f"prompt {i} ({len(p)} tokens, int8 prefill {i8}): FIRST {first} GEN {gen}", flush=True)
                firsts.append(first)
                gens.append(np.array(gen, np.int32))
            out["first" + sfx] = np.array(firsts, np.int32)
            out["gen_lens" + sfx] = np.array([len(g) for g in gens])
            out["gens" + sfx] = np.concatenate(gens)
        for i, p in enumerate(prompts) if (not only or gap_only) else ():
            env = dict(base_env(), ENGINE_K="0", ENGINE_DEBUG_GAP="1")
            env.pop("ENGINE_HEAD_SCREEN", None)
            pf = os.path.join(d, f"gprompt{i}.txt")
            with open(pf, "w") as f:
                f.write(" ".join(map(str, p)) + "\n")
            r = subprocess.run([EXE, d, os.path.join(d, "index.tsv"), pf, str(NNEW)], env=env,
                               capture_output=True, text=True, timeout=1800)
            if r.returncode != 0:
                sys.exit(f"engine failed ({r.returncode}): {r.stderr[-2000:]}")
            gaps = [ln.strip() for ln in r.stderr.splitlines() if ln.startswith("GAP ")]
            gen = [int(x) for x in [ln for ln in r.stdout.splitlines() if ln.startswith("GEN:")][0].split()[1:]]
            want = np.split(out["gens"], np.cumsum(out["gen_lens"])[:-1])[i]
            # one line per head row: the warm-up pass at position 0 (E:1578), then FIRST and each GEN row
            if gen != [int(t) for t in want] or len(gaps) != len(gen) + 1:
                sys.exit(f"prompt {i}: full-head run differs from the screened one: {gen} / {list(want)} / {len(gaps)}")
            print(f"prompt {i}: {len(gaps)} GAP lines, first {gaps[0]}", flush=True)
            out[f"gap_{i}"] = np.array(gaps)
        from oracle import Model
        m = Model(orc, gl.EMBED_SEED, gl.V, 1, 256, 64)
        E = m.get("E", np.uint16, gl.V * gl.H).reshape(gl.V, gl.H)
        m.close()
        gl.write_drafter(orc, d, E)
        lines = "".join(f"{NNEW_D} {' '.join(map(str, p))}\n" for p in prompts)
        for mode, extra in DRAFT_MODES.items():
            if only and mode not in only:
                continue
            env = dict(base_env(), ENGINE_SERVE="1", ENGINE_DRAFTER_DIR=os.path.join(d, "drafter"),
                       ENGINE_DRAFTER_INDEX=os.path.join(d, "drafter_index.tsv"), **extra)
            r = subprocess.run([EXE, d, os.path.join(d, "index.tsv"), "-", "0"], input=lines, env=env,
                               capture_output=True, text=True, timeout=3600)
            if r.returncode != 0:
                sys.exit(f"engine failed ({r.returncode}): {r.stderr[-2000:]}")
            out_lines = r.stdout.splitlines()
            firsts = [int(ln.split()[1]) for ln in out_lines if ln.startswith("FIRST")]
            gens = [np.array([int(x) for x in ln.split()[1:]], np.int32) for ln in out_lines if ln.startswith("GEN:")]
            rank1 = [parse_rank1(ln) for ln in r.stderr.splitlines() if ln.startswith("RANK1")]
            if not (len(firsts) == len(gens) == len(rank1) == len(prompts)):
                sys.exit(f"mode {mode}: unexpected output\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}")
            for i in range(len(prompts)):
                print(f"mode {mode} prompt {i}: GEN {list(gens[i])} RANK1 {rank1[i]}", flush=True)
            out["first_" + mode] = np.array(firsts, np.int32)
            out["gen_lens_" + mode] = np.array([len(g) for g in gens])
            out["gens_" + mode] = np.concatenate(gens)
            out["rank1_" + mode] = np.array(rank1, np.int64)
        raw = np.memmap(os.path.join(d, "model.safetensors"), np.uint8, "r")
        file_crc = crc(np.asarray(raw[:gl.V * gl.H * 2 + (64 << 20)]))
    if only and int(out["crc_head"][0]) != file_crc:
        sys.exit("the checkpoint's CRC differs from the fixture's: regenerate it whole")
    out.update(cpus=np.array([CPUS]), nnew=np.array([NNEW]), ctx=np.array([CTX]), nnew_d=np.array([NNEW_D]),
               prompt_lens=np.array([len(p) for p in prompts]), prompts=np.concatenate(prompts),
               crc_head=np.array([file_crc], np.uint32))
    np.savez_compressed(path, **out)
    print(f"gemma_layout.npz: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main()
