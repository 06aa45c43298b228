"""Write the Gemma-layout fixture from the reference engine run unchanged.

oracle/_ref/gemma4_engine is engine/gemma4_engine.cpp compiled by `make -C oracle` from its own
source.  It runs here on the synthetic checkpoint of gemma_layout.write_checkpoint (35 layers of
head_dim 256 / 512, KV sharing, per-layer inputs, V = 262,144), ENGINE_DECODE_INT8=0,
ENGINE_K=0 (prefill, then one-row decode passes), the certified head (ENGINE_HEAD_SCREEN=1) and
ENGINE_CPUS of 6 CPUs (6 attention splits), twice: exact float prefill (ENGINE_PREFILL_INT8
unset: first, gens) and W4A8 prefill blocks (ENGINE_PREFILL_INT8=1: first_i8, gens_i8).  Each
prompt of cases() is one engine run; its FIRST and GEN lines are stored.

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
    orc = Oracle()
    prompts = cases(orc)
    out = {}
    with tempfile.TemporaryDirectory() as d:
        gl.write_checkpoint(orc, d)
        for sfx, i8 in (("", False), ("_i8", True)):
            env = dict(os.environ, ENGINE_CPUS=",".join(str(c) for c in range(CPUS)), ENGINE_K="0",
                       ENGINE_HEAD_SCREEN="1", ENGINE_DECODE_INT8="0", ENGINE_CTX=str(CTX))
            for k in ("ENGINE_PREFILL_INT8", "ENGINE_SERVE", "ENGINE_STREAM", "ENGINE_ADAPTIVE_THREADS"):
                env.pop(k, None)
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
        raw = np.memmap(os.path.join(d, "model.safetensors"), np.uint8, "r")
        file_crc = crc(np.asarray(raw[:gl.V * gl.H * 2 + (64 << 20)]))
    path = os.path.join(HERE, "gemma_layout.npz")
    np.savez_compressed(path, cpus=np.array([CPUS]), nnew=np.array([NNEW]), ctx=np.array([CTX]),
                        prompt_lens=np.array([len(p) for p in prompts]), prompts=np.concatenate(prompts),
                        crc_head=np.array([file_crc], np.uint32), **out)
    print(f"gemma_layout.npz: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main()
