"""Write the head-screen fixture from the reference engine's own main().

The screen build (engine/gemma4_engine.cpp:1235-1244) is a lambda inside main(), so the only
way to run the reference's code for it is to run main() itself.  oracle/_ref/ref_engine_screen
(built by `make -C oracle` from the reference's sources) does that on a checkpoint directory
written here: model.safetensors holds the embedding of golden_cases.screen_build_embedding()
(the seed-1 synthetic embedding, V = 262,144, with crafted tie rows) followed by a zero region
every other tensor of the engine's index points into (E:1218-1231 reads tensors through the
index offsets only).  The program copies the screen main() builds (SCR.w, SCR.s, SCR.coef) as
soon as main() reports it built.

Stored: CRC-32 of the embedding and of each of the three screen arrays over all 262,144 rows,
and the screen bytes of the tie rows and of golden_cases.SCREEN_SAMPLE_ROWS verbatim.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_screen_build.py
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

from golden_cases import (HEAD_V, SCREEN_BUILD_SEED, SCREEN_SAMPLE_ROWS, SCREEN_TIE_ROWS, crc,  # noqa: E402
                          screen_build_embedding)
from oracle import Oracle  # noqa: E402

H, NL = 1536, 35
EXE = os.path.join(ROOT, "oracle", "_ref", "ref_engine_screen")


def index_lines(e_bytes, zoff):
    """the tensor index (name, dtype, offset, bytes, shape) main() reads (E:1214-1231): the
    embedding at 0, everything else in the zero region at zoff, with the layer shapes of the
    reference's checkpoint (E:1222-1228)"""
    out = [("embed_tokens.weight", "BF16", 0, e_bytes, f"{HEAD_V},{H}"),
           ("embed_tokens_per_layer.weight", "BF16", zoff, 2 * 35 * 256 * 4, f"{HEAD_V},{35 * 256}")]

    def q4(name, N, K):
        out.append((name + ".weight_packed", "I32", zoff, N * K // 2, f"{N},{K // 8}"))
        out.append((name + ".weight_scale", "BF16", zoff, N * K // 16, f"{N},{K // 32}"))

    def vec(name, n):
        out.append((name, "BF16", zoff, 2 * n, f"{n}"))

    for l in range(NL):
        p = f"layers.{l}."
        hd = 256 if l % 5 != 4 else 512
        ff = 6144 if l < 15 else 12288
        q4(p + "self_attn.q_proj", 8 * hd, H)
        if l < 15:
            q4(p + "self_attn.k_proj", hd, H)
            q4(p + "self_attn.v_proj", hd, H)
            vec(p + "self_attn.k_norm.weight", hd)
        q4(p + "self_attn.o_proj", H, 8 * hd)
        q4(p + "mlp.gate_proj", ff, H)
        q4(p + "mlp.up_proj", ff, H)
        q4(p + "mlp.down_proj", H, ff)
        q4(p + "per_layer_input_gate", 256, H)
        q4(p + "per_layer_projection", H, 256)
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm", "post_per_layer_input_norm"):
            vec(p + n + ".weight", H)
        vec(p + "self_attn.q_norm.weight", hd)
        vec(p + "layer_scalar", 1)
    q4("per_layer_model_projection", 35 * 256, H)
    vec("per_layer_projection_norm.weight", 256)
    vec("norm.weight", H)
    return out


def main():
    if not os.path.exists(EXE):
        sys.exit("oracle/_ref/ref_engine_screen is not built (make -C oracle with the reference sources)")
    o = Oracle()
    E = screen_build_embedding(o)
    zbytes = 16 << 20  # >= the largest matrix the index names (gate 12288 x 1536: 10.6 MB)
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "model.safetensors"), "wb") as f:
            f.write(E.tobytes())
            f.truncate(E.nbytes + zbytes)
        with open(os.path.join(d, "index.tsv"), "w") as f:
            for name, dt, off, nb, shape in index_lines(E.nbytes, E.nbytes):
                f.write(f"{name}\t{dt}\t{off}\t{nb}\t{shape}\n")
        with open(os.path.join(d, "prompt.txt"), "w") as f:
            f.write("2\n")
        out = os.path.join(d, "screen.bin")
        env = dict(os.environ, ENGINE_CPUS=",".join(str(c) for c in range(min(8, os.cpu_count() or 1))))
        subprocess.run([EXE, d, os.path.join(d, "index.tsv"), os.path.join(d, "prompt.txt"), out], env=env,
                       check=True)
        raw = np.fromfile(out, np.uint8)
    nw, ns = HEAD_V * 768, HEAD_V * 48 * 2
    assert raw.size == nw + ns + HEAD_V * 4, raw.size
    Wq = raw[:nw].reshape(HEAD_V, 768)
    Sq = raw[nw:nw + ns].view(np.uint16).reshape(HEAD_V, 48)
    coef = raw[nw + ns:].view(np.float32)
    rows = np.array(sorted(set(SCREEN_TIE_ROWS) | set(SCREEN_SAMPLE_ROWS)), np.int64)
    path = os.path.join(HERE, "screen_build.npz")
    np.savez_compressed(path, seed=np.array([SCREEN_BUILD_SEED]), crc_E=np.array([crc(E)], np.uint32),
                        crc_Wq=np.array([crc(Wq)], np.uint32), crc_Sq=np.array([crc(Sq)], np.uint32),
                        crc_coef=np.array([crc(coef)], np.uint32), rows=rows, Wq_rows=Wq[rows], Sq_rows=Sq[rows],
                        coef_rows=coef[rows])
    print(f"screen_build.npz: {os.path.getsize(path)} bytes", flush=True)


if __name__ == "__main__":
    main()
