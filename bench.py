"""Verify-step benchmark on one MI355X.

Workload: one greedy verify pass of the synthetic 35-layer Gemma-4-E2B-shaped int4 stack
(hidden 1536, FFN 6144, 8 query heads / 1 KV head of dim 256, l % 5 != 4 sliding-window
512, vocabulary 262,144 with the certified head screen), context 2048 (the reference's
ENGINE_FAKE_CTX synthetic cache), draft tree of 2 branches x depth 3 with seeded token ids,
greedy longest-prefix acceptance on the device.  A step is one such pass; successive steps
advance the position by the committed tokens, as the engine's run_req does.

Prints one JSON line: accepted tokens per second (value), the verify-step time, the
dominant kernel class against the HBM roofline (HIP events on the library's stream over
the timed region), the whole step's algorithmic bytes against peak HBM (step_hbm_frac), the
device's read and copy bandwidth over 2 GiB / 1 GiB buffers (hbm_stream), an accepted-path
run (drafts the model takes, in branch a and branch b in turn, so acceptance and KV compaction
are timed), the reference's own AVX2 kernels timed on this host (one
thread per physical core and 8 threads, each in a child process, interleaved with a second
GPU run, with the host's read bandwidth and lscpu summary), and the long-prompt workload's
prefill and decode times.

--workload long_prompt runs the long-prompt case instead: a 6,841-token prompt (a seeded
64-token motif repeated, 5% uniform noise tokens) prefilled through the same stack (W4A8
linear layers on the matrix cores), then 256 speculative decode rounds with prompt-lookup
drafts (n-gram 3, up to 3 drafts), or 3 MTP drafts from the synthetic drafter when the lookup
finds none, verified as a chain.  A step is one prefill + 256 rounds.

--workload gemma_layout runs the Gemma-4-E2B layout's passes alone (device-generated weights at
the checkpoint's sizes: a 2,048-token prefill, then verify passes of 1, 4 and 8 rows) and prints
that sub-object of the default line as its own line.
"""
import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "accepted tok/s + verify-step µs at 1 GPU; achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0

V, NL, I, CTXCAP, NCTX, SEED, NA, NB, NSPLIT = 262144, 35, 6144, 4096, 2048, 1, 3, 3, 8
H, HD = 1536, 256
# algorithmic bytes of a step: every layer's int4 matrices with their bf16 scales (N K / 2 + N K / 16
# for q 2048, k 256, v 256, o, gate, up, down), the head screen (int4 + scales + coef), and the
# K and V rows of every layer up to the step's position
LAYER_BYTES = sum(n * k // 2 + n * k // 16 for n, k in [(2048, H), (256, H), (256, H), (H, 2048), (I, H), (I, H),
                                                         (H, I)])
SCREEN_BYTES = V * H // 2 + V * H // 16 + V * 4


def hbm_traffic(cls):
    """bytes read + written per launch of kernel class `cls`, from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs summarised in profiles/hbm_traffic.md (copy-kernel calibrated); None when
    the class was not measured"""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == cls:
            try:
                return int(cells[4].replace(",", "")) + int(cells[5].replace(",", ""))
            except ValueError:
                return None
    return None


def trace_avg_us(cls):
    """the average device duration of kernel class `cls` in the committed rocprofv3 kernel trace of
    this bench (profiles/verify_step_kernels.md, table `class | kernel | launches | avg us`); None
    when the class is not listed"""
    path = os.path.join(ROOT, "profiles", "verify_step_kernels.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 4 and cells[0] == cls:
            try:
                return float(cells[3])
            except ValueError:
                return None
    return None


def load_g4v():
    spec = importlib.util.spec_from_file_location("g4v", os.path.join(ROOT, "gemma4-e2b-laptop-cpu_amd", "g4v.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def drafts(step, conf):
    """seeded draft ids for step `step`: chain a then branch b (stand-ins for the MTP and
    prompt-lookup drafters), confirmed token first"""
    rng = np.random.default_rng(1000 + step)
    d = rng.integers(0, V, size=NA + NB)
    return np.concatenate([[conf], d]).astype(np.int32)


def accepted_drafts(step, conf):
    """drafts the model accepts: the random-init stack's greedy token repeats the row's own token,
    so a branch of copies of the confirmed token is its greedy chain.  Even steps put that chain
    in branch a, odd steps in branch b (committing branch b compacts its KV rows into place)."""
    d = drafts(step, conf)
    if step % 2 == 0:
        d[1:1 + NA] = conf
    else:
        d[1 + NA:] = conf
    return d


def run_steps(verify, nsteps, pos0, conf, step0, draft=None):
    tokens = 0
    draft = draft or drafts
    stats = {"branch_b": 0, "nacc": 0}
    for s in range(nsteps):
        r = verify(draft(step0 + s, conf), pos0)
        tokens += r.ncommit
        pos0 += r.ncommit
        conf = r.commit[r.ncommit - 1]
        stats["branch_b"] += r.branch
        stats["nacc"] += r.nacc
    run_steps.stats = stats
    return tokens, pos0, conf


def host_topology():
    """the host's CPUs as this process may use them: lscpu's summary, the allowed logical CPUs,
    and one logical CPU per physical core (sysfs core / package ids)"""
    import subprocess
    allowed = sorted(os.sched_getaffinity(0))
    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "CPU(s)", "Thread(s) per core", "Core(s) per socket", "Socket(s)"):
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    cores, seen = [], set()
    for c in allowed:
        try:
            base = f"/sys/devices/system/cpu/cpu{c}/topology/"
            key = (open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip())
        except OSError:
            key = ("?", str(c))
        if key not in seen:
            seen.add(key)
            cores.append(c)
    return {"lscpu": info, "allowed_cpus": len(allowed), "physical_cores": len(cores)}, allowed, cores


def cpu_baseline_run(cpus, seconds=10.0):
    """the reference's own kernels (oracle/_ref) with its worker pool pinned to `cpus`, over a
    bounded sample of the same verify steps; the scalar C oracle when the harness was not built"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Model, Oracle, Ref, ref_available

    orc = Oracle()
    m = Model(orc, SEED, V, NL, I, CTXCAP)
    m.fake_ctx(NCTX, 12345)
    if ref_available():
        ref = Ref(cpus=cpus)
        ref.bind_model(m)
        verify = lambda toks, p: ref.verify(toks, NA, NB, p)
        kind, cores = "reference", ref.threads
    else:
        verify = lambda toks, p: m.verify(toks, NA, NB, p, NSPLIT)[0]
        kind, cores = "port", 1
    verify(drafts(0, 11), NCTX)  # warm-up
    t0 = time.perf_counter()
    tokens, steps, pos0, conf = 0, 0, NCTX, 11
    while steps < 100:
        t, pos0, conf = run_steps(verify, 1, pos0, conf, steps)
        tokens += t
        steps += 1
        if time.perf_counter() - t0 > seconds and steps >= 3:
            break
    dt = time.perf_counter() - t0
    bw = orc.host_read_gbs(cpus)
    m.close()
    return {"value": tokens / dt, "unit": "tok/s", "cores": cores, "kind": kind, "cpus": list(cpus),
            "ms_per_step": round(dt * 1e3 / steps, 2), "steps": steps, "host_read_gbs": round(bw, 1)}


def cpu_baseline_child(cpus):
    """cpu_baseline_run in a child process (the reference pool starts once per process)"""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-only", ",".join(map(str, cpus))]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        return {"value": None, "error": r.stderr[-400:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


LP_N, LP_ROUNDS, LP_NGRAM, LP_NGLEN, LP_CTX, LP_K, LP_DSPLIT = 6841, 256, 3, 3, 8192, 3, 6


def long_prompt_tokens():
    rng = np.random.default_rng(11)
    motif = rng.integers(0, V, 64)
    seq = np.resize(motif, LP_N).astype(np.int32)
    noise = rng.random(LP_N) < 0.05
    seq[noise] = rng.integers(0, V, int(noise.sum()))
    return seq


def long_prompt_run(dev, prompt):
    """prefill, then LP_ROUNDS rounds of run_req's loop (E:1617-1661): prompt-lookup drafts, and
    the MTP drafter's chain of LP_K when the lookup finds none (E:1624-1646 with the sibling
    policy off)"""
    dev.sync()
    t0 = time.perf_counter()
    g0, h0 = dev.prefill(prompt, hidden=True)
    t1 = time.perf_counter()
    dev.history_set(np.concatenate([prompt, [g0]]))
    gen, P, app, acc, nd, nmtp = [g0], len(prompt) - 1, [], 0, 0, 0
    for rnd in range(LP_ROUNDS):
        d = dev.prompt_lookup(LP_NGRAM, LP_NGLEN, app)
        if d.size == 0:  # the chain starts from the prefill's (then the last verify step's) hidden state
            d = dev.draft_mtp(gen[-1], h0 if rnd == 0 else None, P, LP_K, LP_DSPLIT)[0]
            nmtp += 1
        r = dev.verify(np.array([gen[-1]] + d.tolist(), np.int32), len(d), 0, P + 1, NSPLIT)
        app = list(r.commit[:r.ncommit])
        gen += app
        P += r.ncommit
        acc += r.nacc
        nd += len(d)
    dev.sync()
    t2 = time.perf_counter()
    return {"prefill_s": t1 - t0, "decode_s": t2 - t1, "tokens": len(gen) - 1, "accepted": acc, "drafted": nd,
            "mtp_rounds": nmtp}


def cpu_prefill_baseline(prompt, nrows=64):
    """the reference's prefill composition (oracle/_ref, 8 workers) over the first `nrows` prompt rows"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Model, Oracle, Ref, ref_available
    if not ref_available():
        return {"value": None, "error": "oracle/_ref not built"}
    orc = Oracle()
    m = Model(orc, SEED, V, NL, I, 256)
    ref = Ref(threads=8)
    ref.bind_model(m)
    ref.prefill(prompt[:32])  # W4A8 repacks of every matrix, once
    t0 = time.perf_counter()
    ref.prefill(prompt[:nrows])
    dt = time.perf_counter() - t0
    m.close()
    return {"value": nrows / dt, "unit": "prefill tok/s", "cores": ref.threads, "kind": "reference",
            "sample": f"prefill of the first {nrows} prompt tokens (35 layers, W4A8, blocks of 32), {dt:.2f} s"}


def long_prompt_summary(g4v):
    """the long-prompt workload (one warm-up run, one timed run) for the verify line"""
    dev = g4v.Device(0)
    dev.model_synth(SEED, V, NL, I, LP_CTX)
    dev.drafter_synth(SEED + 1)
    prompt = long_prompt_tokens()
    long_prompt_run(dev, prompt)
    r = long_prompt_run(dev, prompt)
    dev.close()
    return {"workload": f"{LP_N}-token motif prompt prefilled (blocks of 32), then {LP_ROUNDS} speculative rounds",
            "prefill_ms": round(r["prefill_s"] * 1e3, 2), "prefill_tok_s": round(LP_N / r["prefill_s"], 1),
            "decode_ms": round(r["decode_s"] * 1e3, 2), "decode_tok_s": round(r["tokens"] / r["decode_s"], 1),
            "tokens_per_round": round(r["tokens"] / LP_ROUNDS, 3),
            "drafts_accepted": f"{r['accepted']}/{r['drafted']}", "mtp_rounds": r["mtp_rounds"]}


GM_MLP = [6144 if l < 15 else 12288 for l in range(35)]  # the checkpoint's MLP widths
GM_CTX = 2048


def gemma_pass_bytes(M, pos0=GM_CTX):
    """algorithmic bytes of one verify pass of M rows at pos0 on the Gemma-4-E2B layout: every
    layer's int4 matrices with their bf16 group scales (q/k/v of the owner layers, o, gate, up,
    down, the per-layer-input gate and projection), the per-layer-input projection and the rows'
    per-layer embeddings, the head screen, and the K / V rows each layer attends (window 512 for
    head dim 256, the whole context for 512)"""
    q4 = lambda n, k: n * k // 2 + n * k // 16
    b = q4(35 * 256, H) + M * 35 * 256 * 2 + SCREEN_BYTES
    for l in range(35):
        hd = 512 if l % 5 == 4 else 256
        b += q4(8 * hd, H) + q4(H, 8 * hd) + 2 * q4(GM_MLP[l], H) + q4(H, GM_MLP[l]) + q4(256, H) + q4(H, 256)
        if l < 15:
            b += 2 * q4(hd, H)
        npos = pos0 + M if hd == 512 else min(pos0 + M, 512 + M - 1)
        b += npos * hd * 2 * 2
    return b


def components_summary(dev, iters=30):
    """configs 1-3 of the workload on their own, device-timed per launch (g4v_*_time): warm (the
    launches repeat, operands stay in the caches) and cold (a 512 MB read before each launch evicts
    the 256 MB last-level cache, outside the timed events).  The head of one row (config 1); the
    W4G32 products 1536 x 1536, 6144 x 1536, the fused gate + up pair (2 x 6144 x 1536) and the
    down projection (1536 x 6144) at 1, 2, 4 and 8 rows, and their W4A8 form at 2, 4 and 8 rows
    (config 2); split-KV attention of 4 rows, 8 splits, at ctx 512, 2048, 6841 and with the 512
    window at 6841 (config 3).  Bytes are the algorithmic ones (int4 + bf16 scales; K and V rows
    attended), hbm_frac = bytes / cold time / 8 TB/s."""
    rng = np.random.default_rng(SEED + 3)

    def mat(N, K):
        W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
        s = rng.uniform(0.005, 0.02, (N, K // 32)).astype(np.float32)
        return dev.w4_upload(W, (s.view(np.uint32) >> 16).astype(np.uint16))

    frac = lambda b, us: round(b / (us * 1e-6) / (HBM_PEAK_GBS * 1e9), 4)
    out = {"timing": "device events per launch on the library stream; cold = 512 MB read before each launch",
           "iters": iters}
    hrow = rng.standard_normal(1536).astype(np.float32)
    hw, ns, fb = dev.head_time(hrow, iters, False)
    hc = dev.head_time(hrow, iters, True)[0]
    out["head_1row"] = {"bytes": SCREEN_BYTES, "warm_us": round(hw, 2), "cold_us": round(hc, 2),
                        "survivors": ns, "fallback_full_head": fb, "cold_hbm_frac_screen_bytes": frac(SCREEN_BYTES, hc)}
    g = {}
    for name, shp in (("1536x1536", [(1536, 1536)]), ("6144x1536", [(6144, 1536)]),
                      ("gate_up_2x6144x1536", [(6144, 1536), (6144, 1536)]), ("down_1536x6144", [(1536, 6144)])):
        ms = [mat(N, K) for N, K in shp]
        nb = sum(N * K // 2 + N * K // 16 for N, K in shp)
        row = {"bytes": nb}
        for M in (1, 2, 4, 8):
            w = dev.w4g32_time(ms, M, iters, cold=False)
            c = dev.w4g32_time(ms, M, iters, cold=True)
            row[f"m{M}"] = {"warm_us": round(w, 2), "cold_us": round(c, 2), "cold_hbm_frac": frac(nb, c)}
        for M in (2, 4, 8):
            c = dev.w4g32_time(ms, M, iters, cold=True, w4a8=True)
            row[f"w4a8_m{M}"] = {"cold_us": round(c, 2), "cold_hbm_frac": frac(nb, c)}
        g[name] = row
    out["w4g32"] = g
    a = {}
    for ctx, window in ((512, False), (2048, False), (6841, False), (6841, True)):
        keys = min(ctx, 512 + 3) if window else ctx
        nb = keys * HD * 2 * 2
        w = dev.attn_time(ctx, 4, 8, window, iters, cold=False)
        c = dev.attn_time(ctx, 4, 8, window, iters, cold=True)
        a[f"ctx{ctx}" + ("_window512" if window else "")] = {"bytes": nb, "warm_us": round(w, 2), "cold_us": round(c, 2),
                                                          "cold_hbm_frac": frac(nb, c)}
    out["attn_4rows_8splits"] = a
    return out


GM_SHAPES = ((1, False), (4, False), (8, False), (4, True), (8, True))


def gemma_layout_summary(g4v, reps=10, shapes=GM_SHAPES, graphs=True):
    """verify passes on the Gemma-4-E2B layer layout at the checkpoint's sizes (device-generated
    weights): a 2048-token context prefilled with W4A8 blocks, then one-row decode passes and
    chain passes of 3 and 7 drafts at position 2048 (the passes re-run at the same position), in
    exact float and, for the chains, with W4A8 products (ENGINE_DECODE_INT8, the server's mode).
    shapes: (rows, W4A8) of the passes timed; graphs = False launches their kernels eagerly (for a
    kernel trace: the tracer follows graph replays less reliably)"""
    dev = g4v.Device(0)
    if not graphs:
        dev.set_graphs(False)
    dev.model_synth_gemma(SEED + 7, V, GM_MLP, 4096)
    dev.set_prefill_int8(True)
    rng = np.random.default_rng(11)
    ctx = rng.integers(0, V, GM_CTX).astype(np.int32)
    dev.prefill(ctx, 0, 32, 6)
    dev.sync()
    t0 = time.perf_counter()
    dev.prefill(ctx, 0, 32, 6)
    dev.sync()
    out = {"workload": f"Gemma-4-E2B layout (35 layers, head dim 256 / 512, KV shared past layer 14, MLP 6144 / "
                       f"12288, per-layer inputs, V {V}), context {GM_CTX}, 6 KV splits",
           "prefill_ms": round((time.perf_counter() - t0) * 1e3, 2)}
    for M, i8 in shapes:
        dev.set_decode_int8(i8)
        blk = rng.integers(0, V, M).astype(np.int32)
        for _ in range(2):
            dev.verify(blk, M - 1, 0, GM_CTX, 6)
        dev.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            dev.verify(blk, M - 1, 0, GM_CTX, 6)
        dev.sync()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        out[f"verify_{M}_rows{'_w4a8' if i8 else ''}_ms"] = round(ms, 3)
        out[f"verify_{M}_rows{'_w4a8' if i8 else ''}_hbm_frac"] = round(
            gemma_pass_bytes(M) / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4)
    dev.set_decode_int8(False)
    dev.close()
    return out


def main_long_prompt(args, g4v):
    dev = g4v.Device(0)
    info = dev.info()
    dev.model_synth(SEED, V, NL, I, LP_CTX)
    dev.drafter_synth(SEED + 1)
    prompt = long_prompt_tokens()
    for _ in range(args.warmup):
        long_prompt_run(dev, prompt)
    runs = [long_prompt_run(dev, prompt) for _ in range(args.steps)]
    dev.close()
    pf = sum(r["prefill_s"] for r in runs) / len(runs)
    dc = sum(r["decode_s"] for r in runs) / len(runs)
    last = runs[-1]
    out = {
        "metric": METRIC,
        "value": round(last["tokens"] / dc, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((pf + dc) * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (prefill linear layers: int8 x int4 on the matrix cores)",
        "data": "synthetic (seeded random-init weights, seeded motif prompt)",
        "config": {"workload": f"long prompt: {LP_N}-token motif prompt prefilled (blocks of 32), then {LP_ROUNDS} "
                               f"speculative rounds with prompt-lookup drafts (n-gram {LP_NGRAM}, <= {LP_NGLEN}), "
                               f"else {LP_K} MTP drafts",
                   "prefill_ms": round(pf * 1e3, 2), "prefill_tok_s": round(LP_N / pf, 1),
                   "decode_ms": round(dc * 1e3, 2), "tokens_per_step": round(last["tokens"] / LP_ROUNDS, 3),
                   "drafts_accepted": f"{last['accepted']}/{last['drafted']}",
                   "mtp_rounds": last["mtp_rounds"], "device": info["name"]},
    }
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_prefill_baseline(prompt)
        except Exception as e:
            out["cpu_baseline"] = {"value": None, "error": str(e)}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--workload", choices=["verify", "long_prompt", "gemma_layout", "components"], default="verify")
    ap.add_argument("--cpu-only", default=None, help=argparse.SUPPRESS)  # child process of the CPU baseline
    ap.add_argument("--no-long-prompt", action="store_true", help="skip the long-prompt sub-measurement")
    ap.add_argument("--no-gemma", action="store_true", help="skip the Gemma-4-E2B layout sub-measurement")
    ap.add_argument("--no-components", action="store_true",
                    help="skip the components sub-measurement (head, products, attention on their own)")
    ap.add_argument("--gemma-shapes", default=None,
                    help="gemma_layout: the passes to time, e.g. 1,4,8,4i8,8i8 (rows; i8: W4A8 products)")
    ap.add_argument("--no-graphs", action="store_true", help="gemma_layout: launch the passes' kernels eagerly")
    args = ap.parse_args()
    if args.cpu_only is not None:
        print(json.dumps(cpu_baseline_run([int(c) for c in args.cpu_only.split(",")])), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the verify path is single-GPU by design (asked for {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "long_prompt":
        main_long_prompt(args, load_g4v())
        return
    if args.workload == "components":  # configs 1-3 on their own (the line's sub-object as a line)
        g4v = load_g4v()
        dev = g4v.Device(0)
        dev.model_synth(SEED, V, NL, I, CTXCAP)
        print(json.dumps(components_summary(dev)), flush=True)
        return
    if args.workload == "gemma_layout":  # the Gemma-4-E2B layout's passes alone (its sub-object as a line)
        shapes = GM_SHAPES
        if args.gemma_shapes:
            shapes = tuple((int(t[:-2] if t.endswith("i8") else t), t.endswith("i8"))
                           for t in args.gemma_shapes.split(","))
        print(json.dumps(gemma_layout_summary(load_g4v(), shapes=shapes, graphs=not args.no_graphs)), flush=True)
        return

    g4v = load_g4v()
    dev = g4v.Device(0)
    info = dev.info()
    t0 = time.time()
    dev.model_synth(SEED, V, NL, I, CTXCAP)
    dev.fake_ctx(NCTX, 12345)
    setup_s = time.time() - t0
    verify = lambda toks, p: dev.verify(toks, NA, NB, p, NSPLIT)

    # warm-up on the replayed graph (the first call of the shape runs eagerly, the second captures it)
    _, pos0, conf = run_steps(verify, args.warmup, NCTX, 11, 0)

    # timed region: replayed graphs, wall clock around K steps
    dev.sync()
    t0 = time.perf_counter()
    tokens, pos0, conf = run_steps(verify, args.steps, pos0, conf, args.warmup)
    dev.sync()
    dt = time.perf_counter() - t0

    # kernel classes: HIP events recorded on the library's stream around every launch of a class.
    # Event nodes inside a replayed graph do not wait for the preceding kernel, so these steps
    # launch eagerly (same kernels, same grids); the event pairs then bracket each launch.
    dev.set_graphs(False)
    dev.profile(None)
    nprof = max(3, args.steps // 4)
    run_steps(verify, nprof, pos0, conf, args.warmup + args.steps)
    prof_all = dev.profile_read()
    dev.profile([])
    dev.set_graphs(True)
    dominant = max(prof_all, key=lambda k: prof_all[k]["ms"])
    prof = prof_all[dominant]
    timing = "hip events around each launch on the library stream, eager launches of the same steps"

    # the accepted path: drafts the model takes, branch a and branch b (KV compaction) in turn
    dev.sync()
    nacc_steps = max(8, args.steps // 2)
    t1 = time.perf_counter()
    acc_tokens, pos0, conf = run_steps(verify, nacc_steps, pos0, conf, 0, accepted_drafts)
    dev.sync()
    dt_acc = time.perf_counter() - t1
    acc_stats = dict(run_steps.stats)

    ms_per_step = dt * 1e3 / args.steps
    step_ctx = NCTX + args.warmup + tokens // 2  # mean position of the timed steps
    step_bytes = NL * LAYER_BYTES + SCREEN_BYTES + NL * step_ctx * HD * 2 * 2
    per_launch_ms = prof["ms"] / max(prof["launches"], 1)
    per_launch_bytes = prof["bytes"] / max(prof["launches"], 1)
    achieved = per_launch_bytes / (per_launch_ms * 1e-3) / 1e9 if per_launch_ms > 0 else 0.0
    classes = {k: round(v["ms"] / nprof * 1e3, 1) for k, v in prof_all.items() if v["launches"]}

    out = {
        "metric": METRIC,
        "value": round(tokens / dt, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded random-init weights, fake KV context, seeded draft ids)",
        "config": {"workload": "verify step: 35-layer int4 G32 stack, hidden 1536, FFN 6144, 8q/1kv heads hd 256, "
                               "vocab 262144 certified head, ctx 2048, 2x3 draft tree, 8 KV splits",
                   "verify_step_us": round(ms_per_step * 1e3, 1), "tokens_per_step": round(tokens / args.steps, 3),
                   "device": info["name"]},
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": hbm_traffic(dominant),
                     "launch_us": round(per_launch_ms * 1e3, 2), "bytes_per_launch": int(per_launch_bytes),
                     "timing": timing},
        "step_hbm_frac": round(step_bytes / (ms_per_step * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "step_bytes": int(step_bytes),
        "accepted_path": {"ms_per_step": round(dt_acc * 1e3 / nacc_steps, 4), "steps": nacc_steps,
                          "tokens_per_step": round(acc_tokens / nacc_steps, 3),
                          "tok_s": round(acc_tokens / dt_acc, 1), "branch_b_commits": acc_stats["branch_b"],
                          "drafts_accepted": acc_stats["nacc"]},
        "kernel_classes_us_per_step": classes,
        "setup_s": round(setup_s, 1),
    }
    tus = trace_avg_us(dominant)
    if tus:  # the same bytes over the kernel's device duration in the committed trace (no launch overhead)
        out["roofline"].update({"trace_us": tus, "trace_achieved": round(per_launch_bytes / (tus * 1e-6) / 1e9, 1),
                                "trace_frac": round(per_launch_bytes / (tus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                "trace_source": "profiles/verify_step_kernels.md (rocprofv3 --kernel-trace --stats "
                                                "of this bench, device kernel durations)"})
    # the device's streaming bandwidth beside the 8 TB/s peak (bench/stream_bw.cpp:10-19 method)
    out["hbm_stream"] = {"read_gbs": round(dev.hbm_stream(2 << 30, 5), 1),
                         "copy_gbs": round(dev.hbm_stream(1 << 30, 5, copy=True), 1), "read_buffer": 2 << 30,
                         "copy_buffer": 1 << 30, "passes": 5}
    # the same steps with W4A8 products (ENGINE_PREFILL_INT8=1 with ENGINE_DECODE_INT8 on, E:1600:
    # the reference server's mode), replayed graphs
    dev.set_prefill_int8(True)
    dev.set_decode_int8(True)
    run_steps(verify, 2, pos0, conf, 8000)
    dev.sync()
    t3 = time.perf_counter()
    tok3, _, _ = run_steps(verify, args.steps, pos0, conf, 8000)
    dev.sync()
    out["w4a8_step"] = {"ms_per_step": round((time.perf_counter() - t3) * 1e3 / args.steps, 4), "steps": args.steps,
                        "tokens_per_step": round(tok3 / args.steps, 3)}
    dev.set_decode_int8(False)
    if not args.no_components:  # configs 1-3 on their own, warm and cold
        out["components"] = components_summary(dev)
    if not args.no_cpu:
        # A (GPU) and B (CPU) interleaved: A1 above, B1 one thread per physical core, A2, B2 8 threads
        try:
            topo, allowed, cores = host_topology()
            per_core = cores[:16]
            eight = (cores if len(cores) >= 8 else allowed)[:8]
            b1 = cpu_baseline_child(per_core)
            dev.sync()
            t2 = time.perf_counter()
            tok2, pos0, conf = run_steps(verify, args.steps, pos0, conf, 7000)
            dev.sync()
            a2_ms = (time.perf_counter() - t2) * 1e3 / args.steps
            b2 = cpu_baseline_child(eight)
            best = b1 if (b1.get("value") or 0) >= (b2.get("value") or 0) else b2
            out["cpu_baseline"] = {
                "value": best.get("value"), "unit": "tok/s", "cores": best.get("cores"), "kind": best.get("kind"),
                "sample": "bounded sample (about 10 s) of the same verify steps (2x3 tree, ctx 2048, 35 layers, "
                          "V 262144) with the reference's own kernels (oracle/_ref) on this host",
                "one_thread_per_core": b1, "eight_threads": b2, "host": topo,
                "abab_gpu_ms_per_step": [round(ms_per_step, 4), round(a2_ms, 4)]}
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"value": None, "error": str(e)}
    dev.close()
    if not args.no_long_prompt:
        try:
            out["long_prompt"] = long_prompt_summary(g4v)
        except Exception as e:
            out["long_prompt"] = {"error": str(e)}
    if not args.no_gemma:
        try:
            out["gemma_layout"] = gemma_layout_summary(g4v)
        except Exception as e:
            out["gemma_layout"] = {"error": str(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
