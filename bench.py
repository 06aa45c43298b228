"""Verify-step benchmark on one MI355X.

Workload: one greedy verify pass of the synthetic 35-layer Gemma-4-E2B-shaped int4 stack
(hidden 1536, FFN 6144, 8 query heads / 1 KV head of dim 256, l % 5 != 4 sliding-window
512, vocabulary 262,144 with the certified head screen), context 2048 (the reference's
ENGINE_FAKE_CTX synthetic cache), draft tree of 2 branches x depth 3 with seeded token ids,
greedy longest-prefix acceptance on the device.  A step is one such pass; successive steps
advance the position by the committed tokens, as the engine's run_req does.

Prints one JSON line: accepted tokens per second (value), the verify-step time, the
dominant kernel class against the HBM roofline (HIP events on the library's stream over
the timed region) and the reference's own AVX2 kernels timed on this host as a baseline.

--workload long_prompt runs the long-prompt case instead: a 6,841-token prompt (a seeded
64-token motif repeated, 5% uniform noise tokens) prefilled through the same stack (W4A8
linear layers on the matrix cores), then 256 speculative decode rounds with prompt-lookup
drafts (n-gram 3, up to 3 drafts), or 3 MTP drafts from the synthetic drafter when the lookup
finds none, verified as a chain.  A step is one prefill + 256 rounds.
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


def run_steps(verify, nsteps, pos0, conf, step0):
    tokens = 0
    for s in range(nsteps):
        r = verify(drafts(step0 + s, conf), pos0)
        tokens += r.ncommit
        pos0 += r.ncommit
        conf = r.commit[r.ncommit - 1]
    return tokens, pos0, conf


def cpu_baseline(seconds_cap=30.0):
    """the reference's own kernels (oracle/_ref, 8 worker threads as the engine uses past
    1,024 tokens) on this host over a bounded sample of the same workload; falls back to the
    scalar C oracle when the harness was not built"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Model, Oracle, Ref, ref_available

    orc = Oracle()
    m = Model(orc, SEED, V, NL, I, CTXCAP)
    m.fake_ctx(NCTX, 12345)
    if ref_available():
        ref = Ref(threads=8)
        ref.bind_model(m)
        verify = lambda toks, p: ref.verify(toks, NA, NB, p)
        kind, cores = "reference", ref.threads
    else:
        verify = lambda toks, p: m.verify(toks, NA, NB, p, NSPLIT)[0]
        kind, cores = "port", int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    verify(drafts(0, 11), NCTX)  # warm-up
    t0 = time.perf_counter()
    tokens, steps, pos0, conf = 0, 0, NCTX, 11
    while steps < 100:
        t, pos0, conf = run_steps(verify, 1, pos0, conf, steps)
        tokens += t
        steps += 1
        if time.perf_counter() - t0 > min(seconds_cap, 10.0) and steps >= 3:
            break
    dt = time.perf_counter() - t0
    m.close()
    return {"value": tokens / dt, "unit": "tok/s", "cores": cores, "kind": kind,
            "sample": f"{steps} verify steps (2x3 tree, ctx 2048, 35 layers, V 262144) on the host, "
                      f"{dt * 1e3 / steps:.1f} ms/step"}


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
    ap.add_argument("--workload", choices=["verify", "long_prompt"], default="verify")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the verify path is single-GPU by design (asked for {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "long_prompt":
        main_long_prompt(args, load_g4v())
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

    ms_per_step = dt * 1e3 / args.steps
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
        "kernel_classes_us_per_step": classes,
        "setup_s": round(setup_s, 1),
    }
    dev.close()
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline()
        except Exception as e:  # the baseline is reported, never required
            out["cpu_baseline"] = {"value": None, "error": str(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
