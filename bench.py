#!/usr/bin/env python3
"""Batched Q8_0 decode on one MI355X: the continuous-batching step of the
Coheryn engine's Qwen2 graph (inference/batch.rs:64-273) at Qwen2.5-0.5B shape.

Workload (and its 128-lane form): seeded N(0,0.02)
weights quantized to Q8_0 and written as GGUF; N ragged decode lanes whose
f32 KV caches are pre-filled with seeded values to lengths drawn U[64, 2048];
one greedy token per lane per step.  A step = one cohx_step over all lanes.

Prints one JSON line.  `value` is the 128-lane tok/s; the 32-lane run rides
along under "secondary".  `roofline` is the dominant kernel's algorithmic
bytes / its average launch time (HIP events on the library's stream);
`step_roofline` is the whole step's algorithmic bytes / step time.
`cpu_baseline` times the CPU oracle (the engine's algorithm restated in C,
16-lane units as batch.rs:65 allows) on a bounded sample of the same lanes.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "coheryn-ai-studio_amd"), os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import cohx  # noqa: E402
import gguf  # noqa: E402
import synth  # noqa: E402

METRIC = "batched decode tok/s, Qwen2.5-0.5B Q8_0 @32 & 128 ragged seqs; % of HBM peak"
HBM_PEAK = 8.0e12
KV_LO, KV_HI = 64, 2048


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_file(seed):
    path = f"/tmp/cohx_qwen25_05b_q8_0_seed{seed}.gguf"
    if not os.path.exists(path):
        log(f"[bench] writing seeded Q8_0 GGUF {path}")
        t0 = time.time()
        synth.write_model(path + ".part", synth.config(), "q8_0", seed=seed)
        os.replace(path + ".part", path)
        log(f"[bench] model written in {time.time() - t0:.1f}s")
    return path


def step_bytes(cfg, kv_lens, matrix_bytes):
    """Algorithmic HBM bytes of one decode step (f32 KV, no logits copied):
    weights + K/V rows attended (kv+1 each) + K/V rows appended + embedding rows
    + norm/bias vectors."""
    L, H = cfg["layers"], cfg["hidden"]
    kvd = cfg["kv_heads"] * cfg["head_dim"]
    per_tok = L * kvd * 4 * 2
    n = len(kv_lens)
    vectors = L * (2 * H + H + 2 * kvd) * 4 + H * 4
    return (matrix_bytes + sum(k + 1 for k in kv_lens) * per_tok + n * per_tok
            + n * H // 32 * 34 + vectors)


def run_workload(model, cfg, lanes, steps, warmup, seed, profile_steps):
    rng = np.random.default_rng(seed + lanes)
    kv = [int(v) for v in rng.integers(KV_LO, KV_HI + 1, lanes)]
    tokens = [int(v) for v in rng.integers(0, cfg["vocabulary"], lanes)]
    seqs = []
    for i in range(lanes):
        s = model.seq_alloc()
        model.seq_fill_synthetic(s, kv[i], seed, i)
        seqs.append(s)
    first = None

    def one_step():
        nonlocal tokens, first
        res = model.step([dict(seq=s, tokens=[t]) for s, t in zip(seqs, tokens)])
        if any(r["status"] for r in res):
            raise RuntimeError(f"lane failure {[r['status'] for r in res]}")
        if first is None:
            first = [r["argmax"] for r in res]
        tokens = [r["argmax"] for r in res]

    start_tokens = list(tokens)
    for _ in range(warmup):
        one_step()
    kv_at_timing = [model.seq_length(s) for s in seqs]
    t0 = time.perf_counter()
    for _ in range(steps):
        one_step()
    elapsed = time.perf_counter() - t0
    # per-kernel profile over a few more steps (events add overhead, so not timed above)
    model.profile(True)
    for _ in range(profile_steps):
        one_step()
    stats = model.profile_read()
    model.profile(False)
    mean_kv = [k + (steps - 1) / 2.0 for k in kv_at_timing]
    sb = step_bytes(cfg, mean_kv, model.matrix_bytes)
    for s in seqs:
        model.seq_free(s)
    return dict(kv=kv, start_tokens=start_tokens, first_argmax=first, elapsed=elapsed,
                stats=stats, step_bytes=sb, tok_s=lanes * steps / elapsed,
                ms_per_step=elapsed * 1e3 / steps)


def roofline(stats):
    top = max(stats, key=lambda s: s["total_ms"])
    avg_s = top["total_ms"] / 1e3 / top["launches"]
    achieved = top["bytes"] / top["launches"] / avg_s
    return {"kernel": top["name"], "bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9,
            "unit": "GB/s", "frac": achieved / HBM_PEAK, "traffic": None,
            "avg_launch_us": avg_s * 1e6, "bytes_per_launch": top["bytes"] / top["launches"],
            "share_of_step": top["total_ms"] / sum(s["total_ms"] for s in stats)}


def cpu_baseline(cfg, tensors, kv, start_tokens, seed, lanes, steps, threads):
    import orc
    m = orc.Model(cfg, tensors, threads=threads)
    ctx = max(kv[:lanes]) + steps + 8
    sess = []
    for i in range(lanes):
        s = m.session(ctx)
        s.fill_synthetic(kv[i], seed, i)
        sess.append(s)
    toks = list(start_tokens[:lanes])
    first = None
    t0 = time.perf_counter()
    for _ in range(steps):
        errs = m.forward_batch(sess, toks)
        assert not errs.any()
        toks = [int(orc.Sampler().sample(s.logits())[1]) for s in sess]
        if first is None:
            first = list(toks)
    elapsed = time.perf_counter() - t0
    return first, lanes * steps / elapsed, elapsed


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--lanes", type=int, default=128)
    ap.add_argument("--secondary-lanes", type=int, default=32)
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--cpu-steps", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the step shards by sequence with no collectives; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    path = model_file(args.seed)
    meta, tensors = gguf.read(path)
    cfg = gguf.qwen2_config(meta)
    ctx_len = KV_HI + args.warmup + args.steps + args.profile_steps + 16
    log(f"[bench] uploading model (max_lanes={args.lanes}, max_context={ctx_len})")
    model = cohx.Model(cfg, tensors, max_lanes=args.lanes, max_rows=args.lanes,
                       max_seqs=args.lanes, max_context=ctx_len)
    results = {}
    for lanes in (args.secondary_lanes, args.lanes):
        log(f"[bench] {lanes} lanes: warmup {args.warmup}, timed {args.steps}")
        results[lanes] = run_workload(model, cfg, lanes, args.steps, args.warmup, args.seed,
                                      args.profile_steps)
        log(f"[bench] {lanes} lanes: {results[lanes]['tok_s']:.0f} tok/s, "
            f"{results[lanes]['ms_per_step']:.3f} ms/step")
    main_r = results[args.lanes]
    line = {
        "metric": METRIC, "value": main_r["tok_s"], "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": main_r["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q8_0 int8 MFMA + f32 fmaf chain; f32 KV, f64 reductions",
        "data": "synthetic (seeded N(0,0.02) weights as Q8_0 GGUF, seeded KV, greedy decode)",
        "config": {"workload": f"Qwen2.5-0.5B-shape Q8_0 decode, {args.lanes} ragged lanes, "
                               f"KV U[{KV_LO},{KV_HI}] f32, 1 token/lane/step",
                   "lanes": args.lanes, "kv_range": [KV_LO, KV_HI], "kv_dtype": "f32",
                   "seed": args.seed},
        "roofline": roofline(main_r["stats"]),
        "step_roofline": {"bound": "hbm", "bytes_per_step": main_r["step_bytes"],
                          "achieved": main_r["step_bytes"] / (main_r["ms_per_step"] / 1e3) / 1e9,
                          "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                          "frac": main_r["step_bytes"] / (main_r["ms_per_step"] / 1e3) / HBM_PEAK},
        "kernels": {s["name"]: {"ms_per_step": s["total_ms"] / args.profile_steps,
                                "launches_per_step": s["launches"] / args.profile_steps,
                                "GB_s": (s["bytes"] / (s["total_ms"] / 1e3) / 1e9) if s["total_ms"] else 0}
                    for s in main_r["stats"] if s["launches"]},
    }
    sec = results[args.secondary_lanes]
    line["secondary"] = {
        "lanes": args.secondary_lanes, "value": sec["tok_s"], "unit": "tok/s",
        "ms_per_step": sec["ms_per_step"],
        "step_frac": sec["step_bytes"] / (sec["ms_per_step"] / 1e3) / HBM_PEAK,
        "roofline": roofline(sec["stats"])}
    if not args.no_cpu_baseline:
        threads = min(16, os.cpu_count() or 1)
        n_cpu = min(16, args.lanes)
        log(f"[bench] cpu baseline: oracle, {n_cpu} lanes x {args.cpu_steps} steps, {threads} threads")
        first, tps, el = cpu_baseline(cfg, tensors, main_r["kv"], main_r["start_tokens"], args.seed,
                                      n_cpu, args.cpu_steps, threads)
        line["cpu_baseline"] = {
            "value": tps, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"first {n_cpu} of the {args.lanes} lanes (one 16-lane unit, batch.rs:65), "
                      f"{args.cpu_steps} decode steps, same weights/KV/tokens; {el:.1f}s"}
        gpu_first = main_r["first_argmax"][:n_cpu]
        line["parity"] = {"lanes": n_cpu, "greedy_equal": int(sum(a == b for a, b in zip(first, gpu_first))),
                          "check": "first-step greedy token, GPU vs CPU oracle, same inputs"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
