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
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on
# this workload, scaled by the same counters on a copy of known size
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_decode128.json")
# profiler category -> the kernel instance it times at the Qwen2.5-0.5B shape
# (qkv, o and down are split-K instances; o and down share one instance and
# grid, so counters cannot tell them apart)
CATEGORY_KERNEL = {"attn_scores": "k_attn_scores<64, 7, 2>", "attn_softmax_stats": "k_attn_exp<7>",
                   "attn_pv": "k_attn_pv<64, 7>", "attn_combine_act": "k_attn_combine<8>",
                   "matvec_qkv": "k_mv_q8s<4, 1, 2, 8, 8>", "matvec_o_residual": "k_mv_q8s<1, 1, 2, 8, 8>",
                   "matvec_gate_up_swiglu": "k_mv_q8w<2, 2, 8, 14, 2, true>",
                   "matvec_down_residual": "k_mv_q8s<1, 1, 2, 8, 8>",
                   "matvec_head_argmax": "k_mv_q8h<8, 14>"}
PMC_CMD = ("COHX_GRAPHS=0 rocprofv3 --pmc {counter} --kernel-include-regex \"k_attn|k_mv\" --output-format csv "
           "-d <dir> -o <name> -- python3 bench.py --steps 2 --warmup 1 --secondary-lanes 0 "
           "--no-cpu-baseline --no-c3 --no-c4 --no-c5")
COPY_CMD = ("rocprofv3 --pmc {counter} --output-format csv -d <dir> -o <name> -- "
            "python3 bench.py --copy-probe")
TRACE_CMD = ("COHX_GRAPHS=0 rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o <name> -- "
             "python3 bench.py --no-cpu-baseline --no-c3 --no-c4 --no-c5")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_info():
    """The host the CPU baselines run on: logical CPUs, the ones this process
    may use, and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def model_file(seed, dtype="q8_0"):
    path = f"/tmp/cohx_qwen25_05b_{dtype}_seed{seed}.gguf"
    if not os.path.exists(path):
        log(f"[bench] writing seeded {dtype} GGUF {path}")
        t0 = time.time()
        synth.write_model(path + ".part", synth.config(), dtype, seed=seed)
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


def run_workload(model, cfg, lanes, steps, warmup, seed):
    """Warm up, time `steps` plain steps (the throughput figure), then rewind
    every sequence to where the timed region began and replay the same steps
    with per-kernel timing events (identical work: greedy decode is
    deterministic, which the replay checks)."""
    rng = np.random.default_rng(seed + lanes)
    kv = [int(v) for v in rng.integers(KV_LO, KV_HI + 1, lanes)]
    tokens = [int(v) for v in rng.integers(0, cfg["vocabulary"], lanes)]
    seqs = []
    for i in range(lanes):
        s = model.seq_alloc()
        model.seq_fill_synthetic(s, kv[i], seed, i)
        seqs.append(s)
    first = None
    seq_arr = np.asarray(seqs, np.uint32)

    def one_step(toks):
        status, argmax = model.step_decode(seq_arr, toks)
        if status.any():
            raise RuntimeError(f"lane failure {status.tolist()}")
        return argmax

    start_tokens = list(tokens)
    tokens = np.asarray(tokens, np.uint32)
    for _ in range(warmup):
        tokens = one_step(tokens)
        if first is None:
            first = tokens.tolist()
    if first is None:
        tokens = one_step(tokens)
        first = tokens.tolist()
    kv_at_timing = [model.seq_length(s) for s in seqs]
    timed_tokens = tokens.copy()
    trace = []
    t0 = time.perf_counter()
    for _ in range(steps):
        tokens = one_step(tokens)
        trace.append(tokens)
    elapsed = time.perf_counter() - t0
    # replay of the timed region with dispatch-packet timing events
    for s, n in zip(seqs, kv_at_timing):
        model.seq_truncate(s, n)
    tokens = timed_tokens
    model.profile(True)
    replay_equal = True
    tp = time.perf_counter()
    for i in range(steps):
        tokens = one_step(tokens)
        replay_equal &= bool(np.array_equal(tokens, trace[i]))
    prof_elapsed = time.perf_counter() - tp
    stats = model.profile_read()
    model.profile(False)
    log(f"[bench] {lanes} lanes: replay with timing events {prof_elapsed * 1e3 / steps:.3f} ms/step, "
        f"same tokens: {replay_equal}")
    mean_kv = [k + (steps - 1) / 2.0 for k in kv_at_timing]
    sb = step_bytes(cfg, mean_kv, model.matrix_bytes)
    for s in seqs:
        model.seq_free(s)
    return dict(kv=kv, start_tokens=start_tokens, first_argmax=first, elapsed=elapsed,
                stats=stats, step_bytes=sb, tok_s=lanes * steps / elapsed,
                ms_per_step=elapsed * 1e3 / steps, replay_equal=replay_equal,
                replay_ms_per_step=prof_elapsed * 1e3 / steps)


C4_GROUPS, C4_GROUP, C4_PREFIX, C4_CONTEXT = 8, 16, 256, 4096


def run_c4(seed, steps, warmup):
    """Q4_0 weights, 128 decode lanes in groups of 16 that
    share a 256-token prefix through forked page tables (full pages shared,
    copy on write), private suffixes up to context 4096, greedy decode.
    Algorithmic KV bytes count each group's prefix once per step."""
    path = model_file(seed, "q4_0")
    meta, tensors = gguf.read(path)
    cfg = gguf.qwen2_config(meta)
    lanes = C4_GROUPS * C4_GROUP
    model = cohx.Model(cfg, tensors, max_lanes=lanes, max_rows=lanes, max_seqs=lanes + C4_GROUPS,
                       max_context=C4_CONTEXT)
    rng = np.random.default_rng(seed + 4)
    hi = C4_CONTEXT - C4_PREFIX - warmup - steps - 8
    suffix = [int(v) for v in rng.integers(0, hi + 1, lanes)]
    seqs = []
    for g in range(C4_GROUPS):
        base = model.seq_alloc()
        model.seq_fill_synthetic(base, C4_PREFIX, seed, 1000 + g)
        for k in range(C4_GROUP):
            i = g * C4_GROUP + k
            s = model.seq_fork(base, C4_PREFIX)
            model.seq_fill_synthetic(s, C4_PREFIX + suffix[i], seed, i)
            seqs.append(s)
        model.seq_free(base)
    seq_arr = np.asarray(seqs, np.uint32)
    tokens = rng.integers(0, cfg["vocabulary"], lanes).astype(np.uint32)
    init_tokens, first_out = tokens.tolist(), None
    for _ in range(warmup):
        st, tokens = model.step_decode(seq_arr, tokens)
        assert not st.any()
        if first_out is None:
            first_out = tokens.tolist()
    kv0 = [model.seq_length(s) for s in seqs]
    start = tokens.copy()
    trace = []
    t0 = time.perf_counter()
    for _ in range(steps):
        st, tokens = model.step_decode(seq_arr, tokens)
        assert not st.any()
        trace.append(tokens)
    elapsed = time.perf_counter() - t0
    for s, n in zip(seqs, kv0):
        model.seq_truncate(s, n)
    model.profile(True)
    tokens, same = start, True
    for i in range(steps):
        st, tokens = model.step_decode(seq_arr, tokens)
        same &= bool(np.array_equal(tokens, trace[i]))
    stats = model.profile_read()
    model.profile(False)
    matrix_bytes = model.matrix_bytes
    del model
    L, kvd = cfg["layers"], cfg["kv_heads"] * cfg["head_dim"]
    per_tok = L * kvd * 4 * 2
    mean_private = sum(n - C4_PREFIX + 1 + (steps - 1) / 2.0 for n in kv0)
    unique_kv = (C4_GROUPS * C4_PREFIX + mean_private) * per_tok + lanes * per_tok
    sb = matrix_bytes + unique_kv + lanes * cfg["hidden"] // 32 * 18
    ms = elapsed * 1e3 / steps
    top = max(stats, key=lambda x: x["total_ms"])
    log(f"[bench] c4: {lanes * steps / elapsed:.0f} tok/s, {ms:.3f} ms/step, replay same tokens: {same}")
    return {"workload": "Qwen2.5-0.5B-shape Q4_0 decode, 128 lanes in 8 groups of 16 sharing a "
                        "256-token prefix (forked page tables), private suffixes, context <= 4096",
            "value": lanes * steps / elapsed, "unit": "tok/s", "ms_per_step": ms, "steps": steps,
            "step_roofline": {"bound": "hbm", "bytes_per_step": sb,
                              "note": "unique KV: each group's prefix counted once per step",
                              "achieved": sb / (ms / 1e3) / 1e9, "peak": HBM_PEAK / 1e9,
                              "unit": "GB/s", "frac": sb / (ms / 1e3) / HBM_PEAK},
            "dominant_kernel": {"kernel": top["name"],
                                "avg_launch_us": top["total_ms"] * 1e3 / top["launches"]},
            "replay_same_tokens": same,
            "_cpu": dict(cfg=cfg, tensors=tensors, init=init_tokens, first=first_out, seed=seed,
                         suffix=suffix)}


def c4_cpu_baseline(c, steps, threads):
    """The oracle on the first 16-lane group of the C4 workload (a 16-lane
    unit, batch.rs:65): the same Q4_0 weights, the group's shared 256-token
    prefix and private suffixes and the same first tokens as the GPU run;
    `steps` decode steps.  Also checks the first step's greedy ids against
    the GPU's first (warm-up) step."""
    import orc
    m = orc.Model(c["cfg"], c["tensors"], threads=threads)
    sess = []
    for i in range(C4_GROUP):
        s = m.session(C4_CONTEXT)
        s.fill_synthetic(C4_PREFIX, c["seed"], 1000)
        s.fill_synthetic(C4_PREFIX + c["suffix"][i], c["seed"], i)
        sess.append(s)
    toks = c["init"][:C4_GROUP]
    first = None
    t0 = time.perf_counter()
    for _ in range(steps):
        errs = m.forward_batch(sess, toks)
        assert not errs.any()
        toks = [int(orc.Sampler().sample(s.logits())[1]) for s in sess]
        if first is None:
            first = list(toks)
    el = time.perf_counter() - t0
    return {"value": C4_GROUP * steps / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle, the first group's {C4_GROUP} lanes (one unit), {steps} decode steps "
                      f"from the GPU run's initial state; {el:.1f}s",
            "greedy_equal_first_step": int(sum(a == b for a, b in zip(first, c["first"][:C4_GROUP]))),
            "host": host_info()}


C3_CHUNKS, C3_DECODE, C3_CONTEXT = 8, 56, 4608
MFMA_F16_PEAK = 2.5e15


def run_c3(seed, steps, warmup, dtype="f16"):
    """F16 weights; every step packs 8 prompt chunks of
    U[128,512] tokens (each sequence continuing its prompt) with 56 greedy
    decode rows over KV U[256,4096].  Linears of packed batches run on the
    matrix cores (f32 sums; tolerance-checked by the tests).  Reports packed
    rows/s and the linears' achieved TFLOP/s against the dense fp16 peak.
    dtype "q8_0": the same schedule on Q8_0 weights in the regime's quantized
    form (the weight tiles dequantized to binary16 in LDS, the activations
    rounded as the reference's Q8_0 operands and held as binary16, fp16 MFMA
    with f32 sums; chunk attention): the quantized prefill rate, the linears
    against the same fp16 peak."""
    path = model_file(seed, dtype)
    meta, tensors = gguf.read(path)
    cfg = gguf.qwen2_config(meta)
    n = C3_CHUNKS + C3_DECODE
    rng = np.random.default_rng(seed + 3)
    total = warmup + steps
    chunk_len = rng.integers(128, 513, (total, C3_CHUNKS))
    max_rows = int(chunk_len.sum(axis=1).max()) + C3_DECODE
    model = cohx.Model(cfg, tensors, max_lanes=n, max_rows=max_rows, max_seqs=n, max_context=C3_CONTEXT)
    pre = [model.seq_alloc() for _ in range(C3_CHUNKS)]
    dec = []
    kv = [int(v) for v in rng.integers(256, 4097 - total - 8, C3_DECODE)]
    for i, k in enumerate(kv):
        s = model.seq_alloc()
        model.seq_fill_synthetic(s, k, seed, 500 + i)
        dec.append(s)
    chunks = [[[int(v) for v in rng.integers(0, cfg["vocabulary"], chunk_len[t, j])]
               for j in range(C3_CHUNKS)] for t in range(total)]
    dec_tok = [int(v) for v in rng.integers(0, cfg["vocabulary"], C3_DECODE)]

    def one_step(t, toks):
        lanes = [dict(seq=s, tokens=chunks[t][j]) for j, s in enumerate(pre)]
        lanes += [dict(seq=s, tokens=[tk]) for s, tk in zip(dec, toks)]
        res = model.step(lanes)
        if any(r["status"] for r in res):
            raise RuntimeError(f"lane failure {[r['status'] for r in res]}")
        return [r["argmax"] for r in res[C3_CHUNKS:]]

    for t in range(warmup):
        dec_tok = one_step(t, dec_tok)
    lengths = [model.seq_length(s) for s in pre + dec]
    start, trace = list(dec_tok), []
    rows = int(sum(chunk_len[t].sum() for t in range(warmup, total))) + C3_DECODE * steps
    t0 = time.perf_counter()
    for t in range(warmup, total):
        dec_tok = one_step(t, dec_tok)
        trace.append(dec_tok)
    elapsed = time.perf_counter() - t0
    for s, k in zip(pre + dec, lengths):
        model.seq_truncate(s, k)
    model.profile(True)
    toks, same = start, True
    for i, t in enumerate(range(warmup, total)):
        toks = one_step(t, toks)
        same &= toks == trace[i]
    stats = model.profile_read()
    model.profile(False)
    del model
    lin = [x for x in stats if x["name"] in ("matvec_qkv", "matvec_o_residual", "matvec_gate_up_swiglu",
                                            "matvec_down_residual")]
    lin_flops = sum(x["flops"] for x in lin)
    lin_ms = sum(x["total_ms"] for x in lin)
    ms = elapsed * 1e3 / steps
    tflops = lin_flops / (lin_ms / 1e3) / 1e12 if lin_ms else 0.0
    log(f"[bench] c3 {dtype}: {rows / elapsed:.0f} packed rows/s, {ms:.2f} ms/step, linears "
        f"{tflops:.0f} TFLOP/s, replay same tokens: {same}")
    if dtype != "f16":
        return {"workload": f"Qwen2.5-0.5B-shape {dtype.upper()}, C3's schedule (8 prompt chunks U[128,512] + "
                            "56 decode rows over KV U[256,4096]) in the packed-prefill regime: Q8_0 tiles "
                            "dequantized to binary16 in LDS, Q8_0-rounded activations as binary16, fp16 MFMA "
                            "(f32 sums), chunk attention",
                "value": rows / elapsed, "unit": "packed rows/s", "ms_per_step": ms, "steps": steps,
                "mean_rows_per_step": rows / steps,
                "roofline": {"bound": "mfma", "kernel": "linears (k_gemm_q, fp16 MFMA)",
                             "achieved": tflops, "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                             "frac": tflops * 1e12 / MFMA_F16_PEAK},
                "kernels": {x["name"]: {"ms_per_step": x["total_ms"] / steps} for x in stats if x["launches"]},
                "replay_same_tokens": same}
    return {"workload": "Qwen2.5-0.5B-shape F16, each step 8 prompt chunks U[128,512] + 56 decode "
                        "rows over KV U[256,4096]; linears on the matrix cores (f32 sums)",
            "value": rows / elapsed, "unit": "packed rows/s", "ms_per_step": ms, "steps": steps,
            "mean_rows_per_step": rows / steps,
            "roofline": {"bound": "mfma", "kernel": "linears (k_gemm, the matrix-core GEMM of steps with prompt rows)",
                         "achieved": tflops, "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                         "frac": tflops * 1e12 / MFMA_F16_PEAK},
            "attention_chunk": chunk_roofline(stats, steps),
            "kernels": {x["name"]: {"ms_per_step": x["total_ms"] / steps} for x in stats if x["launches"]},
            "replay_same_tokens": same,
            "_cpu": dict(cfg=cfg, tensors=tensors, chunks=chunks[warmup], kv=kv, seed=seed)}


def chunk_roofline(stats, steps):
    """The prefill chunks' attention on the matrix cores: QK^T and PV flops of
    the chunk rows (4 * heads * head_dim per attended position) over its time,
    and the per-layer pass that converts the key tiles into its binary16
    operands."""
    x = next((x for x in stats if x["name"] == "attn_chunk_mfma" and x["launches"]), None)
    if not x:
        return None
    st = next((y for y in stats if y["name"] == "attn_chunk_stage" and y["launches"]), None)
    tf = x["flops"] / (x["total_ms"] / 1e3) / 1e12
    return {"bound": "mfma", "kernel": "k_attn_chunk", "achieved": tf, "peak": MFMA_F16_PEAK / 1e12,
            "unit": "TFLOP/s", "frac": tf * 1e12 / MFMA_F16_PEAK, "ms_per_step": x["total_ms"] / steps,
            "staging_ms_per_step": st["total_ms"] / steps if st else None,
            "note": "S = (K_hi + K_lo) Q^T takes two binary16 products per f32 product, O = V P one; "
                    "the peak is one product's"}


C3_CPU_TOKENS = 24


def c3_cpu_baseline(c, threads):
    """The oracle on a sample of one C3 step: the 8 chunk lanes' first
    C3_CPU_TOKENS prompt tokens (the engine forwards prompts one token per
    lane per step, docs/BATCHING.md:23, in 16-lane units) and one step of the
    56 decode lanes over their seeded KV (4 units), on the same F16 weights."""
    import orc
    m = orc.Model(c["cfg"], c["tensors"], threads=threads)
    pre = [m.session(C3_CONTEXT) for _ in range(C3_CHUNKS)]
    dec = []
    for i, k in enumerate(c["kv"]):
        s = m.session(C3_CONTEXT)
        s.fill_synthetic(k, c["seed"], 500 + i)
        dec.append(s)
    toks = [int(v) for v in np.random.default_rng(7).integers(0, c["cfg"]["vocabulary"], C3_DECODE)]
    t0 = time.perf_counter()
    for j in range(C3_CPU_TOKENS):
        errs = m.forward_batch(pre, [ch[j] for ch in c["chunks"]])
        assert not errs.any()
    for u in range(0, C3_DECODE, 16):
        errs = m.forward_batch(dec[u:u + 16], toks[u:u + 16])
        assert not errs.any()
    el = time.perf_counter() - t0
    rows = C3_CHUNKS * C3_CPU_TOKENS + C3_DECODE
    return {"value": rows / el, "unit": "packed rows/s", "cores": threads, "kind": "port",
            "sample": f"oracle, the first {C3_CPU_TOKENS} tokens of the 8 prompt chunks and one step of "
                      f"the 56 decode lanes ({rows} rows); {el:.1f}s", "host": host_info()}


def measured_traffic(category, lanes):
    """HBM bytes per launch of `category`'s kernel from the committed counter
    summary, or None when it does not cover this kernel and workload."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(CATEGORY_KERNEL.get(category, ""))
    if not k or t.get("lanes") != lanes:
        return None
    return k["hbm_bytes_per_launch"]


def roofline(stats, lanes):
    top = max(stats, key=lambda s: s["total_ms"])
    avg_s = top["total_ms"] / 1e3 / top["launches"]
    achieved = top["bytes"] / top["launches"] / avg_s
    return {"kernel": top["name"], "bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9,
            "unit": "GB/s", "frac": achieved / HBM_PEAK, "traffic": measured_traffic(top["name"], lanes),
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


def kernel_instance(name):
    import re
    m = re.search(r"\b(k_\w+)(<[^>]*>)?\(", name)
    if m:
        return m.group(1) + (m.group(2) or "")
    return name


def counter_means(path):
    """{kernel instance: mean counter value (KiB) per dispatch} of a
    rocprofv3 --pmc counter_collection.csv."""
    import csv
    acc = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            k = kernel_instance(row["Kernel_Name"])
            v = acc.setdefault(k, [0.0, 0])
            v[0] += float(row["Counter_Value"])
            v[1] += 1
    return {k: (v[0] / v[1], v[1]) for k, v in acc.items()}


def summarize_counters(fetch_csv, write_csv, copy_fetch_csv, copy_write_csv, lanes):
    """Scale FETCH_SIZE / WRITE_SIZE (KiB per dispatch) to bytes with the same
    counters read over a device copy of 1 GiB; write the traffic summary."""
    copy_bytes = float(1 << 30)
    cf = counter_means(copy_fetch_csv)["__amd_rocclr_copyBuffer"][0] * 1024
    cw = counter_means(copy_write_csv)["__amd_rocclr_copyBuffer"][0] * 1024
    ff, fw = copy_bytes / cf, copy_bytes / cw
    fetch, write = counter_means(fetch_csv), counter_means(write_csv)
    kernels = {}
    for k, (fk, n) in sorted(fetch.items()):
        wk = write.get(k, (0.0, 0))[0]
        kernels[k] = {"dispatches": n, "fetch_kib": fk, "write_kib": wk,
                      "hbm_bytes_per_launch": fk * 1024 * ff + wk * 1024 * fw}
    out = {"workload": "Qwen2.5-0.5B-shape Q8_0 decode, 128 ragged lanes, KV U[64,2048] f32",
           "lanes": lanes,
           "calibration": {"copy_bytes": copy_bytes, "fetch_counter_bytes": cf,
                           "write_counter_bytes": cw, "fetch_factor": ff, "write_factor": fw},
           "commands": {"fetch": PMC_CMD.format(counter="FETCH_SIZE"),
                        "write": PMC_CMD.format(counter="WRITE_SIZE"),
                        "copy_fetch": COPY_CMD.format(counter="FETCH_SIZE"),
                        "copy_write": COPY_CMD.format(counter="WRITE_SIZE")},
           "kernels": kernels}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


def summarize_trace(trace_csv, bench_json):
    """Markdown summary of a rocprofv3 --kernel-trace run of the default bench
    command: per kernel instance and grid shape (x tells the 32- and 128-lane
    workloads apart, z the KV depth of the attention passes, which separates
    the 128-lane decode from the longer-context workloads) the dispatch count
    and mean duration, next to the dispatch-event means of a plain run of the
    same command on the same machine (under the tracer those events also time
    the tracer's work)."""
    import csv
    groups = {}
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            k = (kernel_instance(row["Kernel_Name"]),
                 f'{row["Grid_Size_X"]}x{row["Grid_Size_Y"]}x{row["Grid_Size_Z"]}')
            g = groups.setdefault(k, [])
            g.append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    with open(bench_json) as f:
        line = json.loads(f.read().strip().splitlines()[-1])
    print(f"Command: `{TRACE_CMD}`\n")
    print(f"Plain run of the same command: {line['value']:.0f} tok/s, {line['ms_per_step']:.3f} ms/step; "
          f"dominant kernel {line['roofline']['kernel']} {line['roofline']['avg_launch_us']:.2f} us "
          f"per launch (dispatch events over the replayed timed region).\n")
    print("Plain-run dispatch-event means, 128 lanes (us per launch):\n")
    for name, v in line["kernels"].items():
        print(f"- {name}: {v['ms_per_step'] * 1e3 / v['launches_per_step']:.2f}")
    print("\n| kernel | grid (threads) | dispatches | mean us | min us | max us | total ms |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for (name, gx), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        if sum(d) < 1000:
            continue
        print(f"| {name} | {gx} | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} | "
              f"{sum(d) / 1e3:.2f} |")


C5_TRACE_CMD = ("rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o <name> -- "
                "python3 bench.py --c5-only --no-cpu-baseline")
C5_PMC_CMD = ("rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_BF16 "
              "GRBM_GUI_ACTIVE --kernel-include-regex \"k_gemm\" --output-format csv -d <dir> -o <name> -- "
              "python3 bench.py --c5-only --no-cpu-baseline")


def summarize_c5_trace(trace_csv, bench_json, mfma_csv=None):
    """Markdown summary of a rocprofv3 --kernel-trace run of the C5 workload:
    per kernel and grid shape (the grid's y extent counts row groups, so the
    one-token schedule's 16-row steps separate from the prompt chunks) the
    dispatch count and mean duration, and the per-step time of the 16-row
    decode steps by kernel."""
    import csv
    groups = {}
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            k = (kernel_instance(row["Kernel_Name"]),
                 f'{row["Grid_Size_X"]}x{row["Grid_Size_Y"]}x{row["Grid_Size_Z"]}')
            groups.setdefault(k, []).append(
                (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    with open(bench_json) as f:
        line = json.loads(f.read().strip().splitlines()[-1])
    es = line["engine_schedule"]
    print(f"Command: `{C5_TRACE_CMD}`\n")
    ex = line["chunked_exact"]
    print(f"Plain run of the same command: prompts in chunks of {line['prompt_chunk']} (packed-prefill "
          f"regime): {line['value']:.0f} generated tok/s ({line['rows_per_s']:.0f} rows/s); the same "
          f"schedule exact: {ex['value']:.0f} generated tok/s; one token per sequence per step: "
          f"{es['ms_per_step']:.3f} ms/step ({es['rows_per_s']:.0f} rows/s); same tokens in the exact "
          f"schedules: {line['same_tokens_both_exact_schedules']}, regime against exact: "
          f"{line['regime_same_tokens_as_exact']}.\n")
    print("| kernel | grid (threads) | dispatches | mean us | min us | max us | total ms |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for (name, gx), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:30]:
        print(f"| {name} | {gx} | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} | "
              f"{sum(d) / 1e3:.2f} |")
    print("\nThe 30 largest (kernel, grid) groups by total time, over the three runs.  Grid y of the\n"
          "matvec kernels counts row groups: `k_q35_mvpc` 36864x4 and `k_q35_mvd` 131584x1 / 114688x1\n"
          "are the 16-row steps of the one-token schedule (o/out/down projections; mix; gate+up with SwiGLU, `k_q35_mvd<3, ...>`),\n"
          "`k_q35_mvd<2, ...>` is the LM head with its argmax, and `k_q35_mv` with grid y in the hundreds\n"
          "are the 256-token prompt chunks (up to 4096 rows) of the exact run; `k_gemm<1, true, ...>` is\n"
          "the regime's matrix-core GEMM over hi/lo operands, `k_q35_split` their split.\n\n"
          f"Summary: `python bench.py --summarize-c5-trace <dir>/<name>_kernel_trace.csv <bench stdout> "
          f"[<mfma counter_collection.csv>]`")
    if mfma_csv:
        print_mfma_table(mfma_csv, C5_PMC_CMD)


LEG_TRACE_CMD = ("COHX_GRAPHS=0 rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o <name> -- "
                 "python3 bench.py --only {leg}")
LEG_PMC_CMD = ("COHX_GRAPHS=0 rocprofv3 --pmc {counters} --kernel-include-regex \"{regex}\" --output-format csv "
               "-d <dir> -o <name> -- python3 bench.py --only {leg}")
MFMA_COUNTERS = "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_MOPS_BF16 GRBM_GUI_ACTIVE"
MI355X_CUS = 256


def print_mfma_table(mfma_csv, cmd):
    """Per matrix-core kernel instance: dispatches, MFMA busy share
    (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 256 CUs)), the MOPS
    counters (units of 512 flops) and the counted TFLOP/s over the dispatches'
    own durations."""
    import csv
    acc = {}
    with open(mfma_csv) as f:
        for row in csv.DictReader(f):
            k = kernel_instance(row["Kernel_Name"])
            a = acc.setdefault(k, {"_d": set(), "_ns": 0.0})
            a[row["Counter_Name"]] = a.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
            if row["Dispatch_Id"] not in a["_d"]:
                a["_d"].add(row["Dispatch_Id"])
                a["_ns"] += int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    print(f"\nMatrix cores: `{cmd}`\n")
    print("| kernel | dispatches | MFMA busy share | MOPS f16 (x512 flop) | MOPS bf16 (x512 flop) | "
          "counted TFLOP/s |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, a in sorted(acc.items()):
        busy = a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / max(a.get("GRBM_GUI_ACTIVE", 1.0) * MI355X_CUS, 1.0)
        mops = a.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) + a.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        tf = mops * 512 / (a["_ns"] * 1e-9) / 1e12 if a["_ns"] else 0.0
        print(f"| {k} | {len(a['_d'])} | {busy:.3f} | {a.get('SQ_INSTS_VALU_MFMA_MOPS_F16', 0.0):.3g} | "
              f"{a.get('SQ_INSTS_VALU_MFMA_MOPS_BF16', 0.0):.3g} | {tf:.0f} |")
    print("\nThe counted rate covers every MFMA issued (the chunk attention's two binary16 products for "
          "each score, the Qwen3.5 regime's hi and lo GEMMs); the bench's TFLOP/s count the "
          "algorithmic flops once.")


def summarize_leg(leg, trace_csv, bench_json, fetch_csv=None, write_csv=None, mfma_csv=None,
                  copy_fetch_csv=None, copy_write_csv=None):
    """Markdown summary of the rocprofv3 runs of one workload (`bench.py
    --only <leg>`): per kernel instance and grid the dispatch count and mean
    duration (kernel trace); HBM bytes per dispatch from FETCH_SIZE /
    WRITE_SIZE scaled by the same counters over a 1 GiB copy; for the matrix-
    core kernels the MFMA counters (SQ_INSTS_VALU_MFMA_MOPS_* count units of
    512 flops; busy share = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x
    256 CUs))."""
    import csv
    groups = {}
    with open(trace_csv) as f:
        for row in csv.DictReader(f):
            k = (kernel_instance(row["Kernel_Name"]),
                 f'{row["Grid_Size_X"]}x{row["Grid_Size_Y"]}x{row["Grid_Size_Z"]}')
            groups.setdefault(k, []).append((int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1e3)
    with open(bench_json) as f:
        line = json.loads(f.read().strip().splitlines()[-1])
    print(f"# {leg.upper()}: kernel trace and counters\n")
    print(f"Workload: {line['workload']}.\n")
    print(f"Plain run (`python3 bench.py --only {leg}`): {line['value']:.0f} {line['unit']}, "
          f"{line['ms_per_step']:.3f} ms/step.\n")
    print(f"Kernel trace: `{LEG_TRACE_CMD.format(leg=leg)}`\n")
    print("| kernel | grid (threads) | dispatches | mean us | min us | max us | total ms |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for (name, gx), d in sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:25]:
        print(f"| {name} | {gx} | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} | "
              f"{sum(d) / 1e3:.2f} |")
    if fetch_csv and write_csv and copy_fetch_csv and copy_write_csv:
        cf = counter_means(copy_fetch_csv)["__amd_rocclr_copyBuffer"][0] * 1024
        cw = counter_means(copy_write_csv)["__amd_rocclr_copyBuffer"][0] * 1024
        ff, fw = float(1 << 30) / cf, float(1 << 30) / cw
        fetch, write = counter_means(fetch_csv), counter_means(write_csv)
        print(f"\nHBM traffic: `{LEG_PMC_CMD.format(counters='FETCH_SIZE', regex='k_', leg=leg)}`, then "
              f"`WRITE_SIZE`; scaled by the same counters over a 1 GiB copy (`{COPY_CMD.format(counter='FETCH_SIZE')}`: "
              f"factors {ff:.4f} fetch, {fw:.4f} write).\n")
        print("| kernel | dispatches | FETCH KiB | WRITE KiB | HBM bytes per launch |")
        print("|---|---:|---:|---:|---:|")
        for k, (fk, n) in sorted(fetch.items(), key=lambda kv: -kv[1][0]):
            wk = write.get(k, (0.0, 0))[0]
            print(f"| {k} | {n} | {fk:.0f} | {wk:.0f} | {(fk * ff + wk * fw) * 1024 / 1e6:.2f} MB |")
    if mfma_csv:
        print_mfma_table(mfma_csv, LEG_PMC_CMD.format(counters=MFMA_COUNTERS, regex='k_gemm|k_attn_chunk',
                                                      leg=leg))
    print(f"\nSummary: `python3 bench.py --summarize-leg {leg} <trace.csv> <bench stdout> [<fetch.csv> "
          f"<write.csv> <mfma.csv or -> <copy_fetch.csv> <copy_write.csv>]`")


def copy_probe():
    """A plain device copy of known size, for scaling the FETCH_SIZE and
    WRITE_SIZE counters to bytes (the tensors are plumbing, not the product)."""
    import torch
    n = 1 << 28  # 2^28 floats = 1 GiB
    src = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "copies": 4}),
          flush=True)


def read_probe():
    """The HBM read rate this device reaches with a plain streaming kernel
    (libcohx_probe.so): 1 GiB and 4 GiB buffers (past the 256 MB last-level
    cache) read with float4 loads by grids of 1024 to 8192 workgroups."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "coheryn-ai-studio_amd", "libcohx_probe.so"))
    lib.cohx_probe_read.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_float)]
    out = []
    for mib in (1024, 4096):
        for blocks in (1024, 2048, 4096, 8192):
            ms = ctypes.c_float()
            rc = lib.cohx_probe_read(mib, blocks, 10, ctypes.byref(ms))
            if rc:
                raise RuntimeError(f"probe failed ({rc})")
            out.append({"mib": mib, "workgroups": blocks, "ms": ms.value,
                        "read_TBps": (mib << 20) / (ms.value * 1e-3) / 1e12})
    print(json.dumps({"read_probe": out, "best_read_TBps": max(o["read_TBps"] for o in out)}), flush=True)


def mfma_probe():
    """The f16 matrix-core rate (libcohx_probe.so, k_probe_mfma): workgroups of
    4 waves, each wave 8 independent 16x16x32 MFMA chains on registers."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "coheryn-ai-studio_amd", "libcohx_probe.so"))
    lib.cohx_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    out = []
    for blocks in (1024, 2048, 4096):
        ms = ctypes.c_float()
        if lib.cohx_probe_mfma(blocks, 256, ctypes.byref(ms)):
            raise RuntimeError("probe failed")
        flops = blocks * 4 * 8 * 256 * 16384
        out.append({"workgroups": blocks, "ms": ms.value, "TFLOPs": flops / (ms.value * 1e-3) / 1e12})
    print(json.dumps({"mfma_probe": out}), flush=True)


def measured_peaks():
    """The rates this device reaches, measured in the same run (libcohx_probe.so):
    a plain streaming read of 1 GiB (`--read-probe`) and back-to-back f16
    MFMAs (`--mfma-probe`); None when the probe library is absent."""
    import ctypes
    try:
        lib = ctypes.CDLL(os.path.join(ROOT, "coheryn-ai-studio_amd", "libcohx_probe.so"))
    except OSError:
        return None
    lib.cohx_probe_read.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_float)]
    lib.cohx_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    rd, mf = ctypes.c_float(), ctypes.c_float()
    if lib.cohx_probe_read(1024, 1024, 5, ctypes.byref(rd)) or lib.cohx_probe_mfma(2048, 256, ctypes.byref(mf)):
        return None
    return {"hbm_read_GBps": (1 << 30) / (rd.value * 1e-3) / 1e9,
            "mfma_f16_TFLOPs": 2048 * 4 * 8 * 256 * 16384 / (mf.value * 1e-3) / 1e12,
            "note": "streaming read of 1 GiB (float4 loads, 1024 workgroups) and back-to-back "
                    "v_mfma_f32_16x16x32_f16 (2048 workgroups); the roofline fractions use the published peaks"}


C5_SEQS, C5_PROMPT, C5_GEN, C5_CHUNK = 16, (64, 1024), 64, 256


def c5_generate(model, prompts, chunk, head_every_row=False):
    """Continuous batching of the hybrid graph (qwen35/generation.rs:335-406):
    every step gives each unfinished sequence its next `chunk` prompt tokens
    (prompt rows that do not end the prompt skip the head, generation.rs:368)
    or its last greedy token; the step on a prompt's last row yields the first
    greedy token, and a sequence stops after C5_GEN tokens.  chunk=1 is the
    engine's own schedule (one token per state per step_batch call)."""
    seqs = [model.seq_alloc() for _ in prompts]
    cursor = [0] * len(prompts)
    out = [[] for _ in prompts]
    steps = rows = 0
    while any(len(o) < C5_GEN for o in out):
        lanes, idx = [], []
        for i, p in enumerate(prompts):
            if len(out[i]) >= C5_GEN:
                continue
            if cursor[i] < len(p):
                toks = p[cursor[i]:cursor[i] + chunk]
                ends = cursor[i] + len(toks) == len(p)
                lanes.append(dict(seq=seqs[i], tokens=toks,
                                  skip_head=not ends and not head_every_row))
            else:
                toks = [out[i][-1]]
                lanes.append(dict(seq=seqs[i], tokens=toks))
            idx.append((i, len(toks)))
        res = model.step(lanes)
        for (i, n), r in zip(idx, res):
            if r["status"]:
                raise RuntimeError(f"c5 lane {i} failed with status {r['status']}")
            if cursor[i] < len(prompts[i]):
                cursor[i] += n
                if cursor[i] == len(prompts[i]):
                    out[i].append(int(r["argmax"]))
            else:
                out[i].append(int(r["argmax"]))
        steps += 1
        rows += sum(n for _, n in idx)
    for s in seqs:
        model.seq_free(s)
    return out, steps, rows


def run_c5(seed, cpu_steps, threads, with_cpu=True):
    """the Qwen3.5-0.8B hybrid shape (bf16 N(0,0.02)
    weights), 16 sequences with prompts U[64,1024] of random ids, 64 greedy
    tokens each.  Timed from fresh sequences: with prompts in chunks of
    C5_CHUNK rows per lane per step (steps of 128+ rows in the packed-prefill
    regime, the default: linears on the matrix-core BF16 GEMM with f32 sums, within
    the stated tolerance), the same schedule with the regime off (exact, bit
    for bit against the oracle), and the engine's one-token-per-step schedule
    (exact).  The two exact runs must generate the same tokens; the regime's
    agreement is reported.  The CPU baseline steps the oracle over the first
    prompt tokens of all 16 sequences (one token per sequence per step)."""
    import synth35
    t0 = time.perf_counter()
    cfg, tensors = synth35.in_memory(synth35.config(), seed=seed + 5)
    log(f"[bench] c5: synthetic Qwen3.5-0.8B weights in {time.perf_counter() - t0:.1f}s")
    rng = np.random.default_rng(seed + 5)
    plen = [int(v) for v in rng.integers(C5_PROMPT[0], C5_PROMPT[1] + 1, C5_SEQS)]
    prompts = [[int(v) for v in rng.integers(0, cfg["vocabulary"], n)] for n in plen]
    ctx = C5_PROMPT[1] + C5_GEN + 8

    def make(regime):
        old = os.environ.get("COHX_PREFILL_MFMA")
        os.environ["COHX_PREFILL_MFMA"] = "1" if regime else "0"
        try:
            return cohx.Qwen35(cfg, tensors, max_lanes=C5_SEQS, max_rows=C5_SEQS * C5_CHUNK,
                               max_seqs=C5_SEQS, max_context=ctx)
        finally:
            if old is None:
                os.environ.pop("COHX_PREFILL_MFMA", None)
            else:
                os.environ["COHX_PREFILL_MFMA"] = old

    res = {}
    for regime, runs in ((True, (("chunked", C5_CHUNK),)),
                         (False, (("chunked_exact", C5_CHUNK), ("engine_schedule", 1)))):
        model = make(regime)
        c5_generate(model, [p[:C5_CHUNK + 3] for p in prompts[:4]], C5_CHUNK)  # warm-up
        for name, chunk in runs:
            t0 = time.perf_counter()
            toks, steps, rows = c5_generate(model, prompts, chunk)
            el = time.perf_counter() - t0
            res[name] = dict(tokens=toks, steps=steps, rows=rows, elapsed=el)
            log(f"[bench] c5 {name}: {C5_SEQS * C5_GEN / el:.0f} generated tok/s, {rows / el:.0f} rows/s, "
                f"{steps} steps, {el:.2f}s")
        matrix_bytes = model.matrix_bytes
        del model
    ch, ex, es = res["chunked"], res["chunked_exact"], res["engine_schedule"]
    line = {"workload": f"Qwen3.5-0.8B-shape hybrid (bf16 weights, f32 state), {C5_SEQS} sequences, "
                        f"prompts U[{C5_PROMPT[0]},{C5_PROMPT[1]}], {C5_GEN} greedy tokens each; prompt "
                        f"steps of 128+ rows in the packed-prefill regime (matrix-core BF16 GEMM, f32 sums)",
            "value": C5_SEQS * C5_GEN / ch["elapsed"], "unit": "generated tok/s (whole job)",
            "rows_per_s": ch["rows"] / ch["elapsed"], "elapsed_s": ch["elapsed"],
            "steps": ch["steps"], "prompt_chunk": C5_CHUNK, "prompt_rows": sum(plen),
            "matrix_bytes": matrix_bytes,
            "chunked_exact": {"value": C5_SEQS * C5_GEN / ex["elapsed"], "rows_per_s": ex["rows"] / ex["elapsed"],
                              "elapsed_s": ex["elapsed"], "steps": ex["steps"]},
            "engine_schedule": {"value": C5_SEQS * C5_GEN / es["elapsed"],
                                "rows_per_s": es["rows"] / es["elapsed"], "steps": es["steps"],
                                "ms_per_step": es["elapsed"] * 1e3 / es["steps"],
                                "elapsed_s": es["elapsed"]},
            "same_tokens_both_exact_schedules": ex["tokens"] == es["tokens"],
            "regime_same_tokens_as_exact": ch["tokens"] == ex["tokens"],
            "regime_tokens_differing": sum(a != b for x, y in zip(ch["tokens"], ex["tokens"])
                                           for a, b in zip(x, y)),
            "seed": seed + 5}
    # one-token schedule: each step reads every weight once and each
    # sequence's recurrent state (conv ring and delta memory, read and written)
    lin = sum(1 for f in cfg["full"] if not f)
    conv_ch = 2 * cfg["key_heads"] * cfg["key_dim"] + cfg["value_heads"] * cfg["value_dim"]
    state = lin * (cfg["value_heads"] * cfg["key_dim"] * cfg["value_dim"] + conv_ch * cfg["conv_kernel"]) * 4 * 2
    sb = matrix_bytes + C5_SEQS * state
    es_s = es["elapsed"] / es["steps"]
    line["engine_schedule"]["step_roofline"] = {
        "bound": "hbm", "bytes_per_step": sb, "achieved": sb / es_s / 1e9, "peak": HBM_PEAK / 1e9,
        "unit": "GB/s", "frac": sb / es_s / HBM_PEAK,
        "note": "weights once plus each sequence's delta memory read and written; the exact step is "
                "bound by one wave's issue rate on its f64 chains, not by HBM"}
    if with_cpu:
        import orc
        m = orc.Qwen35Model(cfg, tensors, threads=threads)
        sess = [m.session(ctx) for _ in prompts]
        t0 = time.perf_counter()
        for j in range(cpu_steps):
            errs = m.forward_batch(sess, [p[j] for p in prompts], logits=[0] * C5_SEQS)
            assert not errs.any()
        el = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": C5_SEQS * cpu_steps / el, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"oracle, the first {cpu_steps} prompt tokens of all {C5_SEQS} sequences, "
                      f"one token per sequence per step, no head (prompt rows); {el:.1f}s",
            "gpu_engine_schedule_rows_per_s": es["rows"] / es["elapsed"], "host": host_info()}
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--lanes", type=int, default=128)
    ap.add_argument("--secondary-lanes", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-c4", action="store_true", help="skip the Q4_0 shared-prefix workload")
    ap.add_argument("--no-c3", action="store_true", help="skip the F16 packed-prefill workload")
    ap.add_argument("--no-c5", action="store_true", help="skip the Qwen3.5 hybrid workload")
    ap.add_argument("--c5-only", action="store_true",
                    help="run only the Qwen3.5 hybrid workload and print its JSON")
    ap.add_argument("--only", choices=["c3", "c3q8", "c4", "c5"],
                    help="run only this workload and print its JSON (profiling runs)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 1 GiB device-to-device 4 times (counter calibration)")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="only time back-to-back f16 MFMAs (the reachable matrix-core rate)")
    ap.add_argument("--read-probe", action="store_true",
                    help="only time a plain streaming read of 1 and 4 GiB (the reachable HBM read rate)")
    ap.add_argument("--summarize-counters", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="write the traffic summary from rocprofv3 --pmc csv files (no GPU)")
    ap.add_argument("--summarize-c5-trace", nargs="+", metavar="ARG",
                    help="KERNEL_TRACE_CSV BENCH_JSON [MFMA_CSV]: markdown summary of the rocprofv3 runs "
                         "of --c5-only")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("KERNEL_TRACE_CSV", "BENCH_JSON"),
                    help="print a markdown summary of a rocprofv3 --kernel-trace run (no GPU)")
    ap.add_argument("--summarize-leg", nargs="+", metavar="ARG",
                    help="LEG TRACE_CSV BENCH_JSON [FETCH WRITE MFMA COPY_FETCH COPY_WRITE]: markdown "
                         "summary of the rocprofv3 runs of `--only LEG` (no GPU)")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe()
        return
    if args.read_probe:
        read_probe()
        return
    if args.mfma_probe:
        mfma_probe()
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters, lanes=args.lanes)
        return
    if args.summarize_c5_trace:
        summarize_c5_trace(*args.summarize_c5_trace)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.summarize_leg:
        a = [None if x == "-" else x for x in args.summarize_leg] + [None] * (8 - len(args.summarize_leg))
        summarize_leg(a[0], a[1], a[2], fetch_csv=a[3], write_csv=a[4], mfma_csv=a[5], copy_fetch_csv=a[6],
                      copy_write_csv=a[7])
        return
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(the step shards by sequence with no collectives; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    threads = min(16, host_info()["usable_cpus"] or 1)
    if args.c5_only or args.only == "c5":
        print(json.dumps(run_c5(args.seed, args.cpu_steps // 2, threads,
                                with_cpu=not args.no_cpu_baseline)), flush=True)
        return
    if args.only == "c4":
        r = run_c4(args.seed, 128, args.warmup)
        r.pop("_cpu")
        print(json.dumps(r), flush=True)
        return
    if args.only == "c3":
        r = run_c3(args.seed, 8, 2)
        r.pop("_cpu")
        print(json.dumps(r), flush=True)
        return
    if args.only == "c3q8":
        print(json.dumps(run_c3(args.seed, 8, 2, "q8_0")), flush=True)
        return
    path = model_file(args.seed)
    meta, tensors = gguf.read(path)
    cfg = gguf.qwen2_config(meta)
    ctx_len = KV_HI + args.warmup + args.steps + 16
    log(f"[bench] uploading model (max_lanes={args.lanes}, max_context={ctx_len})")
    model = cohx.Model(cfg, tensors, max_lanes=args.lanes, max_rows=args.lanes,
                       max_seqs=args.lanes, max_context=ctx_len)
    results = {}
    for lanes in ([args.secondary_lanes] if args.secondary_lanes else []) + [args.lanes]:
        log(f"[bench] {lanes} lanes: warmup {args.warmup}, timed {args.steps}")
        results[lanes] = run_workload(model, cfg, lanes, args.steps, args.warmup, args.seed)
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
        "roofline": roofline(main_r["stats"], args.lanes),
        "step_roofline": {"bound": "hbm", "bytes_per_step": main_r["step_bytes"],
                          "achieved": main_r["step_bytes"] / (main_r["ms_per_step"] / 1e3) / 1e9,
                          "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                          "frac": main_r["step_bytes"] / (main_r["ms_per_step"] / 1e3) / HBM_PEAK},
        "timing_replay": {"ms_per_step": main_r["replay_ms_per_step"], "same_tokens": main_r["replay_equal"],
                          "note": "timed steps replayed from the same KV lengths with per-kernel "
                                  "dispatch-packet events; roofline and kernels come from it"},
        "kernels": {s["name"]: {"ms_per_step": s["total_ms"] / args.steps,
                                "launches_per_step": s["launches"] / args.steps,
                                "GB_s": (s["bytes"] / (s["total_ms"] / 1e3) / 1e9) if s["total_ms"] else 0}
                    for s in main_r["stats"] if s["launches"]},
    }
    sec = results.get(args.secondary_lanes)
    line["secondary"] = None if sec is None else {
        "lanes": args.secondary_lanes, "value": sec["tok_s"], "unit": "tok/s",
        "ms_per_step": sec["ms_per_step"],
        "step_frac": sec["step_bytes"] / (sec["ms_per_step"] / 1e3) / HBM_PEAK,
        "roofline": roofline(sec["stats"], args.secondary_lanes)}
    peaks = measured_peaks()
    line["measured_peaks"] = peaks
    if peaks:
        line["roofline"]["frac_of_measured_read"] = line["roofline"]["achieved"] / peaks["hbm_read_GBps"]
    if not args.no_c4:
        del model
        line["c4"] = run_c4(args.seed, 128, args.warmup)
        c4c = line["c4"].pop("_cpu")
        if not args.no_cpu_baseline:
            log(f"[bench] c4 cpu baseline: oracle, {C4_GROUP} lanes x 8 steps, {threads} threads")
            line["c4"]["cpu_baseline"] = c4_cpu_baseline(c4c, 8, threads)
        del c4c
    if not args.no_c3:
        line["c3"] = run_c3(args.seed, 8, 2)
        if peaks:
            line["c3"]["roofline"]["frac_of_measured_mfma"] = (line["c3"]["roofline"]["achieved"] /
                                                               peaks["mfma_f16_TFLOPs"])
        c3c = line["c3"].pop("_cpu")
        if not args.no_cpu_baseline:
            log(f"[bench] c3 cpu baseline: oracle, {threads} threads")
            line["c3"]["cpu_baseline"] = c3_cpu_baseline(c3c, threads)
        del c3c
        line["c3_q8_0"] = run_c3(args.seed, 8, 2, "q8_0")
    if not args.no_c5:
        line["c5"] = run_c5(args.seed, args.cpu_steps // 2, threads, with_cpu=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        n_cpu = min(16, args.lanes)
        log(f"[bench] cpu baseline: oracle, {n_cpu} lanes x {args.cpu_steps} steps, {threads} threads")
        first, tps, el = cpu_baseline(cfg, tensors, main_r["kv"], main_r["start_tokens"], args.seed,
                                      n_cpu, args.cpu_steps, threads)
        log(f"[bench] cpu baseline: oracle, {n_cpu} lanes x 2 steps, 1 thread")
        _, tps1, el1 = cpu_baseline(cfg, tensors, main_r["kv"], main_r["start_tokens"], args.seed,
                                    n_cpu, 2, 1)
        line["cpu_baseline"] = {
            "value": tps, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"first {n_cpu} of the {args.lanes} lanes (one 16-lane unit, batch.rs:65), "
                      f"{args.cpu_steps} decode steps, same weights/KV/tokens; {el:.1f}s",
            "threads_1": {"value": tps1, "unit": "tok/s", "cores": 1,
                          "sample": f"the same lanes, 2 decode steps on one thread; {el1:.1f}s"},
            "host": host_info()}
        gpu_first = main_r["first_argmax"][:n_cpu]
        line["parity"] = {"lanes": n_cpu, "greedy_equal": int(sum(a == b for a, b in zip(first, gpu_first))),
                          "check": "first-step greedy token, GPU vs CPU oracle, same inputs"}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
