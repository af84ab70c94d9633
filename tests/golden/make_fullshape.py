#!/usr/bin/env python3
"""Writes the full-shape oracle fixtures tests/golden/fullshape_<case>.json.

Runs the CPU oracle (oracle/liborc.so, the C restatement of the engine's
forward step) over the BASELINE.json workloads at their stated sizes, as
tests/fullshape_cases.py specifies them, and records per lane the SHA-256 of
the float32 logits, the greedy id, the top-2 values and the SHA-256 of the
K/V rows each step appends.  tests/test_gpu_baseline_shapes.py runs the same
inputs through the HIP library and compares.

    python tests/golden/make_fullshape.py [case ...]   # c2_32 c2_128 c4 c1 c3 c5 q4km_32

The oracle runs on this machine's cores (minutes per case; C5 the longest).
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "coheryn-ai-studio_amd"),
                os.path.join(ROOT, "oracle")]

import numpy as np  # noqa: E402

import fullshape_cases as fc  # noqa: E402
import orc  # noqa: E402
import synth  # noqa: E402

THREADS = min(16, os.cpu_count() or 1)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rows_digest(sess, layers, first, count):
    return fc.kv_rows_digest([(sess.kv(l, False)[first:first + count],
                               sess.kv(l, True)[first:first + count]) for l in layers])


def decode_steps(o, sess, tokens, steps):
    out, toks = [], list(tokens)
    for step in range(steps):
        t0 = time.time()
        errs = o.forward_batch(sess, toks)
        assert not errs.any(), errs
        sums = [fc.summary(s.logits()) for s in sess]
        out.append(sums)
        toks = [x["argmax"] for x in sums]
        log(f"  step {step}: {len(sess)} lanes in {time.time() - t0:.1f}s")
    return out


def run_c2(lanes, spec=None):
    spec = spec or fc.c2(lanes)
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    o = orc.Model(c, t, threads=THREADS)
    sess = []
    for i, n in enumerate(spec["kv"]):
        s = o.session(spec["context"])
        assert s.fill_synthetic(n, spec["fill_seed"], i) == 0
        sess.append(s)
    steps = decode_steps(o, sess, spec["tokens"], spec["steps"])
    kv = [rows_digest(s, spec["kv_check_layers"], n, spec["steps"]) for s, n in zip(sess, spec["kv"])]
    return spec, {"steps": steps, "kv_appended": kv}


def run_c4():
    spec = fc.c4()
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    o = orc.Model(c, t, threads=THREADS)
    sess, starts = [], []
    for g in range(spec["groups"]):
        for k in range(spec["group"]):
            i = g * spec["group"] + k
            s = o.session(spec["context"])
            assert s.fill_synthetic(spec["prefix"], spec["fill_seed"], 1000 + g) == 0
            assert s.fill_synthetic(spec["prefix"] + spec["suffix"][i], spec["fill_seed"], i) == 0
            sess.append(s)
            starts.append(spec["prefix"] + spec["suffix"][i])
    steps = decode_steps(o, sess, spec["tokens"], spec["steps"])
    kv = [rows_digest(s, spec["kv_check_layers"], n, spec["steps"]) for s, n in zip(sess, starts)]
    return spec, {"steps": steps, "kv_appended": kv}


def run_c1():
    """Each lane alone (batched == individual holds for the oracle): prompt
    tokens one per forward, then greedy tokens until max_tokens or an
    end-of-generation id (the state machine of generation.rs:279-394)."""
    spec = fc.c1()
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    o = orc.Model(c, t, threads=THREADS)
    eog = {c["eos_token_id"]} if c.get("eos_token_id") is not None else set()
    lanes = []
    for p in spec["prompts"]:
        s = o.session(spec["context"])
        for tok in p:
            assert o.forward_batch([s], [tok])[0] == 0
        ids, sums = [], []
        while True:
            sm = fc.summary(s.logits())
            sums.append(sm)
            ids.append(sm["argmax"])
            if sm["argmax"] in eog or len(ids) == spec["max_tokens"]:
                break
            assert o.forward_batch([s], [sm["argmax"]])[0] == 0
        lanes.append({"ids": ids, "samples": sums})
        log(f"  c1 prompt {len(p)}: {ids}")
    return spec, {"lanes": lanes}


def run_c3():
    spec = fc.c3()
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    o = orc.Model(c, t, threads=THREADS)
    chunk_sess = []
    for i, n in enumerate(spec["prefix"]):
        s = o.session(spec["context"])
        assert s.fill_synthetic(n, spec["fill_seed"], i) == 0
        chunk_sess.append(s)
    width = max(len(ch) for ch in spec["chunks"])
    t0 = time.time()
    for j in range(width):
        live = [(s, ch[j]) for s, ch in zip(chunk_sess, spec["chunks"]) if j < len(ch)]
        errs = o.forward_batch([s for s, _ in live], [tok for _, tok in live])
        assert not errs.any()
        if j % 64 == 0:
            log(f"  c3 chunk row {j}/{width} ({time.time() - t0:.0f}s)")
    dec_sess = []
    for i, n in enumerate(spec["kv"]):
        s = o.session(spec["context"])
        assert s.fill_synthetic(n, spec["fill_seed"], 100 + i) == 0
        dec_sess.append(s)
    errs = o.forward_batch(dec_sess, spec["tokens"])
    assert not errs.any()
    layers = spec["kv_check_layers"]
    chunk = [{"summary": fc.summary(s.logits()),
              "kv_appended": rows_digest(s, layers, n, len(ch))}
             for s, n, ch in zip(chunk_sess, spec["prefix"], spec["chunks"])]
    dec = [{"summary": fc.summary(s.logits()), "kv_appended": rows_digest(s, layers, n, 1)}
           for s, n in zip(dec_sess, spec["kv"])]
    return spec, {"chunk_lanes": chunk, "decode_lanes": dec}


def run_c5():
    import synth35
    spec = fc.c5()
    cfg, t = synth35.in_memory(synth35.config(), seed=spec["model_seed"])
    o = orc.Qwen35Model(cfg, t, threads=THREADS)
    prompts = spec["prompts"]
    sess = [o.session(spec["context"]) for _ in prompts]
    width = max(len(p) for p in prompts)
    t0 = time.time()
    samples = [[] for _ in prompts]
    for j in range(width):
        live = [i for i, p in enumerate(prompts) if j < len(p)]
        want = [1 if j == len(prompts[i]) - 1 else 0 for i in live]
        errs = o.forward_batch([sess[i] for i in live], [prompts[i][j] for i in live], logits=want)
        assert not errs.any()
        for i in live:
            if j == len(prompts[i]) - 1:
                samples[i].append(fc.summary(sess[i].logits()))
        if j % 64 == 0:
            log(f"  c5 prompt row {j}/{width} ({time.time() - t0:.0f}s)")
    for g in range(spec["generate"]):
        toks = [samples[i][-1]["argmax"] for i in range(len(prompts))]
        errs = o.forward_batch(sess, toks)
        assert not errs.any()
        for i, s in enumerate(sess):
            samples[i].append(fc.summary(s.logits()))
    full = [l for l, f in enumerate(cfg["full"]) if f]
    lin = [l for l, f in enumerate(cfg["full"]) if not f]
    state = []
    for i, s in enumerate(sess):
        n = s.position()
        kvd = cfg["kv_heads"] * cfg["head_dim"]
        kl = full[-1]
        k = s.state(kl, 0).reshape(n, kvd)[-(spec["generate"] + 1):]
        v = s.state(kl, 1).reshape(n, kvd)[-(spec["generate"] + 1):]
        state.append({"kv_tail_layer": kl, "kv_tail": fc.kv_rows_digest([(k, v)]),
                      "linear_layer": lin[-1], "conv": fc.digest(s.state(lin[-1], 2)),
                      "delta": fc.digest(s.state(lin[-1], 3))})
    return spec, {"samples": samples, "state": state}


CASES = {"c2_32": lambda: run_c2(32), "c2_128": lambda: run_c2(128), "c4": run_c4, "c1": run_c1,
         "c3": run_c3, "c5": run_c5, "q4km_32": lambda: run_c2(32, fc.q4km(32))}


def main():
    names = sys.argv[1:] or list(CASES)
    for name in names:
        t0 = time.time()
        log(f"[make_fullshape] {name} on {THREADS} threads")
        spec, result = CASES[name]()
        out = {"case": name, "spec_sha256": fc.spec_digest(spec), "oracle_threads": THREADS,
               "generated_s": round(time.time() - t0, 1), **result}
        path = os.path.join(HERE, f"fullshape_{name}.json")
        with open(path, "w") as f:
            json.dump(out, f, indent=0, sort_keys=True)
        log(f"[make_fullshape] {name}: wrote {path} in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
