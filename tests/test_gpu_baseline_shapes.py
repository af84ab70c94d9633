"""GPU parity at BASELINE.json's workloads at their stated sizes, against the
CPU oracle's results for the same inputs (tests/golden/fullshape_<case>.json,
written by tests/golden/make_fullshape.py from tests/fullshape_cases.py).

Each lane's float32 logits are compared through their SHA-256 (all V values
bit for bit), with the greedy id; the K/V rows a step appends through the
SHA-256 of their bytes.  A differing lane is reported with its top-1 / top-2
values next to the oracle's, and the test fails.  The packed-prefill regime
(C3, matrix-core linears with f32 sums) is held to north_star's F16 tolerance
(max-abs 1e-2) against the exact path, which itself equals the oracle bit for
bit on the same step.
"""
import json
import os

import numpy as np
import pytest

import cohx
import fullshape_cases as fc
import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture(name, spec):
    with open(os.path.join(GOLDEN, f"fullshape_{name}.json")) as f:
        fx = json.load(f)
    assert fx["spec_sha256"] == fc.spec_digest(spec), f"{name}: inputs differ from the fixture's"
    return fx


def compare(got_logits, want, what, diffs):
    got = fc.summary(got_logits)
    if got["sha256"] != want["sha256"]:
        diffs.append(f"{what}: logits differ; gpu top1 {got['top1']!r} top2 {got['top2']!r} "
                     f"argmax {got['argmax']}, oracle top1 {want['top1']!r} top2 {want['top2']!r} "
                     f"argmax {want['argmax']}")
    return got["argmax"]


def appended_rows(m, seq, layers, first, count):
    return fc.kv_rows_digest([(m.seq_read_kv_rows(seq, l, first, count),
                               m.seq_read_kv_rows(seq, l, first, count, values=True)) for l in layers])


def run_decode(m, seqs, starts, spec, fx, name):
    """The fixture's greedy decode steps with logits on every lane, then the
    appended K/V rows, then the same steps again without logits through the
    vectorized decode entry (the benchmark's path): same greedy ids."""
    diffs, toks = [], list(spec["tokens"])
    for step, want in enumerate(fx["steps"]):
        print(f"case {name}: step {step}, {len(seqs)} lanes with logits", flush=True)
        res = m.step([dict(seq=s, tokens=[tk], logits=True) for s, tk in zip(seqs, toks)])
        for i, (r, w) in enumerate(zip(res, want)):
            assert r["status"] == 0, (i, r["status"])
            assert compare(r["logits"], w, f"step {step} lane {i}", diffs) == w["argmax"]
            assert r["argmax"] == w["argmax"], (step, i, r["argmax"], w["argmax"])
        toks = [w["argmax"] for w in want]
    for i, (s, n) in enumerate(zip(seqs, starts)):
        got = appended_rows(m, s, spec["kv_check_layers"], n, spec["steps"])
        if got != fx["kv_appended"][i]:
            diffs.append(f"lane {i}: appended K/V rows differ")
    print(f"case {name}: {len(diffs)} differing lanes of {len(seqs) * len(fx['steps'])}", flush=True)
    for d in diffs[:16]:
        print("  " + d, flush=True)
    assert not diffs
    for s, n in zip(seqs, starts):
        m.seq_truncate(s, n)
    toks = np.asarray(spec["tokens"], np.uint32)
    arr = np.asarray(seqs, np.uint32)
    for step, want in enumerate(fx["steps"]):
        print(f"case {name}: step {step} again, argmax only", flush=True)
        st, am = m.step_decode(arr, toks)
        assert not st.any()
        assert am.tolist() == [w["argmax"] for w in want]
        toks = am


@pytest.fixture(scope="module")
def q8_model():
    print("building the Q8_0 Qwen2.5-0.5B-shape model", flush=True)
    return synth.in_memory(synth.config(), "q8_0", seed=fc.SEED_Q8)


@pytest.mark.parametrize("lanes", [32, 128])
def test_c2_q8_0_ragged_decode_matches_oracle(q8_model, lanes):
    """configs[1] (32 lanes) and the 128-lane headline: KV U[64, 2048]."""
    spec = fc.c2(lanes)
    fx = fixture(f"c2_{lanes}", spec)
    c, t = q8_model
    m = cohx.Model(c, t, max_lanes=lanes, max_rows=lanes, max_seqs=lanes, max_context=spec["context"])
    seqs = []
    for i, n in enumerate(spec["kv"]):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, spec["fill_seed"], i)
        seqs.append(s)
    run_decode(m, seqs, spec["kv"], spec, fx, f"c2_{lanes}")
    m.close()


def test_q4_k_m_full_shape_decode_matches_oracle():
    """The Qwen2.5-0.5B shape with the publisher Q4_K_M file's dtypes (Q5_0,
    Q8_0, Q4_K, Q6_K; untied Q8_0 head): 32 decode lanes over KV U[64, 2048]."""
    spec = fc.q4km(32)
    fx = fixture("q4km_32", spec)
    print("building the Q4_K_M-style Qwen2.5-0.5B-shape model", flush=True)
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    lanes = len(spec["kv"])
    m = cohx.Model(c, t, max_lanes=lanes, max_rows=lanes, max_seqs=lanes, max_context=spec["context"])
    seqs = []
    for i, n in enumerate(spec["kv"]):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, spec["fill_seed"], i)
        seqs.append(s)
    run_decode(m, seqs, spec["kv"], spec, fx, "q4km_32")
    m.close()


def test_c4_q4_0_shared_prefix_groups_match_oracle():
    """8 groups of 16 lanes forked from 256-token prefixes
    (shared pages, copy on write), contexts up to 4096."""
    spec = fc.c4()
    fx = fixture("c4", spec)
    print("building the Q4_0 Qwen2.5-0.5B-shape model", flush=True)
    c, t = synth.in_memory(synth.config(), "q4_0", seed=spec["model_seed"])
    lanes = spec["groups"] * spec["group"]
    m = cohx.Model(c, t, max_lanes=lanes, max_rows=lanes, max_seqs=lanes + spec["groups"],
                   max_context=spec["context"])
    seqs, starts = [], []
    for g in range(spec["groups"]):
        base = m.seq_alloc()
        m.seq_fill_synthetic(base, spec["prefix"], spec["fill_seed"], 1000 + g)
        for k in range(spec["group"]):
            i = g * spec["group"] + k
            s = m.seq_fork(base, spec["prefix"])
            m.seq_fill_synthetic(s, spec["prefix"] + spec["suffix"][i], spec["fill_seed"], i)
            seqs.append(s)
            starts.append(spec["prefix"] + spec["suffix"][i])
        m.seq_free(base)
    # the lanes of a group share their prefix pages
    p0 = m.seq_pages(seqs[0])[:spec["prefix"] // cohx.PAGE]
    assert np.array_equal(m.seq_pages(seqs[1])[:p0.size], p0)
    run_decode(m, seqs, starts, spec, fx, "c4")
    m.close()


def test_c1_f16_continuous_batch_matches_oracle():
    """4 prompts of 16/32/48/64 ids, 16 greedy tokens, context 512,
    one token per lane per step; logits at every sampling point bit for bit,
    then the same run through the generation mirror (cohx_gen_* and
    cohx_step_batch): the same ids."""
    spec = fc.c1()
    fx = fixture("c1", spec)
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    m = cohx.Model(c, t, max_lanes=4, max_rows=4, max_seqs=4, max_context=spec["context"])
    prompts = spec["prompts"]
    seqs = [m.seq_alloc() for _ in prompts]
    cursor = [0] * len(prompts)
    ids = [[] for _ in prompts]
    done = [False] * len(prompts)
    diffs = []
    print("case c1: direct steps", flush=True)
    while not all(done):
        lanes, idx = [], []
        for i, p in enumerate(prompts):
            if done[i]:
                continue
            tok = p[cursor[i]] if cursor[i] < len(p) else ids[i][-1]
            sampling = cursor[i] >= len(p) - 1
            lanes.append(dict(seq=seqs[i], tokens=[tok], logits=sampling))
            idx.append((i, sampling))
        res = m.step(lanes)
        for (i, sampling), r in zip(idx, res):
            assert r["status"] == 0
            cursor[i] += 1
            if not sampling:
                continue
            k = len(ids[i])
            want = fx["lanes"][i]["samples"][k]
            compare(r["logits"], want, f"lane {i} sample {k}", diffs)
            ids[i].append(int(r["argmax"]))
            if len(ids[i]) == len(fx["lanes"][i]["ids"]):
                done[i] = True
    for d in diffs:
        print("  " + d, flush=True)
    assert not diffs
    assert ids == [l["ids"] for l in fx["lanes"]]
    m.close()
    print("case c1: generation mirror", flush=True)
    m = cohx.Model(c, t, max_lanes=4, max_rows=4, max_seqs=4, max_context=spec["context"])
    opts = cohx.GenerationOptions(max_tokens=spec["max_tokens"])
    states = [m.begin_generation(p, opts) for p in prompts]
    while not all(s.is_finished() for s in states):
        lanes = [s for s in states if s.needs_forward()]
        if lanes:
            m.step_batch(lanes)
        for s in states:
            s.sample()
    assert [s.token_ids() for s in states] == [l["ids"] for l in fx["lanes"]]
    for s in states:
        s.free()
    m.close()


def c3_context(c, t, spec, exact):
    rows = sum(len(ch) for ch in spec["chunks"]) + len(spec["kv"])
    lanes = len(spec["chunks"]) + len(spec["kv"])
    old = os.environ.get("COHX_PREFILL_MFMA")
    if exact:
        os.environ["COHX_PREFILL_MFMA"] = "0"
    try:
        m = cohx.Model(c, t, max_lanes=lanes, max_rows=rows, max_seqs=lanes, max_context=spec["context"])
    finally:
        if old is None:
            os.environ.pop("COHX_PREFILL_MFMA", None)
        else:
            os.environ["COHX_PREFILL_MFMA"] = old
    chunk = []
    for i, n in enumerate(spec["prefix"]):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, spec["fill_seed"], i)
        chunk.append(s)
    dec = []
    for i, n in enumerate(spec["kv"]):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, spec["fill_seed"], 100 + i)
        dec.append(s)
    lanes = [dict(seq=s, tokens=ch, logits=True) for s, ch in zip(chunk, spec["chunks"])]
    lanes += [dict(seq=s, tokens=[tk], logits=True) for s, tk in zip(dec, spec["tokens"])]
    res = m.step(lanes)
    assert all(r["status"] == 0 for r in res)
    return m, chunk, dec, res


def test_c3_f16_mixed_prefill_step_matches_oracle():
    """one step packing 8 prompt chunks of U[128, 512] tokens (over
    seeded prefixes) with 56 decode rows over KV U[256, 4096].  The exact path
    equals the oracle bit for bit (logits of every lane, appended K/V rows);
    the packed-prefill regime is within 1e-2 of it, with the same greedy id
    wherever the top-2 margin exceeds twice the difference."""
    spec = fc.c3()
    fx = fixture("c3", spec)
    c, t = synth.in_memory(synth.config(), spec["dtype"], seed=spec["model_seed"])
    layers = spec["kv_check_layers"]
    print("case c3: exact path", flush=True)
    m, chunk, dec, exact = c3_context(c, t, spec, exact=True)
    diffs = []
    want = [x["summary"] for x in fx["chunk_lanes"]] + [x["summary"] for x in fx["decode_lanes"]]
    for i, (r, w) in enumerate(zip(exact, want)):
        compare(r["logits"], w, f"lane {i}", diffs)
        assert r["argmax"] == w["argmax"], i
    kv_exact = {}
    for i, (s, n, ch) in enumerate(zip(chunk, spec["prefix"], spec["chunks"])):
        kv_exact[("c", i)] = [(m.seq_read_kv_rows(s, l, n, len(ch)), m.seq_read_kv_rows(s, l, n, len(ch), True))
                              for l in layers]
        if fc.kv_rows_digest(kv_exact[("c", i)]) != fx["chunk_lanes"][i]["kv_appended"]:
            diffs.append(f"chunk lane {i}: appended K/V rows differ")
    for i, (s, n) in enumerate(zip(dec, spec["kv"])):
        rows = [(m.seq_read_kv_rows(s, l, n, 1), m.seq_read_kv_rows(s, l, n, 1, True)) for l in layers]
        if fc.kv_rows_digest(rows) != fx["decode_lanes"][i]["kv_appended"]:
            diffs.append(f"decode lane {i}: appended K/V rows differ")
    print(f"case c3 exact: {len(diffs)} differing lanes of {len(want)}", flush=True)
    for d in diffs[:16]:
        print("  " + d, flush=True)
    assert not diffs
    m.close()
    print("case c3: packed-prefill regime", flush=True)
    m, chunk, dec, regime = c3_context(c, t, spec, exact=False)
    worst = 0.0
    for i, (r, e) in enumerate(zip(regime, exact)):
        diff = float(np.abs(r["logits"].astype(np.float64) - e["logits"]).max())
        worst = max(worst, diff)
        order = np.sort(e["logits"])
        if order[-1] - order[-2] > 2 * diff:
            assert r["argmax"] == e["argmax"], (i, diff)
        assert diff <= 1e-2, (i, diff)
    kv_worst = 0.0
    for i, (s, n, ch) in enumerate(zip(chunk, spec["prefix"], spec["chunks"])):
        for l, (k, v) in zip(layers, kv_exact[("c", i)]):
            kv_worst = max(kv_worst, float(np.abs(m.seq_read_kv_rows(s, l, n, len(ch)) - k).max()),
                           float(np.abs(m.seq_read_kv_rows(s, l, n, len(ch), True) - v).max()))
    print(f"case c3 regime: worst logit max-abs {worst:.3g}, appended K/V rows {kv_worst:.3g}", flush=True)
    assert kv_worst <= 1e-2
    m.close()


def test_c5_qwen35_prefill_regime_greedy_ids_and_top_logits():
    """configs[4] with the packed-prefill regime on (the default): the prompt
    steps' linears run on the bfloat16 matrix-core GEMM (hi/lo operands, f32
    sums).  Every sampled lane's top-1 and top-2 logits (the fixture keeps
    those values) within 1e-2 of the oracle's, and greedy ids equal to the
    oracle's over the whole 64-token continuation, except where the oracle's
    own top-1/top-2 gap is within twice that deviation: a lane that takes the
    other id there continues on its own tokens, and its check ends at that
    sample."""
    import synth35
    spec = fc.c5()
    fx = fixture("c5", spec)
    print("building the Qwen3.5-0.8B-shape model", flush=True)
    cfg, t = synth35.in_memory(synth35.config(), seed=spec["model_seed"])
    old = os.environ.get("COHX_PREFILL_MFMA")
    os.environ["COHX_PREFILL_MFMA"] = "1"
    try:
        m = cohx.Qwen35(cfg, t, max_lanes=16, max_rows=16 * 256, max_seqs=16, max_context=spec["context"])
    finally:
        if old is None:
            os.environ.pop("COHX_PREFILL_MFMA", None)
        else:
            os.environ["COHX_PREFILL_MFMA"] = old
    prompts = spec["prompts"]
    seqs = [m.seq_alloc() for _ in prompts]
    cursor = [0] * len(prompts)
    got = [[] for _ in prompts]
    done = [False] * len(prompts)  # a lane's check ended (sampled all, or a near-tie took the other id)
    worst, gap, compared, diverged = 0.0, float("inf"), 0, []
    while not all(done):
        lanes, idx = [], []
        for i, p in enumerate(prompts):
            if done[i]:
                continue
            if cursor[i] < len(p):
                toks = p[cursor[i]:cursor[i] + 256]
                ends = cursor[i] + len(toks) == len(p)
                lanes.append(dict(seq=seqs[i], tokens=toks, logits=ends, skip_head=not ends))
                idx.append((i, len(toks), ends))
            else:
                lanes.append(dict(seq=seqs[i], tokens=[got[i][-1]], logits=True))
                idx.append((i, 1, True))
        res = m.step(lanes)
        for (i, n, sampled), r in zip(idx, res):
            assert r["status"] == 0
            cursor[i] += n
            if not sampled:
                continue
            k = len(got[i])
            want = fx["samples"][i][k]
            sm = fc.summary(r["logits"])
            dev = max(abs(sm["top1"] - want["top1"]), abs(sm["top2"] - want["top2"]))
            worst = max(worst, dev)
            gap = min(gap, want["top1"] - want["top2"])
            compared += 1
            got[i].append(int(r["argmax"]))
            if got[i][-1] != want["argmax"]:
                assert want["top1"] - want["top2"] <= 2 * max(dev, 1e-7), (i, k, want, sm)
                diverged.append((i, k))
                done[i] = True
            elif len(got[i]) == spec["generate"] + 1:
                done[i] = True
    print(f"case c5 regime: {compared} samples compared, worst top-1/top-2 logit deviation "
          f"{worst:.3g}, smallest oracle top-1/top-2 gap {gap:.3g}, near-tie divergences "
          f"{diverged}", flush=True)
    assert worst <= 1e-2
    m.close()


def test_c5_qwen35_sixteen_prompts_match_oracle():
    """Qwen3.5-0.8B shape, 16 prompts of U[64, 1024] ids in chunks
    of 256 rows (rows before a prompt's end skip the head), then 64 greedy
    tokens: every sampled lane's logits, the ids, and the last linear layer's
    conv ring and delta memory and the last full layer's K/V tail, bit for bit
    (the packed-prefill regime off: every step on the exact matvecs)."""
    import synth35
    spec = fc.c5()
    fx = fixture("c5", spec)
    print("building the Qwen3.5-0.8B-shape model", flush=True)
    cfg, t = synth35.in_memory(synth35.config(), seed=spec["model_seed"])
    prompts = spec["prompts"]
    old = os.environ.get("COHX_PREFILL_MFMA")
    os.environ["COHX_PREFILL_MFMA"] = "0"
    try:
        m = cohx.Qwen35(cfg, t, max_lanes=16, max_rows=16 * 256, max_seqs=16, max_context=spec["context"])
    finally:
        if old is None:
            os.environ.pop("COHX_PREFILL_MFMA", None)
        else:
            os.environ["COHX_PREFILL_MFMA"] = old
    seqs = [m.seq_alloc() for _ in prompts]
    cursor = [0] * len(prompts)
    got = [[] for _ in prompts]
    diffs = []
    step = 0
    while any(len(g) < spec["generate"] + 1 for g in got):
        lanes, idx = [], []
        for i, p in enumerate(prompts):
            if len(got[i]) >= spec["generate"] + 1:
                continue
            if cursor[i] < len(p):
                toks = p[cursor[i]:cursor[i] + 256]
                ends = cursor[i] + len(toks) == len(p)
                lanes.append(dict(seq=seqs[i], tokens=toks, logits=ends, skip_head=not ends))
                idx.append((i, len(toks), ends))
            else:
                lanes.append(dict(seq=seqs[i], tokens=[got[i][-1]], logits=True))
                idx.append((i, 1, True))
        print(f"case c5: step {step}, {len(lanes)} lanes, {sum(n for _, n, _ in idx)} rows", flush=True)
        res = m.step(lanes)
        step += 1
        for (i, n, sampled), r in zip(idx, res):
            assert r["status"] == 0
            cursor[i] += n
            if sampled:
                k = len(got[i])
                compare(r["logits"], fx["samples"][i][k], f"seq {i} sample {k}", diffs)
                got[i].append(int(r["argmax"]))
    assert got == [[x["argmax"] for x in s] for s in fx["samples"]]
    for i, s in enumerate(seqs):
        st = fx["state"][i]
        n = m.seq_length(s)
        kvd = cfg["kv_heads"] * cfg["head_dim"]
        tail = spec["generate"] + 1
        k = m.read_state(s, st["kv_tail_layer"], 0).reshape(n, kvd)[-tail:]
        v = m.read_state(s, st["kv_tail_layer"], 1).reshape(n, kvd)[-tail:]
        if fc.kv_rows_digest([(k, v)]) != st["kv_tail"]:
            diffs.append(f"seq {i}: K/V tail differs")
        if fc.digest(m.read_state(s, st["linear_layer"], 2)) != st["conv"]:
            diffs.append(f"seq {i}: conv ring differs")
        if fc.digest(m.read_state(s, st["linear_layer"], 3)) != st["delta"]:
            diffs.append(f"seq {i}: delta memory differs")
    print(f"case c5: {len(diffs)} differences", flush=True)
    for d in diffs[:16]:
        print("  " + d, flush=True)
    assert not diffs
    m.close()
