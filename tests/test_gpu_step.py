"""GPU parity: the HIP step (through the C ABI) against the CPU oracle.

Bit-exact targets: packing (cu_seqlens, positions, slots, lanes), KV rows,
greedy token ids.  Logits are compared bitwise too: the kernels keep the
reference's reduction orders (exact int8 block sums + the fmaf block chain for
Q8_0; q.k in element order), and the remaining f64 tree sums agree with the
sequential ones unless a partial sum rounds — the test reports any such
difference with its size rather than hiding it (tolerance: max-abs <= 1e-2 for
F16, <= 3e-2 for quantized, the bound stated for this path).
"""
import os

import numpy as np
import pytest

import cohx
import orc
import synth

pytestmark = pytest.mark.gpu

TINY = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                    vocabulary=300, context=512)
TOL = {"f16": 1e-2, "q8_0": 3e-2, "q4_0": 3e-2}


def build(dtype, seed, cfg=TINY, exact=False, **kw):
    """exact: the context keeps the exact kernels at every row count (the
    packed-prefill regime, held to a tolerance by test_gpu_prefill.py, off)."""
    c, t = synth.in_memory(cfg, dtype, seed=seed)
    kw.setdefault("max_lanes", 8)
    kw.setdefault("max_rows", 64)
    kw.setdefault("max_seqs", 8)
    kw.setdefault("max_context", 256)
    old = os.environ.get("COHX_PREFILL_MFMA")
    if exact:
        os.environ["COHX_PREFILL_MFMA"] = "0"
    try:
        m = cohx.Model(c, t, **kw)
    finally:
        if old is None:
            os.environ.pop("COHX_PREFILL_MFMA", None)
        else:
            os.environ["COHX_PREFILL_MFMA"] = old
    return c, t, m, orc.Model(c, t, threads=8)


def compare_logits(got, want, dtype, what):
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    diff = float(np.abs(got.astype(np.float64) - want).max())
    print(f"{what}: {bad.size} of {got.size} logits differ in bits, max-abs {diff:.3g}",
          flush=True)
    assert diff <= TOL[dtype], what
    return bad.size


def test_pack_matches_oracle():
    print("case: pack", flush=True)
    c, t, m, o = build("q8_0", 1)
    seqs = [m.seq_alloc() for _ in range(4)]
    for s, n in zip(seqs, (0, 17, 40, 5)):
        if n:
            m.seq_fill_synthetic(s, n, 7, s)
    lanes = [dict(seq=s, tokens=list(range(k))) for s, k in zip(seqs, (3, 1, 5, 16))]
    cu, pos, slot, lane = m.pack(lanes)
    pages = [m.seq_pages(s) for s in seqs]
    width = max(len(p) for p in pages)
    table = np.full((len(seqs), width), -1, np.int32)
    for i, p in enumerate(pages):
        table[i, :len(p)] = p
    rc, cu2, pos2, slot2, lane2 = orc.pack([3, 1, 5, 16], [0, 17, 40, 5], table, cohx.PAGE)
    assert rc == 0
    assert np.array_equal(cu, cu2) and np.array_equal(pos, pos2)
    assert np.array_equal(slot, slot2) and np.array_equal(lane, lane2)


@pytest.mark.parametrize("dtype", ["q8_0", "f16", "q4_0"])
def test_ragged_steps_match_oracle(dtype):
    print(f"case: ragged steps {dtype}", flush=True)
    c, t, m, o = build(dtype, 2)
    rng = np.random.default_rng(3)
    V = c["vocabulary"]
    seqs = [m.seq_alloc() for _ in range(3)]
    sess = [o.session(256) for _ in range(3)]
    # (lane -> n_tokens) per step: mixed prefill chunks and single decode rows
    plan = [{0: 5, 1: 3}, {0: 1, 1: 1, 2: 4}, {0: 1, 2: 1}, {1: 2, 2: 1, 0: 1}]
    mismatched = 0
    for step, spec in enumerate(plan):
        lanes, toks = [], {}
        for i, n in spec.items():
            toks[i] = [int(v) for v in rng.integers(0, V, n)]
            lanes.append(dict(seq=seqs[i], tokens=toks[i], logits=True))
        res = m.step(lanes)
        for (i, n), r in zip(spec.items(), res):
            assert r["status"] == 0
            for tok in toks[i]:
                assert o.forward_batch([sess[i]], [tok])[0] == 0
            want = sess[i].logits()
            mismatched += compare_logits(r["logits"], want, dtype, f"step {step} lane {i}")
            assert r["argmax"] == orc.Sampler().sample(want)[1]
    for i in range(3):
        assert m.seq_length(seqs[i]) == sess[i].position
        for layer in range(c["layers"]):
            for values in (False, True):
                got, want = m.seq_read_kv(seqs[i], layer, values), sess[i].kv(layer, values)
                assert np.array_equal(got, want), (i, layer, values)
    assert mismatched == 0


def run_generation(m, prompts, options, arrive=None):
    """tests/batching.rs:40-125 protocol: step every lane that needs a forward,
    sample each, admit a late arrival, retire finished lanes."""
    arrive = arrive or {}
    states = {i: m.begin_generation(p, options[i]) for i, p in enumerate(prompts)
              if i not in arrive}
    done = {}
    for rnd in range(400):
        for i, r in arrive.items():
            if r == rnd:
                states[i] = m.begin_generation(prompts[i], options[i])
        lanes = [s for s in states.values() if s.needs_forward()]
        if lanes:
            m.step_batch(lanes)
        for i in list(states):
            s = states[i]
            s.sample()
            if s.is_finished():
                done[i] = (s.token_ids(), s.finish_reason())
                s.free()
                del states[i]
        if len(done) == len(prompts):
            break
    return done


def oracle_generate(o, prompt, opt, eos):
    s = o.session(256)
    sampler = orc.Sampler(opt.temperature, opt.top_k, opt.top_p, opt.seed,
                          opt.repetition_penalty, opt.frequency_penalty, opt.presence_penalty)
    sampler.history(o.config["vocabulary"], prompt)  # generation.rs:151
    for tok in prompt:
        assert o.forward_batch([s], [tok])[0] == 0
    ids = []
    while len(ids) < opt.max_tokens:
        rc, tok = sampler.sample(s.logits())
        assert rc == 0
        sampler.observe(tok)
        ids.append(tok)
        if tok == eos:
            return ids, "stop"
        if len(ids) == opt.max_tokens:
            break
        assert o.forward_batch([s], [tok])[0] == 0
    return ids, "length"


@pytest.mark.parametrize("dtype", ["q8_0", "f16", "q4_0"])
def test_batched_generation_equals_individual_and_oracle(dtype):
    print(f"case: generation {dtype}", flush=True)
    c, t, m, o = build(dtype, 4)
    rng = np.random.default_rng(5)
    prompts = [[int(v) for v in rng.integers(0, c["vocabulary"], n)] for n in (2, 9, 5)]
    opts = [cohx.GenerationOptions(max_tokens=6),
            cohx.GenerationOptions(max_tokens=7, temperature=0.7, top_k=16, top_p=0.9, seed=48,
                                   repetition_penalty=1.1, frequency_penalty=0.2,
                                   presence_penalty=0.3),
            cohx.GenerationOptions(max_tokens=5, temperature=0.9, seed=49)]
    batched = run_generation(m, prompts, opts, arrive={2: 4})
    for i, p in enumerate(prompts):
        single = cohx.generate(m, p, opts[i])
        assert single.token_ids() == batched[i][0]
        want, reason = oracle_generate(o, p, opts[i], c["eos_token_id"])
        assert batched[i] == (want, reason), i
        single.free()


def test_lane_errors_are_isolated():
    print("case: lane errors", flush=True)
    c, t, m, o = build("q8_0", 6)
    a, b, d = m.seq_alloc(), m.seq_alloc(capacity=2), m.seq_alloc()
    m.step([dict(seq=a, tokens=[1, 2]), dict(seq=b, tokens=[3, 4])])
    res = m.step([dict(seq=a, tokens=[c["vocabulary"] + 1]), dict(seq=b, tokens=[5]),
                  dict(seq=d, tokens=[7], logits=True)])
    assert res[0]["status"] == cohx.INVALID_REQUEST
    assert res[1]["status"] == cohx.RESOURCE
    assert res[2]["status"] == 0
    s = o.session(256)
    o.forward_batch([s], [7])
    assert np.array_equal(res[2]["logits"], s.logits())
    assert m.seq_length(a) == 2 and m.seq_length(b) == 2


def test_zero_weights_give_token_zero_and_eos_stops():
    print("case: closed forms", flush=True)
    c, t = synth.in_memory(TINY, "q8_0", seed=0)
    for name, tensor in t.items():
        if len(tensor.shape) == 2:
            tensor.data[:] = 0
    m = cohx.Model(c, t, max_lanes=2, max_rows=8, max_seqs=4, max_context=64)
    st = cohx.generate(m, [5, 6], cohx.GenerationOptions(max_tokens=4))
    assert st.token_ids() == [0, 0, 0, 0] and st.finish_reason() == "length"
    # EOS (tests/engine.rs:187-217): embeddings of ones, zero matrices and an
    # output row of ones for the end-of-generation id make it the argmax.
    c2, t2 = synth.in_memory(TINY, "q8_0", seed=0, eos_token_id=258, tied=False)
    ones = np.tile(np.r_[np.frombuffer(np.float16(1.0).tobytes(), np.uint8),
                         np.ones(32, np.uint8)], c2["hidden"] // 32)
    for name, tensor in t2.items():
        if len(tensor.shape) == 2:
            tensor.data[:] = 0
    t2["token_embd.weight"].data.reshape(c2["vocabulary"], -1)[:] = ones
    t2["output.weight"].data.reshape(c2["vocabulary"], -1)[258] = ones
    m2 = cohx.Model(c2, t2, max_lanes=2, max_rows=8, max_seqs=4, max_context=64)
    st = cohx.generate(m2, [5, 6], cohx.GenerationOptions(max_tokens=4))
    assert st.token_ids() == [258] and st.finish_reason() == "stop"


@pytest.mark.parametrize("dtype", ["q8_0", "q4_0"])
def test_shared_prefix_fork_equals_recompute(dtype):
    print(f"case: fork {dtype}", flush=True)
    c, t, m, o = build(dtype, 7)
    base = m.seq_alloc()
    prefix = list(range(1, 40))
    m.step([dict(seq=base, tokens=prefix)])
    fa, fb = m.seq_fork(base, 32), m.seq_fork(base, 37)
    fresh = m.seq_alloc()
    m.step([dict(seq=fresh, tokens=prefix[:37])])
    ra = m.step([dict(seq=fa, tokens=[9], logits=True), dict(seq=fb, tokens=[11], logits=True),
                 dict(seq=fresh, tokens=[11], logits=True)])
    s = o.session(256)
    for tok in prefix[:32] + [9]:
        o.forward_batch([s], [tok])
    assert np.array_equal(ra[0]["logits"], s.logits())
    assert np.array_equal(ra[1]["logits"], ra[2]["logits"])
    # the shared source is untouched by the forks' writes (copy on write)
    for layer in range(c["layers"]):
        assert np.array_equal(m.seq_read_kv(fb, layer)[:37], m.seq_read_kv(base, layer)[:37])


def test_step_decode_matches_lane_step():
    """The vectorized decode path (start position COHX_AT_END) and the per-lane
    step advance identical contexts identically, and an explicit wrong start
    position fails only its own lane."""
    print("case: step_decode vs step", flush=True)
    c, t, m1, o = build("q8_0", 5)
    m2 = cohx.Model(c, t, max_lanes=8, max_rows=64, max_seqs=8, max_context=256)
    kv = [37, 5, 90, 16, 64]
    s1, s2 = [], []
    for i, n in enumerate(kv):
        a, b = m1.seq_alloc(), m2.seq_alloc()
        m1.seq_fill_synthetic(a, n, 3, i)
        m2.seq_fill_synthetic(b, n, 3, i)
        s1.append(a)
        s2.append(b)
    toks = np.array([11, 250, 3, 299, 0], np.uint32)
    for step in range(3):
        res = m1.step([dict(seq=a, tokens=[int(x)], start=m1.seq_length(a)) for a, x in zip(s1, toks)])
        status, argmax = m2.step_decode(s2, toks)
        assert not status.any()
        assert [r["argmax"] for r in res] == argmax.tolist(), step
        toks = argmax
    for a, b in zip(s1, s2):
        assert m1.seq_length(a) == m2.seq_length(b)
        assert np.array_equal(m1.seq_read_kv(a, 1, True), m2.seq_read_kv(b, 1, True))
    res = m1.step([dict(seq=s1[0], tokens=[1], start=m1.seq_length(s1[0]) + 1),
                   dict(seq=s1[1], tokens=[1])])
    assert res[0]["status"] == 1 and res[1]["status"] == 0


def test_graph_replays_match_direct_launches():
    """Steps replayed from captured graphs equal directly launched steps, bit
    for bit, on every replay: across a KV-length bucket change (a new graph),
    with logits requested (another graph), and with eager work (KV reads,
    host synchronization) between the replays."""
    import os
    print("case: graph replay vs direct launches", flush=True)
    c, t, mg, o = build("q8_0", 9, max_context=512)
    os.environ["COHX_GRAPHS"] = "0"
    try:
        md = cohx.Model(c, t, max_lanes=8, max_rows=64, max_seqs=8, max_context=512)
    finally:
        del os.environ["COHX_GRAPHS"]
    kv = [250, 3, 128, 254]
    sg, sd = [], []
    for i, n in enumerate(kv):
        a, b = mg.seq_alloc(), md.seq_alloc()
        mg.seq_fill_synthetic(a, n, 4, i)
        md.seq_fill_synthetic(b, n, 4, i)
        sg.append(a)
        sd.append(b)
    toks = np.array([7, 8, 9, 10], np.uint32)
    for step in range(8):
        if step % 3 == 2:
            lg = mg.step([dict(seq=a, tokens=[int(x)], logits=True) for a, x in zip(sg, toks)])
            ld = md.step([dict(seq=b, tokens=[int(x)], logits=True) for b, x in zip(sd, toks)])
            for x, y in zip(lg, ld):
                assert x["status"] == 0 and y["status"] == 0
                assert np.array_equal(x["logits"].view(np.uint32), y["logits"].view(np.uint32)), step
            ag = np.array([r["argmax"] for r in lg], np.uint32)
            ad = np.array([r["argmax"] for r in ld], np.uint32)
        else:
            st_g, ag = mg.step_decode(sg, toks)
            st_d, ad = md.step_decode(sd, toks)
            assert not st_g.any() and not st_d.any()
        assert np.array_equal(ag, ad), step
        # eager work between replays
        assert np.array_equal(mg.seq_read_kv(sg[0], 1), md.seq_read_kv(sd[0], 1)), step
        toks = ag
    for a, b in zip(sg, sd):
        assert np.array_equal(mg.seq_read_kv(a, 0, True), md.seq_read_kv(b, 0, True))


# Shapes off the Qwen2.5-0.5B path: the intermediate width is an odd number of
# 32-element blocks per 64 (F % 64 == 32: gate+up cannot quantize the down
# operand in its epilogue), and a hidden width above 1024 (gate+up and the head
# leave the short-K kernels).
ODD_F = synth.config(layers=2, hidden=128, intermediate=224, heads=4, kv_heads=2, vocabulary=300,
                     context=512)
WIDE_H = synth.config(layers=2, hidden=1152, intermediate=256, heads=18, kv_heads=9,
                      vocabulary=300, context=512)


@pytest.mark.parametrize("shape", ["tiny", "odd_f", "wide_h"])
@pytest.mark.parametrize("dtype", ["q8_0", "q4_0"])
def test_tall_ragged_steps_match_oracle(dtype, shape):
    """Packed steps of 197 rows (13 batch tiles: more than one row of the
    8-tile gate+up workgroups, the second one partial) on the exact kernels
    (the packed-prefill regime off), then a decode step, bit for bit against
    the oracle: logits of every lane, greedy ids, the K/V rows of every
    layer."""
    cfg = {"tiny": TINY, "odd_f": ODD_F, "wide_h": WIDE_H}[shape]
    print(f"case: tall ragged steps {dtype} {shape}", flush=True)
    c, t, m, o = build(dtype, 12, cfg=cfg, exact=True, max_lanes=4, max_rows=200, max_seqs=4,
                       max_context=256)
    rng = np.random.default_rng(13)
    V = c["vocabulary"]
    seqs = [m.seq_alloc() for _ in range(3)]
    sess = [o.session(256) for _ in range(3)]
    m.seq_fill_synthetic(seqs[2], 21, 6, 2)
    sess[2].fill_synthetic(21, 6, 2)
    mismatched = 0
    for step, lens in enumerate(((90, 70, 37), (1, 1, 1))):
        toks = [[int(v) for v in rng.integers(0, V, n)] for n in lens]
        res = m.step([dict(seq=s, tokens=tk, logits=True) for s, tk in zip(seqs, toks)])
        width = max(lens)
        for j in range(width):
            live = [i for i in range(3) if j < lens[i]]
            errs = o.forward_batch([sess[i] for i in live], [toks[i][j] for i in live])
            assert not errs.any()
        for i, r in enumerate(res):
            assert r["status"] == 0
            want = sess[i].logits()
            mismatched += compare_logits(r["logits"], want, dtype, f"{shape} step {step} lane {i}")
            assert r["argmax"] == orc.Sampler().sample(want)[1]
    for i in range(3):
        for layer in range(c["layers"]):
            for values in (False, True):
                assert np.array_equal(m.seq_read_kv(seqs[i], layer, values), sess[i].kv(layer, values))
    assert mismatched == 0


LONG = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2, vocabulary=300,
                    context=8192)


@pytest.mark.parametrize("dtype", ["q8_0", "f16"])
def test_long_rows_match_oracle(dtype):
    """Decode steps whose rows attend to up to 4700 positions (19 score
    chunks of 256 keys, 37 value chunks of 128) beside rows of 2 to 30
    positions, bit for bit against the oracle: logits of every lane, greedy
    ids, the K/V rows appended."""
    print(f"case: long rows {dtype}", flush=True)
    c, t, m, o = build(dtype, 14, cfg=LONG, max_lanes=4, max_rows=8, max_seqs=4, max_context=4800)
    rng = np.random.default_rng(15)
    mismatched = 0
    for k, lens in enumerate(((4599, 30, 1000), (4699, 2, 4200))):
        seqs = [m.seq_alloc() for _ in lens]
        sess = [o.session(4800) for _ in lens]
        for i, n in enumerate(lens):
            m.seq_fill_synthetic(seqs[i], n, 8, i)
            sess[i].fill_synthetic(n, 8, i)
        for step in range(2):
            toks = [int(v) for v in rng.integers(0, c["vocabulary"], len(lens))]
            res = m.step([dict(seq=s, tokens=[x], logits=True) for s, x in zip(seqs, toks)])
            assert not o.forward_batch(sess, toks).any()
            for i, r in enumerate(res):
                assert r["status"] == 0
                want = sess[i].logits()
                mismatched += compare_logits(r["logits"], want, dtype, f"case {k} step {step} lane {i}")
                assert r["argmax"] == orc.Sampler().sample(want)[1]
        for i, n in enumerate(lens):
            for values in (False, True):
                got = m.seq_read_kv_rows(seqs[i], 1, n, 2, values)
                assert np.array_equal(got, sess[i].kv(1, values)[n:n + 2]), (k, i, values)
            m.seq_free(seqs[i])
    assert mismatched == 0
