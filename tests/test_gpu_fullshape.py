"""GPU parity at the Qwen2.5-0.5B shape against the
CPU oracle: Q8_0 ragged decode over seeded KV (config 2's form), a mixed
prefill-chunk + decode step, and an F16 continuous batch (config 1's form,
shortened so the oracle finishes in seconds).  Logits bit-for-bit, greedy ids
and KV rows exact; any bit difference is printed with its size
(tolerance max-abs 1e-2 for F16, 3e-2 for Q8_0)."""
import numpy as np
import pytest

import cohx
import orc
import synth

pytestmark = pytest.mark.gpu

FULL = synth.config()


@pytest.fixture(scope="module")
def q8_model():
    c, t = synth.in_memory(FULL, "q8_0", seed=21)
    return c, t


def check(got, want, tol, what):
    nbits = int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
    diff = float(np.abs(got.astype(np.float64) - want).max())
    order = np.sort(want)
    print(f"{what}: {nbits} differing logits, max-abs {diff:.3g}, "
          f"top1-top2 margin {order[-1] - order[-2]:.3g}", flush=True)
    assert diff <= tol
    return nbits


def test_q8_0_ragged_decode_over_seeded_kv(q8_model):
    print("case: full-shape Q8_0 decode, 4 lanes, KV 33..1500", flush=True)
    c, t = q8_model
    m = cohx.Model(c, t, max_lanes=4, max_rows=24, max_seqs=4, max_context=1600)
    o = orc.Model(c, t, threads=16)
    kv = [1500, 33, 700, 160]
    seqs, sess = [], []
    for i, n in enumerate(kv):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, 99, i)
        seqs.append(s)
        x = o.session(1600)
        x.fill_synthetic(n, 99, i)
        sess.append(x)
    for layer in (0, 23):
        assert np.array_equal(m.seq_read_kv(seqs[0], layer, True), sess[0].kv(layer, True))
    rng = np.random.default_rng(1)
    toks = [int(v) for v in rng.integers(0, c["vocabulary"], 4)]
    bits = 0
    for step in range(2):
        res = m.step([dict(seq=s, tokens=[tk], logits=True) for s, tk in zip(seqs, toks)])
        o.forward_batch(sess, toks)
        nxt = []
        for i, r in enumerate(res):
            assert r["status"] == 0
            want = sess[i].logits()
            bits += check(r["logits"], want, 3e-2, f"step {step} lane {i}")
            assert r["argmax"] == orc.Sampler().sample(want)[1]
            nxt.append(r["argmax"])
        toks = nxt
    for i in range(4):
        got = m.seq_read_kv(seqs[i], 5)
        assert np.array_equal(got[-2:], sess[i].kv(5)[-2:])
    assert bits == 0


def test_q8_0_mixed_prefill_chunk_and_decode(q8_model):
    print("case: full-shape Q8_0 prefill chunk (40 rows) + 2 decode rows", flush=True)
    c, t = q8_model
    m = cohx.Model(c, t, max_lanes=4, max_rows=64, max_seqs=4, max_context=512)
    o = orc.Model(c, t, threads=16)
    a, b, d = m.seq_alloc(), m.seq_alloc(), m.seq_alloc()
    m.seq_fill_synthetic(b, 300, 5, 1)
    m.seq_fill_synthetic(d, 64, 5, 2)
    sa, sb, sd = o.session(512), o.session(512), o.session(512)
    sb.fill_synthetic(300, 5, 1)
    sd.fill_synthetic(64, 5, 2)
    rng = np.random.default_rng(2)
    chunk = [int(v) for v in rng.integers(0, c["vocabulary"], 40)]
    res = m.step([dict(seq=a, tokens=chunk, logits=True), dict(seq=b, tokens=[17], logits=True),
                  dict(seq=d, tokens=[4242], logits=True)])
    for tok in chunk:
        o.forward_batch([sa], [tok])
    o.forward_batch([sb, sd], [17, 4242])
    bits = 0
    for r, s, name in zip(res, (sa, sb, sd), ("chunk", "decode300", "decode64")):
        assert r["status"] == 0
        bits += check(r["logits"], s.logits(), 3e-2, name)
        assert r["argmax"] == orc.Sampler().sample(s.logits())[1]
    assert np.array_equal(m.seq_read_kv(a, 11), sa.kv(11))
    assert bits == 0


def test_f16_continuous_batch_greedy_tokens():
    print("case: full-shape F16 continuous batch, 4 prompts, greedy", flush=True)
    c, t = synth.in_memory(FULL, "f16", seed=22)
    m = cohx.Model(c, t, max_lanes=4, max_rows=4, max_seqs=4, max_context=128)
    o = orc.Model(c, t, threads=16)
    rng = np.random.default_rng(3)
    prompts = [[int(v) for v in rng.integers(0, c["vocabulary"], n)] for n in (2, 4, 6, 8)]
    opts = cohx.GenerationOptions(max_tokens=3)
    states = [m.begin_generation(p, opts) for p in prompts]
    while not all(s.is_finished() for s in states):
        lanes = [s for s in states if s.needs_forward()]
        if lanes:
            m.step_batch(lanes)
        for s in states:
            s.sample()
    for p, st in zip(prompts, states):
        sess = o.session(128)
        for tok in p:
            o.forward_batch([sess], [tok])
        ids = []
        for _ in range(3):
            tok = orc.Sampler().sample(sess.logits())[1]
            ids.append(tok)
            if len(ids) < 3:
                o.forward_batch([sess], [tok])
        print(f"prompt {len(p)}: gpu {st.token_ids()} oracle {ids}", flush=True)
        assert st.token_ids() == ids


def test_q4_0_shared_prefix_groups_decode():
    """Config 4's form at the full shape, shortened so the oracle finishes in
    seconds: Q4_0 weights; two groups of lanes, each forked from one 48-token
    prefix (three full pages shared, copy on write), decoding together.  Every
    lane's logits equal the oracle's unshared recomputation bit for bit, and
    greedy tokens match."""
    print("case: full-shape Q4_0 shared-prefix groups", flush=True)
    c, t = synth.in_memory(FULL, "q4_0", seed=23)
    m = cohx.Model(c, t, max_lanes=8, max_rows=128, max_seqs=8, max_context=128)
    o = orc.Model(c, t, threads=16)
    rng = np.random.default_rng(4)
    P, per_group = 48, 2
    prefixes = [[int(v) for v in rng.integers(0, c["vocabulary"], P)] for _ in range(2)]
    bases = [m.seq_alloc() for _ in prefixes]
    res = m.step([dict(seq=b, tokens=p) for b, p in zip(bases, prefixes)])
    assert all(r["status"] == 0 for r in res)
    lanes = [m.seq_fork(b, P) for b in bases for _ in range(per_group)]
    for b in bases:
        m.seq_free(b)
    sessions = [o.session(128) for _ in lanes]
    for j in range(P):
        o.forward_batch(sessions, [prefixes[i // per_group][j] for i in range(len(lanes))])
    toks = [int(v) for v in rng.integers(0, c["vocabulary"], len(lanes))]
    bits = 0
    for step in range(2):
        res = m.step([dict(seq=a, tokens=[tk], logits=True) for a, tk in zip(lanes, toks)])
        o.forward_batch(sessions, toks)
        nxt = []
        for i, r in enumerate(res):
            assert r["status"] == 0
            bits += check(r["logits"], sessions[i].logits(), 3e-2, f"step {step} lane {i}")
            assert r["argmax"] == orc.Sampler().sample(sessions[i].logits())[1]
            nxt.append(r["argmax"])
        toks = nxt
    for a in lanes[1:per_group]:
        assert np.array_equal(m.seq_read_kv(a, 7)[:P], m.seq_read_kv(lanes[0], 7)[:P])
    assert bits == 0
