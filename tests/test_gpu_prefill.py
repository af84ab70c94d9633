"""Packed-prefill regime (F16 weights, 128+ packed rows): the linears run on
the matrix cores with f32 sums instead of the reference's f64 sums
(cpu.rs:31-35), so this regime is checked to the north_star tolerance for F16
logits (max-abs 1e-2), not bit for bit.  Q8_0/Q5_0/Q4_0 weights take the
regime's quantized GEMM (weights dequantized to binary16 in LDS, binary16
activations, f32 sums) where the reference multiplies Q8_0-quantized
activations with the int8 blocks (quant.rs:245-292): checked to the
quantized tolerance (max-abs 3e-2) on 2-layer models, and at the full
24-layer shape against the reference's own response to a binary16-sized
perturbation (its Q8_0 activation rounding makes that path ill-conditioned
there; see test_mixed_prefill_and_decode_full_shape).  Greedy ids must agree wherever the
reference's top-2 margin exceeds the measured difference.  The same steps
with the matrix-core path switched off (COHX_PREFILL_MFMA=0) stay bit-exact
against the oracle, and so does a decode-only step of the regime's width
(the regime is for steps that carry prompt rows)."""
import os

import numpy as np
import pytest

import cohx
import gguf
import orc
import synth

pytestmark = pytest.mark.gpu

TOL = 1e-2
TOL_Q = 3e-2  # quantized weights


def make(cfg, t, mfma, **kw):
    old = os.environ.get("COHX_PREFILL_MFMA")
    os.environ["COHX_PREFILL_MFMA"] = "1" if mfma else "0"
    try:
        return cohx.Model(cfg, t, **kw)
    finally:
        if old is None:
            del os.environ["COHX_PREFILL_MFMA"]
        else:
            os.environ["COHX_PREFILL_MFMA"] = old


def close(got, want, what, tol=TOL):
    diff = float(np.abs(got.astype(np.float64) - want).max())
    order = np.sort(want)
    margin = float(order[-1] - order[-2])
    print(f"{what}: max-abs {diff:.3g}, top1-top2 margin {margin:.3g}", flush=True)
    assert diff <= tol, what
    if margin > 2 * diff:
        assert int(np.argmax(got)) == int(np.argmax(want)), what
    return diff


def test_prefill_chunk_matches_oracle_within_tolerance():
    print("case: tiny F16 prefill chunk of 150 rows, matrix cores vs oracle", flush=True)
    cfg = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                       vocabulary=300, context=512)
    c, t = synth.in_memory(cfg, "f16", seed=31)
    kw = dict(max_lanes=4, max_rows=256, max_seqs=4, max_context=256)
    mm, me = make(c, t, True, **kw), make(c, t, False, **kw)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(5)
    chunk = [int(v) for v in rng.integers(0, c["vocabulary"], 150)]
    sm, se = mm.seq_alloc(), me.seq_alloc()
    rm = mm.step([dict(seq=sm, tokens=chunk, logits=True)])[0]
    re = me.step([dict(seq=se, tokens=chunk, logits=True)])[0]
    s = o.session(256)
    for tok in chunk:
        o.forward_batch([s], [tok])
    want = s.logits()
    assert rm["status"] == 0 and re["status"] == 0
    assert np.array_equal(re["logits"], want)  # exact kernels: bit for bit
    close(rm["logits"], want, "matrix-core chunk logits")
    for layer in range(c["layers"]):
        kv_diff = float(np.abs(mm.seq_read_kv(sm, layer) - s.kv(layer)).max())
        assert kv_diff < 1e-3, (layer, kv_diff)
    # decoding on after the chunk: one-row steps are exact again
    tok = int(np.argmax(want))
    r1 = mm.step([dict(seq=sm, tokens=[tok], logits=True)])[0]
    o.forward_batch([s], [tok])
    close(r1["logits"], s.logits(), "decode after matrix-core chunk")


@pytest.mark.parametrize("dtype", ["q8_0", "q5_0", "q4_0"])
def test_quantized_prefill_matches_oracle_within_tolerance(dtype):
    """A quantized model's prefill chunk of 150 rows after 40 prompt tokens,
    beside a decode lane (head_dim 64: the chunk attention on the matrix
    cores too), against the oracle: logits and appended K/V rows within the
    quantized tolerance, greedy ids equal where the oracle's margin allows;
    the same step with the regime off is bit-exact."""
    print(f"case: {dtype} prefill chunk of 150 rows + a decode lane, quantized GEMM vs oracle", flush=True)
    cfg = synth.config(layers=2, hidden=256, intermediate=512, heads=4, kv_heads=2,
                       vocabulary=500, context=512)
    c, t = synth.in_memory(cfg, dtype, seed=34)
    kw = dict(max_lanes=4, max_rows=256, max_seqs=4, max_context=512)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(8)
    head = [int(v) for v in rng.integers(0, c["vocabulary"], 40)]
    chunk = [int(v) for v in rng.integers(0, c["vocabulary"], 150)]
    sa, sb = o.session(512), o.session(512)
    for tok in head:
        o.forward_batch([sa], [tok])
    sb.fill_synthetic(300, 9, 1)
    for tok in chunk:
        o.forward_batch([sa], [tok])
    o.forward_batch([sb], [77])
    want = [sa.logits(), sb.logits()]
    for mfma in (True, False):
        m = make(c, t, mfma, **kw)
        a, b = m.seq_alloc(), m.seq_alloc()
        assert m.step([dict(seq=a, tokens=head)])[0]["status"] == 0
        m.seq_fill_synthetic(b, 300, 9, 1)
        res = m.step([dict(seq=a, tokens=chunk, logits=True), dict(seq=b, tokens=[77], logits=True)])
        assert res[0]["status"] == 0 and res[1]["status"] == 0
        if not mfma:
            for r, w in zip(res, want):
                assert np.array_equal(r["logits"], w)  # exact kernels: bit for bit
            m.close()
            continue
        close(res[0]["logits"], want[0], f"{dtype} chunk lane", TOL_Q)
        close(res[1]["logits"], want[1], f"{dtype} decode lane", TOL_Q)
        for layer in range(c["layers"]):
            for v in (False, True):
                kv = float(np.abs(m.seq_read_kv(a, layer, v) - sa.kv(layer, v)).max())
                print(f"layer {layer} {'V' if v else 'K'} rows: max-abs {kv:.3g}", flush=True)
                assert kv <= TOL_Q, (layer, v, kv)
        m.close()


def scaled(t, name, factor):
    """The model with tensor `name` (f32) multiplied by `factor` (in f32)."""
    x = t[name]
    f = (x.data.view(np.float32) * np.float32(factor)).astype(np.float32)
    out = dict(t)
    out[name] = gguf.Tensor(x.name, x.shape, x.dtype, f.view(np.uint8))
    return out


def mixed_step(m, chunks, kv):
    lanes = []
    for ch in chunks:
        lanes.append(dict(seq=m.seq_alloc(), tokens=ch, logits=True))
    for i, n in enumerate(kv):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, n, 8, i)
        lanes.append(dict(seq=s, tokens=[int(10 + i)], logits=True))
    res = m.step(lanes)
    assert all(r["status"] == 0 for r in res)
    return [r["logits"].astype(np.float64) for r in res]


@pytest.mark.parametrize("dtype", ["f16", "q8_0"])
def test_mixed_prefill_and_decode_full_shape(dtype):
    """Config 3's form at the full shape, shortened: two prefill chunks plus
    decode rows over seeded KV in one packed step; the matrix-core context
    against the exact context (itself pinned to the oracle by the other GPU
    tests).

    F16: every lane within 1e-2.  Q8_0: at 24 layers the reference's
    quantized path is ill-conditioned.  Its Q8_0 activation rounding turns a
    last-bit difference into a whole quantization step (which then feeds
    every later layer), so a 1-ulp change of one norm weight vector already
    moves its own logits by about 0.07 max-abs, past the 3e-2 quantized
    tolerance (which the 2-layer tests meet).  The regime rounds operands to
    binary16, so its yardstick is the reference's own response to one
    binary16 step: the exact context with blk.0.attn_norm.weight scaled by
    1 + 2^-11, measured here on the same lanes (about 0.08 max-abs on the
    prefill lanes and 0.2 on the decode lanes over synthetic KV).  Each
    lane's max-abs and rms distance from the exact context must stay within
    twice that lane's yardstick."""
    print(f"case: full-shape {dtype} mixed packed step, matrix cores vs exact", flush=True)
    c, t = synth.in_memory(synth.config(), dtype, seed=32)
    kw = dict(max_lanes=8, max_rows=512, max_seqs=8, max_context=1024)
    rng = np.random.default_rng(6)
    chunks = [[int(v) for v in rng.integers(0, c["vocabulary"], n)] for n in (200, 131)]
    kv = [300, 900, 64, 512]
    got = mixed_step(make(c, t, True, **kw), chunks, kv)
    want = mixed_step(make(c, t, False, **kw), chunks, kv)
    if dtype == "f16":
        worst = max(close(a, b, f"lane {i}") for i, (a, b) in enumerate(zip(got, want)))
        print(f"worst lane max-abs {worst:.3g}", flush=True)
        return
    moved = mixed_step(make(c, scaled(t, "blk.0.attn_norm.weight", 1 + 2**-11), False, **kw), chunks, kv)
    rms = lambda d: float(np.sqrt(np.mean(d * d)))
    for i, (a, b, y) in enumerate(zip(got, want, moved)):
        d_reg, d_y = a - b, y - b
        print(f"lane {i}: regime vs exact max-abs {np.abs(d_reg).max():.3g} rms {rms(d_reg):.3g}; "
              f"exact under a 2^-11 norm change max-abs {np.abs(d_y).max():.3g} rms {rms(d_y):.3g}",
              flush=True)
        assert np.abs(d_y).max() > 0, i  # the yardstick is not degenerate
        assert np.abs(d_reg).max() <= 2 * np.abs(d_y).max(), i
        assert rms(d_reg) <= 2 * rms(d_y), i
        order = np.sort(b)
        if order[-1] - order[-2] > 2 * float(np.abs(d_reg).max()):
            assert int(np.argmax(a)) == int(np.argmax(b)), i


def test_chunk_attention_matches_oracle_within_tolerance():
    """head_dim 64 (the matrix-core chunk attention's shape): a prefill chunk
    continuing a sequence that already holds 40 tokens, next to a decode lane;
    logits of both lanes against the oracle."""
    print("case: D=64 chunk attention, 170-row chunk after 40 tokens + a decode lane", flush=True)
    cfg = synth.config(layers=2, hidden=256, intermediate=512, heads=4, kv_heads=2,
                       vocabulary=500, context=512)
    c, t = synth.in_memory(cfg, "f16", seed=33)
    kw = dict(max_lanes=4, max_rows=256, max_seqs=4, max_context=512)
    m = make(c, t, True, **kw)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(7)
    head = [int(v) for v in rng.integers(0, c["vocabulary"], 40)]
    chunk = [int(v) for v in rng.integers(0, c["vocabulary"], 170)]
    a, b = m.seq_alloc(), m.seq_alloc()
    assert m.step([dict(seq=a, tokens=head)])[0]["status"] == 0
    m.seq_fill_synthetic(b, 300, 9, 1)
    sa, sb = o.session(512), o.session(512)
    for tok in head:
        o.forward_batch([sa], [tok])
    sb.fill_synthetic(300, 9, 1)
    res = m.step([dict(seq=a, tokens=chunk, logits=True), dict(seq=b, tokens=[77], logits=True)])
    for tok in chunk:
        o.forward_batch([sa], [tok])
    o.forward_batch([sb], [77])
    assert res[0]["status"] == 0 and res[1]["status"] == 0
    close(res[0]["logits"], sa.logits(), "chunk lane")
    close(res[1]["logits"], sb.logits(), "decode lane")
    for layer in range(c["layers"]):
        assert float(np.abs(m.seq_read_kv(a, layer, True) - sa.kv(layer, True)).max()) < 1e-3
    # a step of chunk rows only (no row left to the exact passes), 130 rows
    # ending at a ragged 2-row tile
    more = [int(v) for v in rng.integers(0, c["vocabulary"], 130)]
    res = m.step([dict(seq=a, tokens=more, logits=True)])
    for tok in more:
        o.forward_batch([sa], [tok])
    assert res[0]["status"] == 0
    close(res[0]["logits"], sa.logits(), "chunk-only step")


def test_chunk_attention_over_several_key_segments():
    """Chunk rows whose keys span two and three 1024-key segments (segment
    records merged by the combine pass) and end inside a 64-key tile of the
    staged key images: a 160-row chunk after 1500 cached tokens and a
    24-row chunk after 2100, next to a decode lane; logits of every lane and
    the appended K/V rows against the oracle."""
    print("case: D=64 chunk attention across key segments", flush=True)
    cfg = synth.config(layers=2, hidden=256, intermediate=512, heads=4, kv_heads=2,
                       vocabulary=500, context=4096)
    c, t = synth.in_memory(cfg, "f16", seed=35)
    m = make(c, t, True, max_lanes=4, max_rows=256, max_seqs=4, max_context=2400)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(9)
    fill = (1500, 2100, 700)
    seqs = [m.seq_alloc() for _ in fill]
    sess = [o.session(2400) for _ in fill]
    for i, n in enumerate(fill):
        m.seq_fill_synthetic(seqs[i], n, 21, i)
        sess[i].fill_synthetic(n, 21, i)
    toks = [[int(v) for v in rng.integers(0, c["vocabulary"], n)] for n in (160, 24, 1)]
    res = m.step([dict(seq=s, tokens=tk, logits=True) for s, tk in zip(seqs, toks)])
    for i, tk in enumerate(toks):
        for tok in tk:
            assert o.forward_batch([sess[i]], [tok])[0] == 0
    for i, what in enumerate(("two segments", "three segments", "decode lane")):
        assert res[i]["status"] == 0
        close(res[i]["logits"], sess[i].logits(), what)
    for i, n in enumerate(fill):
        for layer in range(c["layers"]):
            for values in (False, True):
                got = m.seq_read_kv_rows(seqs[i], layer, n, len(toks[i]), values)
                assert float(np.abs(got - sess[i].kv(layer, values)[n:]).max()) < 1e-3, (i, layer, values)


def test_regime_head_on_matrix_cores_matches_oracle():
    """A packed-prefill step with 18 logit rows: the F16 head runs on the
    matrix cores too (f32 sums), every lane within tolerance of the oracle,
    greedy ids equal where the margin allows; with the regime off the same
    step is bit-exact."""
    print("case: regime step with 18 lanes (head on the matrix cores)", flush=True)
    cfg = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                       vocabulary=700, context=512)
    c, t = synth.in_memory(cfg, "f16", seed=35)
    kw = dict(max_lanes=20, max_rows=256, max_seqs=20, max_context=256)
    mm, me = make(c, t, True, **kw), make(c, t, False, **kw)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(11)
    chunk = [int(v) for v in rng.integers(0, c["vocabulary"], 140)]
    toks = [int(v) for v in rng.integers(0, c["vocabulary"], 17)]
    res = {}
    for name, m in (("mfma", mm), ("exact", me)):
        a = m.seq_alloc()
        dec = [m.seq_alloc() for _ in toks]
        for i, s in enumerate(dec):
            m.seq_fill_synthetic(s, 20 + 3 * i, 13, i)
        res[name] = m.step([dict(seq=a, tokens=chunk, logits=True)] +
                           [dict(seq=s, tokens=[tk], logits=True) for s, tk in zip(dec, toks)])
    sa = o.session(256)
    for tok in chunk:
        o.forward_batch([sa], [tok])
    sess = []
    for i in range(len(toks)):
        s = o.session(256)
        s.fill_synthetic(20 + 3 * i, 13, i)
        sess.append(s)
    o.forward_batch(sess, toks)
    want = [sa.logits()] + [s.logits() for s in sess]
    for i, w in enumerate(want):
        assert res["mfma"][i]["status"] == 0 and res["exact"][i]["status"] == 0
        assert np.array_equal(res["exact"][i]["logits"], w), i
        close(res["mfma"][i]["logits"], w, f"lane {i}")
        if res["mfma"][i]["argmax"] != res["exact"][i]["argmax"]:
            order = np.sort(w)
            assert order[-1] - order[-2] <= 2 * float(np.abs(res["mfma"][i]["logits"] - w).max()), i


def test_wide_f16_decode_step_stays_exact():
    """A decode-only F16 step of 130 rows, as wide as the regime's steps,
    keeps the exact kernels (one f64 chain per dot, the exact head): every
    lane's logits and greedy id equal the oracle's bit for bit, with the
    regime switched on."""
    print("case: F16 decode-only step of 130 lanes with the regime on: exact", flush=True)
    cfg = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                       vocabulary=300, context=512)
    c, t = synth.in_memory(cfg, "f16", seed=37)
    n = 130
    m = make(c, t, True, max_lanes=n, max_rows=n, max_seqs=n, max_context=256)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(17)
    toks = [int(v) for v in rng.integers(0, c["vocabulary"], n)]
    seqs, sess = [], []
    for i in range(n):
        s = m.seq_alloc()
        m.seq_fill_synthetic(s, 10 + i, 19, i)
        seqs.append(s)
        so = o.session(256)
        so.fill_synthetic(10 + i, 19, i)
        sess.append(so)
    res = m.step([dict(seq=s, tokens=[tk], logits=True) for s, tk in zip(seqs, toks)])
    for u in range(0, n, 16):  # the oracle's units of at most 16 lanes
        o.forward_batch(sess[u:u + 16], toks[u:u + 16])
    differ = 0
    for i, (r, so) in enumerate(zip(res, sess)):
        assert r["status"] == 0, i
        want = so.logits()
        differ += int(np.count_nonzero(r["logits"].view(np.uint32) != want.view(np.uint32)))
        assert r["argmax"] == orc.Sampler().sample(want)[1], i
    print(f"case: {differ} differing logits of {n * c['vocabulary']}", flush=True)
    assert differ == 0
    m.close()
