"""Reduction orders under wide exponent ranges.

Four f64 sums of the exact path run in a fixed order that differs from the
reference's sequential loops (the rms_norm sum of squares, the softmax
denominator, the attention value sums, and the F16 dot under 16 rows).  Each
sums f32 values in f64, so the two orders can differ only in the last f64
bits, and then only when a partial sum rounds, which needs terms that span
more than ~29 binades; the f32 result then differs only when the f64 value
sits within that difference of an f32 rounding boundary.

Synthetic N(0, 0.02) weights never get there.  These models scale every matrix
row, norm weight and bias element by 2^U[-6, 5]: K/V rows span about 2^-22 to
2^8, activations and logits (up to ~130) likewise.  A 4096-token prompt and
a 1500-token prompt are prefilled in chunks beside each other, then decoded,
and every sampled row's logits and every appended K/V row are compared with
the oracle bit for bit.  The number of differing bits is printed.
"""
import os

import numpy as np
import pytest

import cohx
import orc
import synth

pytestmark = pytest.mark.gpu

CFG = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2, vocabulary=300,
                   context=4200)


@pytest.mark.parametrize("dtype", ["q8_0", "f16"])
def test_wide_exponent_range_long_context_matches_oracle(dtype):
    print(f"case: wide exponent range, contexts to 4096, {dtype}", flush=True)
    c, t = synth.in_memory(CFG, dtype, seed=41, spread=(-6, 5))
    old = os.environ.get("COHX_PREFILL_MFMA")
    os.environ["COHX_PREFILL_MFMA"] = "0"  # the exact kernels at every row count
    try:
        m = cohx.Model(c, t, max_lanes=4, max_rows=1100, max_seqs=4, max_context=4200)
    finally:
        if old is None:
            del os.environ["COHX_PREFILL_MFMA"]
        else:
            os.environ["COHX_PREFILL_MFMA"] = old
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(2)
    prompts = [[int(v) for v in rng.integers(0, 300, n)] for n in (4096, 1500)]
    chunks = [512, 500]
    seqs = [m.seq_alloc() for _ in prompts]
    sess = [o.session(4200) for _ in prompts]
    cur = [0, 0]
    nxt = [None, None]
    differing, compared, worst = 0, 0, 0.0
    for step in range(12):
        lanes, idx = [], []
        for i, p in enumerate(prompts):
            if cur[i] < len(p):
                toks = p[cur[i]:cur[i] + chunks[i]]
            else:
                toks = [nxt[i]]
            lanes.append(dict(seq=seqs[i], tokens=toks, logits=True))
            idx.append((i, toks))
        res = m.step(lanes)
        for (i, toks), r in zip(idx, res):
            assert r["status"] == 0, (step, i, r["status"])
            for tok in toks:
                assert o.forward_batch([sess[i]], [tok])[0] == 0
            want = sess[i].logits()
            bad = int((r["logits"].view(np.uint32) != want.view(np.uint32)).sum())
            worst = max(worst, float(np.abs(r["logits"].astype(np.float64) - want).max()))
            differing += bad
            compared += want.size
            nxt[i] = int(orc.Sampler().sample(want)[1])
            assert r["argmax"] == nxt[i], (step, i)
            cur[i] = min(cur[i] + len(toks), len(prompts[i])) if cur[i] < len(prompts[i]) else cur[i]
    kv_bad = 0
    for i in range(2):
        n = m.seq_length(seqs[i])
        assert n == sess[i].position
        for layer in range(c["layers"]):
            for values in (False, True):
                got, want = m.seq_read_kv(seqs[i], layer, values), sess[i].kv(layer, values)
                kv_bad += int((got.view(np.uint32) != want.view(np.uint32)).sum())
    print(f"{dtype}: {differing} of {compared} logits differ in bits (max-abs {worst:.3g}); "
          f"{kv_bad} K/V values differ", flush=True)
    assert differing == 0 and kv_bad == 0
