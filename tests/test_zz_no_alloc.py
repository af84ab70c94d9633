"""cohx_step_noalloc (device scratch from the library's static array, no
allocation) against cohx_step on the same context: two calls in a row, the
second with a smaller batch, each equal bit for bit (logits of every lane,
greedy ids, appended K/V rows); a batch whose scratch exceeds the array is
refused with COHX_RESOURCE and leaves its sequences untouched.

F16 in the packed-prefill regime: both entry points run the same matrix-core
GEMM over the step's rows, so that step is compared bit for bit too."""
import numpy as np
import pytest

import cohx
import synth

pytestmark = pytest.mark.gpu

TINY = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2, vocabulary=300,
                    context=4096)


def snapshot(m, seqs, starts, res):
    kv = [(m.seq_read_kv_rows(s, l, n, m.seq_length(s) - n),
           m.seq_read_kv_rows(s, l, n, m.seq_length(s) - n, True))
          for s, n in zip(seqs, starts) for l in range(m.config["layers"])]
    return [(r["status"], r["argmax"], None if r["logits"] is None else r["logits"].view(np.uint32).copy())
            for r in res], kv


@pytest.mark.parametrize("dtype", ["q8_0", "f16"])
def test_noalloc_step_equals_step(dtype):
    print(f"case: noalloc vs step {dtype}", flush=True)
    c, t = synth.in_memory(TINY, dtype, seed=41)
    m = cohx.Model(c, t, max_lanes=8, max_rows=160, max_seqs=8, max_context=1024)
    seqs = [m.seq_alloc() for _ in range(5)]
    for i, n in enumerate((0, 300, 17, 700, 64)):
        m.seq_fill_synthetic(seqs[i], n, 5, i)
    rng = np.random.default_rng(42)
    calls = [  # a prefill chunk with decode rows (140 rows: F16 takes the matrix cores), then decode only
        [(0, 130, True), (1, 1, True), (2, 4, False), (3, 1, True), (4, 4, True)],
        [(1, 1, True), (3, 1, False)],
    ]
    for k, spec in enumerate(calls):
        lanes = [dict(seq=seqs[i], tokens=[int(v) for v in rng.integers(0, c["vocabulary"], n)], logits=lg)
                 for i, n, lg in spec]
        used = [seqs[i] for i, _, _ in spec]
        starts = [m.seq_length(s) for s in used]
        print(f"call {k}: {len(lanes)} lanes, {sum(n for _, n, _ in spec)} rows", flush=True)
        want = snapshot(m, used, starts, m.step(lanes))
        for s, n in zip(used, starts):
            m.seq_truncate(s, n)
        got = snapshot(m, used, starts, m.step(lanes, noalloc=True))
        for (ws, wa, wl), (gs, ga, gl) in zip(want[0], got[0]):
            assert ws == gs == 0
            assert (wl is None) == (gl is None)
            assert wa == ga
            if wl is not None:
                assert np.array_equal(wl, gl), f"call {k}: logits differ"
        for (wk, wv), (gk, gv) in zip(want[1], got[1]):
            assert np.array_equal(wk, gk) and np.array_equal(wv, gv), f"call {k}: K/V rows differ"
    m.close()


def test_noalloc_refuses_a_step_beyond_its_scratch():
    print("case: noalloc scratch limit", flush=True)
    c, t = synth.in_memory(TINY, "q8_0", seed=43)
    m = cohx.Model(c, t, max_lanes=2, max_rows=320, max_seqs=2, max_context=4096)
    s = m.seq_alloc()
    m.seq_fill_synthetic(s, 3700, 6, 0)
    # 320 rows attending over up to 4020 positions: the score rows alone take
    # 320 rows x 2 KV heads x 4020 positions x 8 slots x 4 bytes = 82.3 MB,
    # more than the 64 MiB (67.1 MB) array
    lanes = [dict(seq=s, tokens=list(range(320)))]
    with pytest.raises(cohx.CohxError) as e:
        m.step(lanes, noalloc=True)
    assert e.value.code == cohx.RESOURCE and "scratch" in str(e.value)
    assert m.seq_length(s) == 3700
    res = m.step([dict(seq=s, tokens=[1, 2, 3], logits=True)], noalloc=True)
    assert res[0]["status"] == 0 and m.seq_length(s) == 3703
    m.close()


def test_noalloc_sizes_scratch_from_lanes_that_can_run():
    """A lane with a bogus explicit start position (or a dead sequence) is
    refused on its own as INVALID_REQUEST, as cohx_step refuses it; it must
    not inflate the scratch estimate and fail the whole call."""
    print("case: noalloc with an invalid lane beside valid ones", flush=True)
    c, t = synth.in_memory(TINY, "q8_0", seed=44)
    m = cohx.Model(c, t, max_lanes=4, max_rows=64, max_seqs=4, max_context=4096)
    a, b = m.seq_alloc(), m.seq_alloc()
    m.seq_fill_synthetic(a, 50, 7, 0)
    m.seq_fill_synthetic(b, 20, 7, 1)
    # start 4000 with 40 tokens would need scores over 4040 positions for 64
    # rows; only lane b (start at its length 20) can run
    lanes = [dict(seq=a, tokens=list(range(40)), start=4000), dict(seq=b, tokens=[3, 4], logits=True)]
    want = m.step(lanes)
    m.seq_truncate(b, 20)
    got = m.step(lanes, noalloc=True)
    assert want[0]["status"] == got[0]["status"] == cohx.INVALID_REQUEST
    assert want[1]["status"] == got[1]["status"] == 0
    assert want[1]["argmax"] == got[1]["argmax"]
    assert np.array_equal(want[1]["logits"].view(np.uint32), got[1]["logits"].view(np.uint32))
    assert m.seq_length(a) == 50 and m.seq_length(b) == 22
    m.close()
