"""cohx_step_noalloc (device scratch from the library's static array, no
allocation) against cohx_step on the same context: two calls in a row, the
second with a smaller batch, each equal bit for bit (logits of every lane,
greedy ids, appended K/V rows); a batch whose scratch exceeds the array is
refused with COHX_RESOURCE and leaves its sequences untouched.

F16 in the packed-prefill regime: cohx_step runs the linears of a step with
prompt rows as library GEMMs, while the allocation-free call keeps them on the
in-house matrix-core kernel; both are f32 sums held to the regime's tolerance
(logits max-abs 1e-2, K/V rows 1e-3), so that step is compared within it, and
bit for bit with the library switched off (COHX_GEMM_LIB=0)."""
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


@pytest.mark.parametrize("dtype,lib", [("q8_0", True), ("f16", False), ("f16", True)])
def test_noalloc_step_equals_step(dtype, lib, monkeypatch):
    print(f"case: noalloc vs step {dtype} (library GEMMs {'on' if lib else 'off'})", flush=True)
    if not lib:
        monkeypatch.setenv("COHX_GEMM_LIB", "0")
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
        exact = not (dtype == "f16" and lib and k == 0)
        for (ws, wa, wl), (gs, ga, gl) in zip(want[0], got[0]):
            assert ws == gs == 0
            assert (wl is None) == (gl is None)
            if exact:
                assert wa == ga
                if wl is not None:
                    assert np.array_equal(wl, gl), f"call {k}: logits differ"
            elif wl is not None:
                a, b = wl.view(np.float32), gl.view(np.float32)
                diff = float(np.abs(a - b).max())
                print(f"call {k}: logits max-abs {diff:.3g}", flush=True)
                assert diff <= 1e-2
                top = np.sort(a)[-2:]
                if top[1] - top[0] > 2e-2:
                    assert wa == ga
        for (wk, wv), (gk, gv) in zip(want[1], got[1]):
            if exact:
                assert np.array_equal(wk, gk) and np.array_equal(wv, gv), f"call {k}: K/V rows differ"
            else:
                assert float(np.abs(wk - gk).max()) <= 1e-3 and float(np.abs(wv - gv).max()) <= 1e-3
    m.close()


def test_noalloc_refuses_a_step_beyond_its_scratch():
    print("case: noalloc scratch limit", flush=True)
    c, t = synth.in_memory(TINY, "q8_0", seed=43)
    m = cohx.Model(c, t, max_lanes=2, max_rows=256, max_seqs=2, max_context=4096)
    s = m.seq_alloc()
    m.seq_fill_synthetic(s, 3800, 6, 0)
    # 256 rows attending over up to 4056 positions: the score rows alone take
    # 256 x 2 heads x 4056 x 32 bytes, more than the 64 MiB array
    lanes = [dict(seq=s, tokens=list(range(256)))]
    with pytest.raises(cohx.CohxError) as e:
        m.step(lanes, noalloc=True)
    assert e.value.code == cohx.RESOURCE and "scratch" in str(e.value)
    assert m.seq_length(s) == 3800
    res = m.step([dict(seq=s, tokens=[1, 2, 3], logits=True)], noalloc=True)
    assert res[0]["status"] == 0 and m.seq_length(s) == 3803
    m.close()
