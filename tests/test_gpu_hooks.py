"""Cooperation with the scheduler during a step (cohx_step_hooked,
cohx_step_batch_hooked): the WorkYield hook (multimodal.rs:6, called between
layers by qwen35/execution.rs:306-309 and used by scheduler/batching.rs:
229-239 to release the compute permit) and per-lane cancellation
(inference.rs:32-68).  Results with hooks equal the plain step's bit for bit;
a stop request fails the step as a shared Cancelled with no lane advanced; a
lane cancelled before or during the step fails alone and its peers are
unchanged."""
import numpy as np
import pytest

import cohx
import orc
import synth

pytestmark = pytest.mark.gpu

TINY = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                    vocabulary=300, context=512)


def model(dtype="q8_0"):
    c, t = synth.in_memory(TINY, dtype, seed=51)
    return c, t, cohx.Model(c, t, max_lanes=4, max_rows=64, max_seqs=8, max_context=256)


def lanes_for(seqs, toks):
    return [dict(seq=s, tokens=tk, logits=True) for s, tk in zip(seqs, toks)]


def test_yield_hook_runs_while_the_device_computes_and_changes_nothing():
    print("case: yield hook, same bits as the plain step", flush=True)
    c, t, m = model()
    toks = [[3, 14, 15, 92], [65], [35, 89]]
    a = [m.seq_alloc() for _ in toks]
    b = [m.seq_alloc() for _ in toks]
    plain = m.step(lanes_for(a, toks))
    calls = []
    hooked = m.step(lanes_for(b, toks), yield_fn=lambda: calls.append(1) and False)
    print(f"yield called {len(calls)} times", flush=True)
    assert calls
    for p, h in zip(plain, hooked):
        assert p["status"] == 0 and h["status"] == 0
        assert np.array_equal(p["logits"], h["logits"]) and p["argmax"] == h["argmax"]
    assert [m.seq_length(s) for s in b] == [len(x) for x in toks]


def test_yield_stop_is_a_shared_cancellation_and_advances_nothing():
    print("case: yield hook asks to stop", flush=True)
    c, t, m = model()
    o = orc.Model(c, t, threads=8)
    s = m.seq_alloc()
    with pytest.raises(cohx.CohxError) as e:
        m.step(lanes_for([s], [[7, 8, 9]]), yield_fn=lambda: True)
    assert e.value.code == cohx.CANCELLED
    assert m.seq_length(s) == 0
    # the same sequence then steps as if the cancelled step never happened
    r = m.step(lanes_for([s], [[7, 8, 9]]))[0]
    sess = o.session(256)
    for tok in (7, 8, 9):
        o.forward_batch([sess], [tok])
    assert r["status"] == 0 and np.array_equal(r["logits"], sess.logits())


def test_lane_cancellation_before_and_during_the_step():
    print("case: per-lane cancellation flags", flush=True)
    c, t, m = model()
    o = orc.Model(c, t, threads=8)
    seqs = [m.seq_alloc() for _ in range(3)]
    toks = [[11, 12], [21], [31, 32, 33]]
    flags = np.array([0, 1, 0], np.uint32)  # lane 1 cancelled before the launch
    res = m.step(lanes_for(seqs, toks), cancel=flags)
    assert res[1]["status"] == cohx.CANCELLED and m.seq_length(seqs[1]) == 0
    sess = [o.session(256) for _ in range(3)]
    for i in (0, 2):
        for tok in toks[i]:
            o.forward_batch([sess[i]], [tok])
        assert res[i]["status"] == 0 and np.array_equal(res[i]["logits"], sess[i].logits())
        assert m.seq_length(seqs[i]) == len(toks[i])
    # lane 2 cancelled while the device computes (from the yield hook)
    flags[:] = 0

    def cancel_lane_2():
        flags[2] = 1
        return False

    res = m.step(lanes_for(seqs, [[13], [22], [34]]), yield_fn=cancel_lane_2, cancel=flags)
    assert res[2]["status"] == cohx.CANCELLED and m.seq_length(seqs[2]) == 3
    for i, tok in ((0, 13), (1, 22)):
        o.forward_batch([sess[i]], [tok])
        assert res[i]["status"] == 0 and np.array_equal(res[i]["logits"], sess[i].logits())


def test_generation_cancelled_during_a_batched_step():
    """cohx_gen_cancel from the yield hook (another thread in a server): the
    decode lane's forward is dropped and the generation finishes as
    cancelled; its peer generates exactly what it generates alone."""
    print("case: generation cancelled mid-step", flush=True)
    c, t, m = model()
    opts = cohx.GenerationOptions(max_tokens=6)
    a = m.begin_generation([5, 6, 7], opts)
    b = m.begin_generation([8, 9], opts)
    assert a.compatible(b)
    alone = cohx.generate(m, [8, 9], opts).token_ids()
    steps = 0
    while not b.is_finished():
        live = [s for s in (a, b) if s.needs_forward()]
        if live:
            hook = (lambda: a.cancel() or False) if steps == 4 else (lambda: False)
            m.step_batch(live, yield_fn=hook)
            steps += 1
        for s in (a, b):
            if not s.is_finished():
                try:
                    s.sample()
                except cohx.CohxError as e:
                    assert s is a and e.code == cohx.CANCELLED
    assert a.is_finished() and a.finish_reason() == "cancelled"
    assert b.token_ids() == alone
    print(f"a: {a.token_ids()} (cancelled), b: {b.token_ids()}", flush=True)
