"""Pins of the Qwen3.5 oracle (oracle/orc_qwen35.c) before it is used as the
checker: the reference's own delta-rule fixture, the closed forms its kernel
tests assert (qwen35/kernels.rs:270-375), an independent float64 textbook of
the hybrid step, and the batched == individual invariant."""
import json
import os

import numpy as np

import orc
import synth35
from qwen35_ref import Qwen35F64

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def tiny():
    return synth35.config(layers=4, hidden=64, intermediate=96, vocabulary=300, heads=2,
                          kv_heads=1, head_dim=32, key_heads=2, value_heads=4, key_dim=16,
                          value_dim=8, rotary_dim=16, context=256)


def test_delta_rule_matches_reference_fixture():
    # fixtures/qwen35/operations-v1.json, used by kernels.rs:275-326
    fx = json.load(open(os.path.join(GOLDEN, "qwen35_operations.json")))
    st = orc.DeltaState(fx["heads"], fx["key_dimension"], fx["value_dimension"])
    for step in fx["steps"]:
        rc, out = st.step(step["q"], step["k"], step["v"], step["log_decay"], step["beta"])
        assert rc == 0
        assert np.abs(out - np.float32(step["output"])).max() < fx["absolute_tolerance"]
        assert np.abs(st.memory - np.float32(step["state"])).max() < fx["absolute_tolerance"]


def test_delta_rule_rejects_growth_and_out_of_range_gates():
    st = orc.DeltaState(1, 2, 2)
    ok = dict(q=[0.5, 0.25], k=[0.25, -0.5], v=[1.0, -1.0])
    assert st.step(**ok, log_decay=[0.5], beta=[0.5])[0] != 0   # decay > 1
    assert st.step(**ok, log_decay=[-0.5], beta=[1.5])[0] != 0  # beta outside [0, 1]
    assert st.step(**ok, log_decay=[-0.5], beta=[1.0])[0] == 0


def test_conv_gates_and_norm_closed_forms():
    # kernels.rs:328-353
    st = orc.ConvState(1, 3)
    for x, y in [(1.0, 3.0), (2.0, 8.0), (-1.0, 2.0), (4.0, 12.0)]:
        rc, out = st.step([x], [1.0, 2.0, 3.0])
        assert rc == 0 and abs(out[0] - orc.q35_silu(y)) < 1e-6
    assert orc.q35_sigmoid(1000.0) == 1.0 and orc.q35_sigmoid(-1000.0) == 0.0
    assert orc.q35_softplus(1000.0) == 1000.0 and orc.q35_softplus(-1000.0) == 0.0
    rc, out = orc.q35_norm([1.0, 2.0, 3.0], [-1.0, 0.0, 1.0], 1e-6, True)
    assert rc == 0 and out[0] == 0.0
    assert abs(out[1] - 2.0 / np.sqrt(np.float32(14.0 / 3.0 + 1e-6))) < 1e-6
    assert orc.q35_norm([3.4e38], [1.0], 1e-6, False)[0] != 0  # reduction overflow
    # softplus against float64 for a spread of arguments
    for v in np.linspace(-30, 30, 241, dtype=np.float32):
        want = np.log1p(np.exp(-abs(float(v)))) + max(float(v), 0.0)
        assert abs(orc.q35_softplus(float(v)) - want) <= 2e-7 * max(1.0, abs(want))


def test_partial_rope_identity_tail_and_closed_form():
    row = np.arange(1, 9, dtype=np.float32)
    rc, out = orc.q35_partial_rope(row, 8, 4, 0, 10000.0)
    assert rc == 0 and np.array_equal(out, row)            # position 0: identity
    rc, out = orc.q35_partial_rope(row, 8, 4, 3, 10000.0)
    assert rc == 0 and np.array_equal(out[4:], row[4:])      # tail untouched
    assert orc.q35_partial_rope(row, 8, 3, 0, 10000.0)[0] != 0
    # kernels.rs:361-374: rotated unit prefix gives (cos, sin) of the angle
    v = np.zeros(256, np.float32)
    v[:32] = 1.0
    rc, out = orc.q35_partial_rope(v, 256, 64, 7, 1e7)
    assert rc == 0
    for j in range(32):
        ang = 7.0 * 1e7 ** (-(2 * j) / 64.0)
        assert abs(out[j] - np.cos(ang)) < 2e-6
        assert abs(out[j + 32] - np.sin(ang)) < 2e-6
    assert not out[64:].any()


def _oracle_logits(cfg, t, toks):
    m = orc.Qwen35Model(cfg, t, threads=4)
    s = m.session(64)
    out = []
    for tok in toks:
        assert m.forward_batch([s], [tok])[0] == 0
        out.append(s.logits())
    return np.array(out)


def test_oracle_matches_float64_textbook_hybrid_step():
    cfg, t = synth35.in_memory(tiny(), seed=1)
    toks = [5, 17, 3, 99, 250, 7, 7, 1, 42, 11]
    got = _oracle_logits(cfg, t, toks)
    ref = Qwen35F64(cfg, t).forward(toks)
    assert np.abs(got - ref).max() < 2e-5, np.abs(got - ref).max()


def test_textbook_check_catches_a_planted_mistake():
    cfg, t = synth35.in_memory(tiny(), seed=1)
    toks = [5, 17, 3, 99, 250, 7]
    got = _oracle_logits(cfg, t, toks)
    bad = Qwen35F64(cfg, t, mistake="conv_taps_reversed").forward(toks)
    assert np.abs(got - bad).max() > 1e-2


def test_batched_equals_individual_bitwise():
    cfg, t = synth35.in_memory(tiny(), seed=2)
    m = orc.Qwen35Model(cfg, t, threads=4)
    prompts = [[1, 2, 3, 4, 5], [9, 8], [100, 200, 250]]
    together = [m.session(32) for _ in prompts]
    alone = [m.session(32) for _ in prompts]
    for step in range(5):
        live = [i for i, p in enumerate(prompts) if step < len(p)]
        m.forward_batch([together[i] for i in live], [prompts[i][step] for i in live])
        for i in live:
            m.forward_batch([alone[i]], [prompts[i][step]])
            assert np.array_equal(together[i].logits(), alone[i].logits())
    for i in range(len(prompts)):
        for layer in range(cfg["layers"]):
            which = (0, 1) if cfg["full"][layer] else (2, 3)
            for w in which:
                assert np.array_equal(together[i].state(layer, w), alone[i].state(layer, w))
