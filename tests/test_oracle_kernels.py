"""Pins the CPU oracle's scalar kernels to the reference's own known answers.

kernels.json / rope.json / sampling-v2.json are the reference's frozen fixtures
(fixtures/quantized, fixtures/constraints), used by
crates/coheryn-engine/tests/quant.rs:28-59,165-192 and sampling.rs:229-250 with
the tolerances stated there.  The closed forms are cpu.rs:215-305's tests plus
brute force in float64 where the fixture leaves a function open.
"""
import json
import math
import os

import numpy as np
import pytest

import orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_kernels_fixture_decode_activation_dot():
    fx = load("kernels.json")
    tol = fx["tolerances"]
    assert len(fx["cases"]) == 100
    for i, case in enumerate(fx["cases"]):
        rc, decoded = orc.decode(case["bytes"], case["dtype"], len(case["decoded"]))
        assert rc == 0, i
        np.testing.assert_array_equal(decoded, np.array(case["decoded"], np.float32),
                                      err_msg=f"decode {i}")
        rc, act, kind = orc.prepare(case["input"], case["dtype"])
        assert rc == 0
        assert kind == case["activation_dtype"]
        assert list(act) == case["activation_bytes"], f"activation {i}"
        rc, dot = orc.qdot(case["bytes"], case["dtype"], act, kind, len(case["input"]))
        assert rc == 0
        assert abs(dot - case["dot"]) <= tol["dot_absolute"] + tol["dot_relative"] * abs(
            case["dot"]), f"dot {i}: {dot} vs {case['dot']}"


def test_hostile_shapes_and_scales_fail():
    # tests/quant.rs:61-85
    for dtype in (2, 6, 8, 12, 14):
        width = 32 if dtype < 12 else 256
        rc, nbytes = orc.row_bytes(dtype, width)
        assert rc == 0
        for length in range(nbytes):
            assert orc.decode(bytes(length), dtype, width)[0] != 0
        bad = bytearray(nbytes)
        off = 208 if dtype == 14 else 0
        bad[off + 1] = 0x7C  # +inf scale
        assert orc.decode(bytes(bad), dtype, width)[0] != 0
        rc, act, kind = orc.prepare(np.zeros(width, np.float32), dtype)
        assert rc == 0
        rc, d = orc.qdot(bytes(nbytes), dtype, act, kind, width)
        assert rc == 0 and d == 0.0
        rc, _, _ = orc.prepare(np.full(width, np.nan, np.float32), dtype)
        assert rc != 0
    assert orc.row_bytes(2, 31)[0] != 0
    assert orc.row_bytes(12, 32)[0] != 0
    assert orc.row_bytes(99, 32)[0] != 0


def test_rope_fixture_and_closed_forms():
    fx = load("rope.json")
    for case in fx["cases"]:
        out = orc.rope(case["input"], case["head_dim"], case["position"], case["base"])
        exp = np.array(case["output"], np.float32)
        assert np.all(np.abs(out - exp) <= 1e-6 + 1e-6 * np.abs(exp)), case["position"]
    # cpu.rs:229-239
    x = orc.rope([1, 2, 3, 4], 4, 0, 10000.0)
    assert list(x) == [1, 2, 3, 4]
    x = orc.rope([1, 2, 3, 4], 4, 1, 10000.0)
    assert abs(x[0] - (math.cos(1) - 3 * math.sin(1))) < 1e-6
    # The angle advances by repeated f32 multiplication (cpu.rs:62,70), not
    # powf(base, -2i/d) per index; at position 4093 the two differ by more
    # than the 1e-6 tolerance for several indices.
    hd, pos, base = 64, 4093, 1e6
    step = np.float32(np.float32(base) ** np.float32(-2.0 / hd))
    angle = np.float32(pos)
    iterative_wins = 0
    for i in range(hd // 2):
        x = np.zeros(hd, np.float32)
        x[i] = 1.0
        out = orc.rope(x, hd, pos, base)
        assert abs(out[i] - math.cos(float(angle))) < 1e-6
        assert abs(out[i + hd // 2] - math.sin(float(angle))) < 1e-6
        direct = np.float32(pos) * np.float32(np.float32(base) ** np.float32(-2.0 * i / hd))
        if abs(math.cos(float(direct)) - out[i]) > 1e-6:
            iterative_wins += 1
        angle = np.float32(angle * step)
    assert iterative_wins > 0


def test_f16_conversion_matches_numpy_rne_on_all_halves_and_sampled_floats():
    halves = np.arange(65536, dtype=np.uint16)
    ref = halves.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(h)) for h in halves], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # include exact ties, subnormal boundaries and the overflow edge
    extra = np.array([65504.0, 65520.0, 65519.996, 2.0**-24, 2.0**-25, 1.5 * 2.0**-25,
                      2.0**-14, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, -0.0], np.float32)
    f = np.concatenate([f, extra])
    ref = f.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in f], np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_cpu_closed_forms():
    # cpu.rs:215-228
    rc, v = orc.decode(bytes([0, 0, 0, 0x3C]), 1, 2)
    assert rc == 0 and list(v) == [0.0, 1.0]
    assert orc.decode(bytes([0xFF] * 4), 0, 1)[0] != 0
    rc, r = orc.round_f16([1.0001, -2.0001])
    assert list(r) == [1.0, -2.0]
    assert orc.dot_f32([1e8, 1.0, -1e8], [1.0, 1.0, 1.0]) == 1.0
    out = orc.rms_norm([3.0, 4.0], [1.0, 1.0], 0.0)
    assert abs(out[0] - 0.84852815) < 1e-6
    # swiglu = silu(g) * u
    g = np.array([-3.0, -0.5, 0.0, 0.5, 4.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -1.0, 0.25], np.float32)
    s = orc.swiglu(g, u)
    ref = g / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(s, ref, rtol=1e-6, atol=1e-7)


def test_attention_rows_matches_double_brute_force():
    # cpu.rs:248-291
    q = np.array([1, -0.5, 0.25, 1, -1, 0.5, 0.5, -0.25], np.float32)
    keys = np.array([(i % 17) / 16 - 0.5 for i in range(129 * 4)], np.float32)
    values = np.array([(i % 23) / 8 - 1 for i in range(129 * 4)], np.float32)
    rc, out = orc.attention_rows(q, keys, values, 2, 2)
    assert rc == 0
    for h in range(4):
        kv = h // 2
        w = np.array([math.exp(sum(float(q[h * 2 + j]) * float(keys[r * 4 + kv * 2 + j])
                                   for j in range(2)) / math.sqrt(2)) for r in range(129)])
        for j in range(2):
            exp = sum(w[r] * float(values[r * 4 + kv * 2 + j]) for r in range(129)) / w.sum()
            assert abs(float(out[h * 2 + j]) - exp) < 1e-6
    assert orc.attention_rows(q, keys, values, 0, 2)[0] != 0


def test_online_attention_matches_explicit_softmax():
    # cpu.rs:240-255
    rc, out = orc.attention_rows([1.0, 0.0], [1.0, 0.0, 0.0, 1.0], [2.0, 4.0, 6.0, 8.0], 1, 2,
                                 online=True)
    p = math.exp(1 / math.sqrt(2))
    assert abs(out[0] - (2 * p + 6) / (p + 1)) < 1e-6
    assert abs(out[1] - (4 * p + 8) / (p + 1)) < 1e-6


def test_q8_0_dot_is_the_blockwise_fma_chain():
    # A plausible mistake (one fused multiply per row, or a float sum of
    # products) fails this: the chain rounds after every block.
    rng = np.random.default_rng(7)
    width = 896
    w = rng.normal(0, 0.02, width).astype(np.float32)
    x = rng.normal(0, 1, width).astype(np.float32)
    rc, wq, _ = orc.prepare(w, 8)
    rc, xq, kind = orc.prepare(x, 8)
    rc, d = orc.qdot(wq, 8, xq, kind, width)
    s = np.float32(0)
    for b in range(width // 32):
        wb, xb = wq[b * 34:(b + 1) * 34], xq[b * 34:(b + 1) * 34]
        dw = np.frombuffer(wb[:2].tobytes(), np.float16)[0].astype(np.float32)
        da = np.frombuffer(xb[:2].tobytes(), np.float16)[0].astype(np.float32)
        isum = int(np.dot(wb[2:].view(np.int8).astype(np.int64), xb[2:].view(np.int8).astype(np.int64)))
        # fmaf(isum, dw*da, s): exact product then one rounding (float64 holds it exactly)
        s = np.float32(np.float64(isum) * np.float64(np.float32(dw * da)) + np.float64(s))
    assert d == s


SAMPLING_EXPECTED_KEYS = ("logits", "allowed", "history", "settings", "penalties", "expected_ids")


def test_sampling_fixture():
    fx = load("sampling-v2.json")
    for case in fx["cases"]:
        st, pen = case["settings"], case["penalties"]
        s = orc.Sampler(st["temperature"], st["top_k"], st["top_p"], st["seed"],
                        pen["repetition_penalty"], pen["frequency_penalty"],
                        pen["presence_penalty"])
        assert s.history(len(case["logits"]), case["history"]) == 0
        for exp in case["expected_ids"]:
            rc, tok = s.sample(case["logits"], case["allowed"])
            assert rc == 0
            assert tok == exp, case["id"]
            s.observe(tok)


def test_sampler_greedy_ties_and_penalties():
    s = orc.Sampler()
    assert s.sample([2.0, 2.0, 1.0]) == (0, 0)
    s = orc.Sampler(repetition_penalty=2.0, frequency_penalty=0.25, presence_penalty=0.5)
    s.history(3, [0, 0, 1, 1])
    assert s.sample([4.0, -2.0, 3.0]) == (0, 2)
    assert s.sample([4.0, -2.0, 3.0], [1, 1, 0]) == (0, 0)
    assert s.sample([1.0, 2.0, 3.0], [0, 0, 0])[0] != 0
    assert orc.Sampler().sample([math.inf])[0] != 0
    with pytest.raises(ValueError):
        orc.Sampler(temperature=float("nan"))
