"""GPU parity for the K-quant and Q5_0 matrices (quant.rs:175-349) and for
mixed-dtype (Q4_K_M-style) models, through the C ABI.

* cohx_matvec runs one matrix against f32 inputs through the step's own
  operand preparation and exact kernels.  On the reference's 100 frozen
  kernel cases (tests/golden/kernels.json, all five packed dtypes) the
  prepared activation bytes and the decoded rows must equal the fixture byte
  for byte, and each dot must equal the oracle's bit for bit (the fixture's
  own dot is within its stated 1e-5).  On random and hostile inputs every dot
  must equal the oracle's.
* A Q4_K_M-style model (Q4_K/Q6_K/Q5_0/Q8_0 matrices, untied Q6_K or Q8_0
  head) runs ragged steps bit for bit against the oracle: logits, greedy ids
  and KV rows.
"""
import json
import os

import numpy as np
import pytest

import cohx
import orc
import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = {2: "q4_0", 6: "q5_0", 8: "q8_0", 12: "q4_k", 14: "q6_k"}


def host_model():
    """Any Qwen2 context: cohx_matvec only borrows its device and stream."""
    cfg = synth.config(layers=1, hidden=128, intermediate=256, heads=4, kv_heads=2,
                       vocabulary=64, context=64)
    c, t = synth.in_memory(cfg, "q8_0", seed=1)
    return cohx.Model(c, t, max_lanes=2, max_rows=2, max_seqs=2, max_context=32)


def oracle_dots(rows, dtype, K, inputs):
    out = np.zeros((len(inputs), len(rows)), np.float32)
    rcs = np.zeros(len(inputs), np.int32)
    for i, x in enumerate(inputs):
        rc, act, kind = orc.prepare(x, dtype)
        if rc:
            rcs[i] = rc
            continue
        for r, row in enumerate(rows):
            rc, v = orc.qdot(row, dtype, act, kind, K)
            if rc:
                rcs[i] = rc
                break
            out[i, r] = v
    return out, rcs


def test_matvec_matches_reference_kernel_fixture():
    print("case: kernels.json through cohx_matvec", flush=True)
    fx = json.load(open(os.path.join(GOLDEN, "kernels.json")))
    m = host_model()
    counts = {}
    for i, case in enumerate(fx["cases"]):
        dt = case["dtype"]
        K = len(case["input"])
        row = np.array(case["bytes"], np.uint8)
        x = np.array(case["input"], np.float32)
        out, act, st, dec = m.matvec(dt, 1, K, row, x[None, :], decode=True)
        assert st[0] == 0, (i, dt, st)
        assert np.array_equal(act[0], np.array(case["activation_bytes"], np.uint8)), (i, dt, "activation bytes")
        assert np.array_equal(dec[0], np.array(case["decoded"], np.float32)), (i, dt, "decoded")
        rc, oact, kind = orc.prepare(x, dt)
        rc2, want = orc.qdot(row, dt, oact, kind, K)
        assert rc == 0 and rc2 == 0
        assert out[0, 0].view(np.uint32) == np.float32(want).view(np.uint32), (i, dt, out[0, 0], want)
        ref = case["dot"]
        assert abs(float(out[0, 0]) - ref) <= 1e-5 + 1e-5 * abs(ref), (i, dt)
        counts[NAMES[dt]] = counts.get(NAMES[dt], 0) + 1
    print(f"bit-exact against the oracle, bytes equal to the fixture: {counts}", flush=True)
    assert sum(counts.values()) == 100


def hostile_inputs(rng, n, K):
    """Wide exponent ranges, zero blocks, ties in magnitude of both signs,
    single spikes, subnormals."""
    xs = []
    for i in range(n):
        kind = i % 6
        if kind == 0:
            x = rng.standard_normal(K).astype(np.float32)
        elif kind == 1:  # |x| from 2^-20 to 2^10
            x = (np.exp2(rng.uniform(-20, 10, K)) * rng.choice([-1, 1], K)).astype(np.float32)
        elif kind == 2:  # zero blocks and lone spikes
            x = np.zeros(K, np.float32)
            x[rng.integers(0, K, 3)] = rng.standard_normal(3).astype(np.float32) * 100
        elif kind == 3:  # equal magnitudes of both signs: the first one sets the sign
            x = rng.choice([-1.0, 1.0, 0.5, -0.5], K).astype(np.float32)
        elif kind == 4:  # subnormal and tiny values next to normal ones
            x = (rng.standard_normal(K) * 1e-38).astype(np.float32)
            x[::7] *= np.float32(1e-3)
        else:
            x = (rng.standard_normal(K) * 0.02).astype(np.float32)
        xs.append(x)
    return np.stack(xs)


@pytest.mark.parametrize("dtype", [12, 14, 6, 8, 2])
def test_matvec_random_and_hostile_inputs_match_oracle(dtype):
    print(f"case: random matvec {NAMES[dtype]}", flush=True)
    rng = np.random.default_rng(dtype)
    m = host_model()
    K, rows, n = 512, 45, 36
    w = (rng.standard_normal((rows, K)) * 0.05).astype(np.float32)
    w[3] = 0.0  # an all-zero row
    payload = synth.encode(w, dtype).reshape(rows, -1)
    xs = hostile_inputs(rng, n, K)
    got, _, st, _ = m.matvec(dtype, rows, K, payload, xs)
    want, rcs = oracle_dots(list(payload), dtype, K, xs)
    ok = rcs == 0
    assert np.array_equal(st != 0, ~ok), (st, rcs)
    diff = got[ok].view(np.uint32) != want[ok].view(np.uint32)
    print(f"{NAMES[dtype]}: {int(diff.sum())} of {diff.size} dots differ in bits; "
          f"{int((~ok).sum())} inputs rejected by both", flush=True)
    assert not diff.any()


def mixed_config(hidden, intermediate, layers=2, vocabulary=300):
    return synth.config(layers=layers, hidden=hidden, intermediate=intermediate, heads=4,
                        kv_heads=2, vocabulary=vocabulary, context=512)


def model_dtypes(t):
    return sorted({NAMES[v.dtype] for v in t.values() if len(v.shape) == 2})


@pytest.mark.parametrize("hidden,intermediate", [(128, 512), (256, 512)],
                         ids=["q5_0-q8_0-with-k-down", "all-k-quant"])
def test_q4_k_m_ragged_steps_match_oracle(hidden, intermediate):
    """hidden 128: q/k/o/gate/up Q5_0, v Q8_0 or Q5_0, down Q6_K or Q4_K, head
    Q8_0 (the publisher 0.5B file's pattern); hidden 256: every matrix a
    K-quant, the head Q6_K."""
    print(f"case: q4_k_m ragged steps H={hidden}", flush=True)
    c, t = synth.in_memory(mixed_config(hidden, intermediate), "q4_k_m", seed=5)
    print("dtypes:", model_dtypes(t), flush=True)
    m = cohx.Model(c, t, max_lanes=8, max_rows=64, max_seqs=8, max_context=256)
    o = orc.Model(c, t, threads=8)
    rng = np.random.default_rng(6)
    V = c["vocabulary"]
    seqs = [m.seq_alloc() for _ in range(3)]
    sess = [o.session(256) for _ in range(3)]
    plan = [{0: 5, 1: 3}, {0: 1, 1: 1, 2: 19}, {0: 1, 2: 1}, {1: 2, 2: 1, 0: 1}]
    mismatched = 0
    for step, spec in enumerate(plan):
        lanes, toks = [], {}
        for i, n in spec.items():
            toks[i] = [int(v) for v in rng.integers(0, V, n)]
            lanes.append(dict(seq=seqs[i], tokens=toks[i], logits=True))
        res = m.step(lanes)
        for (i, n), r in zip(spec.items(), res):
            assert r["status"] == 0, r
            for tok in toks[i]:
                assert o.forward_batch([sess[i]], [tok])[0] == 0
            want = sess[i].logits()
            bad = int((r["logits"].view(np.uint32) != want.view(np.uint32)).sum())
            print(f"step {step} lane {i}: {bad} logits differ in bits", flush=True)
            mismatched += bad
            assert r["argmax"] == orc.Sampler().sample(want)[1]
    for i in range(3):
        for layer in range(c["layers"]):
            for values in (False, True):
                assert np.array_equal(m.seq_read_kv(seqs[i], layer, values), sess[i].kv(layer, values))
    assert mismatched == 0


def test_fused_matrix_families_must_agree():
    """A fused q/k/v (or gate/up) whose parts fall in different device
    families is refused at upload, not computed wrongly."""
    c, t = synth.in_memory(mixed_config(256, 512), "q4_k_m", seed=7)
    bad = dict(t)
    k = bad["blk.0.attn_k.weight"]
    w = np.random.default_rng(0).standard_normal((k.shape[1], k.shape[0])).astype(np.float32) * 0.02
    import gguf
    bad["blk.0.attn_k.weight"] = gguf.Tensor(k.name, k.shape, 8, synth.encode(w, 8))
    with pytest.raises(cohx.CohxError) as e:
        cohx.Model(c, bad, max_lanes=2, max_rows=4, max_seqs=2, max_context=32)
    assert e.value.code == cohx.UNSUPPORTED
