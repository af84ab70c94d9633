"""Pins the oracle's Qwen2 step (inference/batch.rs:117-273) without the Rust
reference: closed forms from crates/coheryn-engine/tests/engine.rs:35-60,187-217,
the batched == individual invariants (tensor.rs:443-582, tests/batching.rs:40-125),
an independent float64 textbook forward, and GGUF/quantizer round trips."""
import os

import numpy as np
import pytest

import gguf
import orc
import synth
from qwen2_ref import Qwen2F64

TINY = synth.config(layers=2, hidden=64, intermediate=128, heads=4, kv_heads=2,
                    vocabulary=97, context=64)


def test_q8_0_quantizer_matches_oracle_prepare():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 0.02, (7, 896)).astype(np.float32)
    x[0, :32] = 0.0  # zero block
    x[1, 5] = 0.5
    x[1, 9] = -0.5  # tie: first wins
    q = synth.quantize_q8_0(x)
    for r in range(x.shape[0]):
        rc, b, kind = orc.prepare(x[r], 8)
        assert rc == 0 and kind == 8
        assert bytes(b) == q[r].tobytes()


def test_q4_0_decodes_close_to_source():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 0.02, (3, 256)).astype(np.float32)
    q = synth.quantize_q4_0(x)
    for r in range(3):
        rc, v = orc.decode(q[r].tobytes(), 2, 256)
        assert rc == 0
        d = np.abs(x[r]).reshape(8, 32).max(1).repeat(32) / 8
        # half a step inside the range; a full step where +7 clips the far end
        assert np.all(np.abs(v - x[r]) <= d * 1.001 + 1e-7)
        assert np.mean(np.abs(v - x[r]) <= d * 0.501 + 1e-7) > 0.9


def test_gguf_round_trip(tmp_path):
    path = str(tmp_path / "m.gguf")
    synth.write_model(path, TINY, "q8_0", seed=1)
    meta, tensors = gguf.read(path)
    cfg = gguf.qwen2_config(meta)
    for k in ("layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim",
              "vocabulary", "context"):
        assert cfg[k] == TINY[k]
    _, mem = synth.in_memory(TINY, "q8_0", seed=1)
    assert set(mem) == set(tensors)
    for n in mem:
        assert tensors[n].shape == mem[n].shape and tensors[n].dtype == mem[n].dtype
        assert np.array_equal(np.asarray(tensors[n].data), mem[n].data)


def zero_model(cfg, dtype):
    c, t = synth.in_memory(cfg, dtype, seed=0)
    for n, tensor in t.items():
        if len(tensor.shape) == 2 and n != "token_embd.weight":
            tensor.data[:] = 0
    # tied head -> zero embedding rows give zero logits
    t["token_embd.weight"].data[:] = 0
    return c, t


@pytest.mark.parametrize("dtype", ["f16", "q8_0", "f32"])
def test_zero_matrices_give_token_zero(dtype):
    # tests/engine.rs:35-60: zero weights -> all-zero logits -> greedy token 0
    c, t = zero_model(TINY, dtype)
    m = orc.Model(c, t, threads=2)
    s = m.session()
    for tok in (5, 17, 3):
        errs = m.forward_batch([s], [tok])
        assert errs[0] == 0
        logits = s.logits()
        assert np.all(logits == 0)
        assert orc.Sampler().sample(logits) == (0, 0)


def greedy_generate(model, prompt, n_new):
    s = model.session()
    sampler = orc.Sampler()
    out = []
    for tok in prompt:
        assert model.forward_batch([s], [tok])[0] == 0
    for _ in range(n_new):
        rc, t = sampler.sample(s.logits())
        out.append(t)
        assert model.forward_batch([s], [t])[0] == 0
    return out, s


@pytest.mark.parametrize("dtype", ["f16", "q8_0", "q4_0"])
def test_batched_equals_individual_bitwise(dtype):
    c, t = synth.in_memory(TINY, dtype, seed=5)
    m = orc.Model(c, t, threads=3)
    rng = np.random.default_rng(9)
    prompts = [list(rng.integers(0, c["vocabulary"], n)) for n in (3, 7, 5)]
    sessions = [m.session() for _ in prompts]
    ref = []
    for p in prompts:
        s1 = m.session()
        logits = []
        for tok in p:
            m.forward_batch([s1], [tok])
            logits.append(s1.logits())
        ref.append(logits)
    # ragged batches: lanes join and retire
    for step in range(max(map(len, prompts))):
        live = [i for i, p in enumerate(prompts) if step < len(p)]
        errs = m.forward_batch([sessions[i] for i in live], [prompts[i][step] for i in live])
        assert not errs.any()
        for i in live:
            assert np.array_equal(sessions[i].logits().view(np.uint32),
                                  ref[i][step].view(np.uint32))


def test_thread_count_does_not_change_bits():
    c, t = synth.in_memory(TINY, "q8_0", seed=6)
    outs = []
    for threads in (1, 4):
        m = orc.Model(c, t, threads=threads)
        s = m.session()
        for tok in (1, 2, 3):
            m.forward_batch([s], [tok])
        outs.append(s.logits())
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("dtype,tol", [("f32", 2e-5), ("f16", 2e-2), ("q8_0", 6e-2)])
def test_oracle_matches_float64_textbook_forward(dtype, tol):
    c, t = synth.in_memory(TINY, dtype, seed=11, tied=False)
    m = orc.Model(c, t, threads=2)
    ref = Qwen2F64(c, t)
    tokens = [3, 50, 7, 96, 0, 12, 33, 8]
    want = ref.forward(tokens)
    s = m.session()
    worst = 0.0
    for i, tok in enumerate(tokens):
        assert m.forward_batch([s], [tok])[0] == 0
        got = s.logits().astype(np.float64)
        scale = np.abs(want[i]).max()
        worst = max(worst, np.abs(got - want[i]).max() / scale)
    # f32 weights: only f32 rounding separates the two; quantized activations
    # (f16 operands, Q8_0 blocks) widen the gap by their step size.
    assert worst < tol, worst


def test_oracle_textbook_check_catches_a_planted_mistake():
    """The float64 comparison is sharp enough to see a transposed operand."""
    c, t = synth.in_memory(TINY, "f32", seed=12, tied=False)
    ref = Qwen2F64(c, t)
    tokens = [3, 50, 7]
    want = ref.forward(tokens)
    w = t["blk.0.attn_output.weight"]
    H = c["hidden"]
    wt = np.frombuffer(w.data.tobytes(), np.float32).reshape(H, H).T.copy()
    t2 = dict(t)
    t2["blk.0.attn_output.weight"] = gguf.Tensor(w.name, w.shape, 0, wt.view(np.uint8).reshape(-1))
    m = orc.Model(c, t2, threads=2)
    s = m.session()
    for tok in tokens:
        m.forward_batch([s], [tok])
    got = s.logits().astype(np.float64)
    assert np.abs(got - want[-1]).max() / np.abs(want[-1]).max() > 1e-3


def test_errors_are_lane_local():
    c, t = synth.in_memory(TINY, "q8_0", seed=7)
    m = orc.Model(c, t, threads=2)
    a, b = m.session(), m.session(context=2)
    m.forward_batch([a, b], [1, 2])
    m.forward_batch([a, b], [3, 4])
    ref = a.logits()
    errs = m.forward_batch([a, b], [c["vocabulary"] + 5, 1])  # a: bad token, b: context full
    assert errs[0] == orc_errors("request") and errs[1] == orc_errors("resource")
    a2 = m.session()
    m.forward_batch([a2], [1])
    m.forward_batch([a2], [3])
    assert np.array_equal(a2.logits(), ref)


def orc_errors(kind):
    return {"request": 1, "invalid": 2, "resource": 3}[kind]


def test_pack_closed_form():
    n_tokens = np.array([1, 4, 1, 3], np.uint32)
    start = np.array([10, 0, 33, 17], np.uint32)
    page = 16
    pages = np.full((4, 8), -1, np.int32)
    pages[0, :1] = [5]
    pages[1, :1] = [2]
    pages[2, :3] = [7, 8, 9]
    pages[3, :2] = [1, 4]
    rc, cu, pos, slot, lane = orc.pack(n_tokens, start, pages, page)
    assert rc == 0
    assert list(cu) == [0, 1, 5, 6, 9]
    assert list(pos) == [10, 0, 1, 2, 3, 33, 17, 18, 19]
    assert list(lane) == [0, 1, 1, 1, 1, 2, 3, 3, 3]
    assert list(slot) == [5 * 16 + 10, 32, 33, 34, 35, 9 * 16 + 1, 4 * 16 + 1, 4 * 16 + 2,
                          4 * 16 + 3]
    # a position beyond the page table is a resource error
    rc, *_ = orc.pack(np.array([1], np.uint32), np.array([200], np.uint32), pages[:1], page)
    assert rc == 3


def test_synthetic_kv_fill_is_seeded_and_bounded():
    c, t = synth.in_memory(TINY, "q8_0", seed=8)
    m = orc.Model(c, t, threads=1)
    s = m.session()
    assert s.fill_synthetic(20, 1234, 3) == 0
    k = s.kv(1)
    assert k.shape == (20, c["kv_heads"] * c["head_dim"])
    assert np.all(np.abs(k) <= 1.0) and k.std() > 0.3
    assert k[4, 7] == orc.synthetic_kv(1234, 3, 1, 0, 4, 7)
    s2 = m.session()
    s2.fill_synthetic(20, 1234, 4)
    assert not np.array_equal(s2.kv(1), k)


def test_synthetic_kv_fill_appends_after_the_current_rows():
    """A second fill keeps rows [0, position) and fills only the new rows with
    its own stream (the GPU contract for a forked, shared prefix)."""
    c, t = synth.in_memory(TINY, "q8_0", seed=8)
    m = orc.Model(c, t, threads=1)
    s = m.session()
    assert s.fill_synthetic(10, 77, 1) == 0
    assert s.fill_synthetic(25, 77, 2) == 0
    assert s.position == 25
    k = s.kv(0, True)
    assert k[9, 3] == orc.synthetic_kv(77, 1, 0, 1, 9, 3)
    assert k[10, 3] == orc.synthetic_kv(77, 2, 0, 1, 10, 3)
    assert s.fill_synthetic(5, 77, 3) != 0  # never shrinks
