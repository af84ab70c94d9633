"""Qwen3.5 hybrid step on the GPU against the oracle (oracle/orc_qwen35.c),
bit for bit: logits of every lane's last row, greedy ids, and the recurrent
state (K/V rows, causal-conv ring, delta-rule memory) after each step.  A lane
may carry a prompt chunk of several tokens; the oracle steps the same tokens
one at a time (Graph::forward_batch, qwen35/execution.rs:257-608)."""
import os

import numpy as np
import pytest

import cohx
import orc
import synth35

pytestmark = pytest.mark.gpu


def tiny(**kw):
    c = dict(layers=4, hidden=64, intermediate=96, vocabulary=300, heads=2, kv_heads=1,
             head_dim=32, key_heads=2, value_heads=4, key_dim=16, value_dim=8, rotary_dim=16,
             context=256)
    c.update(kw)
    return synth35.config(**c)


# The packed-prefill regime's stated tolerance: logits max-abs (the fp16
# bound the engine's tolerance names) and the recurrent state it leaves
# (K/V rows, conv ring, delta memory).  Greedy ids stay exact.
REGIME_LOGITS_TOL = 1e-2
REGIME_STATE_TOL = 1e-3


def make_q35(cfg, t, regime, **kw):
    """A GPU context; regime False keeps every step on the exact matvecs
    (COHX_PREFILL_MFMA=0), True lets steps of 128+ rows take the matrix-core
    GEMM."""
    old = os.environ.get("COHX_PREFILL_MFMA")
    os.environ["COHX_PREFILL_MFMA"] = "1" if regime else "0"
    try:
        return cohx.Qwen35(cfg, t, **kw)
    finally:
        if old is None:
            del os.environ["COHX_PREFILL_MFMA"]
        else:
            os.environ["COHX_PREFILL_MFMA"] = old


class Pair:
    """A GPU context and an oracle model over the same tensors, with one oracle
    session per GPU sequence.  With `tol` (the regime tests) logits and state
    are held to REGIME_*_TOL instead of bit equality; greedy ids stay exact."""

    def __init__(self, cfg, t, threads=8, tol=False, **kw):
        self.cfg = cfg
        self.tol = tol
        self.gpu = make_q35(cfg, t, tol, **kw)
        self.orc = orc.Qwen35Model(cfg, t, threads=threads)
        self.sessions = {}
        self.worst_logit = 0.0
        self.worst_state = 0.0

    def alloc(self):
        s = self.gpu.seq_alloc()
        self.sessions[s] = self.orc.session(self.gpu.max_context)
        return s

    def step(self, lanes, skip=()):
        """lanes: [(seq, tokens)]; every lane asks for logits except the seqs in
        `skip`, whose rows only advance the state.  Checks each lane against
        the oracle and returns the GPU argmax per lane."""
        res = self.gpu.step([dict(seq=s, tokens=toks, logits=s not in skip, skip_head=s in skip)
                             for s, toks in lanes])
        width = max(len(toks) for _, toks in lanes)
        for j in range(width):
            live = [(s, toks[j]) for s, toks in lanes if j < len(toks)]
            errs = self.orc.forward_batch([self.sessions[s] for s, _ in live],
                                          [tok for _, tok in live])
            assert not any(errs), errs
        out = []
        for (s, toks), r in zip(lanes, res):
            assert r["status"] == 0, (s, r["status"])
            if s in skip:
                assert r["argmax"] == cohx.NO_TOKEN and r["logits"] is None
                assert self.gpu.seq_length(s) == self.sessions[s].position()
                out.append(None)
                continue
            want = self.sessions[s].logits()
            got = r["logits"]
            if self.tol:
                err = float(np.abs(got.astype(np.float64) - want).max())
                self.worst_logit = max(self.worst_logit, err)
                assert err <= REGIME_LOGITS_TOL, (s, err)
            elif not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
                bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
                raise AssertionError(f"seq {s}: {bad.size} logits differ, first {bad[:4]}, "
                                     f"max-abs {np.abs(got - want).max():.3g}")
            assert r["argmax"] == int(np.argmax(want)), (s, r["argmax"], int(np.argmax(want)))
            assert self.gpu.seq_length(s) == self.sessions[s].position()
            out.append(r["argmax"])
        return out

    def check_state(self, seq):
        ses = self.sessions[seq]
        for layer, full in enumerate(self.cfg["full"]):
            for which in ((0, 1) if full else (2, 3)):
                got = self.gpu.read_state(seq, layer, which)
                want = ses.state(layer, which).reshape(-1)
                assert got.size == want.size, (layer, which)
                if self.tol:
                    err = float(np.abs(got.astype(np.float64) - want).max()) if got.size else 0.0
                    self.worst_state = max(self.worst_state, err)
                    assert err <= REGIME_STATE_TOL, (seq, layer, which, err)
                else:
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seq, layer, which)


def test_tiny_prefill_decode_and_state_bit_exact():
    print("case: tiny Qwen3.5, 3 lanes prefill (7, 3, 1 tokens) then 5 greedy steps", flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=3)
    p = Pair(cfg, t, max_lanes=4, max_rows=32, max_context=64)
    seqs = [p.alloc() for _ in range(3)]
    prompts = [[5, 17, 3, 99, 250, 7, 7], [1, 2, 3], [299]]
    nxt = p.step(list(zip(seqs, prompts)))
    for s in seqs:
        p.check_state(s)
    for _ in range(5):
        nxt = p.step([(s, [tok]) for s, tok in zip(seqs, nxt)])
    for s in seqs:
        p.check_state(s)


def test_tiny_ragged_chunks_across_steps():
    print("case: tiny Qwen3.5, one prompt in chunks 8/1/11 beside a decoding lane", flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=4)
    p = Pair(cfg, t, max_lanes=4, max_rows=24, max_context=64)
    a, b = p.alloc(), p.alloc()
    rng = np.random.default_rng(9)
    prompt = [int(v) for v in rng.integers(0, cfg["vocabulary"], 20)]
    (tok_b,) = p.step([(b, [4, 8, 15])])
    for chunk in (prompt[:8], prompt[8:9], prompt[9:]):
        _, tok_b = p.step([(a, chunk), (b, [tok_b])])
    p.check_state(a)
    p.check_state(b)


def _large_packed_tiny(regime):
    cfg, t = synth35.in_memory(tiny(), seed=12)
    p = Pair(cfg, t, tol=regime, max_lanes=4, max_rows=160, max_context=160)
    a, b, c = p.alloc(), p.alloc(), p.alloc()
    rng = np.random.default_rng(13)
    pa = [int(v) for v in rng.integers(0, cfg["vocabulary"], 100)]
    pb = [int(v) for v in rng.integers(0, cfg["vocabulary"], 40)]
    (tc,) = p.step([(c, [5, 6])])
    ta, tb, tc = p.step([(a, pa), (b, pb), (c, [tc])])
    p.step([(a, [ta]), (b, [tb]), (c, [tc])])
    for s_ in (a, b, c):
        p.check_state(s_)
    return p


def test_tiny_large_packed_step_bit_exact():
    print("case: tiny Qwen3.5, 141 packed rows (chunks of 100 and 40 plus a decode row): the "
          "many-rows matvec form, regime off", flush=True)
    _large_packed_tiny(False)


def test_tiny_large_packed_step_prefill_regime_within_tolerance():
    print("case: tiny Qwen3.5, 141 packed rows through the packed-prefill regime (matrix-core "
          "BF16 GEMM on hi/lo activations over the tiled matrices)", flush=True)
    p = _large_packed_tiny(True)
    print(f"case: worst logit max-abs {p.worst_logit:.3g}, worst state {p.worst_state:.3g}", flush=True)


def _full_shape_packed(regime, n_prompt):
    cfg, t = synth35.in_memory(synth35.config(), seed=14)
    p = Pair(cfg, t, threads=16, tol=regime, max_lanes=2, max_rows=128, max_context=160)
    a, b = p.alloc(), p.alloc()
    rng = np.random.default_rng(15)
    pa = [int(v) for v in rng.integers(0, cfg["vocabulary"], n_prompt)]
    (tb,) = p.step([(b, [11])])
    ta, tb = p.step([(a, pa), (b, [tb])])
    p.step([(a, [ta]), (b, [tb])])
    p.check_state(a)
    p.check_state(b)
    return p


def test_full_shape_large_packed_step_bit_exact():
    print("case: Qwen3.5-0.8B shape, one step of 96 + 1 packed rows (many-rows matvec form)",
          flush=True)
    _full_shape_packed(False, 96)


def test_full_shape_prefill_regime_within_tolerance():
    print("case: Qwen3.5-0.8B shape, one step of 127 + 1 packed rows through the packed-prefill "
          "regime, then a decode step", flush=True)
    p = _full_shape_packed(True, 127)
    print(f"case: worst logit max-abs {p.worst_logit:.3g}, worst state {p.worst_state:.3g}", flush=True)


def test_tiny_fused_mixer_matches_oracle_and_split_kernels():
    print("case: tiny Qwen3.5 with one key head per value head (the fused linear mixer) against "
          "the oracle and against the four-kernel mixer", flush=True)
    cfg, t = synth35.in_memory(tiny(key_heads=4, value_heads=4, key_dim=16, value_dim=16),
                               seed=16)
    p = Pair(cfg, t, max_lanes=4, max_rows=96, max_context=96)
    a, b = p.alloc(), p.alloc()
    rng = np.random.default_rng(17)
    pa = [int(v) for v in rng.integers(0, cfg["vocabulary"], 70)]
    ta, tb = p.step([(a, pa[:4]), (b, [1, 2, 3])])          # short chunks: fused
    ta, tb = p.step([(a, pa[4:]), (b, [tb])])               # a long chunk: split
    for _ in range(3):
        ta, tb = p.step([(a, [ta]), (b, [tb])])              # decode: fused
    p.check_state(a)
    p.check_state(b)
    old = os.environ.get("COHX_Q35_SPLIT_LINEAR")
    os.environ["COHX_Q35_SPLIT_LINEAR"] = "1"
    try:
        split = cohx.Qwen35(cfg, t, max_lanes=4, max_rows=96, max_context=96)
    finally:
        if old is None:
            del os.environ["COHX_Q35_SPLIT_LINEAR"]
        else:
            os.environ["COHX_Q35_SPLIT_LINEAR"] = old
    sa, fused = split.seq_alloc(), p.gpu.seq_alloc()
    for chunk in (pa[:3], pa[3:7], pa[7:8]):
        r = split.step([dict(seq=sa, tokens=chunk, logits=True)])[0]
        f = p.gpu.step([dict(seq=fused, tokens=chunk, logits=True)])[0]
        assert np.array_equal(r["logits"].view(np.uint32), f["logits"].view(np.uint32))
    for layer, full in enumerate(cfg["full"]):
        for which in ((0, 1) if full else (2, 3)):
            assert np.array_equal(split.read_state(sa, layer, which).view(np.uint32),
                                  p.gpu.read_state(fused, layer, which).view(np.uint32))


def test_tiny_prompt_chunks_without_head():
    print("case: tiny Qwen3.5, prompt chunks that skip the head, then the last chunk with it",
          flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=8)
    p = Pair(cfg, t, max_lanes=4, max_rows=24, max_context=64)
    a, b, c = p.alloc(), p.alloc(), p.alloc()
    p.step([(a, [1, 2, 3, 4, 5]), (b, [6]), (c, [7, 8])], skip={a, c})
    p.step([(a, [9, 10]), (b, [11]), (c, [12])], skip={b})
    p.step([(a, [13]), (b, [14, 15, 16]), (c, [17])], skip={a, b, c})
    p.step([(a, [18]), (b, [19]), (c, [20])])
    for s in (a, b, c):
        p.check_state(s)


def test_tiny_fork_snapshot_then_diverge():
    print("case: tiny Qwen3.5, fork at the source length, both branches step", flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=5)
    p = Pair(cfg, t, max_lanes=4, max_rows=16, max_context=64)
    a = p.alloc()
    prompt = [11, 22, 33, 44, 55, 66]
    p.step([(a, prompt)])
    f = p.gpu.seq_fork(a, len(prompt))
    # the oracle branch replays the prompt in a fresh session
    p.sessions[f] = p.orc.session(p.gpu.max_context)
    for tok in prompt:
        assert p.orc.forward_batch([p.sessions[f]], [tok])[0] == 0
    p.check_state(f)
    p.step([(a, [1]), (f, [2])])
    p.step([(a, [3, 4]), (f, [5])])
    p.check_state(a)
    p.check_state(f)
    with pytest.raises(cohx.CohxError):
        p.gpu.seq_fork(a, 2)           # recurrent state cannot be forked mid-sequence
    with pytest.raises(cohx.CohxError):
        p.gpu.seq_truncate(a, 3)       # nor rewound


def test_tiny_request_errors():
    print("case: tiny Qwen3.5, invalid lanes rejected without touching the others", flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=6)
    p = Pair(cfg, t, max_lanes=4, max_rows=8, max_context=16)
    a, b = p.alloc(), p.alloc()
    res = p.gpu.step([dict(seq=a, tokens=[cfg["vocabulary"]], logits=True),
                      dict(seq=b, tokens=[1, 2], logits=True)])
    assert res[0]["status"] == cohx.INVALID_REQUEST
    assert res[1]["status"] == 0
    assert p.gpu.seq_length(a) == 0 and p.gpu.seq_length(b) == 2
    res = p.gpu.step([dict(seq=b, tokens=list(range(15)), logits=True)])  # past capacity
    assert res[0]["status"] == cohx.INVALID_REQUEST
    res = p.gpu.step([dict(seq=a, tokens=list(range(9)), logits=True)])   # past max_rows
    assert res[0]["status"] == cohx.RESOURCE


def test_full_shape_prefill_and_decode_bit_exact():
    print("case: Qwen3.5-0.8B shape (random weights), 2 lanes prefill 5/3 then 2 steps",
          flush=True)
    cfg, t = synth35.in_memory(synth35.config(), seed=7)
    p = Pair(cfg, t, threads=16, max_lanes=4, max_rows=16, max_context=64)
    a, b = p.alloc(), p.alloc()
    nxt = p.step([(a, [100, 2000, 30000, 248000, 5]), (b, [7, 77, 777])])
    for _ in range(2):
        nxt = p.step([(a, [nxt[0]]), (b, [nxt[1]])])
    p.check_state(a)
    p.check_state(b)


def _oracle_greedy(o, cfg, prompt, n, context):
    s = o.session(context)
    out = []
    for tok in prompt:
        assert o.forward_batch([s], [tok])[0] == 0
    for _ in range(n):
        nxt = int(np.argmax(s.logits()))
        out.append(nxt)
        if len(out) == n:
            break
        assert o.forward_batch([s], [nxt])[0] == 0
    return out


def test_tiny_generation_api_greedy_and_prefix_takeover():
    print("case: tiny Qwen3.5 through the generation mirror: greedy vs oracle, batched == alone, "
          "prefix takeover", flush=True)
    cfg, t = synth35.in_memory(tiny(), seed=9)
    m = cohx.Qwen35(cfg, t, max_lanes=4, max_rows=8, max_seqs=16, max_context=48)
    o = orc.Qwen35Model(cfg, t, threads=8)
    prompts = [[3, 1, 4, 1, 5], [9, 2, 6], [5, 3, 5, 8, 9, 7, 9]]
    opts = cohx.GenerationOptions(max_tokens=6)
    states = [m.begin_generation(p, opts) for p in prompts]
    while not all(s.is_finished() for s in states):
        live = [s for s in states if s.needs_forward()]
        if live:
            m.step_batch(live)
        for s in states:
            s.sample()
    for p, s in zip(prompts, states):
        assert s.token_ids() == _oracle_greedy(o, cfg, p, 6, 48), p
    # seeded sampling: batched == alone
    sopts = cohx.GenerationOptions(max_tokens=5, temperature=0.8, top_k=20, top_p=0.9, seed=11)
    together = [m.begin_generation(p, sopts) for p in prompts[:2]]
    while not all(s.is_finished() for s in together):
        live = [s for s in together if s.needs_forward()]
        if live:
            m.step_batch(live)
        for s in together:
            s.sample()
    for p, s in zip(prompts[:2], together):
        assert cohx.generate(m, p, sopts).token_ids() == s.token_ids()
    # a finished generation whose whole history prefixes the next prompt is taken over
    first = states[0]
    hist = prompts[0] + first.token_ids()[:-1]
    nxt = m.begin_generation(hist + [7, 7], opts, prior=first)
    while not nxt.is_finished():
        if nxt.needs_forward():
            m.step_generation(nxt)
        nxt.sample()
    assert nxt.token_ids() == _oracle_greedy(o, cfg, hist + [7, 7], 6, 48)
