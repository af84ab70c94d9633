"""The BASELINE.json workloads at their stated sizes, as deterministic input
specifications shared by the fixture generator (tests/golden/make_fullshape.py,
which runs the CPU oracle) and the GPU parity tests
(tests/test_gpu_baseline_shapes.py, which run the HIP path and compare with
the committed oracle results).

Every input is a function of the seeds below: weights come from synth /
synth35 (numpy generators), cached K/V rows from the seeded hash that both
the oracle (orc_session_fill_synthetic) and the library
(cohx_seq_fill_synthetic) implement, token ids from numpy generators.

Results are compared through digests: the SHA-256 of a lane's float32 logits
bytes (bit-exact equality of all V logits), the greedy id, the top-2 margin,
and the SHA-256 of the K/V rows a step appends.
"""
import hashlib

import numpy as np

V_QWEN2 = 151936

# model seeds (weights) per workload
SEED_Q8 = 31      # C2 / C2': Q8_0
SEED_Q4 = 32      # C4: Q4_0
SEED_F16_C1 = 33  # C1: F16
SEED_F16_C3 = 34  # C3: F16
SEED_Q35 = 35     # C5: Qwen3.5-0.8B bf16
SEED_Q4KM = 36    # Q4_K_M-style mixed dtypes (the reference's published decode format)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def summary(logits):
    """Digest, greedy id (lowest id on ties, sampling.rs:160-173) and the
    top-1 / top-2 values of one lane's logits."""
    logits = np.ascontiguousarray(logits, np.float32)
    top = int(np.argmax(logits))  # numpy returns the first maximum
    rest = np.delete(logits, top)
    return {"sha256": digest(logits), "argmax": top, "top1": float(logits[top]),
            "top2": float(rest.max())}


def kv_rows_digest(rows_by_layer):
    """rows_by_layer: [(K rows, V rows)] per layer, float32."""
    h = hashlib.sha256()
    for k, v in rows_by_layer:
        h.update(np.ascontiguousarray(k, np.float32).tobytes())
        h.update(np.ascontiguousarray(v, np.float32).tobytes())
    return h.hexdigest()


def c2(lanes):
    """BASELINE configs[1] (32 lanes) and its 128-lane headline form: Q8_0
    weights, decode-only lanes over seeded KV of U[64, 2048] tokens, one
    greedy token per lane per step: 16 steps at 32 lanes, 8 at 128 (each
    step's greedy ids feed the next, so a lane's whole continuation is
    checked)."""
    rng = np.random.default_rng(1000 + lanes)
    kv = [int(v) for v in rng.integers(64, 2049, lanes)]
    tokens = [int(v) for v in rng.integers(0, V_QWEN2, lanes)]
    return {"model_seed": SEED_Q8, "dtype": "q8_0", "fill_seed": 7000 + lanes, "kv": kv,
            "tokens": tokens, "steps": 16 if lanes <= 32 else 8, "context": 2048 + 24,
            "kv_check_layers": [0, 11, 23]}


def q4km(lanes=32):
    """The Qwen2.5-0.5B shape in the dtype pattern of the publisher's Q4_K_M
    file (synth.q4_k_m_dtype: Q5_0 q/k/o/gate/up and embedding, Q8_0 or Q5_0
    v, Q6_K or Q4_K down, untied Q8_0 head), as configs[1]: decode-only
    lanes over seeded KV of U[64, 2048] tokens, two greedy steps."""
    rng = np.random.default_rng(1100 + lanes)
    kv = [int(v) for v in rng.integers(64, 2049, lanes)]
    tokens = [int(v) for v in rng.integers(0, V_QWEN2, lanes)]
    return {"model_seed": SEED_Q4KM, "dtype": "q4_k_m", "fill_seed": 7200 + lanes, "kv": kv,
            "tokens": tokens, "steps": 2, "context": 2048 + 8, "kv_check_layers": [0, 11, 23]}


C4_GROUPS, C4_GROUP, C4_PREFIX, C4_CONTEXT = 8, 16, 256, 4096


def c4():
    """Q4_0 weights, 128 decode lanes in 8 groups of 16
    forked from one 256-token prefix per group (the prefix rows are filled
    once with the group's stream; each lane's private suffix with its own),
    contexts up to 4096, eight greedy steps."""
    rng = np.random.default_rng(4004)
    lanes = C4_GROUPS * C4_GROUP
    suffix = [int(v) for v in rng.integers(0, C4_CONTEXT - C4_PREFIX - 8 + 1, lanes)]
    tokens = [int(v) for v in rng.integers(0, V_QWEN2, lanes)]
    return {"model_seed": SEED_Q4, "dtype": "q4_0", "fill_seed": 8004, "groups": C4_GROUPS,
            "group": C4_GROUP, "prefix": C4_PREFIX, "suffix": suffix, "tokens": tokens, "steps": 8,
            "context": C4_CONTEXT, "kv_check_layers": [0, 23]}


def c1():
    """F16 weights, a continuous batch of 4 sequences with
    prompts of 16/32/48/64 uniform-random ids, 16 greedy tokens each, context
    512; one token per lane per step (batch.rs:64-116)."""
    rng = np.random.default_rng(1001)
    prompts = [[int(v) for v in rng.integers(0, V_QWEN2, n)] for n in (16, 32, 48, 64)]
    return {"model_seed": SEED_F16_C1, "dtype": "f16", "prompts": prompts, "max_tokens": 16,
            "context": 512}


def c3():
    """F16 weights, one mixed ragged step packing 8 prompt
    chunks of U[128, 512] tokens (each continuing a sequence with a seeded
    prefix of U[0, 512] cached rows) with 56 decode rows over seeded KV of
    U[256, 4096] tokens."""
    rng = np.random.default_rng(1003)
    chunk_len = [int(v) for v in rng.integers(128, 513, 8)]
    prefix = [int(v) for v in rng.integers(0, 513, 8)]
    chunks = [[int(v) for v in rng.integers(0, V_QWEN2, n)] for n in chunk_len]
    kv = [int(v) for v in rng.integers(256, 4097, 56)]
    tokens = [int(v) for v in rng.integers(0, V_QWEN2, 56)]
    return {"model_seed": SEED_F16_C3, "dtype": "f16", "fill_seed": 9003, "prefix": prefix,
            "chunks": chunks, "kv": kv, "tokens": tokens, "context": 4096 + 8,
            "kv_check_layers": [0, 23]}


def c5():
    """the Qwen3.5-0.8B hybrid shape (bf16 weights), 16
    sequences with prompts of U[64, 1024] random ids, through the prompt's end
    and the configuration's 64 greedy tokens."""
    rng = np.random.default_rng(1005)
    plen = [int(v) for v in rng.integers(64, 1025, 16)]
    prompts = [[int(v) for v in rng.integers(0, 248320, n)] for n in plen]
    return {"model_seed": SEED_Q35, "prompts": prompts, "generate": 64, "context": 1024 + 72}


def spec_digest(spec):
    """Digest of an input specification, stored with its expected results so a
    change of the inputs cannot go unnoticed."""
    import json
    return hashlib.sha256(json.dumps(spec, sort_keys=True).encode()).hexdigest()
