"""Seeded synthetic Qwen2-family models, written as GGUF.

Weights are N(0, 0.02) float32 draws (norm weights = 1, biases N(0, 0.02)),
stored as F16, Q8_0 (quantized with the engine's Q8_0 block rule,
quant.rs:197-213: signed max-|x| element, d = |m|/127, q = round-half-away(x/d))
or Q4_0 (ggml's Q4_0 rule: d = m/-8, q = min(15, trunc(x/d + 8.5))).
The tensor set and metadata are those compat.rs:54-221 validates, modelled on
the reference's test builder crates/coheryn-engine/tests/common/mod.rs:83-251.
"""
import numpy as np

import gguf

QWEN25_05B = dict(layers=24, hidden=896, intermediate=4864, heads=14, kv_heads=2,
                  vocabulary=151936, context=32768, rope_base=1e6, norm_epsilon=1e-6)

DTYPES = {"f32": 0, "f16": 1, "q4_0": 2, "q5_0": 6, "q8_0": 8, "q4_k": 12, "q6_k": 14}


def quantize_q8_0(x):
    """[rows, width] float32 -> [rows, width/32 * 34] uint8 (quant.rs:197-213)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    b = x.reshape(rows, width // 32, 32)
    idx = np.abs(b).argmax(axis=2)  # first element of maximal magnitude
    m = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    d = (np.abs(m) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1.0) / d).astype(np.float32)
    v = (b * inv[..., None]).astype(np.float32).astype(np.float64)
    q = np.trunc(v + np.copysign(0.5, v))  # round half away from zero, exact in f64
    q = np.clip(q, -128, 127).astype(np.int8)
    out = np.empty((rows, width // 32, 34), np.uint8)
    out[..., :2] = d.astype(np.float16).view(np.uint8).reshape(rows, width // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(rows, -1)


def quantize_q4_0(x):
    """[rows, width] float32 -> [rows, width/32 * 18] uint8 (ggml Q4_0 reference rule)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    b = x.reshape(rows, width // 32, 32)
    idx = np.abs(b).argmax(axis=2)
    m = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    d = (m / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1.0) / d).astype(np.float32)
    v = (b * inv[..., None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(np.trunc(v.astype(np.float32)), 15).astype(np.int32)
    q = np.clip(q, 0, 15).astype(np.uint8)
    out = np.empty((rows, width // 32, 18), np.uint8)
    out[..., :2] = d.astype(np.float16).view(np.uint8).reshape(rows, width // 32, 2)
    out[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(rows, -1)


def quantize_q5_0(x):
    """[rows, width] float32 -> [rows, width/32 * 22] uint8 (ggml's Q5_0 rule:
    d = m/-16, q = min(31, trunc(x/d + 16.5)); layout of quant.rs:102-114)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    b = x.reshape(rows, width // 32, 32)
    idx = np.abs(b).argmax(axis=2)
    m = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    d = (m / np.float32(-16.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1.0) / d).astype(np.float32)
    v = (b * inv[..., None]).astype(np.float32) + np.float32(16.5)
    q = np.clip(np.minimum(np.trunc(v), 31), 0, 31).astype(np.uint32)
    high = ((q[..., :16] >> 4) << np.arange(16, dtype=np.uint32)).sum(axis=2) | \
           ((q[..., 16:] >> 4) << np.arange(16, 32, dtype=np.uint32)).sum(axis=2)
    out = np.empty((rows, width // 32, 22), np.uint8)
    out[..., :2] = d.astype(np.float16).view(np.uint8).reshape(rows, width // 32, 2)
    out[..., 2:6] = high.astype("<u4").view(np.uint8).reshape(rows, width // 32, 4)
    out[..., 6:] = ((q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)).astype(np.uint8)
    return out.reshape(rows, -1)


def quantize_q4_k(x):
    """[rows, width] float32 -> [rows, width/256 * 144] uint8.  A plain
    min/max fit per 32-value group (not ggml's search): 6-bit group scales and
    mins under binary16 d and dmin, 4-bit values; the block layout is the one
    quant.rs:44-55,116-133 decodes."""
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    nb = width // 256
    g = x.reshape(rows, nb, 8, 32).astype(np.float64)
    lo = np.minimum(g.min(axis=3), 0.0)
    scale = (g.max(axis=3) - lo) / 15.0
    d = scale.max(axis=2) / 63.0
    dmin = (-lo).max(axis=2) / 63.0
    d16, dm16 = d.astype(np.float16), dmin.astype(np.float16)
    dd, dm = d16.astype(np.float64), dm16.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(dd[..., None] > 0, np.rint(scale / dd[..., None]), 0).clip(0, 63).astype(np.int64)
        mn = np.where(dm[..., None] > 0, np.rint(-lo / dm[..., None]), 0).clip(0, 63).astype(np.int64)
        step = dd[..., None] * sc
        q = np.where(step[..., None] > 0, np.rint((g + (dm[..., None] * mn)[..., None]) / step[..., None]), 0)
    q = q.clip(0, 15).astype(np.uint8)
    out = np.zeros((rows, nb, 144), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(rows, nb, 2)
    out[..., 2:4] = dm16.view(np.uint8).reshape(rows, nb, 2)
    for j in range(4):
        out[..., 4 + j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., 8 + j] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[..., 12 + j] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    for j in range(4):
        out[..., 16 + j * 32:16 + (j + 1) * 32] = q[:, :, 2 * j, :] | (q[:, :, 2 * j + 1, :] << 4)
    return out.reshape(rows, -1)


def quantize_q6_k(x):
    """[rows, width] float32 -> [rows, width/256 * 210] uint8: int8 scales per
    16 values under a binary16 d, 6-bit values (q + 32) split into 4 low bits
    and 2 high bits in the layout quant.rs:56-64 decodes."""
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    nb = width // 256
    g = x.reshape(rows, nb, 16, 16).astype(np.float64)
    scale = np.abs(g).max(axis=3) / 31.0
    d16 = (scale.max(axis=2) / 127.0).astype(np.float16)
    dd = d16.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(dd[..., None] > 0, np.rint(scale / dd[..., None]), 0).clip(-128, 127).astype(np.int64)
        step = dd[..., None] * sc
        q = np.where(step[..., None] > 0, np.rint(g / step[..., None]), 0)
    q = (q.clip(-32, 31).astype(np.int64) + 32).reshape(rows, nb, 256)
    out = np.zeros((rows, nb, 210), np.uint8)
    i = np.arange(256)
    half, grp, ln = i // 128, (i % 128) // 32, i % 32
    low_at = half * 64 + (grp % 2) * 32 + ln
    high_at = 128 + half * 32 + ln
    for k in range(256):
        v = q[..., k]
        if grp[k] < 2:
            out[..., low_at[k]] |= (v & 15).astype(np.uint8)
        else:
            out[..., low_at[k]] |= ((v & 15) << 4).astype(np.uint8)
        out[..., high_at[k]] |= (((v >> 4) & 3) << (2 * grp[k])).astype(np.uint8)
    out[..., 192:208] = sc.astype(np.int8).view(np.uint8)
    out[..., 208:210] = d16.view(np.uint8).reshape(rows, nb, 2)
    return out.reshape(rows, -1)


# Layers whose attn_v / ffn_down get the wider type in the publisher's
# Qwen2.5-0.5B Q4_K_M file (fixtures/quantized/qwen2.5-0.5b-instruct-q4_k_m
# .inventory.json: attn_v Q8_0 and ffn_down Q6_K in exactly these layers).
Q4_K_M_MORE_BITS_24 = (0, 1, 3, 6, 7, 8, 9, 10, 13, 16, 19, 21)


def q4_k_m_dtype(name, width, layer, layers):
    """Per-tensor dtype of a Q4_K_M-style file: Q4_K, with Q6_K for the head
    and for attn_v / ffn_down of the wider layers; a width that is not a
    multiple of 256 falls back to Q5_0 (for Q4_K) or Q8_0 (for Q6_K), which is
    how the publisher's 0.5B file ends up Q5_0/Q8_0/Q4_K/Q6_K."""
    more = layer is not None and (layer in Q4_K_M_MORE_BITS_24 if layers == 24 else layer % 2 == 0)
    if name == "output.weight":
        want = 14
    elif name in ("attn_v.weight", "ffn_down.weight"):
        want = 14 if more else 12
    else:
        want = 12
    if width % 256:
        want = 8 if want == 14 else 6
    return want


def encode(x, dtype):
    """x: [rows, width] float32 -> payload bytes for `dtype` (GGUF layout)."""
    if dtype == 0:
        return np.ascontiguousarray(x, np.float32).view(np.uint8).reshape(-1)
    if dtype == 1:
        return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint8).reshape(-1)
    if dtype == 8:
        return quantize_q8_0(x).reshape(-1)
    if dtype == 2:
        return quantize_q4_0(x).reshape(-1)
    if dtype == 6:
        return quantize_q5_0(x).reshape(-1)
    if dtype == 12:
        return quantize_q4_k(x).reshape(-1)
    if dtype == 14:
        return quantize_q6_k(x).reshape(-1)
    raise ValueError(dtype)


def config(**overrides):
    c = dict(QWEN25_05B)
    c.update(overrides)
    c["head_dim"] = c["hidden"] // c["heads"]
    return c


def build(cfg, dtype="q8_0", seed=0, eos_token_id=None, tied=None, std=0.02, spread=None):
    """Returns (metadata, [(name, shape, dtype, payload)]) for a seeded model.
    dtype "q4_k_m" gives each matrix the dtype q4_k_m_dtype picks (and an
    untied head, as the publisher's file has); tied defaults to True otherwise.
    spread=(lo, hi) multiplies every matrix row, norm weight and bias element
    by 2^U[lo, hi] (integer exponents): activations, K/V rows and products
    then span many binades (tests of the reduction orders)."""
    mixed = dtype == "q4_k_m"
    wdt = None if mixed else (DTYPES[dtype] if isinstance(dtype, str) else dtype)
    tied = (not mixed) if tied is None else tied
    rng = np.random.default_rng(seed)
    H, F, V, L = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"], cfg["layers"]
    kvd = cfg["kv_heads"] * cfg["head_dim"]
    eos = V - 1 if eos_token_id is None else eos_token_id

    def scale(shape):
        if spread is None:
            return np.float32(1.0)
        return np.exp2(rng.integers(spread[0], spread[1] + 1, shape)).astype(np.float32)

    def normal(rows, width):
        return rng.standard_normal((rows, width), dtype=np.float32) * np.float32(std) * scale((rows, 1))

    def ones(n):
        return np.ones((1, n), np.float32) * scale((1, n))

    def mat(name, rows, width, layer=None):
        t = q4_k_m_dtype(name, width, layer, L) if mixed else wdt
        return t, encode(normal(rows, width), t)

    tensors = [("token_embd.weight", (H, V), *mat("token_embd.weight", V, H)),
               ("output_norm.weight", (H,), 0, encode(ones(H), 0))]
    if not tied:
        tensors.append(("output.weight", (H, V), *mat("output.weight", V, H)))
    for i in range(L):
        p = f"blk.{i}."
        tensors += [
            (p + "attn_norm.weight", (H,), 0, encode(ones(H), 0)),
            (p + "ffn_norm.weight", (H,), 0, encode(ones(H), 0)),
            (p + "attn_q.weight", (H, H), *mat("attn_q.weight", H, H, i)),
            (p + "attn_k.weight", (H, kvd), *mat("attn_k.weight", kvd, H, i)),
            (p + "attn_v.weight", (H, kvd), *mat("attn_v.weight", kvd, H, i)),
            (p + "attn_q.bias", (H,), 0, encode(normal(1, H) * scale((1, H)), 0)),
            (p + "attn_k.bias", (kvd,), 0, encode(normal(1, kvd) * scale((1, kvd)), 0)),
            (p + "attn_v.bias", (kvd,), 0, encode(normal(1, kvd) * scale((1, kvd)), 0)),
            (p + "attn_output.weight", (H, H), *mat("attn_output.weight", H, H, i)),
            (p + "ffn_gate.weight", (H, F), *mat("ffn_gate.weight", F, H, i)),
            (p + "ffn_up.weight", (H, F), *mat("ffn_up.weight", F, H, i)),
            (p + "ffn_down.weight", (F, H), *mat("ffn_down.weight", H, F, i)),
        ]
    meta = {
        "general.architecture": "qwen2",
        "qwen2.block_count": cfg["layers"],
        "qwen2.embedding_length": H,
        "qwen2.feed_forward_length": F,
        "qwen2.attention.head_count": cfg["heads"],
        "qwen2.attention.head_count_kv": cfg["kv_heads"],
        "qwen2.context_length": cfg["context"],
        "qwen2.attention.layer_norm_rms_epsilon": float(cfg["norm_epsilon"]),
        "qwen2.rope.freq_base": float(cfg["rope_base"]),
        "tokenizer.ggml.model": "gpt2",
        "tokenizer.ggml.tokens": [f"<{i}>" for i in range(V)],
        "tokenizer.ggml.eos_token_id": eos,
    }
    return meta, tensors


def write_model(path, cfg, dtype="q8_0", seed=0, **kw):
    meta, tensors = build(cfg, dtype, seed, **kw)
    gguf.write(path, meta, tensors)
    return path


def in_memory(cfg, dtype="q8_0", seed=0, **kw):
    """The same model without a file: (config, {name: gguf.Tensor})."""
    meta, tensors = build(cfg, dtype, seed, **kw)
    out = {n: gguf.Tensor(n, s, d, np.ascontiguousarray(p)) for n, s, d, p in tensors}
    c = dict(cfg)
    c["eos_token_id"] = meta["tokenizer.ggml.eos_token_id"]
    return c, out
