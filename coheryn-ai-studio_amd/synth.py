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

DTYPES = {"f32": 0, "f16": 1, "q4_0": 2, "q8_0": 8}


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
    raise ValueError(dtype)


def config(**overrides):
    c = dict(QWEN25_05B)
    c.update(overrides)
    c["head_dim"] = c["hidden"] // c["heads"]
    return c


def build(cfg, dtype="q8_0", seed=0, eos_token_id=None, tied=True, std=0.02):
    """Returns (metadata, [(name, shape, dtype, payload)]) for a seeded model."""
    wdt = DTYPES[dtype] if isinstance(dtype, str) else dtype
    rng = np.random.default_rng(seed)
    H, F, V = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"]
    kvd = cfg["kv_heads"] * cfg["head_dim"]
    eos = V - 1 if eos_token_id is None else eos_token_id

    def normal(rows, width):
        return rng.standard_normal((rows, width), dtype=np.float32) * np.float32(std)

    tensors = [("token_embd.weight", (H, V), wdt, encode(normal(V, H), wdt)),
               ("output_norm.weight", (H,), 0, encode(np.ones((1, H), np.float32), 0))]
    if not tied:
        tensors.append(("output.weight", (H, V), wdt, encode(normal(V, H), wdt)))
    for i in range(cfg["layers"]):
        p = f"blk.{i}."
        tensors += [
            (p + "attn_norm.weight", (H,), 0, encode(np.ones((1, H), np.float32), 0)),
            (p + "ffn_norm.weight", (H,), 0, encode(np.ones((1, H), np.float32), 0)),
            (p + "attn_q.weight", (H, H), wdt, encode(normal(H, H), wdt)),
            (p + "attn_k.weight", (H, kvd), wdt, encode(normal(kvd, H), wdt)),
            (p + "attn_v.weight", (H, kvd), wdt, encode(normal(kvd, H), wdt)),
            (p + "attn_q.bias", (H,), 0, encode(normal(1, H), 0)),
            (p + "attn_k.bias", (kvd,), 0, encode(normal(1, kvd), 0)),
            (p + "attn_v.bias", (kvd,), 0, encode(normal(1, kvd), 0)),
            (p + "attn_output.weight", (H, H), wdt, encode(normal(H, H), wdt)),
            (p + "ffn_gate.weight", (H, F), wdt, encode(normal(F, H), wdt)),
            (p + "ffn_up.weight", (H, F), wdt, encode(normal(F, H), wdt)),
            (p + "ffn_down.weight", (F, H), wdt, encode(normal(H, F), wdt)),
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
