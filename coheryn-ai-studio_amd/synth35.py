"""Seeded synthetic Qwen3.5 hybrid text models (no file; tensors in memory).

The tensor set and shapes are those qwen35/config.rs:193-309 validates, under
the safetensors names the reference binds (qwen35/execution.rs:168-219).
Matrices are BF16 (round-to-nearest-even of float32 N(0, std) draws);
vectors are F32: norm weights N(0, 0.02) (the zero-centred norms scale by
w + 1; the linear-attention output norm by w, so it draws around 1),
A_log = log(U[1, 16]), dt_bias = 1 + N(0, 0.1), causal-conv taps N(0, 0.25).
"""
import numpy as np

import gguf

BF16, F32 = 30, 0

# Qwen3.5-0.8B text shape (fixtures/qualification/a1-metadata-runtime.json:25-68)
QWEN35_08B = dict(layers=24, hidden=1024, intermediate=3584, vocabulary=248320, heads=8,
                  kv_heads=2, head_dim=256, key_heads=16, value_heads=16, key_dim=128,
                  value_dim=128, conv_kernel=4, rotary_dim=64, rope_base=1e7, epsilon=1e-6,
                  context=262144, pattern="LLLF")


def config(**overrides):
    c = dict(QWEN35_08B)
    c.update(overrides)
    pat = c["pattern"]
    c["full"] = [pat[i % len(pat)] == "F" for i in range(c["layers"])]
    return c


def to_bf16(x):
    """float32 -> bfloat16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _t(name, shape, dtype, arr):
    data = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    return gguf.Tensor(name, shape, dtype, data)


def in_memory(cfg, seed=0, std=0.02, tied=True):
    """(config, {name: gguf.Tensor}) with GGML-order shapes (ne0 = width, ne1 = rows)."""
    rng = np.random.default_rng(seed)
    H, F, V = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"]
    D, NH, NKV = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    keys = cfg["key_heads"] * cfg["key_dim"]
    vals = cfg["value_heads"] * cfg["value_dim"]
    ch = 2 * keys + vals
    out = {}

    def mat(name, rows, width):
        w = rng.standard_normal((rows, width), dtype=np.float32) * np.float32(std)
        out[name] = _t(name, (width, rows), BF16, to_bf16(w))

    def vec(name, v):
        v = np.asarray(v, np.float32).reshape(-1)
        out[name] = _t(name, (v.size,), F32, v)

    mat("model.language_model.embed_tokens.weight", V, H)
    vec("model.language_model.norm.weight", rng.standard_normal(H, dtype=np.float32) * 0.02)
    if not tied:
        mat("lm_head.weight", V, H)
    for i, full in enumerate(cfg["full"]):
        p = f"model.language_model.layers.{i}"
        vec(f"{p}.input_layernorm.weight", rng.standard_normal(H, dtype=np.float32) * 0.02)
        vec(f"{p}.post_attention_layernorm.weight", rng.standard_normal(H, dtype=np.float32) * 0.02)
        mat(f"{p}.mlp.gate_proj.weight", F, H)
        mat(f"{p}.mlp.up_proj.weight", F, H)
        mat(f"{p}.mlp.down_proj.weight", H, F)
        if full:
            a = f"{p}.self_attn"
            mat(f"{a}.q_proj.weight", 2 * NH * D, H)
            mat(f"{a}.k_proj.weight", NKV * D, H)
            mat(f"{a}.v_proj.weight", NKV * D, H)
            mat(f"{a}.o_proj.weight", H, NH * D)
            vec(f"{a}.q_norm.weight", rng.standard_normal(D, dtype=np.float32) * 0.02)
            vec(f"{a}.k_norm.weight", rng.standard_normal(D, dtype=np.float32) * 0.02)
        else:
            a = f"{p}.linear_attn"
            mat(f"{a}.in_proj_qkv.weight", ch, H)
            mat(f"{a}.in_proj_z.weight", vals, H)
            mat(f"{a}.in_proj_a.weight", cfg["value_heads"], H)
            mat(f"{a}.in_proj_b.weight", cfg["value_heads"], H)
            mat(f"{a}.out_proj.weight", H, vals)
            conv = rng.standard_normal((ch, 1, cfg["conv_kernel"]), dtype=np.float32) * 0.25
            out[f"{a}.conv1d.weight"] = _t(f"{a}.conv1d.weight", (cfg["conv_kernel"], 1, ch), F32,
                                           conv)
            vec(f"{a}.A_log", np.log(rng.uniform(1.0, 16.0, cfg["value_heads"])).astype(np.float32))
            vec(f"{a}.dt_bias", 1.0 + rng.standard_normal(cfg["value_heads"], dtype=np.float32) * 0.1)
            vec(f"{a}.norm.weight", 1.0 + rng.standard_normal(cfg["value_dim"], dtype=np.float32) * 0.02)
    c = dict(cfg)
    c["tied"] = tied
    return c, out
