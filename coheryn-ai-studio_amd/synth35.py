"""Seeded synthetic Qwen3.5 hybrid text models (no file; tensors in memory).

The tensor set and shapes are those qwen35/config.rs:193-309 validates, under
the safetensors names the reference binds (qwen35/execution.rs:168-219).
Matrices are BF16 (round-to-nearest-even of float32 N(0, std) draws);
vectors are F32: norm weights N(0, 0.02) (the zero-centred norms scale by
w + 1; the linear-attention output norm by w, so it draws around 1),
A_log = log(U[1, 16]), dt_bias = 1 + N(0, 0.1), causal-conv taps N(0, 0.25).
"""
import os

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
    """float32 -> bfloat16 bits, round to nearest even (finite inputs: the sum
    stays below 2^32, so 32-bit arithmetic suffices)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(
        np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _t(name, shape, dtype, arr):
    data = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    return gguf.Tensor(name, shape, dtype, data)


def _plan(cfg, tied):
    """(name, kind, GGML shape, draw) for every tensor, in a fixed order; draw
    maps a Generator to the float32 values."""
    H, F, V = cfg["hidden"], cfg["intermediate"], cfg["vocabulary"]
    D, NH, NKV = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    VH, VD, K = cfg["value_heads"], cfg["value_dim"], cfg["conv_kernel"]
    keys = cfg["key_heads"] * cfg["key_dim"]
    vals = VH * VD
    ch = 2 * keys + vals
    plan = []

    def mat(name, rows, width):
        plan.append((name, BF16, (width, rows), lambda g, n=rows * width: g.standard_normal(
            n, dtype=np.float32)))

    def vec(name, n, draw):
        plan.append((name, F32, (n,), draw))

    def normal(n, std, mean=0.0):
        return lambda g: np.float32(mean) + g.standard_normal(n, dtype=np.float32) * np.float32(std)

    mat("model.language_model.embed_tokens.weight", V, H)
    vec("model.language_model.norm.weight", H, normal(H, 0.02))
    if not tied:
        mat("lm_head.weight", V, H)
    for i, full in enumerate(cfg["full"]):
        p = f"model.language_model.layers.{i}"
        vec(f"{p}.input_layernorm.weight", H, normal(H, 0.02))
        vec(f"{p}.post_attention_layernorm.weight", H, normal(H, 0.02))
        mat(f"{p}.mlp.gate_proj.weight", F, H)
        mat(f"{p}.mlp.up_proj.weight", F, H)
        mat(f"{p}.mlp.down_proj.weight", H, F)
        if full:
            a = f"{p}.self_attn"
            mat(f"{a}.q_proj.weight", 2 * NH * D, H)
            mat(f"{a}.k_proj.weight", NKV * D, H)
            mat(f"{a}.v_proj.weight", NKV * D, H)
            mat(f"{a}.o_proj.weight", H, NH * D)
            vec(f"{a}.q_norm.weight", D, normal(D, 0.02))
            vec(f"{a}.k_norm.weight", D, normal(D, 0.02))
        else:
            a = f"{p}.linear_attn"
            mat(f"{a}.in_proj_qkv.weight", ch, H)
            mat(f"{a}.in_proj_z.weight", vals, H)
            mat(f"{a}.in_proj_a.weight", VH, H)
            mat(f"{a}.in_proj_b.weight", VH, H)
            mat(f"{a}.out_proj.weight", H, vals)
            plan.append((f"{a}.conv1d.weight", F32, (K, 1, ch), normal(ch * K, 0.25)))
            vec(f"{a}.A_log", VH, lambda g, n=VH: np.log(g.uniform(1.0, 16.0, n)).astype(np.float32))
            vec(f"{a}.dt_bias", VH, normal(VH, 0.1, 1.0))
            vec(f"{a}.norm.weight", VD, normal(VD, 0.02, 1.0))
    return plan


def in_memory(cfg, seed=0, std=0.02, tied=True, threads=None):
    """(config, {name: gguf.Tensor}) with GGML-order shapes (ne0 = width, ne1 = rows).
    Every tensor draws from its own child of SeedSequence(seed), so the values
    do not depend on the thread count; the draws run on a thread pool."""
    from concurrent.futures import ThreadPoolExecutor
    plan = _plan(cfg, tied)
    kids = np.random.SeedSequence(seed).spawn(len(plan))

    def make(i):
        name, dtype, shape, draw = plan[i]
        v = draw(np.random.default_rng(kids[i]))
        if dtype == BF16:
            v *= np.float32(std)
            return _t(name, shape, BF16, to_bf16(v))
        return _t(name, shape, F32, v.astype(np.float32))

    workers = threads or min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(workers) as ex:
        tensors = list(ex.map(make, range(len(plan))))
    out = {t.name: t for t in tensors}
    c = dict(cfg)
    c["tied"] = tied
    return c, out
