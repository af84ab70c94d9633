"""Textbook Qwen2 decoder in float64 numpy — an independent derivation used to
pin the oracle's graph structure (not a restatement of the reference code).

RMSNorm, biased Q/K/V, NeoX rotary embedding (theta_i = pos * base^(-2i/d)),
causal grouped-query softmax attention, SwiGLU MLP, pre-norm residuals, tied
or untied LM head.
"""
import numpy as np


def dequant(t):
    """gguf.Tensor -> float64 [rows, width]."""
    import orc
    width = t.shape[0]
    rows = t.shape[1] if len(t.shape) > 1 else 1
    rb = orc.row_bytes(t.dtype, width)[1]
    out = np.zeros((rows, width), np.float64)
    for r in range(rows):
        rc, v = orc.decode(t.data[r * rb:(r + 1) * rb].tobytes(), t.dtype, width)
        assert rc == 0
        out[r] = v
    return out


class Qwen2F64:
    def __init__(self, cfg, tensors):
        self.c = cfg
        self.w = {n: dequant(t) for n, t in tensors.items()}

    def forward(self, tokens):
        """Teacher-forced logits for every position: [len(tokens), V]."""
        c, w = self.c, self.w
        H, nh, nkv, d = c["hidden"], c["heads"], c["kv_heads"], c["head_dim"]
        T = len(tokens)
        x = w["token_embd.weight"][np.asarray(tokens)]
        pos = np.arange(T, dtype=np.float64)
        inv = c["rope_base"] ** (-2.0 * np.arange(d // 2) / d)
        ang = pos[:, None] * inv[None, :]
        cos, sin = np.cos(ang), np.sin(ang)

        def rms(v, g):
            return v / np.sqrt((v * v).mean(-1, keepdims=True) + c["norm_epsilon"]) * g

        def rope(v):  # [T, heads, d]
            a, b = v[..., :d // 2], v[..., d // 2:]
            return np.concatenate([a * cos[:, None] - b * sin[:, None],
                                   a * sin[:, None] + b * cos[:, None]], -1)

        for i in range(c["layers"]):
            p = f"blk.{i}."
            h = rms(x, w[p + "attn_norm.weight"][0])
            q = h @ w[p + "attn_q.weight"].T + w[p + "attn_q.bias"][0]
            k = h @ w[p + "attn_k.weight"].T + w[p + "attn_k.bias"][0]
            v = h @ w[p + "attn_v.weight"].T + w[p + "attn_v.bias"][0]
            q = rope(q.reshape(T, nh, d))
            k = rope(k.reshape(T, nkv, d))
            v = v.reshape(T, nkv, d)
            g = nh // nkv
            out = np.zeros((T, nh, d))
            for hh in range(nh):
                s = q[:, hh] @ k[:, hh // g].T / np.sqrt(d)
                s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
                s = np.exp(s - s.max(-1, keepdims=True))
                s /= s.sum(-1, keepdims=True)
                out[:, hh] = s @ v[:, hh // g]
            x = x + out.reshape(T, H) @ w[p + "attn_output.weight"].T
            h = rms(x, w[p + "ffn_norm.weight"][0])
            gt = h @ w[p + "ffn_gate.weight"].T
            up = h @ w[p + "ffn_up.weight"].T
            x = x + (gt / (1 + np.exp(-gt)) * up) @ w[p + "ffn_down.weight"].T
        h = rms(x, w["output_norm.weight"][0])
        head = w.get("output.weight", w["token_embd.weight"])
        return h @ head.T
