"""Textbook Qwen3.5 hybrid text decoder in float64 numpy: an independent
derivation used to pin the oracle's graph structure (not a restatement of the
reference code).

Written from the architecture's published description: zero-centred RMSNorm
(scale 1 + w); Gated DeltaNet linear attention (causal depthwise conv + SiLU
on the q/k/v channels, L2-normalised q and k with q scaled by 1/sqrt(d_k),
per-head decay g = -exp(A_log) * softplus(a + dt_bias), write strength
beta = sigmoid(b), state update S <- S*exp(g) + k (beta (v - S^T k))^T,
read o = S^T q, output RMSNorm over d_v times SiLU(z)); gated softmax
attention (per-head q/k RMSNorm, rotary embedding on the first rotary_dim
dims with angle pos * base^(-2i/rotary_dim), causal GQA softmax scaled by
1/sqrt(head_dim), output times sigmoid(gate)); SwiGLU MLP; pre-norm
residuals; tied head.
"""
import numpy as np


def _w(t):
    """gguf.Tensor (F32 or BF16) -> float64 array in [rows, width] order."""
    raw = t.data
    if t.dtype == 30:
        f = (np.frombuffer(raw.tobytes(), np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        f = np.frombuffer(raw.tobytes(), np.float32)
    width = t.shape[0]
    return f.astype(np.float64).reshape(-1, width) if len(t.shape) > 1 else f.astype(np.float64)


def _rms(x, w, eps, centred):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * ((1.0 + w) if centred else w)


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _silu(x):
    return x * _sigmoid(x)


def _softplus(x):
    return np.log1p(np.exp(-np.abs(x))) + np.maximum(x, 0.0)


class Qwen35F64:
    def __init__(self, cfg, tensors, mistake=None):
        self.c = cfg
        self.mistake = mistake
        self.w = {}
        for n, t in tensors.items():
            if n.endswith("conv1d.weight"):
                k = cfg["conv_kernel"]
                self.w[n] = np.frombuffer(t.data.tobytes(), np.float32).astype(np.float64).reshape(-1, k)
            else:
                self.w[n] = _w(t)

    def forward(self, tokens):
        """Teacher-forced logits for every position: [len(tokens), V]."""
        c, w = self.c, self.w
        eps = c["epsilon"]
        D, NH, NKV = c["head_dim"], c["heads"], c["kv_heads"]
        KH, VH, KD, VD = c["key_heads"], c["value_heads"], c["key_dim"], c["value_dim"]
        K = c["conv_kernel"]
        T = len(tokens)
        x = w["model.language_model.embed_tokens.weight"][np.asarray(tokens)]
        pos = np.arange(T, dtype=np.float64)
        half = c["rotary_dim"] // 2
        ang = pos[:, None] * c["rope_base"] ** (-2.0 * np.arange(half) / c["rotary_dim"])
        cos, sin = np.cos(ang), np.sin(ang)

        def rotate(v):  # v [T, heads, D]
            a, b = v[..., :half].copy(), v[..., half:2 * half].copy()
            v = v.copy()
            v[..., :half] = a * cos[:, None, :] - b * sin[:, None, :]
            v[..., half:2 * half] = b * cos[:, None, :] + a * sin[:, None, :]
            return v

        for i, full in enumerate(c["full"]):
            p = f"model.language_model.layers.{i}"
            h = _rms(x, w[f"{p}.input_layernorm.weight"], eps, True)
            if full:
                a = f"{p}.self_attn"
                qg = (h @ w[f"{a}.q_proj.weight"].T).reshape(T, NH, 2 * D)
                q, gate = qg[..., :D], qg[..., D:].reshape(T, NH * D)
                k = (h @ w[f"{a}.k_proj.weight"].T).reshape(T, NKV, D)
                v = (h @ w[f"{a}.v_proj.weight"].T).reshape(T, NKV, D)
                q = rotate(_rms(q, w[f"{a}.q_norm.weight"], eps, True))
                k = rotate(_rms(k, w[f"{a}.k_norm.weight"], eps, True))
                out = np.zeros((T, NH, D))
                g = NH // NKV
                for hh in range(NH):
                    s = q[:, hh] @ k[:, hh // g].T / np.sqrt(D)
                    s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
                    pr = np.exp(s - s.max(axis=1, keepdims=True))
                    out[:, hh] = (pr / pr.sum(axis=1, keepdims=True)) @ v[:, hh // g]
                mixed = out.reshape(T, NH * D) * _sigmoid(gate)
                x = x + mixed @ w[f"{a}.o_proj.weight"].T
            else:
                a = f"{p}.linear_attn"
                qkv = h @ w[f"{a}.in_proj_qkv.weight"].T
                z = h @ w[f"{a}.in_proj_z.weight"].T
                av = h @ w[f"{a}.in_proj_a.weight"].T
                bv = h @ w[f"{a}.in_proj_b.weight"].T
                taps = w[f"{a}.conv1d.weight"]
                if self.mistake == "conv_taps_reversed":
                    taps = taps[:, ::-1]
                padded = np.vstack([np.zeros((K - 1, qkv.shape[1])), qkv])
                conv = np.stack([(padded[t:t + K] * taps.T).sum(axis=0) for t in range(T)])
                conv = _silu(conv)
                keys = KH * KD
                q = conv[:, :keys].reshape(T, KH, KD)
                k = conv[:, keys:2 * keys].reshape(T, KH, KD)
                v = conv[:, 2 * keys:].reshape(T, VH, VD)
                rep = VH // KH
                q = np.repeat(q, rep, axis=1)
                k = np.repeat(k, rep, axis=1)
                q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(KD)
                k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
                gdecay = -np.exp(w[f"{a}.A_log"]) * _softplus(av + w[f"{a}.dt_bias"])
                beta = _sigmoid(bv)
                S = np.zeros((VH, KD, VD))
                o = np.zeros((T, VH, VD))
                for t in range(T):
                    S = S * np.exp(gdecay[t])[:, None, None]
                    pred = np.einsum("hkv,hk->hv", S, k[t])
                    S = S + np.einsum("hk,hv->hkv", k[t], beta[t][:, None] * (v[t] - pred))
                    o[t] = np.einsum("hkv,hk->hv", S, q[t])
                o = _rms(o, w[f"{a}.norm.weight"], eps, False) * _silu(z.reshape(T, VH, VD))
                x = x + o.reshape(T, VH * VD) @ w[f"{a}.out_proj.weight"].T
            h = _rms(x, w[f"{p}.post_attention_layernorm.weight"], eps, True)
            gt = h @ w[f"{p}.mlp.gate_proj.weight"].T
            up = h @ w[f"{p}.mlp.up_proj.weight"].T
            x = x + (_silu(gt) * up) @ w[f"{p}.mlp.down_proj.weight"].T
        h = _rms(x, w["model.language_model.norm.weight"], eps, True)
        head = w.get("lm_head.weight", w["model.language_model.embed_tokens.weight"])
        return h @ head.T
