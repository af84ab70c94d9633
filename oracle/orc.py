"""ctypes binding of the CPU oracle (liborc.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path.  Importable
from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg; the
product library never loads it.  See orc.h for what each function restates
(reference file:line) and what pins it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_sz = ctypes.c_size_t


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_row_bytes": (ctypes.c_int, [ctypes.c_uint32, _sz, ctypes.POINTER(_sz)]),
        "orc_decode": (ctypes.c_int, [_u8p, _sz, ctypes.c_uint32, _f32p, _sz]),
        "orc_dot_f32": (ctypes.c_float, [_f32p, _f32p, _sz]),
        "orc_round_f16": (ctypes.c_int, [_f32p, _f32p, _sz]),
        "orc_rms_norm": (None, [_f32p, _f32p, ctypes.c_float, _f32p, _sz]),
        "orc_rope": (None, [_f32p, _sz, _sz, _sz, ctypes.c_float]),
        "orc_swiglu": (None, [_f32p, _f32p, _sz]),
        "orc_prepare": (ctypes.c_int, [_f32p, _sz, ctypes.c_uint32, _u8p, _sz,
                                       ctypes.POINTER(_sz), _u32p]),
        "orc_qdot": (ctypes.c_int, [_u8p, _sz, ctypes.c_uint32, _u8p, ctypes.c_uint32, _sz,
                                    _f32p]),
        "orc_attention_rows": (ctypes.c_int, [_f32p, _sz, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
        "orc_attention": (ctypes.c_int, [_f32p, _sz, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
        "orc_sampler_new": (ctypes.c_int, [ctypes.c_float, ctypes.c_uint32, ctypes.c_float,
                                           ctypes.c_uint64, ctypes.c_float, ctypes.c_float,
                                           ctypes.c_float, ctypes.POINTER(ctypes.c_void_p)]),
        "orc_sampler_free": (None, [ctypes.c_void_p]),
        "orc_sampler_history": (ctypes.c_int, [ctypes.c_void_p, _sz, _u32p, _sz]),
        "orc_sampler_observe": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
        "orc_sampler_sample": (ctypes.c_int, [ctypes.c_void_p, _f32p, _sz, _u8p, _u32p]),
        "orc_model_new": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]),
        "orc_model_free": (None, [ctypes.c_void_p]),
        "orc_session_new": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32,
                                           ctypes.POINTER(ctypes.c_void_p)]),
        "orc_session_free": (None, [ctypes.c_void_p]),
        "orc_session_position": (ctypes.c_uint32, [ctypes.c_void_p]),
        "orc_session_truncate": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
        "orc_session_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                          ctypes.c_int, _f32p]),
        "orc_session_logits": (_f32p, [ctypes.c_void_p]),
        "orc_synthetic_kv": (ctypes.c_float, [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
        "orc_session_fill_synthetic": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p,
                                                      ctypes.c_uint32, ctypes.c_uint64,
                                                      ctypes.c_uint32]),
        "orc_forward_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _u32p, _sz,
                                             _i32p]),
        "orc_forward_batch_trace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _u32p, _sz,
                                                   _i32p, _f32p]),
        "orc_pack": (ctypes.c_int, [_sz, _u32p, _u32p, _i32p, ctypes.c_uint32, ctypes.c_uint32,
                                    _u32p, _u32p, _i64p, _u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def ptr(a, t):
    return a.ctypes.data_as(t)


def f16_to_f32(h):
    return lib.orc_f16_to_f32(h)


def f32_to_f16(f):
    return lib.orc_f32_to_f16(f)


def row_bytes(dtype, width):
    out = _sz()
    rc = lib.orc_row_bytes(dtype, width, ctypes.byref(out))
    return rc, out.value


def decode(data, dtype, n):
    data = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
    out = np.zeros(n, np.float32)
    rc = lib.orc_decode(ptr(data, _u8p), data.size, dtype, ptr(out, _f32p), n)
    return rc, out


def dot_f32(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib.orc_dot_f32(ptr(a, _f32p), ptr(b, _f32p), a.size)


def round_f16(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    rc = lib.orc_round_f16(ptr(x, _f32p), ptr(out, _f32p), x.size)
    return rc, out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib.orc_rms_norm(ptr(x, _f32p), ptr(w, _f32p), eps, ptr(out, _f32p), x.size)
    return out


def rope(x, head_dim, position, base):
    x = np.array(x, np.float32)
    lib.orc_rope(ptr(x, _f32p), x.size, head_dim, position, base)
    return x


def swiglu(g, u):
    g = np.array(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    lib.orc_swiglu(ptr(g, _f32p), ptr(u, _f32p), g.size)
    return g


def prepare(x, weight_dtype):
    x = np.ascontiguousarray(x, np.float32)
    cap = (x.size // 32 + 1) * 292
    out = np.zeros(cap, np.uint8)
    used = _sz()
    kind = ctypes.c_uint32()
    rc = lib.orc_prepare(ptr(x, _f32p), x.size, weight_dtype, ptr(out, _u8p), cap,
                         ctypes.byref(used), ctypes.byref(kind))
    return rc, out[:used.value].copy(), kind.value


def qdot(row, dtype, act, act_kind, width):
    row = np.ascontiguousarray(np.frombuffer(bytes(row), np.uint8))
    act = np.ascontiguousarray(np.frombuffer(bytes(act), np.uint8))
    out = ctypes.c_float()
    rc = lib.orc_qdot(ptr(row, _u8p), row.size, dtype, ptr(act, _u8p), act_kind, width,
                      ctypes.byref(out))
    return rc, out.value


def attention_rows(q, keys, values, kv_heads, head_dim, online=False):
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    out = np.zeros_like(q)
    rows = keys.size // (kv_heads * head_dim) if kv_heads * head_dim else 0
    fn = lib.orc_attention if online else lib.orc_attention_rows
    rc = fn(ptr(q, _f32p), q.size, ptr(keys, _f32p), ptr(values, _f32p), rows, kv_heads,
            head_dim, ptr(out, _f32p))
    return rc, out


class Sampler:
    """sampling.rs Sampler (temperature 0 = greedy, lowest id on ties)."""

    def __init__(self, temperature=0.0, top_k=0, top_p=1.0, seed=0, repetition_penalty=1.0,
                 frequency_penalty=0.0, presence_penalty=0.0):
        h = ctypes.c_void_p()
        rc = lib.orc_sampler_new(temperature, top_k, top_p, seed, repetition_penalty,
                                 frequency_penalty, presence_penalty, ctypes.byref(h))
        if rc:
            raise ValueError(f"sampler rejected ({rc})")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_sampler_free(self.h)
            self.h = None

    def history(self, vocabulary, tokens):
        t = np.ascontiguousarray(tokens, np.uint32)
        return lib.orc_sampler_history(self.h, vocabulary, ptr(t, _u32p), t.size)

    def observe(self, token):
        return lib.orc_sampler_observe(self.h, token)

    def sample(self, logits, allowed=None):
        logits = np.ascontiguousarray(logits, np.float32)
        a = None
        if allowed is not None:
            a = np.ascontiguousarray(allowed, np.uint8)
        tok = ctypes.c_uint32()
        rc = lib.orc_sampler_sample(self.h, ptr(logits, _f32p), logits.size,
                                    ptr(a, _u8p) if a is not None else None, ctypes.byref(tok))
        return rc, tok.value


class OrcConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim",
                 "vocabulary", "context")] + [("rope_base", ctypes.c_float),
                                             ("norm_epsilon", ctypes.c_float)]


class OrcTensor(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint32), ("ne0", ctypes.c_uint64), ("ne1", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("bytes", ctypes.c_uint64)]


LAYER_SLOTS = ["attn_norm.weight", "ffn_norm.weight", "attn_q.weight", "attn_k.weight",
               "attn_v.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias",
               "attn_output.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"]


class Model:
    """Oracle Qwen2 model over in-memory GGUF tensors (dict name -> Tensor)."""

    def __init__(self, config, tensors, threads=None):
        self.config = config
        self.tensors = tensors  # keep buffers alive
        c = OrcConfig(**{k: config[k] for k in (
            "layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim", "vocabulary",
            "context", "rope_base", "norm_epsilon")})

        def ot(name):
            t = tensors.get(name)
            if t is None:
                return OrcTensor(0, 0, 0, None, 0)
            ne1 = t.shape[1] if len(t.shape) > 1 else 1
            return OrcTensor(t.dtype, t.shape[0], ne1, t.data.ctypes.data, t.data.nbytes)

        g = (OrcTensor * 3)(ot("token_embd.weight"), ot("output_norm.weight"),
                            ot("output.weight"))
        L = config["layers"]
        lt = (OrcTensor * (L * len(LAYER_SLOTS)))()
        for i in range(L):
            for j, slot in enumerate(LAYER_SLOTS):
                lt[i * len(LAYER_SLOTS) + j] = ot(f"blk.{i}.{slot}")
        h = ctypes.c_void_p()
        threads = threads or min(16, os.cpu_count() or 1)
        rc = lib.orc_model_new(ctypes.byref(c), g, lt, threads, ctypes.byref(h))
        if rc:
            raise ValueError(f"oracle model rejected ({rc})")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_model_free(self.h)
            self.h = None

    def session(self, context=None):
        return Session(self, context or self.config["context"])

    def forward_batch(self, sessions, tokens, trace=False):
        n = len(sessions)
        arr = (ctypes.c_void_p * n)(*[s.h for s in sessions])
        toks = np.ascontiguousarray(tokens, np.uint32)
        errs = np.array([s.error for s in sessions], np.int32)
        if trace:
            tr = np.zeros((n, self.config["layers"], self.config["hidden"]), np.float32)
            lib.orc_forward_batch_trace(self.h, arr, ptr(toks, _u32p), n, ptr(errs, _i32p),
                                        ptr(tr, _f32p))
        else:
            lib.orc_forward_batch(self.h, arr, ptr(toks, _u32p), n, ptr(errs, _i32p))
        for s, e in zip(sessions, errs):
            s.error = int(e)
        return (errs, tr) if trace else errs


class Session:
    def __init__(self, model, context):
        self.model = model
        h = ctypes.c_void_p()
        rc = lib.orc_session_new(model.h, context, ctypes.byref(h))
        if rc:
            raise ValueError(f"oracle session rejected ({rc})")
        self.h = h
        self.error = 0

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_session_free(self.h)
            self.h = None

    @property
    def position(self):
        return lib.orc_session_position(self.h)

    def truncate(self, rows):
        return lib.orc_session_truncate(self.h, rows)

    def logits(self):
        V = self.model.config["vocabulary"]
        p = lib.orc_session_logits(self.h)
        return np.ctypeslib.as_array(p, shape=(V,)).copy()

    def kv(self, layer, values=False):
        c = self.model.config
        out = np.zeros((self.position, c["kv_heads"] * c["head_dim"]), np.float32)
        lib.orc_session_kv(self.model.h, self.h, layer, 1 if values else 0, ptr(out, _f32p))
        return out

    def fill_synthetic(self, rows, seed, stream):
        return lib.orc_session_fill_synthetic(self.model.h, self.h, rows, seed, stream)


def synthetic_kv(seed, stream, layer, which, position, element):
    return lib.orc_synthetic_kv(seed, stream, layer, which, position, element)


def pack(n_tokens, start, pages, page_size):
    n_tokens = np.ascontiguousarray(n_tokens, np.uint32)
    start = np.ascontiguousarray(start, np.uint32)
    pages = np.ascontiguousarray(pages, np.int32)
    n = n_tokens.size
    max_pages = pages.shape[1] if pages.ndim == 2 else 0
    R = int(n_tokens.sum())
    cu = np.zeros(n + 1, np.uint32)
    pos = np.zeros(R, np.uint32)
    slot = np.zeros(R, np.int64)
    lane = np.zeros(R, np.uint32)
    rc = lib.orc_pack(n, ptr(n_tokens, _u32p), ptr(start, _u32p), ptr(pages, _i32p), max_pages,
                      page_size, ptr(cu, _u32p), ptr(pos, _u32p), ptr(slot, _i64p),
                      ptr(lane, _u32p))
    return rc, cu, pos, slot, lane

# ---- Qwen3.5 hybrid text model -------------------------------------------------

class OrcQ35Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("layers", "hidden", "intermediate", "vocabulary", "heads", "kv_heads",
                 "head_dim", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel",
                 "rotary_dim", "context")] + [("epsilon", ctypes.c_float),
                                              ("rope_base", ctypes.c_float),
                                              ("full", ctypes.c_uint8 * 128)]


Q35_SLOTS = ["input_layernorm.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
             "mlp.up_proj.weight", "mlp.down_proj.weight", "self_attn.q_proj.weight",
             "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
             "self_attn.q_norm.weight", "self_attn.k_norm.weight",
             "linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight",
             "linear_attn.in_proj_a.weight", "linear_attn.in_proj_b.weight",
             "linear_attn.out_proj.weight", "linear_attn.conv1d.weight", "linear_attn.A_log",
             "linear_attn.dt_bias", "linear_attn.norm.weight"]

_q35_sig = {
    "orc_q35_sigmoid": (ctypes.c_float, [ctypes.c_float]),
    "orc_q35_silu": (ctypes.c_float, [ctypes.c_float]),
    "orc_q35_softplus": (ctypes.c_float, [ctypes.c_float]),
    "orc_q35_norm": (ctypes.c_int, [_f32p, _f32p, ctypes.c_float, ctypes.c_int, _f32p, _sz]),
    "orc_q35_conv_step": (ctypes.c_int, [_f32p, _u32p, _sz, _sz, _f32p, _f32p, _f32p]),
    "orc_q35_delta_step": (ctypes.c_int, [_f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p,
                                          _f32p, _f32p]),
    "orc_q35_partial_rope": (ctypes.c_int, [_f32p, _sz, _sz, _sz, _sz, ctypes.c_float]),
    "orc_q35_model_new": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]),
    "orc_q35_model_free": (None, [ctypes.c_void_p]),
    "orc_q35_session_new": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32,
                                           ctypes.POINTER(ctypes.c_void_p)]),
    "orc_q35_session_free": (None, [ctypes.c_void_p]),
    "orc_q35_session_position": (ctypes.c_uint32, [ctypes.c_void_p]),
    "orc_q35_session_logits": (_f32p, [ctypes.c_void_p]),
    "orc_q35_session_state": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                             ctypes.c_int, _f32p]),
    "orc_q35_forward_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _u32p, _u8p, _sz,
                                             _i32p]),
}
for _name, (_res, _args) in _q35_sig.items():
    _fn = getattr(lib, _name)
    _fn.restype, _fn.argtypes = _res, _args


def q35_sigmoid(x):
    return float(lib.orc_q35_sigmoid(x))


def q35_silu(x):
    return float(lib.orc_q35_silu(x))


def q35_softplus(x):
    return float(lib.orc_q35_softplus(x))


def q35_norm(x, w, eps, zero_centered):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    rc = lib.orc_q35_norm(ptr(x, _f32p), ptr(w, _f32p), eps, int(zero_centered), ptr(out, _f32p),
                          x.size)
    return rc, out


class ConvState:
    """kernels.rs:54-120 ConvState over [channels][kernel]."""

    def __init__(self, channels, kernel):
        self.history = np.zeros(channels * kernel, np.float32)
        self.cursor = np.zeros(1, np.uint32)
        self.channels, self.kernel = channels, kernel

    def step(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.zeros(self.channels, np.float32)
        rc = lib.orc_q35_conv_step(ptr(self.history, _f32p), ptr(self.cursor, _u32p),
                                   self.channels, self.kernel, ptr(x, _f32p), ptr(w, _f32p),
                                   ptr(out, _f32p))
        return rc, out


class DeltaState:
    """kernels.rs:122-214 DeltaState over [heads][key][value]."""

    def __init__(self, heads, key, value):
        self.memory = np.zeros(heads * key * value, np.float32)
        self.shape = (heads, key, value)

    def step(self, q, k, v, log_decay, beta):
        h, kd, vd = self.shape
        a = [np.ascontiguousarray(x, np.float32) for x in (q, k, v, log_decay, beta)]
        out = np.zeros(h * vd, np.float32)
        rc = lib.orc_q35_delta_step(ptr(self.memory, _f32p), h, kd, vd, *[ptr(x, _f32p) for x in a],
                                    ptr(out, _f32p))
        return rc, out


def q35_partial_rope(x, head, rotary, position, base):
    x = np.array(x, np.float32)
    rc = lib.orc_q35_partial_rope(ptr(x, _f32p), x.size, head, rotary, position, base)
    return rc, x


class Qwen35Model:
    """Oracle Qwen3.5 hybrid model over in-memory tensors (dict name -> Tensor)."""

    def __init__(self, config, tensors, threads=None):
        self.config = config
        self.tensors = tensors
        c = OrcQ35Config()
        for k in ("layers", "hidden", "intermediate", "vocabulary", "heads", "kv_heads",
                  "head_dim", "key_heads", "value_heads", "key_dim", "value_dim", "conv_kernel",
                  "rotary_dim", "context"):
            setattr(c, k, config[k])
        c.epsilon, c.rope_base = config["epsilon"], config["rope_base"]
        for i, f in enumerate(config["full"]):
            c.full[i] = 1 if f else 0

        def ot(name):
            t = tensors.get(name)
            if t is None:
                return OrcTensor(0, 0, 0, None, 0)
            n = int(np.prod(t.shape))
            ne0 = t.shape[0]
            return OrcTensor(t.dtype, ne0, n // ne0, t.data.ctypes.data, t.data.nbytes)

        g = (OrcTensor * 3)(ot("model.language_model.embed_tokens.weight"),
                            ot("model.language_model.norm.weight"), ot("lm_head.weight"))
        L = config["layers"]
        lt = (OrcTensor * (L * len(Q35_SLOTS)))()
        for i in range(L):
            for j, slot in enumerate(Q35_SLOTS):
                lt[i * len(Q35_SLOTS) + j] = ot(f"model.language_model.layers.{i}.{slot}")
        h = ctypes.c_void_p()
        threads = threads or min(16, os.cpu_count() or 1)
        rc = lib.orc_q35_model_new(ctypes.byref(c), g, lt, threads, ctypes.byref(h))
        if rc:
            raise ValueError(f"oracle Qwen3.5 model rejected ({rc})")
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_q35_model_free(self.h)
            self.h = None

    def session(self, context):
        return Qwen35Session(self, context)

    def forward_batch(self, sessions, tokens, logits=None):
        n = len(sessions)
        arr = (ctypes.c_void_p * n)(*[s.h for s in sessions])
        toks = np.ascontiguousarray(tokens, np.uint32)
        want = np.ascontiguousarray([1] * n if logits is None else logits, np.uint8)
        errs = np.array([s.error for s in sessions], np.int32)
        lib.orc_q35_forward_batch(self.h, arr, ptr(toks, _u32p), ptr(want, _u8p), n,
                                  ptr(errs, _i32p))
        for s, e in zip(sessions, errs):
            s.error = int(e)
        return errs


class Qwen35Session:
    def __init__(self, model, context):
        self.model = model
        h = ctypes.c_void_p()
        rc = lib.orc_q35_session_new(model.h, context, ctypes.byref(h))
        if rc:
            raise ValueError(f"oracle session rejected ({rc})")
        self.h = h
        self.error = 0

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_q35_session_free(self.h)
            self.h = None

    def position(self):
        return int(lib.orc_q35_session_position(self.h))

    def logits(self):
        p = lib.orc_q35_session_logits(self.h)
        return np.ctypeslib.as_array(p, (self.model.config["vocabulary"],)).copy()

    def state(self, layer, which):
        """0/1: K/V rows [0, position); 2: conv ring; 3: delta memory; 4: conv cursor."""
        c = self.model.config
        kw = c["kv_heads"] * c["head_dim"]
        ch = 2 * c["key_heads"] * c["key_dim"] + c["value_heads"] * c["value_dim"]
        n = {0: self.position() * kw, 1: self.position() * kw, 2: ch * c["conv_kernel"],
             3: c["value_heads"] * c["key_dim"] * c["value_dim"], 4: 1}[which]
        out = np.zeros(max(n, 1), np.float32)
        rc = lib.orc_q35_session_state(self.model.h, self.h, layer, which, ptr(out, _f32p))
        if rc:
            raise ValueError(f"state {which} of layer {layer}: {rc}")
        return out[:n]
