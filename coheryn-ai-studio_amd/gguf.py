"""GGUF v3 container: writer and memory-mapped reader.

Layout follows the reader at crates/coheryn-engine/src/gguf.rs:311-496 (header,
metadata key/values, tensor table, `general.alignment`-aligned data section,
GGML dimension order with the contiguous input dimension first) and the dtype
table at gguf.rs:104-128.  Tensors are returned as raw little-endian payload
bytes; decoding is the library's job.
"""
import struct
from dataclasses import dataclass

import numpy as np

# gguf.rs:104-128 — (name, block elements, block bytes)
ENCODING = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 40),
    10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144),
    13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8),
    28: ("F64", 1, 8), 30: ("BF16", 1, 2),
}

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


@dataclass
class Tensor:
    name: str
    shape: tuple  # GGML order: (ne0 = input width, ne1 = rows)
    dtype: int
    data: np.ndarray  # uint8 payload

    @property
    def rows(self):
        return self.shape[1] if len(self.shape) > 1 else 1


def tensor_bytes(dtype, shape):
    _, block, size = ENCODING[dtype]
    n = 1
    for d in shape:
        n *= d
    if shape[0] % block:
        raise ValueError("row is not block aligned")
    return n // block * size


class Value:
    """Explicitly typed metadata value."""

    def __init__(self, kind, value, elem=None):
        self.kind, self.value, self.elem = kind, value, elem


def _pack_str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v):
    if not isinstance(v, Value):
        if isinstance(v, bool):
            v = Value(T_BOOL, v)
        elif isinstance(v, int):
            v = Value(T_U32, v)
        elif isinstance(v, float):
            v = Value(T_F32, v)
        elif isinstance(v, str):
            v = Value(T_STR, v)
        elif isinstance(v, (list, tuple)):
            elem = T_STR if (v and isinstance(v[0], str)) else T_U32
            v = Value(T_ARR, list(v), elem)
        else:
            raise TypeError(type(v))
    out = struct.pack("<I", v.kind)
    if v.kind == T_STR:
        out += _pack_str(v.value)
    elif v.kind == T_ARR:
        out += struct.pack("<IQ", v.elem, len(v.value))
        if v.elem == T_STR:
            out += b"".join(_pack_str(s) for s in v.value)
        else:
            out += np.asarray(v.value, dtype=np.dtype(_SCALAR[v.elem][1:]).newbyteorder("<")
                              ).tobytes()
    else:
        out += struct.pack(_SCALAR[v.kind], v.value)
    return out


def write(path, metadata, tensors, alignment=32):
    """tensors: iterable of (name, shape, dtype, payload bytes/ndarray)."""
    tensors = list(tensors)
    header = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(metadata))
    for k, v in metadata.items():
        header += _pack_str(k) + _pack_value(v)
    offset = 0
    infos = []
    for name, shape, dtype, payload in tensors:
        nbytes = tensor_bytes(dtype, shape)
        payload = np.frombuffer(memoryview(payload), np.uint8) if not isinstance(
            payload, np.ndarray) else payload.view(np.uint8).reshape(-1)
        if payload.size != nbytes:
            raise ValueError(f"{name}: payload {payload.size} != {nbytes}")
        offset = (offset + alignment - 1) // alignment * alignment
        infos.append((name, shape, dtype, offset, payload))
        header += _pack_str(name) + struct.pack("<I", len(shape))
        header += b"".join(struct.pack("<Q", d) for d in shape)
        header += struct.pack("<IQ", dtype, offset)
        offset += nbytes
    pad = (-len(header)) % alignment
    with open(path, "wb") as f:
        f.write(header + b"\0" * pad)
        pos = 0
        for name, shape, dtype, off, payload in infos:
            if off > pos:
                f.write(b"\0" * (off - pos))
                pos = off
            f.write(payload.tobytes())
            pos += payload.size


class _Reader:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if self.pos + n > len(self.buf):
            raise ValueError("truncated GGUF")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def unpack(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        n = self.unpack("<Q")
        if n > 1 << 24:
            raise ValueError("string too long")
        return bytes(self.take(n)).decode("utf-8")

    def value(self, kind):
        if kind == T_STR:
            return self.string()
        if kind == T_ARR:
            elem, n = self.unpack("<I"), self.unpack("<Q")
            if elem == T_STR:
                return [self.string() for _ in range(n)]
            fmt = _SCALAR[elem]
            size = struct.calcsize(fmt)
            return np.frombuffer(self.take(size * n), np.dtype(fmt[1:]).newbyteorder("<")).tolist()
        return self.unpack(_SCALAR[kind])


def read(path):
    """Returns (metadata dict, {name: Tensor}) with payloads memory-mapped."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    r = _Reader(memoryview(mm))
    if bytes(r.take(4)) != b"GGUF":
        raise ValueError("not a GGUF file")
    version = r.unpack("<I")
    if version != 3:
        raise ValueError("only GGUF v3 is supported")
    n_tensors, n_kv = r.unpack("<Q"), r.unpack("<Q")
    meta = {}
    for _ in range(n_kv):
        key = r.string()
        meta[key] = r.value(r.unpack("<I"))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.unpack("<I")
        shape = tuple(r.unpack("<Q") for _ in range(nd))
        dtype, off = r.unpack("<I"), r.unpack("<Q")
        if dtype not in ENCODING:
            raise ValueError(f"unknown dtype {dtype}")
        infos.append((name, shape, dtype, off))
    alignment = int(meta.get("general.alignment", 32))
    data = (r.pos + alignment - 1) // alignment * alignment
    tensors = {}
    for name, shape, dtype, off in infos:
        if off % alignment:
            raise ValueError("misaligned tensor")
        nbytes = tensor_bytes(dtype, shape)
        start = data + off
        if start + nbytes > mm.size:
            raise ValueError("tensor outside file")
        tensors[name] = Tensor(name, shape, dtype, mm[start:start + nbytes])
    return meta, tensors


def qwen2_config(meta):
    """compat.rs:54-159 configuration_for(..., "qwen2")."""
    a = meta.get("general.architecture")
    if a != "qwen2":
        raise ValueError("only the Qwen2 decoder graph is implemented")
    g = lambda k: meta[f"qwen2.{k}"]
    hidden, heads, kv = g("embedding_length"), g("attention.head_count"), g(
        "attention.head_count_kv")
    if hidden % heads or heads % kv or (hidden // heads) % 2:
        raise ValueError("invalid Qwen2 GQA or RoPE dimensions")
    return dict(layers=g("block_count"), hidden=hidden, intermediate=g("feed_forward_length"),
                heads=heads, kv_heads=kv, head_dim=hidden // heads,
                vocabulary=len(meta["tokenizer.ggml.tokens"]), context=g("context_length"),
                rope_base=float(meta.get("qwen2.rope.freq_base", 10000.0)),
                norm_epsilon=float(g("attention.layer_norm_rms_epsilon")),
                eos_token_id=meta.get("tokenizer.ggml.eos_token_id"))
