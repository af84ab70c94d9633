"""The library's GGUF loader (cohx_gguf_inspect / cohx_load_gguf): parsing and
validation run on the host, so these run without a GPU.

Which files load, and the status class of each rejection, follow the engine:
the v3 parser rules (crates/coheryn-engine/src/gguf.rs:304-496), the Qwen2
configuration and graph checks (compat.rs:54-221), big-endian files refused
(compat.rs:228-233) and the end-of-generation ids (tokenizer.rs:224-236,
304-306), with the engine's error classes (Error::invalid -> invalid_gguf;
UnsupportedGgufVersion / UnsupportedGgufTensorType / UnsupportedFeature /
UnsupportedModelArchitecture -> unsupported).  The message texts are the
library's own; each check below names the fault it reports.
"""
import os
import struct

import numpy as np
import pytest

import cohx
import gguf
import synth

TINY = synth.config(layers=2, hidden=128, intermediate=256, heads=4, kv_heads=2,
                    vocabulary=300, context=512)


def write(tmp_path, name, meta, tensors, **kw):
    path = os.path.join(tmp_path, name)
    gguf.write(path, meta, tensors, **kw)
    return path


def model(dtype="q8_0", cfg=TINY, **kw):
    return synth.build(cfg, dtype, seed=3, **kw)


@pytest.mark.parametrize("dtype", ["q8_0", "f16", "q4_0", "q4_k_m"])
def test_inspect_reads_the_configuration(tmp_path, dtype):
    cfg = synth.config(layers=2, hidden=128, intermediate=512, heads=4, kv_heads=2,
                       vocabulary=300, context=512) if dtype == "q4_k_m" else TINY
    meta, tensors = model(dtype, cfg)
    path = write(tmp_path, "m.gguf", meta, tensors)
    rc, d, msg = cohx.inspect_gguf(path)
    assert rc == 0, msg
    want = gguf.qwen2_config(gguf.read(path)[0])  # the Python reader, independently
    for k in ("layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim", "vocabulary", "context"):
        assert getattr(d, k) == want[k], k
    assert d.rope_base == np.float32(want["rope_base"]) and d.norm_epsilon == np.float32(want["norm_epsilon"])
    mats = {t[2] for t in tensors if len(t[1]) == 2}
    assert d.weight_dtype == (mats.pop() if len(mats) == 1 else cohx.MIXED)
    assert d.tied == (0 if any(t[0] == "output.weight" for t in tensors) else 1)
    assert [d.eog[i] for i in range(d.n_eog)] == [cfg["vocabulary"] - 1]
    assert (d.max_lanes, d.max_rows, d.max_seqs, d.max_context) == (16, 16, 16, 512)


def test_end_of_generation_ids(tmp_path):
    meta, tensors = model()
    meta["tokenizer.ggml.tokens"] = [f"<{i}>" for i in range(299)] + ["<|endoftext|>"]
    meta["tokenizer.ggml.eos_token_id"] = 7
    meta["tokenizer.ggml.eot_token_id"] = 11
    rc, d, msg = cohx.inspect_gguf(write(tmp_path, "m.gguf", meta, tensors))
    assert rc == 0, msg
    assert [d.eog[i] for i in range(d.n_eog)] == [7, 11, 299]


def rejected(tmp_path, meta, tensors, code, text, **kw):
    rc, _, msg = cohx.inspect_gguf(write(tmp_path, "bad.gguf", meta, tensors, **kw))
    assert rc == code, (rc, msg)
    assert text in msg, msg


def test_graph_and_configuration_rejections(tmp_path):
    meta, tensors = model()
    rejected(tmp_path, meta, [t for t in tensors if t[0] != "blk.1.ffn_up.weight"],
             cohx.INVALID_GGUF, "tensor blk.1.ffn_up.weight is required but absent")
    extra = tensors + [("blk.0.attn_output.bias", (128,), 0, np.zeros(512, np.uint8))]
    rejected(tmp_path, meta, extra, cohx.UNSUPPORTED, "'blk.0.attn_output.bias' is not part of the Qwen2 graph")
    wrong = [(n, (s[0], s[1] + 16) if n == "blk.0.attn_k.weight" else s, d,
              synth.encode(np.zeros((s[1] + 16, s[0]), np.float32), d) if n == "blk.0.attn_k.weight" else p)
             for n, s, d, p in tensors]
    rejected(tmp_path, meta, wrong, cohx.INVALID_GGUF, "tensor blk.0.attn_k.weight has shape [128, 80], expected [128, 64]")
    for key, value, code, text in [
            ("general.architecture", "llama", cohx.UNSUPPORTED, "'llama'; this loader builds the qwen2 graph"),
            ("qwen2.rope.scaling.type", "yarn", cohx.UNSUPPORTED, "Qwen2 variant this loader does not implement"),
            ("qwen2.attention.key_length", 48, cohx.UNSUPPORTED, "qwen2.attention.key_length = 48 differs from the head size 32"),
            ("qwen2.attention.layer_norm_rms_epsilon", 0.0, cohx.INVALID_GGUF, "must be positive and finite"),
            ("qwen2.attention.head_count_kv", 3, cohx.INVALID_GGUF, "head layout does not fit"),
            ("qwen2.block_count", 0, cohx.INVALID_GGUF, "qwen2.block_count = 0 is out of range"),
            ("split.count", 2, cohx.UNSUPPORTED, "split over 2 files"),
            ("tokenizer.ggml.eos_token_id", 300, cohx.UNSUPPORTED, "eos_token_id must be an unsigned id below the vocabulary size 300")]:
        m = dict(meta)
        m[key] = value
        rejected(tmp_path, m, tensors, code, text)
    m = {k: v for k, v in meta.items() if k != "qwen2.attention.layer_norm_rms_epsilon"}
    rejected(tmp_path, m, tensors, cohx.INVALID_GGUF, "layer_norm_rms_epsilon is required")
    m = {k: v for k, v in meta.items() if k != "tokenizer.ggml.tokens"}
    rejected(tmp_path, m, tensors, cohx.INVALID_GGUF, "tokenizer.ggml.tokens (the vocabulary) is required")


def test_container_rejections(tmp_path):
    meta, tensors = model()
    path = write(tmp_path, "m.gguf", meta, tensors)
    raw = open(path, "rb").read()

    def check(blob, code, text):
        p = os.path.join(tmp_path, "raw.gguf")
        with open(p, "wb") as f:
            f.write(blob)
        rc, _, msg = cohx.inspect_gguf(p)
        assert rc == code, (rc, msg)
        assert text in msg, msg

    check(b"GGUX" + raw[4:], cohx.INVALID_GGUF, "not a GGUF file")
    check(raw[:4] + struct.pack("<I", 2) + raw[8:], cohx.UNSUPPORTED, "format version 2 (only version 3 is read)")
    check(raw[:200], cohx.INVALID_GGUF, "more than the file can hold")
    check(raw[:1500], cohx.INVALID_GGUF, "array of 300 elements runs past the end of the file")
    check(raw[:raw.index(b"output_norm.weight") + 5], cohx.INVALID_GGUF, "header truncated: tensor name")
    check(raw[:-1000], cohx.INVALID_GGUF, "lies past the end of the file")
    # a 64-byte alignment claim over offsets laid out at 32
    m = dict(meta)
    m["general.alignment"] = 64
    p = write(tmp_path, "align.gguf", m, tensors, alignment=32)
    rc, _, msg = cohx.inspect_gguf(p)
    assert rc == cohx.INVALID_GGUF and "is not a multiple of the alignment 64" in msg, msg
    m["general.alignment"] = 48
    rc, _, msg = cohx.inspect_gguf(write(tmp_path, "align2.gguf", m, tensors))
    assert rc == cohx.INVALID_GGUF and "power of two no larger than 65536" in msg, msg
    # an unknown tensor dtype: the byte extent cannot be validated
    blob = bytearray(raw)
    name = b"output_norm.weight"
    at = raw.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    nd = struct.unpack_from("<I", raw, at)[0]
    struct.pack_into("<I", blob, at + 4 + 8 * nd, 99)
    check(bytes(blob), cohx.UNSUPPORTED, "unknown ggml type 99")
    rc, _, msg = cohx.inspect_gguf(os.path.join(tmp_path, "missing.gguf"))
    assert rc == cohx.INVALID_REQUEST


def test_matrix_dtypes_the_step_does_not_run(tmp_path):
    """The engine also runs F32 matrices (tensor.rs:81-105); this library
    refuses them at upload rather than computing them differently.  Parsing
    accepts the file; the dtype check is the upload's (no device needed to
    see it named by the inspect step)."""
    meta, tensors = model("f32")
    rc, d, msg = cohx.inspect_gguf(write(tmp_path, "f32.gguf", meta, tensors))
    assert rc == 0 and d.weight_dtype == 0, msg


def test_big_endian_files_are_refused(tmp_path):
    """compat.rs:228-233: a big-endian file parses in the engine but is refused
    as unsupported before any numeric work; here the header's byte order is
    enough to refuse it, with the same class."""
    meta, tensors = model()
    raw = open(write(tmp_path, "m.gguf", meta, tensors), "rb").read()
    p = os.path.join(tmp_path, "be.gguf")
    with open(p, "wb") as f:
        f.write(raw[:4] + struct.pack(">I", 3) + raw[8:])
    rc, _, msg = cohx.inspect_gguf(p)
    assert rc == cohx.UNSUPPORTED and "big-endian" in msg, (rc, msg)


def test_signed_eot_id_is_ignored(tmp_path):
    """tokenizer.rs:228-232 reads the EOT id only when it is stored unsigned;
    a signed value leaves it absent rather than failing the load."""
    meta, tensors = model()
    meta["tokenizer.ggml.eos_token_id"] = 7
    meta["tokenizer.ggml.eot_token_id"] = gguf.Value(gguf.T_I32, 11)
    rc, d, msg = cohx.inspect_gguf(write(tmp_path, "m.gguf", meta, tensors))
    assert rc == 0, msg
    assert [d.eog[i] for i in range(d.n_eog)] == [7]
