"""Python binding of libcohx.so (the MI355X step's C ABI, include/cohx.h).

Mirrors the engine's API for this path so parity tests read like the
reference's own (crates/coheryn-engine/tests/batching.rs):

    model = Model.from_gguf(path, max_lanes=16, max_context=512)
    state = model.begin_generation(prompt_ids, GenerationOptions(max_tokens=8))
    while not state.is_finished():
        if state.needs_forward():
            model.step_batch([state])
        state.sample()

The product path is the HIP library: importing this module on a machine
without the built library raises, and nothing here falls back to the CPU.
"""
import ctypes
import os
import weakref

import numpy as np

import gguf

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcohx.so")

OK, INVALID_REQUEST, INVALID_GGUF, RESOURCE, CANCELLED, UNSUPPORTED, DEAD_END, DEVICE = range(8)
STATUS_NAMES = {0: "ok", 1: "invalid_request", 2: "invalid_gguf", 3: "resource",
                4: "cancelled", 5: "unsupported", 6: "dead_end", 7: "device"}
FINISH = {0: None, 1: "stop", 2: "length", 3: "cancelled"}
PAGE = 16


class CohxError(RuntimeError):
    def __init__(self, code, msg=""):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {msg}")
        self.code = code


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim", "vocabulary",
        "context")] + [("rope_base", ctypes.c_float), ("norm_epsilon", ctypes.c_float)] + [
        (n, ctypes.c_uint32) for n in (
            "weight_dtype", "tied", "kv_dtype", "max_lanes", "max_rows", "max_seqs",
            "max_context", "kv_pages", "n_eog")] + [("eog", ctypes.c_uint32 * 4)]


class Lane(ctypes.Structure):
    _fields_ = [("seq", ctypes.c_uint32), ("n_tokens", ctypes.c_uint32),
                ("tokens", ctypes.POINTER(ctypes.c_uint32)), ("start_position", ctypes.c_uint32),
                ("want_logits", ctypes.c_uint32)]


class Batch(ctypes.Structure):
    _fields_ = [("n_lanes", ctypes.c_uint32), ("lanes", ctypes.POINTER(Lane))]


class LaneOut(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int32), ("argmax", ctypes.c_uint32),
                ("logits", ctypes.POINTER(ctypes.c_float))]


AT_END = 0xFFFFFFFF  # COHX_AT_END: the sequence's current length
SKIP_HEAD = 2        # COHX_SKIP_HEAD: rows only advance the state (Qwen3.5 prompt chunks)
NO_TOKEN = 0xFFFFFFFF  # COHX_NO_TOKEN: argmax of a lane that skipped the head

# numpy views of the same layouts, for building a whole step without per-lane Python work
LANE_DTYPE = np.dtype({"names": ["seq", "n_tokens", "tokens", "start_position", "want_logits"],
                       "formats": [np.uint32, np.uint32, np.uint64, np.uint32, np.uint32],
                       "offsets": [0, 4, 8, 16, 20], "itemsize": ctypes.sizeof(Lane)})
LANE_OUT_DTYPE = np.dtype({"names": ["status", "argmax", "logits"],
                           "formats": [np.int32, np.uint32, np.uint64],
                           "offsets": [0, 4, 8], "itemsize": ctypes.sizeof(LaneOut)})


class StepOut(ctypes.Structure):
    _fields_ = [("lanes", ctypes.POINTER(LaneOut)), ("width", ctypes.c_uint32),
                ("rows", ctypes.c_uint32), ("matrix_bytes", ctypes.c_uint64),
                ("kv_bytes", ctypes.c_uint64), ("elapsed_ns", ctypes.c_uint64)]


class Qwen35Desc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "layers", "hidden", "intermediate", "vocabulary", "heads", "kv_heads", "head_dim",
        "linear_key_heads", "linear_value_heads", "linear_key_dim", "linear_value_dim",
        "conv_kernel", "rotary_dim", "context", "tied")] + [
        ("epsilon", ctypes.c_float), ("rope_base", ctypes.c_float),
        ("full_attention", ctypes.c_uint8 * 128)] + [(n, ctypes.c_uint32) for n in (
            "max_lanes", "max_rows", "max_seqs", "max_context", "n_eog")] + [
        ("eog", ctypes.c_uint32 * 4)]


class GenOptions(ctypes.Structure):
    _fields_ = [("max_tokens", ctypes.c_uint32), ("temperature", ctypes.c_float),
                ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float), ("seed", ctypes.c_uint64),
                ("repetition_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float),
                ("presence_penalty", ctypes.c_float), ("n_stop_tokens", ctypes.c_uint32),
                ("stop_tokens", ctypes.POINTER(ctypes.c_uint32)), ("context", ctypes.c_uint32)]


YIELD_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)


class StepHooks(ctypes.Structure):
    _fields_ = [("yield_", YIELD_FN), ("user", ctypes.c_void_p),
                ("cancel", ctypes.POINTER(ctypes.c_uint32))]


class KernelStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("launches", ctypes.c_uint64),
                ("total_ms", ctypes.c_double), ("bytes", ctypes.c_double),
                ("flops", ctypes.c_double)]


class BatchStepC(ctypes.Structure):
    _fields_ = [("width", ctypes.c_uint32), ("completed_tokens", ctypes.c_uint32),
                ("matrix_tiles", ctypes.c_uint64), ("matrix_bytes", ctypes.c_uint64)]


EXPORTS = {
    "cohx_create": (ctypes.c_int, [ctypes.POINTER(ModelDesc), ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_void_p)]),
    "cohx_create_qwen35": (ctypes.c_int, [ctypes.POINTER(Qwen35Desc), ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_void_p)]),
    "cohx_destroy": (None, [ctypes.c_void_p]),
    "cohx_last_error": (ctypes.c_char_p, [ctypes.c_void_p]),
    "cohx_upload_tensor": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint32,
                                          ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p,
                                          ctypes.c_size_t]),
    "cohx_finalize": (ctypes.c_int, [ctypes.c_void_p]),
    "cohx_load_gguf": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ModelDesc),
                                      ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p, ctypes.c_size_t]),
    "cohx_gguf_inspect": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ModelDesc), ctypes.c_char_p,
                                         ctypes.c_size_t]),
    "cohx_seq_alloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_uint32)]),
    "cohx_seq_fork": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]),
    "cohx_seq_free": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32]),
    "cohx_seq_truncate": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32]),
    "cohx_seq_length": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32,
                                       ctypes.POINTER(ctypes.c_uint32)]),
    "cohx_seq_pages": (ctypes.c_uint32, [ctypes.c_void_p, ctypes.c_uint32,
                                         ctypes.POINTER(ctypes.c_int32), ctypes.c_uint32]),
    "cohx_seq_read_kv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                        ctypes.c_int, ctypes.POINTER(ctypes.c_float)]),
    "cohx_seq_read_kv_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32,
                                             ctypes.POINTER(ctypes.c_float)]),
    "cohx_seq_fill_synthetic": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                               ctypes.c_uint64, ctypes.c_uint32]),
    "cohx_step": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Batch), ctypes.POINTER(StepOut)]),
    "cohx_step_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Batch), ctypes.POINTER(StepOut)]),
    "cohx_step_hooked": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Batch), ctypes.POINTER(StepOut),
                                        ctypes.POINTER(StepHooks)]),
    "cohx_step_batch_hooked": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint32,
                                              ctypes.c_void_p, YIELD_FN, ctypes.c_void_p]),
    "cohx_gen_compatible": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "cohx_pack": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Batch),
                                 ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                                 ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint32)]),
    "cohx_matvec": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32,
                                   ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
                                   ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float),
                                   ctypes.POINTER(ctypes.c_int32)]),
    "cohx_profile": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "cohx_profile_read": (ctypes.c_uint32, [ctypes.c_void_p, ctypes.POINTER(KernelStat),
                                            ctypes.c_uint32]),
    "cohx_gen_begin": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32),
                                      ctypes.c_uint32, ctypes.POINTER(GenOptions), ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_void_p)]),
    "cohx_step_batch": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                       ctypes.c_uint32, ctypes.POINTER(BatchStepC)]),
    "cohx_step_generation": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "cohx_gen_sample": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64)]),
    "cohx_gen_needs_forward": (ctypes.c_int, [ctypes.c_void_p]),
    "cohx_gen_is_finished": (ctypes.c_int, [ctypes.c_void_p]),
    "cohx_gen_is_prefilling": (ctypes.c_int, [ctypes.c_void_p]),
    "cohx_gen_finish_reason": (ctypes.c_uint32, [ctypes.c_void_p]),
    "cohx_gen_tokens": (ctypes.c_uint32, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32),
                                          ctypes.c_uint32]),
    "cohx_gen_cancel": (None, [ctypes.c_void_p]),
    "cohx_gen_free": (None, [ctypes.c_void_p]),
}


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise OSError(f"{path} is not built (run __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(path)
    for name, (res, args) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def _u32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def inspect_gguf(path):
    """cohx_gguf_inspect: the library's parse and validation of a file; returns
    (status, desc or None, message)."""
    d = ModelDesc()
    err = ctypes.create_string_buffer(512)
    rc = lib().cohx_gguf_inspect(os.fsencode(path), ctypes.byref(d), err, 512)
    return rc, (d if rc == 0 else None), err.value.decode()


DTYPE = {"f16": 1, "q8_0": 8, "q4_0": 2, "q5_0": 6, "q4_k": 12, "q6_k": 14}
MIXED = 0x100  # COHX_MIXED: each matrix takes the dtype of its tensor
# bytes of one prepared operand block and the values it covers (Q8_0 / Q8_K / F16)
ACT_BLOCK = {1: (2, 1), 2: (34, 32), 6: (34, 32), 8: (34, 32), 12: (292, 256), 14: (292, 256)}


class Model:
    """An MI355X context holding one Qwen2 model (Model::load, inference.rs:238-297)."""

    def __init__(self, config, tensors, max_lanes=16, max_rows=None, max_seqs=None,
                 max_context=None, kv_pages=0, device=0, eog=None):
        self.config = dict(config)
        L = lib()
        mats = [t for n, t in tensors.items() if len(t.shape) == 2]
        # one dtype for every matrix, or COHX_MIXED (a Q4_K_M-style file)
        wdt = mats[0].dtype if len({t.dtype for t in mats}) == 1 else MIXED
        d = ModelDesc()
        for k in ("layers", "hidden", "intermediate", "heads", "kv_heads", "head_dim",
                  "vocabulary", "context"):
            setattr(d, k, int(config[k]))
        d.rope_base = float(config["rope_base"])
        d.norm_epsilon = float(config["norm_epsilon"])
        d.weight_dtype = wdt
        d.tied = 0 if "output.weight" in tensors else 1
        d.kv_dtype = 0
        d.max_lanes = max_lanes
        d.max_rows = max_rows or max_lanes
        d.max_seqs = max_seqs or max_lanes
        d.max_context = max_context or min(int(config["context"]), 4096)
        d.kv_pages = kv_pages
        eog = list(eog if eog is not None else ([config["eos_token_id"]]
                                                 if config.get("eos_token_id") is not None else []))
        d.n_eog = len(eog)
        for i, e in enumerate(eog):
            d.eog[i] = e
        self.desc = d
        h = ctypes.c_void_p()
        rc = L.cohx_create(ctypes.byref(d), device, ctypes.byref(h))
        if rc:
            raise CohxError(rc, "cohx_create")
        self.h = h
        self.max_lanes = max_lanes
        self.max_context = d.max_context
        for name, t in tensors.items():
            data = np.ascontiguousarray(t.data)
            ne1 = t.shape[1] if len(t.shape) > 1 else 1
            rc = L.cohx_upload_tensor(h, name.encode(), t.dtype, t.shape[0], ne1,
                                      data.ctypes.data, data.nbytes)
            self._check(rc)
        self._check(L.cohx_finalize(h))

    @classmethod
    def from_gguf(cls, path, **kw):
        meta, tensors = gguf.read(path)
        return cls(gguf.qwen2_config(meta), tensors, **kw)

    @classmethod
    def load(cls, path, max_lanes=16, max_rows=None, max_seqs=None, max_context=0, kv_pages=0,
             device=0):
        """Model::load through the library's own GGUF loader (cohx_load_gguf):
        the file is parsed, validated and uploaded in C++."""
        d = ModelDesc()
        d.max_lanes, d.max_rows, d.max_seqs = max_lanes, max_rows or max_lanes, max_seqs or max_lanes
        d.max_context, d.kv_pages = max_context, kv_pages
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        rc = lib().cohx_load_gguf(os.fsencode(path), device, ctypes.byref(d), ctypes.byref(h), err, 512)
        if rc:
            raise CohxError(rc, err.value.decode())
        self = cls.__new__(cls)
        self.config = {k: getattr(d, k) for k in ("layers", "hidden", "intermediate", "heads", "kv_heads",
                                                   "head_dim", "vocabulary", "context")}
        self.config.update(rope_base=d.rope_base, norm_epsilon=d.norm_epsilon)
        self.desc, self.h = d, h
        self.max_lanes, self.max_context = d.max_lanes, d.max_context
        return self

    def _check(self, rc):
        if rc:
            raise CohxError(rc, lib().cohx_last_error(self.h).decode())

    def close(self):
        if getattr(self, "h", None):
            # generation states hold sequences of this context: release them first
            for st in list(getattr(self, "_states", ())):
                st.free()
            lib().cohx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def matvec(self, dtype, rows, K, payload, inputs, decode=False):
        """cohx_matvec: one matrix (GGUF payload) against f32 input rows through
        the step's operand preparation and exact kernels.  Returns (out [n][rows],
        prepared operand bytes [n][...], statuses [n], decoded rows or None)."""
        x = np.ascontiguousarray(inputs, np.float32).reshape(-1, K)
        n = x.shape[0]
        w = np.ascontiguousarray(payload, np.uint8)
        out = np.zeros((n, rows), np.float32)
        bb, bv = ACT_BLOCK[dtype]
        act = np.zeros((n, K // bv * bb), np.uint8)
        st = np.zeros(n, np.int32)
        dec = np.zeros((rows, K), np.float32) if decode else None
        fp = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
        self._check(lib().cohx_matvec(
            self.h, dtype, rows, K, w.ctypes.data, w.nbytes, n, fp(x), fp(out),
            act.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), fp(dec) if decode else None,
            st.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))))
        return out, act, st, dec

    # ---- sequences ---------------------------------------------------------
    def seq_alloc(self, capacity=None):
        s = ctypes.c_uint32()
        self._check(lib().cohx_seq_alloc(self.h, capacity or self.max_context, ctypes.byref(s)))
        return s.value

    def seq_fork(self, src, rows, capacity=None):
        s = ctypes.c_uint32()
        self._check(lib().cohx_seq_fork(self.h, src, rows, capacity or self.max_context,
                                        ctypes.byref(s)))
        return s.value

    def seq_free(self, seq):
        self._check(lib().cohx_seq_free(self.h, seq))

    def seq_truncate(self, seq, rows):
        self._check(lib().cohx_seq_truncate(self.h, seq, rows))

    def seq_length(self, seq):
        n = ctypes.c_uint32()
        self._check(lib().cohx_seq_length(self.h, seq, ctypes.byref(n)))
        return n.value

    def seq_pages(self, seq):
        n = lib().cohx_seq_pages(self.h, seq, None, 0)
        out = np.zeros(n, np.int32)
        lib().cohx_seq_pages(self.h, seq, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), n)
        return out

    def seq_read_kv(self, seq, layer, values=False):
        c = self.config
        out = np.zeros((self.seq_length(seq), c["kv_heads"] * c["head_dim"]), np.float32)
        self._check(lib().cohx_seq_read_kv(self.h, seq, layer, 1 if values else 0,
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def seq_read_kv_rows(self, seq, layer, first, count, values=False):
        c = self.config
        out = np.zeros((count, c["kv_heads"] * c["head_dim"]), np.float32)
        self._check(lib().cohx_seq_read_kv_rows(self.h, seq, layer, 1 if values else 0, first, count,
                                                out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def seq_fill_synthetic(self, seq, rows, seed, stream):
        self._check(lib().cohx_seq_fill_synthetic(self.h, seq, rows, seed, stream))

    # ---- the device step -----------------------------------------------------
    def _batch(self, lanes):
        arr = (Lane * len(lanes))()
        keep = []
        for i, ln in enumerate(lanes):
            toks = np.ascontiguousarray(ln["tokens"], np.uint32)
            keep.append(toks)
            arr[i].seq = ln["seq"]
            arr[i].n_tokens = toks.size
            arr[i].tokens = _u32p(toks)
            arr[i].start_position = ln.get("start", AT_END)
            arr[i].want_logits = 1 if ln.get("logits") else (SKIP_HEAD if ln.get("skip_head") else 0)
        return Batch(len(lanes), arr), keep

    def step(self, lanes, noalloc=False, yield_fn=None, cancel=None):
        """lanes: [{"seq", "tokens", "start"?, "logits"?: bool, "skip_head"?: bool}] -> list
        of dicts (status, argmax, logits).  noalloc: through cohx_step_noalloc
        (device scratch from the library's static array).  yield_fn (called
        while the device computes; a true return asks to stop) and cancel (a
        uint32 array of per-lane flags, read before the launch and after the
        device finishes) go through cohx_step_hooked."""
        batch, keep = self._batch(lanes)
        outs = (LaneOut * len(lanes))()
        bufs = []
        V = self.config["vocabulary"]
        for i, ln in enumerate(lanes):
            if ln.get("logits"):
                b = np.zeros(V, np.float32)
                bufs.append(b)
                outs[i].logits = b.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
            else:
                bufs.append(None)
        so = StepOut()
        so.lanes = outs
        if yield_fn is not None or cancel is not None:
            cb = YIELD_FN((lambda _u: int(bool(yield_fn()))) if yield_fn else 0)
            hk = StepHooks(cb, None, cancel.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
                           if cancel is not None else None)
            rc = lib().cohx_step_hooked(self.h, ctypes.byref(batch), ctypes.byref(so), ctypes.byref(hk))
            res = [dict(status=outs[i].status, argmax=outs[i].argmax, logits=bufs[i])
                   for i in range(len(lanes))]
            if rc:
                raise CohxError(rc, lib().cohx_last_error(self.h).decode())
            return res
        entry = lib().cohx_step_noalloc if noalloc else lib().cohx_step
        self._check(entry(self.h, ctypes.byref(batch), ctypes.byref(so)))
        res = [dict(status=outs[i].status, argmax=outs[i].argmax, logits=bufs[i])
               for i in range(len(lanes))]
        self._last_out = so
        return res

    def step_decode(self, seqs, tokens):
        """One decode token per lane, vectorized: seqs and tokens are equal-length
        uint32 arrays.  Returns (status, argmax) int32/uint32 arrays.  The lane,
        token and output buffers of the last sequence list are kept and reused
        while the list stays the same (a decode loop's per-step Python work is
        then one token copy and the call)."""
        seqs = np.ascontiguousarray(seqs, np.uint32)
        n = seqs.size
        if np.size(tokens) != n:
            raise ValueError("one token per sequence")
        key = seqs.tobytes()
        cache = getattr(self, "_decode_bufs", None)
        if cache is None or cache[0] != key:
            tok = np.zeros(n, np.uint32)
            lanes = np.zeros(n, LANE_DTYPE)
            lanes["seq"] = seqs
            lanes["n_tokens"] = 1
            lanes["tokens"] = tok.ctypes.data + 4 * np.arange(n, dtype=np.uint64)
            lanes["start_position"] = AT_END
            outs = np.zeros(n, LANE_OUT_DTYPE)
            batch = Batch(n, lanes.ctypes.data_as(ctypes.POINTER(Lane)))
            so = StepOut()
            so.lanes = outs.ctypes.data_as(ctypes.POINTER(LaneOut))
            cache = self._decode_bufs = (key, tok, lanes, outs, batch, so, ctypes.byref(batch),
                                         ctypes.byref(so))
        _, tok, _, outs, _, so, batch_ref, so_ref = cache
        np.copyto(tok, tokens, casting="unsafe")
        self._check(lib().cohx_step(self.h, batch_ref, so_ref))
        self._last_out = so  # read by last_step when asked for
        return outs["status"].copy(), outs["argmax"].copy()

    @property
    def last_step(self):
        """The last step's width, rows, matrix and KV bytes and host time."""
        so = self._last_out
        return dict(width=so.width, rows=so.rows, matrix_bytes=so.matrix_bytes, kv_bytes=so.kv_bytes,
                    elapsed_ns=so.elapsed_ns)

    @property
    def matrix_bytes(self):
        return self.last_step["matrix_bytes"]

    def profile(self, enable):
        self._check(lib().cohx_profile(self.h, 1 if enable else 0))

    def profile_read(self):
        n = lib().cohx_profile_read(self.h, None, 0)
        arr = (KernelStat * n)()
        lib().cohx_profile_read(self.h, arr, n)
        return [dict(name=a.name.decode(), launches=a.launches, total_ms=a.total_ms,
                     bytes=a.bytes, flops=a.flops) for a in arr]

    def pack(self, lanes):
        batch, keep = self._batch(lanes)
        n = len(lanes)
        R = sum(len(l["tokens"]) for l in lanes)
        cu = np.zeros(n + 1, np.uint32)
        pos = np.zeros(R, np.uint32)
        slot = np.zeros(R, np.int64)
        lane = np.zeros(R, np.uint32)
        self._check(lib().cohx_pack(self.h, ctypes.byref(batch), _u32p(cu), _u32p(pos),
                                    slot.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                    _u32p(lane)))
        return cu, pos, slot, lane

    # ---- generation API (generation.rs / batch.rs mirror) --------------------
    def begin_generation(self, prompt, options=None, prior=None):
        o = options or GenerationOptions()
        p = np.ascontiguousarray(prompt, np.uint32)
        stops = np.ascontiguousarray(o.stop_tokens, np.uint32)
        c = GenOptions(o.max_tokens, o.temperature, o.top_k, o.top_p, o.seed,
                       o.repetition_penalty, o.frequency_penalty, o.presence_penalty,
                       stops.size, _u32p(stops), o.context)
        h = ctypes.c_void_p()
        rc = lib().cohx_gen_begin(self.h, _u32p(p), p.size, ctypes.byref(c),
                                  prior.h if prior is not None else None, ctypes.byref(h))
        self._check(rc)
        st = GenerationState(self, h)
        if not hasattr(self, "_states"):
            self._states = weakref.WeakSet()
        self._states.add(st)
        return st

    def step_batch(self, states, yield_fn=None):
        """Model::step_batch; yield_fn: the WorkYield hook (cohx_step_batch_hooked)."""
        arr = (ctypes.c_void_p * len(states))(*[s.h for s in states])
        st = BatchStepC()
        if yield_fn is None:
            self._check(lib().cohx_step_batch(self.h, arr, len(states), ctypes.byref(st)))
        else:
            cb = YIELD_FN(lambda _u: int(bool(yield_fn())))
            self._check(lib().cohx_step_batch_hooked(self.h, arr, len(states), ctypes.byref(st), cb, None))
        return dict(width=st.width, completed_tokens=st.completed_tokens,
                    matrix_tiles=st.matrix_tiles, matrix_bytes=st.matrix_bytes)

    def step_generation(self, state):
        rc = lib().cohx_step_generation(self.h, state.h)
        if rc:
            raise CohxError(rc, lib().cohx_last_error(self.h).decode())


class GenerationOptions:
    def __init__(self, max_tokens=128, temperature=0.0, top_k=0, top_p=1.0, seed=0,
                 repetition_penalty=1.0, frequency_penalty=0.0, presence_penalty=0.0,
                 stop_tokens=(), context=0):
        self.max_tokens, self.temperature, self.top_k, self.top_p = (max_tokens, temperature,
                                                                     top_k, top_p)
        self.seed, self.repetition_penalty = seed, repetition_penalty
        self.frequency_penalty, self.presence_penalty = frequency_penalty, presence_penalty
        self.stop_tokens, self.context = list(stop_tokens), context


class GenerationState:
    def __init__(self, model, h):
        self.model, self.h = model, h

    def __del__(self):
        self.free()

    def free(self):
        if getattr(self, "h", None):
            if getattr(self.model, "h", None):  # a closed context already released it
                lib().cohx_gen_free(self.h)
            self.h = None

    def needs_forward(self):
        return bool(lib().cohx_gen_needs_forward(self.h))

    def is_finished(self):
        return bool(lib().cohx_gen_is_finished(self.h))

    def is_prefilling(self):
        return bool(lib().cohx_gen_is_prefilling(self.h))

    def finish_reason(self):
        return FINISH[lib().cohx_gen_finish_reason(self.h)]

    def sample(self):
        t = ctypes.c_int64()
        rc = lib().cohx_gen_sample(self.h, ctypes.byref(t))
        if rc:
            raise CohxError(rc, "sample")
        return None if t.value < 0 else t.value

    def token_ids(self):
        n = lib().cohx_gen_tokens(self.h, None, 0)
        out = np.zeros(n, np.uint32)
        lib().cohx_gen_tokens(self.h, _u32p(out), n)
        return [int(v) for v in out]

    def cancel(self):
        lib().cohx_gen_cancel(self.h)

    def compatible(self, other):
        return bool(lib().cohx_gen_compatible(self.h, other.h))


def generate(model, prompt, options):
    """Model::generate's token loop (inference.rs:641-684) on one lane."""
    st = model.begin_generation(prompt, options)
    while not st.is_finished():
        if st.needs_forward():
            model.step_generation(st)
        st.sample()
    return st


class Qwen35(Model):
    """An MI355X context holding one Qwen3.5 hybrid text model (qwen35::Model,
    qwen35/mod.rs:103-193): tensors by their safetensors names, BF16
    matrices.  Steps, sequences and errors behave as for Model; a fork is a
    full snapshot copy, and read_state exposes the recurrent state."""

    def __init__(self, config, tensors, max_lanes=16, max_rows=None, max_seqs=None,
                 max_context=None, device=0, eog=None):
        self.config = dict(config)
        L = lib()
        d = Qwen35Desc()
        for k, v in (("layers", "layers"), ("hidden", "hidden"), ("intermediate", "intermediate"),
                     ("vocabulary", "vocabulary"), ("heads", "heads"), ("kv_heads", "kv_heads"),
                     ("head_dim", "head_dim"), ("linear_key_heads", "key_heads"),
                     ("linear_value_heads", "value_heads"), ("linear_key_dim", "key_dim"),
                     ("linear_value_dim", "value_dim"), ("conv_kernel", "conv_kernel"),
                     ("rotary_dim", "rotary_dim"), ("context", "context")):
            setattr(d, k, int(config[v]))
        d.tied = 1 if config.get("tied", True) else 0
        d.epsilon = float(config["epsilon"])
        d.rope_base = float(config["rope_base"])
        for i, f in enumerate(config["full"]):
            d.full_attention[i] = 1 if f else 0
        d.max_lanes = max_lanes
        d.max_rows = max_rows or max_lanes
        d.max_seqs = max_seqs or max_lanes
        d.max_context = max_context or min(int(config["context"]), 4096)
        eog = list(eog or [])
        d.n_eog = len(eog)
        for i, e in enumerate(eog):
            d.eog[i] = e
        self.desc = d
        h = ctypes.c_void_p()
        rc = L.cohx_create_qwen35(ctypes.byref(d), device, ctypes.byref(h))
        if rc:
            raise CohxError(rc, "cohx_create_qwen35")
        self.h = h
        self.max_lanes = max_lanes
        self.max_context = d.max_context
        for name, t in tensors.items():
            data = np.ascontiguousarray(t.data)
            n = int(np.prod(t.shape))
            rc = L.cohx_upload_tensor(h, name.encode(), t.dtype, t.shape[0], n // t.shape[0],
                                      data.ctypes.data, data.nbytes)
            self._check(rc)
        self._check(L.cohx_finalize(h))

    def read_state(self, seq, layer, which):
        """0/1: K/V rows [0, length) of a full-attention layer; 2: conv ring
        [channels * kernel]; 3: delta memory [value_heads * key_dim * value_dim]."""
        c = self.config
        n = {0: self.seq_length(seq) * c["kv_heads"] * c["head_dim"],
             1: self.seq_length(seq) * c["kv_heads"] * c["head_dim"],
             2: (2 * c["key_heads"] * c["key_dim"] + c["value_heads"] * c["value_dim"])
             * c["conv_kernel"],
             3: c["value_heads"] * c["key_dim"] * c["value_dim"]}[which]
        out = np.zeros(max(n, 1), np.float32)
        self._check(lib().cohx_seq_read_kv(self.h, seq, layer, which,
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out[:n]

