// GGUF v3 file loading for the Qwen2 graph: Model::load's file side.
//
// The header reader follows the engine's bounded parser
// (crates/coheryn-engine/src/gguf.rs:304-496: magic, v3 only, either byte
// order, metadata and tensor-descriptor limits, alignment, block-aligned
// rows, aligned non-overlapping in-file payloads); the configuration and
// graph checks follow compat.rs:54-221 (qwen2 metadata keys and bounds, GQA
// and RoPE dimensions, the exact tensor set and shapes); the end-of-generation
// ids follow tokenizer.rs:224-236,304-306 (eos, eot, "<|endoftext|>").
// Payloads are read from a read-only mapping of the file and uploaded into
// the context's HBM layout; nothing of the file is kept afterwards.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "internal.h"

namespace {

// gguf.rs:23-45 ParseLimits::default()
constexpr uint64_t kMaxEntries = 65536, kMaxTensors = 100000, kMaxArray = 1000000,
                   kMaxString = 8u << 20, kMaxHeader = 128u << 20, kMaxAlloc = 256u << 20;
constexpr int kMaxDepth = 4;

struct Value {
  enum Kind { U, I, F, B, S, A } kind = U;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0.0;
  bool b = false;
  std::string s;
  std::vector<Value> a;
};

struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t dtype = 0;
  uint64_t offset = 0, bytes = 0;
};

struct LoadError {
  int code;
  std::string msg;
};

// gguf.rs:104-128 encoding(): (block values, block bytes)
bool encoding(uint32_t t, uint64_t &block, uint64_t &size) {
  switch (t) {
    case 0: block = 1; size = 4; return true;
    case 1: block = 1; size = 2; return true;
    case 2: block = 32; size = 18; return true;
    case 3: block = 32; size = 20; return true;
    case 6: block = 32; size = 22; return true;
    case 7: block = 32; size = 24; return true;
    case 8: block = 32; size = 34; return true;
    case 9: block = 32; size = 40; return true;
    case 10: block = 256; size = 84; return true;
    case 11: block = 256; size = 110; return true;
    case 12: block = 256; size = 144; return true;
    case 13: block = 256; size = 176; return true;
    case 14: block = 256; size = 210; return true;
    case 15: block = 256; size = 292; return true;
    case 24: block = 1; size = 1; return true;
    case 25: block = 1; size = 2; return true;
    case 26: block = 1; size = 4; return true;
    case 27: case 28: block = 1; size = 8; return true;
    case 30: block = 1; size = 2; return true;
    default: return false;
  }
}

struct Reader {
  const uint8_t *p;
  uint64_t length, pos = 0, alloc = 0;
  bool big = false;

  void guard(uint64_t n) const {
    if (n > length || pos > length - n || pos + n > kMaxHeader)
      throw LoadError{COHX_INVALID_GGUF, "header exceeds file or parser byte limit"};
  }
  void charge(uint64_t n) {
    if (n > kMaxAlloc || alloc + n > kMaxAlloc)
      throw LoadError{COHX_RESOURCE, "metadata allocation limit exceeded"};
    alloc += n;
  }
  uint64_t uint(int n) {
    guard(n);
    uint64_t v = 0;
    for (int k = 0; k < n; k++) {
      const uint64_t byte = p[pos + k];
      v |= big ? byte << (8 * (n - 1 - k)) : byte << (8 * k);
    }
    pos += n;
    return v;
  }
  std::string string(uint64_t max) {
    const uint64_t n = uint(8);
    if (n > std::min(max, kMaxString)) throw LoadError{COHX_INVALID_GGUF, "string length exceeds parser limit"};
    guard(n);
    charge(n + 24);
    std::string s(reinterpret_cast<const char *>(p + pos), n);
    pos += n;
    return s;
  }
  Value value(uint32_t ty, int depth) {
    Value v;
    switch (ty) {
      case 0: v.u = uint(1); break;
      case 1: v.kind = Value::I; v.i = (int8_t)uint(1); break;
      case 2: v.u = uint(2); break;
      case 3: v.kind = Value::I; v.i = (int16_t)uint(2); break;
      case 4: v.u = uint(4); break;
      case 5: v.kind = Value::I; v.i = (int32_t)uint(4); break;
      case 6: {
        v.kind = Value::F;
        const uint32_t bits = (uint32_t)uint(4);
        float f;
        std::memcpy(&f, &bits, 4);
        v.f = f;
        break;
      }
      case 7: {
        const uint64_t b = uint(1);
        if (b > 1) throw LoadError{COHX_INVALID_GGUF, "invalid boolean"};
        v.kind = Value::B;
        v.b = b == 1;
        break;
      }
      case 8: v.kind = Value::S; v.s = string(kMaxString); break;
      case 9: {
        if (depth >= kMaxDepth) throw LoadError{COHX_INVALID_GGUF, "metadata nesting limit exceeded"};
        const uint32_t item = (uint32_t)uint(4);
        if (item > 12) throw LoadError{COHX_INVALID_GGUF, "unknown array element type"};
        const uint64_t n = uint(8);
        if (n > kMaxArray) throw LoadError{COHX_INVALID_GGUF, "array count exceeds parser limit"};
        const uint64_t minimum = (item <= 1 || item == 7) ? 1 : item <= 3 ? 2 : item <= 6 ? 4 : item == 9 ? 12 : 8;
        guard(n * minimum);
        charge(n * 48);
        v.kind = Value::A;
        v.a.reserve(n);
        for (uint64_t k = 0; k < n; k++) v.a.push_back(value(item, depth + 1));
        break;
      }
      case 10: v.u = uint(8); break;
      case 11: v.kind = Value::I; v.i = (int64_t)uint(8); break;
      case 12: {
        v.kind = Value::F;
        const uint64_t bits = uint(8);
        std::memcpy(&v.f, &bits, 8);
        break;
      }
      default: throw LoadError{COHX_INVALID_GGUF, "unknown metadata value type"};
    }
    return v;
  }
};

struct Parsed {
  std::map<std::string, Value> meta;
  std::vector<TensorInfo> tensors;
  uint64_t data_offset = 0;
  const TensorInfo *find(const std::string &n) const {
    for (const auto &t : tensors)
      if (t.name == n) return &t;
    return nullptr;
  }
  const Value *get(const std::string &k) const {
    auto it = meta.find(k);
    return it == meta.end() ? nullptr : &it->second;
  }
  // Value::uint(): unsigned kinds only (gguf.rs:57-63)
  bool uint(const std::string &k, uint64_t &out) const {
    const Value *v = get(k);
    if (!v || v->kind != Value::U) return false;
    out = v->u;
    return true;
  }
};

Parsed parse(const uint8_t *p, uint64_t length) {
  Reader r{p, length};
  Parsed d;
  r.guard(4);
  if (std::memcmp(p, "GGUF", 4) != 0) throw LoadError{COHX_INVALID_GGUF, "GGUF magic is missing"};
  r.pos = 4;
  r.guard(4);
  const uint32_t be = ((uint32_t)p[4] << 24) | ((uint32_t)p[5] << 16) | ((uint32_t)p[6] << 8) | p[7];
  r.big = be == 3;
  const uint32_t version = (uint32_t)r.uint(4);
  if (version != 3)
    throw LoadError{COHX_UNSUPPORTED, "GGUF version " + std::to_string(version) + "; expected v3"};
  const uint64_t n_tensors = r.uint(8), n_meta = r.uint(8);
  if (n_tensors > kMaxTensors || n_meta > kMaxEntries)
    throw LoadError{COHX_INVALID_GGUF, "descriptor count exceeds parser limit"};
  r.guard(n_meta * 13);
  r.charge(n_meta * 128);
  for (uint64_t k = 0; k < n_meta; k++) {
    std::string key = r.string(65535);
    if (key.empty() || std::any_of(key.begin(), key.end(), [](char c) { return (unsigned char)c > 127; }))
      throw LoadError{COHX_INVALID_GGUF, "metadata key must be nonempty ASCII"};
    const uint32_t ty = (uint32_t)r.uint(4);
    Value v = r.value(ty, 0);
    if (!d.meta.emplace(std::move(key), std::move(v)).second)
      throw LoadError{COHX_INVALID_GGUF, "duplicate metadata key"};
  }
  uint64_t alignment = 32;
  if (const Value *a = d.get("general.alignment")) {
    if (a->kind != Value::U || !a->u || (a->u & (a->u - 1)) || a->u > 65536)
      throw LoadError{COHX_INVALID_GGUF, "alignment must be a positive power of two <= 65536"};
    alignment = a->u;
  }
  r.guard(n_tensors * 32);
  r.charge(n_tensors * 256);
  std::set<std::string> names;
  for (uint64_t k = 0; k < n_tensors; k++) {
    TensorInfo t;
    t.name = r.string(64);
    if (t.name.empty() || !names.insert(t.name).second)
      throw LoadError{COHX_INVALID_GGUF, "empty or duplicate tensor name"};
    const uint32_t nd = (uint32_t)r.uint(4);
    if (nd < 1 || nd > 4) throw LoadError{COHX_INVALID_GGUF, "tensor rank must be 1..=4"};
    unsigned __int128 elements = 1;
    for (uint32_t j = 0; j < nd; j++) {
      const uint64_t dim = r.uint(8);
      if (!dim) throw LoadError{COHX_INVALID_GGUF, "zero tensor dimension"};
      elements *= dim;
      if (elements > UINT64_MAX) throw LoadError{COHX_INVALID_GGUF, "tensor shape overflow"};
      t.dims.push_back(dim);
    }
    t.dtype = (uint32_t)r.uint(4);
    uint64_t block, size;
    if (!encoding(t.dtype, block, size))
      throw LoadError{COHX_UNSUPPORTED, "cannot validate byte extent of tensor " + t.name + ": dtype " +
                                            std::to_string(t.dtype)};
    if (t.dims[0] % block) throw LoadError{COHX_INVALID_GGUF, "tensor row is not divisible by encoding block size"};
    const unsigned __int128 bytes = (elements / block) * size;
    if (bytes > UINT64_MAX) throw LoadError{COHX_INVALID_GGUF, "tensor byte size overflow"};
    t.bytes = (uint64_t)bytes;
    t.offset = r.uint(8);
    if (t.offset % alignment) throw LoadError{COHX_INVALID_GGUF, "unaligned tensor offset"};
    d.tensors.push_back(std::move(t));
  }
  d.data_offset = (r.pos + alignment - 1) / alignment * alignment;
  if (d.data_offset > length) throw LoadError{COHX_INVALID_GGUF, "tensor data starts beyond file"};
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (const auto &t : d.tensors) ranges.emplace_back(t.offset, t.bytes);
  std::sort(ranges.begin(), ranges.end());
  uint64_t last = 0;
  for (const auto &rg : ranges) {
    if (rg.first < last || rg.second > length - d.data_offset || rg.first > length - d.data_offset - rg.second)
      throw LoadError{COHX_INVALID_GGUF, "overlapping or out-of-file tensor payload"};
    last = rg.first + rg.second;
  }
  return d;
}

// compat.rs:38-49 positive()
uint64_t positive(const Parsed &d, const std::string &key, uint64_t max) {
  uint64_t n;
  if (!d.uint(key, n)) throw LoadError{COHX_INVALID_GGUF, "missing unsigned metadata " + key};
  if (!n || n > max) throw LoadError{COHX_INVALID_GGUF, key + " outside supported dimension bounds"};
  return n;
}

// Value::float(): float kinds only
bool get_float(const Parsed &d, const std::string &key, double &out) {
  const Value *v = d.get(key);
  if (!v || v->kind != Value::F) return false;
  out = v->f;
  return true;
}

// compat.rs:54-159 configuration_for(d, "qwen2"), the tensor graph of
// compat.rs:161-221, and the EOG ids of tokenizer.rs:224-236.
void configure(const Parsed &d, cohx_model_desc &c) {
  const Value *arch = d.get("general.architecture");
  if (!arch || arch->kind != Value::S || arch->s != "qwen2")
    throw LoadError{COHX_UNSUPPORTED, "only the Qwen2 decoder graph is implemented"};
  static const char *kKeys[] = {"block_count", "context_length", "embedding_length", "feed_forward_length",
                                "attention.head_count", "attention.head_count_kv",
                                "attention.layer_norm_rms_epsilon", "rope.freq_base", "rope.dimension_count",
                                "attention.key_length", "attention.value_length"};
  for (const auto &kv : d.meta) {
    if (kv.first.rfind("qwen2.", 0) != 0) continue;
    const std::string suffix = kv.first.substr(6);
    if (std::find(std::begin(kKeys), std::end(kKeys), suffix) == std::end(kKeys))
      throw LoadError{COHX_UNSUPPORTED, "unimplemented architecture metadata " + kv.first};
  }
  const uint64_t hidden = positive(d, "qwen2.embedding_length", 32768);
  const uint64_t heads = positive(d, "qwen2.attention.head_count", 512);
  const uint64_t kv_heads = positive(d, "qwen2.attention.head_count_kv", 512);
  if (hidden % heads || heads % kv_heads || (hidden / heads) % 2)
    throw LoadError{COHX_INVALID_GGUF, "invalid Qwen2 GQA or RoPE dimensions"};
  const Value *toks = d.get("tokenizer.ggml.tokens");
  if (!toks || toks->kind != Value::A || toks->a.empty() || toks->a.size() > 1000000)
    throw LoadError{COHX_INVALID_GGUF, "missing or invalid tokenizer vocabulary"};
  const uint64_t vocabulary = toks->a.size();
  double rope_base = 10000.0, eps = 0.0;
  (void)get_float(d, "qwen2.rope.freq_base", rope_base);
  if (!get_float(d, "qwen2.attention.layer_norm_rms_epsilon", eps))
    throw LoadError{COHX_INVALID_GGUF, "missing RMSNorm epsilon"};
  const float rb = (float)rope_base, ne = (float)eps;
  if (!std::isfinite(rb) || rb <= 0.0f || !std::isfinite(ne) || ne <= 0.0f)
    throw LoadError{COHX_INVALID_GGUF, "invalid RoPE base or norm epsilon"};
  const uint64_t head_dim = hidden / heads;
  for (const char *k : {"attention.key_length", "attention.value_length", "rope.dimension_count"}) {
    uint64_t n;
    if (d.uint(std::string("qwen2.") + k, n) && n != head_dim)
      throw LoadError{COHX_UNSUPPORTED, std::string("nonstandard ") + k};
  }
  uint64_t split;
  if (d.uint("split.count", split) && split > 1)
    throw LoadError{COHX_UNSUPPORTED, "multi-file GGUF shards are not implemented"};
  for (const auto &kv : d.meta)
    if (kv.first.rfind("qwen2.rope.scaling.", 0) == 0 || kv.first == "qwen2.attention.sliding_window")
      throw LoadError{COHX_UNSUPPORTED, "RoPE scaling and sliding-window variants are not implemented"};
  c.layers = (uint32_t)positive(d, "qwen2.block_count", 256);
  c.hidden = (uint32_t)hidden;
  c.intermediate = (uint32_t)positive(d, "qwen2.feed_forward_length", 131072);
  c.heads = (uint32_t)heads;
  c.kv_heads = (uint32_t)kv_heads;
  c.head_dim = (uint32_t)head_dim;
  c.vocabulary = (uint32_t)vocabulary;
  c.context = (uint32_t)positive(d, "qwen2.context_length", 1048576);
  c.rope_base = rb;
  c.norm_epsilon = ne;
  // graph (compat.rs:161-221)
  auto expect = [&](const std::string &name, std::initializer_list<uint64_t> dims) {
    const TensorInfo *t = d.find(name);
    if (!t) throw LoadError{COHX_INVALID_GGUF, "missing required tensor " + name};
    if (!std::equal(t->dims.begin(), t->dims.end(), dims.begin(), dims.end()))
      throw LoadError{COHX_INVALID_GGUF, "incorrect shape for " + name};
  };
  const uint64_t H = hidden, F = c.intermediate, V = vocabulary, KVD = kv_heads * head_dim;
  expect("token_embd.weight", {H, V});
  expect("output_norm.weight", {H});
  const bool untied = d.find("output.weight") != nullptr;
  if (untied) expect("output.weight", {H, V});
  for (uint32_t l = 0; l < c.layers; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    expect(p + "attn_norm.weight", {H});
    expect(p + "ffn_norm.weight", {H});
    expect(p + "attn_q.weight", {H, H});
    expect(p + "attn_q.bias", {H});
    expect(p + "attn_k.weight", {H, KVD});
    expect(p + "attn_k.bias", {KVD});
    expect(p + "attn_v.weight", {H, KVD});
    expect(p + "attn_v.bias", {KVD});
    expect(p + "attn_output.weight", {H, H});
    expect(p + "ffn_gate.weight", {H, F});
    expect(p + "ffn_up.weight", {H, F});
    expect(p + "ffn_down.weight", {F, H});
  }
  if (d.tensors.size() != 2 + (untied ? 1u : 0u) + (size_t)c.layers * 12)
    throw LoadError{COHX_UNSUPPORTED, "unexpected tensors in Qwen2 graph"};
  // one dtype for every matrix, or per-matrix dtypes
  std::set<uint32_t> mats;
  for (const auto &t : d.tensors)
    if (t.dims.size() == 2) mats.insert(t.dtype);
  c.weight_dtype = mats.size() == 1 ? *mats.begin() : COHX_MIXED;
  c.tied = untied ? 0 : 1;
  c.kv_dtype = 0;
  // end of generation: eos (required), eot, "<|endoftext|>"
  uint64_t eos, eot;
  if (!d.uint("tokenizer.ggml.eos_token_id", eos) || eos >= vocabulary)
    throw LoadError{COHX_UNSUPPORTED, "missing or invalid EOS token"};
  std::vector<uint32_t> eog = {(uint32_t)eos};
  if (d.get("tokenizer.ggml.eot_token_id")) {
    if (!d.uint("tokenizer.ggml.eot_token_id", eot) || eot >= vocabulary)
      throw LoadError{COHX_UNSUPPORTED, "invalid EOT token"};
    eog.push_back((uint32_t)eot);
  }
  for (size_t k = 0; k < toks->a.size(); k++)
    if (toks->a[k].kind == Value::S && toks->a[k].s == "<|endoftext|>") {
      eog.push_back((uint32_t)k);
      break;
    }
  std::sort(eog.begin(), eog.end());
  eog.erase(std::unique(eog.begin(), eog.end()), eog.end());
  c.n_eog = (uint32_t)eog.size();
  for (size_t k = 0; k < eog.size(); k++) c.eog[k] = eog[k];
}

struct Mapping {
  const uint8_t *p = nullptr;
  uint64_t length = 0;
  int fd = -1;
  ~Mapping() {
    if (p && length) munmap(const_cast<uint8_t *>(p), length);
    if (fd >= 0) close(fd);
  }
};

void map_file(const char *path, Mapping &m) {
  if (!path) throw LoadError{COHX_INVALID_REQUEST, "null path"};
  m.fd = open(path, O_RDONLY | O_CLOEXEC);
  if (m.fd < 0) throw LoadError{COHX_INVALID_REQUEST, std::string("cannot open ") + path};
  struct stat st;
  if (fstat(m.fd, &st) != 0 || !S_ISREG(st.st_mode))
    throw LoadError{COHX_INVALID_REQUEST, std::string("not a regular file: ") + path};
  m.length = (uint64_t)st.st_size;
  if (!m.length) throw LoadError{COHX_INVALID_GGUF, "header exceeds file or parser byte limit"};
  void *addr = mmap(nullptr, m.length, PROT_READ, MAP_PRIVATE, m.fd, 0);
  if (addr == MAP_FAILED) throw LoadError{COHX_RESOURCE, "cannot map the file"};
  m.p = static_cast<const uint8_t *>(addr);
}

void set_err(char *err, size_t cap, const std::string &msg) {
  if (!err || !cap) return;
  const size_t n = std::min(cap - 1, msg.size());
  std::memcpy(err, msg.data(), n);
  err[n] = 0;
}

// Capacities the caller asks for, defaults filled in (max_context: at most
// the file's context and 4096).
void capacities(const cohx_model_desc &in, cohx_model_desc &c) {
  c.max_lanes = in.max_lanes ? in.max_lanes : 16;
  c.max_rows = in.max_rows ? in.max_rows : c.max_lanes;
  c.max_seqs = in.max_seqs ? in.max_seqs : c.max_lanes;
  c.max_context = in.max_context ? in.max_context : std::min<uint32_t>(c.context, 4096);
  c.kv_pages = in.kv_pages;
}

}  // namespace

extern "C" int cohx_gguf_inspect(const char *path, cohx_model_desc *desc, char *err, size_t err_cap) {
  if (!desc) return COHX_INVALID_REQUEST;
  try {
    Mapping m;
    map_file(path, m);
    const Parsed d = parse(m.p, m.length);
    cohx_model_desc c = *desc;
    configure(d, c);
    capacities(*desc, c);
    *desc = c;
    set_err(err, err_cap, "");
    return COHX_OK;
  } catch (const LoadError &e) {
    set_err(err, err_cap, e.msg);
    return e.code;
  } catch (const std::bad_alloc &) {
    set_err(err, err_cap, "host allocation failed");
    return COHX_RESOURCE;
  }
}

extern "C" int cohx_load_gguf(const char *path, int device, cohx_model_desc *desc, cohx_ctx **out, char *err,
                              size_t err_cap) {
  if (!desc || !out) return COHX_INVALID_REQUEST;
  *out = nullptr;
  cohx_ctx *ctx = nullptr;
  try {
    Mapping m;
    map_file(path, m);
    const Parsed d = parse(m.p, m.length);
    cohx_model_desc c = *desc;
    configure(d, c);
    capacities(*desc, c);
    if (c.max_context > c.context) throw LoadError{COHX_INVALID_REQUEST, "max_context exceeds the file's context"};
    int rc = cohx_create(&c, device, &ctx);
    if (rc) throw LoadError{rc, "cohx_create failed"};
    for (const auto &t : d.tensors) {
      rc = cohx_upload_tensor(ctx, t.name.c_str(), t.dtype, t.dims[0], t.dims.size() > 1 ? t.dims[1] : 1,
                              m.p + d.data_offset + t.offset, (size_t)t.bytes);
      if (rc) throw LoadError{rc, cohx_last_error(ctx)};
    }
    rc = cohx_finalize(ctx);
    if (rc) throw LoadError{rc, cohx_last_error(ctx)};
    *desc = c;
    *out = ctx;
    set_err(err, err_cap, "");
    return COHX_OK;
  } catch (const LoadError &e) {
    set_err(err, err_cap, e.msg);
    if (ctx) cohx_destroy(ctx);
    return e.code;
  } catch (const std::bad_alloc &) {
    set_err(err, err_cap, "host allocation failed");
    if (ctx) cohx_destroy(ctx);
    return COHX_RESOURCE;
  }
}
