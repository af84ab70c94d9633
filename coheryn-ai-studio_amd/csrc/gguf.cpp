// GGUF v3 files for the Qwen2 graph: the file side of Model::load
// (crates/coheryn-engine/src/inference.rs:238-297).
//
// How it works.  The header is read in one forward pass by a bounds-checked
// cursor over a read-only mapping of the file.  Nothing of the header is
// copied: a metadata value becomes a fixed-size `Meta` record (scalars by
// value, strings as views into the mapping, arrays as element type and
// count, walked once for validity), and a tensor descriptor keeps its name as
// a view.  The parser's memory is therefore proportional to the number of
// entries, not to the file (a 151,936-string vocabulary is one record, with
// the index of "<|endoftext|>" noted during the walk).  The Qwen2 checks are
// driven by two tables: the model keys this loader understands (`kModelKeys`)
// and the per-layer tensor set (`kLayerTensors`).
//
// Acceptance is the engine's, so the same files load and a rejected file gets
// the same status class: the parser rules of gguf.rs:304-496 (v3 only, known
// value and tensor types, whole encoding blocks per row, aligned offsets,
// in-file non-overlapping payloads), the Qwen2 configuration and graph rules
// of compat.rs:54-221, big-endian files refused as unsupported
// (compat.rs:228-233), and the end-of-generation ids of
// tokenizer.rs:224-236,304-306.  The messages are this library's own.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "internal.h"

namespace {

struct Reject {
  int code;
  std::string text;
};

[[noreturn]] void reject(int code, std::string text) { throw Reject{code, "gguf: " + std::move(text)}; }

std::string quoted(std::string_view s) { return "'" + std::string(s) + "'"; }

// ---------------------------------------------------------------------------
// Format tables

// GGUF metadata value types and the byte width of the scalar ones (0: not a
// fixed-width scalar).
enum : uint32_t { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64, kTypes };
constexpr uint8_t kWidth[kTypes] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
constexpr bool is_unsigned_type(uint32_t t) { return t == kU8 || t == kU16 || t == kU32 || t == kU64; }
constexpr bool is_signed_type(uint32_t t) { return t == kI8 || t == kI16 || t == kI32 || t == kI64; }

// ggml tensor types this loader can size: values per encoding block and bytes
// per block (the GGUF format's own table; gguf.rs:104-128 sizes the same set).
struct Encoding {
  uint32_t type, block, bytes;
  const char *name;
};
constexpr Encoding kEncodings[] = {
    {0, 1, 4, "F32"},      {1, 1, 2, "F16"},       {2, 32, 18, "Q4_0"},   {3, 32, 20, "Q4_1"},
    {6, 32, 22, "Q5_0"},   {7, 32, 24, "Q5_1"},    {8, 32, 34, "Q8_0"},   {9, 32, 40, "Q8_1"},
    {10, 256, 84, "Q2_K"}, {11, 256, 110, "Q3_K"}, {12, 256, 144, "Q4_K"}, {13, 256, 176, "Q5_K"},
    {14, 256, 210, "Q6_K"}, {15, 256, 292, "Q8_K"}, {24, 1, 1, "I8"},     {25, 1, 2, "I16"},
    {26, 1, 4, "I32"},     {27, 1, 8, "I64"},      {28, 1, 8, "F64"},     {30, 1, 2, "BF16"},
};

const Encoding *encoding_of(uint32_t type) {
  for (const Encoding &e : kEncodings)
    if (e.type == type) return &e;
  return nullptr;
}

// Structural limits of this parser.  Lengths follow the GGUF specification
// (keys up to 65,535 bytes, tensor names up to 64, rank up to 4); nesting of
// arrays is bounded so a hostile file cannot recurse deeply.
constexpr uint64_t kMaxKey = 65535, kMaxTensorName = 64;
constexpr int kMaxRank = 4, kMaxNesting = 3;
constexpr uint64_t kMaxAlignment = 65536;

// ---------------------------------------------------------------------------
// The header

struct Meta {
  uint32_t type = kU8;
  uint64_t bits = 0;            // scalar payload (little-endian value, zero-extended)
  std::string_view text;        // kStr
  uint32_t elem = 0;            // kArr: element type
  uint64_t count = 0;           // kArr: element count
  int64_t endoftext = -1;       // kArr of kStr: first index of "<|endoftext|>"

  bool is_unsigned() const { return is_unsigned_type(type); }
  bool is_float() const { return type == kF32 || type == kF64; }
  double real() const {
    if (type == kF32) {
      float f;
      const uint32_t b = (uint32_t)bits;
      std::memcpy(&f, &b, 4);
      return f;
    }
    double d;
    std::memcpy(&d, &bits, 8);
    return d;
  }
};

struct Tensor {
  std::string_view name;
  uint32_t rank = 0;
  uint64_t dims[kMaxRank] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0, bytes = 0;  // offset from the data section's start
};

struct Header {
  std::unordered_map<std::string_view, Meta> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string_view, size_t> by_name;
  uint64_t data_start = 0;

  const Meta *find(std::string_view key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
  }
  const Tensor *tensor(std::string_view name) const {
    auto it = by_name.find(name);
    return it == by_name.end() ? nullptr : &tensors[it->second];
  }
};

class Cursor {
 public:
  Cursor(const uint8_t *base, uint64_t size) : base_(base), size_(size) {}

  uint64_t at() const { return at_; }
  uint64_t left() const { return size_ - at_; }

  const uint8_t *take(uint64_t n, const char *what) {
    if (n > left())
      reject(COHX_INVALID_GGUF, std::string("header truncated: ") + what + " at byte " + std::to_string(at_) +
                                    " needs " + std::to_string(n) + " bytes, " + std::to_string(left()) + " remain");
    const uint8_t *p = base_ + at_;
    at_ += n;
    return p;
  }
  uint64_t le(uint32_t width, const char *what) {
    const uint8_t *p = take(width, what);
    uint64_t v = 0;
    for (uint32_t k = width; k-- > 0;) v = (v << 8) | p[k];
    return v;
  }
  uint32_t u32(const char *what) { return (uint32_t)le(4, what); }
  uint64_t u64(const char *what) { return le(8, what); }
  std::string_view str(uint64_t max_len, const char *what) {
    const uint64_t n = u64(what);
    if (n > max_len)
      reject(COHX_INVALID_GGUF, std::string(what) + " of " + std::to_string(n) + " bytes is longer than the " +
                                    std::to_string(max_len) + " allowed");
    return std::string_view(reinterpret_cast<const char *>(take(n, what)), n);
  }

 private:
  const uint8_t *base_;
  uint64_t size_, at_ = 0;
};

// One value of type `type`; arrays are walked element by element.
Meta read_value(Cursor &c, uint32_t type, int depth) {
  Meta m;
  m.type = type;
  if (type >= kTypes) reject(COHX_INVALID_GGUF, "unknown metadata value type " + std::to_string(type));
  if (kWidth[type]) {
    m.bits = c.le(kWidth[type], "metadata value");
    if (type == kBool && m.bits > 1) reject(COHX_INVALID_GGUF, "boolean metadata value is neither 0 nor 1");
    return m;
  }
  if (type == kStr) {
    m.text = c.str(c.left(), "string value");
    return m;
  }
  if (depth >= kMaxNesting) reject(COHX_INVALID_GGUF, "arrays nested deeper than " + std::to_string(kMaxNesting));
  m.elem = c.u32("array element type");
  m.count = c.u64("array length");
  if (m.elem >= kTypes) reject(COHX_INVALID_GGUF, "unknown array element type " + std::to_string(m.elem));
  if (kWidth[m.elem]) {
    // fixed-width elements: one bounds check, one pass for booleans
    const uint64_t w = kWidth[m.elem];
    if (m.count > c.left() / w) reject(COHX_INVALID_GGUF, "array of " + std::to_string(m.count) + " elements runs past the end of the file");
    const uint8_t *p = c.take(m.count * w, "array");
    if (m.elem == kBool)
      for (uint64_t k = 0; k < m.count; k++)
        if (p[k] > 1) reject(COHX_INVALID_GGUF, "boolean array element is neither 0 nor 1");
    return m;
  }
  // strings (8-byte length each) and arrays (12-byte header each) at least
  const uint64_t least = m.elem == kStr ? 8 : 12;
  if (m.count > c.left() / least) reject(COHX_INVALID_GGUF, "array of " + std::to_string(m.count) + " elements runs past the end of the file");
  for (uint64_t k = 0; k < m.count; k++) {
    const Meta e = read_value(c, m.elem, depth + 1);
    if (m.elem == kStr && m.endoftext < 0 && e.text == "<|endoftext|>") m.endoftext = (int64_t)k;
  }
  return m;
}

Header read_header(const uint8_t *file, uint64_t size) {
  Cursor c(file, size);
  Header h;
  if (size < 4 || std::memcmp(c.take(4, "magic"), "GGUF", 4) != 0)
    reject(COHX_INVALID_GGUF, "not a GGUF file: the first four bytes are not the GGUF magic");
  const uint32_t version = c.u32("version");
  const uint32_t swapped = __builtin_bswap32(version);
  if (version != 3 && swapped == 3)
    reject(COHX_UNSUPPORTED, "big-endian file: its numeric payloads would need byte swapping, which is not done");
  if (version != 3)
    reject(COHX_UNSUPPORTED, "format version " + std::to_string(version) + " (only version 3 is read)");
  const uint64_t n_tensors = c.u64("tensor count");
  const uint64_t n_meta = c.u64("metadata count");
  // every entry is at least 13 bytes (key length, one-byte key, type), every
  // descriptor at least 29 (name length, one-byte name, rank, one dim, type, offset)
  if (n_meta > c.left() / 13 || n_tensors > c.left() / 29)
    reject(COHX_INVALID_GGUF, "header declares " + std::to_string(n_meta) + " metadata entries and " +
                                  std::to_string(n_tensors) + " tensors, more than the file can hold");
  h.meta.reserve(n_meta);
  for (uint64_t k = 0; k < n_meta; k++) {
    const std::string_view key = c.str(kMaxKey, "metadata key");
    if (key.empty()) reject(COHX_INVALID_GGUF, "empty metadata key");
    for (unsigned char ch : key)
      if (ch > 127) reject(COHX_INVALID_GGUF, "metadata key " + quoted(key) + " is not ASCII");
    const uint32_t type = c.u32("metadata type");
    if (!h.meta.emplace(key, read_value(c, type, 0)).second)
      reject(COHX_INVALID_GGUF, "metadata key " + quoted(key) + " appears twice");
  }
  uint64_t alignment = 32;
  if (const Meta *a = h.find("general.alignment")) {
    if (!a->is_unsigned() || a->bits == 0 || (a->bits & (a->bits - 1)) || a->bits > kMaxAlignment)
      reject(COHX_INVALID_GGUF, "general.alignment must be an unsigned power of two no larger than 65536");
    alignment = a->bits;
  }
  h.tensors.resize(n_tensors);
  h.by_name.reserve(n_tensors);
  for (uint64_t k = 0; k < n_tensors; k++) {
    Tensor &t = h.tensors[k];
    t.name = c.str(kMaxTensorName, "tensor name");
    if (t.name.empty()) reject(COHX_INVALID_GGUF, "tensor " + std::to_string(k) + " has an empty name");
    if (!h.by_name.emplace(t.name, k).second) reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " appears twice");
    t.rank = c.u32("tensor rank");
    if (t.rank < 1 || t.rank > (uint32_t)kMaxRank)
      reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " has rank " + std::to_string(t.rank) + " (1 to 4 allowed)");
    unsigned __int128 elements = 1;
    for (uint32_t j = 0; j < t.rank; j++) {
      t.dims[j] = c.u64("tensor dimension");
      elements *= t.dims[j];
      if (t.dims[j] == 0 || elements > UINT64_MAX)
        reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " has a zero or overflowing dimension");
    }
    t.type = c.u32("tensor type");
    const Encoding *e = encoding_of(t.type);
    if (!e)
      reject(COHX_UNSUPPORTED, "tensor " + quoted(t.name) + " has unknown ggml type " + std::to_string(t.type) +
                                   ", so its size cannot be checked");
    if (t.dims[0] % e->block)
      reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " rows of " + std::to_string(t.dims[0]) +
                                    " values are not whole " + e->name + " blocks");
    const unsigned __int128 bytes = (unsigned __int128)(elements / e->block) * e->bytes;
    if (bytes > UINT64_MAX) reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " is too large to address");
    t.bytes = (uint64_t)bytes;
    t.offset = c.u64("tensor offset");
    if (t.offset % alignment)
      reject(COHX_INVALID_GGUF, "tensor " + quoted(t.name) + " offset " + std::to_string(t.offset) +
                                    " is not a multiple of the alignment " + std::to_string(alignment));
  }
  h.data_start = (c.at() + alignment - 1) / alignment * alignment;
  if (h.data_start > size) reject(COHX_INVALID_GGUF, "the data section would start past the end of the file");
  const uint64_t data_size = size - h.data_start;
  // payloads in offset order: each inside the data section, none overlapping
  std::vector<const Tensor *> order;
  order.reserve(h.tensors.size());
  for (const Tensor &t : h.tensors) order.push_back(&t);
  std::sort(order.begin(), order.end(), [](const Tensor *a, const Tensor *b) { return a->offset < b->offset; });
  uint64_t end = 0;
  for (const Tensor *t : order) {
    if (t->offset < end)
      reject(COHX_INVALID_GGUF, "tensor " + quoted(t->name) + " payload overlaps the previous tensor's");
    if (t->bytes > data_size || t->offset > data_size - t->bytes)
      reject(COHX_INVALID_GGUF, "tensor " + quoted(t->name) + " payload of " + std::to_string(t->bytes) +
                                    " bytes at offset " + std::to_string(t->offset) + " lies past the end of the file");
    end = t->offset + t->bytes;
  }
  return h;
}

// ---------------------------------------------------------------------------
// Qwen2 configuration

// The qwen2.* keys this loader understands.  Any other qwen2.* key (RoPE
// scaling, sliding windows, ...) names a variant it does not implement.
enum class Role { Dim, Epsilon, RopeBase, HeadDim };
struct ModelKey {
  const char *suffix;
  Role role;
  uint64_t max;  // Dim: largest accepted value
};
constexpr ModelKey kModelKeys[] = {
    {"block_count", Role::Dim, 4096},
    {"context_length", Role::Dim, 1u << 24},
    {"embedding_length", Role::Dim, 1u << 16},
    {"feed_forward_length", Role::Dim, 1u << 20},
    {"attention.head_count", Role::Dim, 4096},
    {"attention.head_count_kv", Role::Dim, 4096},
    {"attention.layer_norm_rms_epsilon", Role::Epsilon, 0},
    {"rope.freq_base", Role::RopeBase, 0},
    {"rope.dimension_count", Role::HeadDim, 0},
    {"attention.key_length", Role::HeadDim, 0},
    {"attention.value_length", Role::HeadDim, 0},
};
constexpr std::string_view kArch = "qwen2.";

const ModelKey *model_key(std::string_view suffix) {
  for (const ModelKey &k : kModelKeys)
    if (suffix == k.suffix) return &k;
  return nullptr;
}

uint64_t dimension(const Header &h, const char *suffix) {
  const std::string key = std::string(kArch) + suffix;
  const Meta *m = h.find(key);
  if (!m || !m->is_unsigned()) reject(COHX_INVALID_GGUF, key + " is required as an unsigned integer");
  const uint64_t max = model_key(suffix)->max;
  if (m->bits == 0 || m->bits > max)
    reject(COHX_INVALID_GGUF, key + " = " + std::to_string(m->bits) + " is out of range [1, " + std::to_string(max) + "]");
  return m->bits;
}

// The per-layer tensors of the Qwen2 graph: name suffix and shape, in units
// of H (hidden), F (feed-forward) and KVD (kv heads x head size).
enum Extent : uint8_t { H, F, KVD };
struct LayerTensor {
  const char *suffix;
  uint8_t rank;
  Extent d0, d1;
};
constexpr LayerTensor kLayerTensors[] = {
    {"attn_norm.weight", 1, H, H},    {"ffn_norm.weight", 1, H, H},      {"attn_q.weight", 2, H, H},
    {"attn_q.bias", 1, H, H},         {"attn_k.weight", 2, H, KVD},      {"attn_k.bias", 1, KVD, KVD},
    {"attn_v.weight", 2, H, KVD},     {"attn_v.bias", 1, KVD, KVD},      {"attn_output.weight", 2, H, H},
    {"ffn_gate.weight", 2, H, F},     {"ffn_up.weight", 2, H, F},        {"ffn_down.weight", 2, F, H},
};

std::string shape_text(const uint64_t *dims, uint32_t rank) {
  std::string s = "[";
  for (uint32_t j = 0; j < rank; j++) s += (j ? ", " : "") + std::to_string(dims[j]);
  return s + "]";
}

void require_tensor(const Header &h, const std::string &name, uint32_t rank, uint64_t d0, uint64_t d1) {
  const Tensor *t = h.tensor(name);
  if (!t) reject(COHX_INVALID_GGUF, "tensor " + name + " is required but absent");
  const uint64_t want[2] = {d0, d1};
  if (t->rank != rank || t->dims[0] != d0 || (rank == 2 && t->dims[1] != d1))
    reject(COHX_INVALID_GGUF, "tensor " + name + " has shape " + shape_text(t->dims, t->rank) + ", expected " +
                                  shape_text(want, rank));
}

void configure(const Header &h, cohx_model_desc &c) {
  const Meta *arch = h.find("general.architecture");
  if (!arch || arch->type != kStr || arch->text != "qwen2")
    reject(COHX_UNSUPPORTED, "general.architecture is " + (arch && arch->type == kStr ? quoted(arch->text) : "absent") +
                                 "; this loader builds the qwen2 graph");
  for (const auto &kv : h.meta) {
    const std::string_view key = kv.first;
    if (key.substr(0, kArch.size()) == kArch && !model_key(key.substr(kArch.size())))
      reject(COHX_UNSUPPORTED, "metadata key " + quoted(key) + " describes a Qwen2 variant this loader does not implement");
  }
  const uint64_t hidden = dimension(h, "embedding_length");
  const uint64_t heads = dimension(h, "attention.head_count");
  const uint64_t kv_heads = dimension(h, "attention.head_count_kv");
  if (hidden % heads || heads % kv_heads || (hidden / heads) % 2)
    reject(COHX_INVALID_GGUF, "head layout does not fit: " + std::to_string(heads) + " query and " +
                                  std::to_string(kv_heads) + " key/value heads over " + std::to_string(hidden) +
                                  " need equal groups and an even head size");
  const Meta *tokens = h.find("tokenizer.ggml.tokens");
  if (!tokens || tokens->type != kArr || tokens->count == 0 || tokens->count > (1u << 24))
    reject(COHX_INVALID_GGUF, "tokenizer.ggml.tokens (the vocabulary) is required as a non-empty array");
  const uint64_t vocabulary = tokens->count;
  const Meta *eps = h.find("qwen2.attention.layer_norm_rms_epsilon");
  if (!eps || !eps->is_float()) reject(COHX_INVALID_GGUF, "qwen2.attention.layer_norm_rms_epsilon is required as a float");
  const Meta *base = h.find("qwen2.rope.freq_base");
  const float rope_base = base && base->is_float() ? (float)base->real() : 10000.0f;
  const float epsilon = (float)eps->real();
  if (!(std::isfinite(rope_base) && rope_base > 0.0f && std::isfinite(epsilon) && epsilon > 0.0f))
    reject(COHX_INVALID_GGUF, "RoPE base and RMSNorm epsilon must be positive and finite");
  const uint64_t head_dim = hidden / heads;
  for (const ModelKey &k : kModelKeys) {
    if (k.role != Role::HeadDim) continue;
    const Meta *m = h.find(std::string(kArch) + k.suffix);
    if (m && m->is_unsigned() && m->bits != head_dim)
      reject(COHX_UNSUPPORTED, std::string("qwen2.") + k.suffix + " = " + std::to_string(m->bits) +
                                   " differs from the head size " + std::to_string(head_dim));
  }
  if (const Meta *split = h.find("split.count"); split && split->is_unsigned() && split->bits > 1)
    reject(COHX_UNSUPPORTED, "the model is split over " + std::to_string(split->bits) + " files; only single files load");

  c.layers = (uint32_t)dimension(h, "block_count");
  c.hidden = (uint32_t)hidden;
  c.intermediate = (uint32_t)dimension(h, "feed_forward_length");
  c.heads = (uint32_t)heads;
  c.kv_heads = (uint32_t)kv_heads;
  c.head_dim = (uint32_t)head_dim;
  c.vocabulary = (uint32_t)vocabulary;
  c.context = (uint32_t)dimension(h, "context_length");
  c.rope_base = rope_base;
  c.norm_epsilon = epsilon;

  // the graph: every expected tensor present with its shape, nothing else
  const uint64_t extent[3] = {hidden, c.intermediate, kv_heads * head_dim};
  require_tensor(h, "token_embd.weight", 2, hidden, vocabulary);
  require_tensor(h, "output_norm.weight", 1, hidden, 0);
  const bool untied = h.tensor("output.weight") != nullptr;
  if (untied) require_tensor(h, "output.weight", 2, hidden, vocabulary);
  for (uint32_t l = 0; l < c.layers; l++)
    for (const LayerTensor &t : kLayerTensors)
      require_tensor(h, "blk." + std::to_string(l) + "." + t.suffix, t.rank, extent[t.d0], extent[t.d1]);
  const size_t expected = 2 + (untied ? 1 : 0) + (size_t)c.layers * (sizeof kLayerTensors / sizeof kLayerTensors[0]);
  if (h.tensors.size() != expected) {
    // name one tensor that is not part of the graph
    std::string extra = "(unnamed)";
    for (const Tensor &t : h.tensors) {
      const std::string n(t.name);
      bool known = n == "token_embd.weight" || n == "output_norm.weight" || n == "output.weight";
      for (uint32_t l = 0; !known && l < c.layers; l++)
        for (const LayerTensor &lt : kLayerTensors)
          if (n == "blk." + std::to_string(l) + "." + lt.suffix) known = true;
      if (!known) {
        extra = n;
        break;
      }
    }
    reject(COHX_UNSUPPORTED, "tensor " + quoted(extra) + " is not part of the Qwen2 graph (" +
                                 std::to_string(h.tensors.size()) + " tensors, " + std::to_string(expected) + " expected)");
  }
  uint32_t matrix_type = ~0u;
  bool mixed = false;
  for (const Tensor &t : h.tensors) {
    if (t.rank != 2) continue;
    if (matrix_type != ~0u && t.type != matrix_type) mixed = true;
    matrix_type = t.type;
  }
  c.weight_dtype = mixed ? COHX_MIXED : matrix_type;
  c.tied = untied ? 0 : 1;
  c.kv_dtype = 0;

  // end of generation: eos (required), eot (when stored unsigned), the
  // "<|endoftext|>" entry of the vocabulary
  const Meta *eos = h.find("tokenizer.ggml.eos_token_id");
  if (!eos || !eos->is_unsigned() || eos->bits >= vocabulary)
    reject(COHX_UNSUPPORTED, "tokenizer.ggml.eos_token_id must be an unsigned id below the vocabulary size " +
                                 std::to_string(vocabulary));
  std::vector<uint32_t> eog = {(uint32_t)eos->bits};
  if (const Meta *eot = h.find("tokenizer.ggml.eot_token_id"); eot && eot->is_unsigned()) {
    if (eot->bits >= vocabulary)
      reject(COHX_UNSUPPORTED, "tokenizer.ggml.eot_token_id " + std::to_string(eot->bits) + " is outside the vocabulary");
    eog.push_back((uint32_t)eot->bits);
  }
  if (tokens->endoftext >= 0) eog.push_back((uint32_t)tokens->endoftext);
  std::sort(eog.begin(), eog.end());
  eog.erase(std::unique(eog.begin(), eog.end()), eog.end());
  c.n_eog = (uint32_t)eog.size();
  std::copy(eog.begin(), eog.end(), c.eog);
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

// ---------------------------------------------------------------------------
// The file

class MappedFile {
 public:
  explicit MappedFile(const char *path) {
    if (!path) throw Reject{COHX_INVALID_REQUEST, "gguf: no path given"};
    fd_ = open(path, O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw Reject{COHX_INVALID_REQUEST, std::string("gguf: cannot open ") + path};
    struct stat st;
    if (fstat(fd_, &st) != 0 || !S_ISREG(st.st_mode))
      throw Reject{COHX_INVALID_REQUEST, std::string("gguf: ") + path + " is not a regular file"};
    size_ = (uint64_t)st.st_size;
    if (size_ == 0) reject(COHX_INVALID_GGUF, "empty file");
    void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) throw Reject{COHX_RESOURCE, "gguf: cannot map the file"};
    data_ = static_cast<const uint8_t *>(p);
  }
  ~MappedFile() {
    if (data_) munmap(const_cast<uint8_t *>(data_), size_);
    if (fd_ >= 0) close(fd_);
  }
  MappedFile(const MappedFile &) = delete;
  MappedFile &operator=(const MappedFile &) = delete;

  const uint8_t *data() const { return data_; }
  uint64_t size() const { return size_; }

 private:
  int fd_ = -1;
  const uint8_t *data_ = nullptr;
  uint64_t size_ = 0;
};

void write_error(char *err, size_t cap, const std::string &text) {
  if (!err || !cap) return;
  const size_t n = std::min(cap - 1, text.size());
  std::memcpy(err, text.data(), n);
  err[n] = 0;
}

// Runs `body`, turning a rejection or a host allocation failure into a status
// and its text.
template <typename F>
int guarded(char *err, size_t cap, F &&body) {
  try {
    body();
    write_error(err, cap, "");
    return COHX_OK;
  } catch (const Reject &r) {
    write_error(err, cap, r.text);
    return r.code;
  } catch (const std::bad_alloc &) {
    write_error(err, cap, "gguf: host allocation failed");
    return COHX_RESOURCE;
  }
}

}  // namespace

extern "C" int cohx_gguf_inspect(const char *path, cohx_model_desc *desc, char *err, size_t err_cap) {
  if (!desc) return COHX_INVALID_REQUEST;
  return guarded(err, err_cap, [&] {
    const MappedFile file(path);
    const Header h = read_header(file.data(), file.size());
    cohx_model_desc c = *desc;
    configure(h, c);
    capacities(*desc, c);
    *desc = c;
  });
}

extern "C" int cohx_load_gguf(const char *path, int device, cohx_model_desc *desc, cohx_ctx **out, char *err,
                              size_t err_cap) {
  if (!desc || !out) return COHX_INVALID_REQUEST;
  *out = nullptr;
  cohx_ctx *ctx = nullptr;
  const int rc = guarded(err, err_cap, [&] {
    const MappedFile file(path);
    const Header h = read_header(file.data(), file.size());
    cohx_model_desc c = *desc;
    configure(h, c);
    capacities(*desc, c);
    if (c.max_context > c.context)
      throw Reject{COHX_INVALID_REQUEST, "gguf: max_context " + std::to_string(c.max_context) +
                                             " is larger than the file's context " + std::to_string(c.context)};
    if (int r = cohx_create(&c, device, &ctx)) throw Reject{r, "gguf: the device context could not be created"};
    const uint8_t *data = file.data() + h.data_start;
    for (const Tensor &t : h.tensors) {
      const std::string name(t.name);
      if (int r = cohx_upload_tensor(ctx, name.c_str(), t.type, t.dims[0], t.rank > 1 ? t.dims[1] : 1,
                                     data + t.offset, (size_t)t.bytes))
        throw Reject{r, cohx_last_error(ctx)};
    }
    if (int r = cohx_finalize(ctx)) throw Reject{r, cohx_last_error(ctx)};
    *desc = c;
  });
  if (rc == COHX_OK) {
    *out = ctx;
  } else if (ctx) {
    cohx_destroy(ctx);
  }
  return rc;
}
