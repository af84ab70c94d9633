// Host-side state of a cohx context (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/cohx.h"
#include "kernels.h"

namespace cohx {

// One (possibly fused) matrix; allocated in its device format by the first
// part uploaded (view.dtype 0 until then).
struct DeviceMatrix {
  MatrixView view{};
  int8_t *qs = nullptr;
  uint16_t *ds = nullptr;
  uint16_t *f16 = nullptr;
  uint32_t *ksc = nullptr;  // K-quant side data (device.h kq_*)
  uint16_t *kdm = nullptr;
  uint8_t *kmin = nullptr;
  uint64_t gguf_bytes = 0;  // bytes of the GGUF payload(s) it holds
};

struct Layer {
  float *attn_norm = nullptr, *ffn_norm = nullptr, *bqkv = nullptr;
  DeviceMatrix qkv, o, gu, down;
};

struct Sequence {
  bool live = false;
  uint32_t length = 0, capacity = 0;
  std::vector<int32_t> pages;  // logical page -> physical page
};

// Device scratch of one step, carved from one block of device memory by
// layout_workspace (the context's own block, sized for its capacities).
struct Workspace {
  // one upload region: lane_info [lanes][4], tokens [rows], then the exact
  // attention passes' work list (StepDims::att_items)
  uint32_t *lane_info = nullptr, *tokens = nullptr, *att_items = nullptr;
  uint32_t *cu = nullptr, *row_pos = nullptr, *row_lane = nullptr, *row_token = nullptr,
           *row_seq = nullptr, *lane_last = nullptr, *row_err = nullptr;
  int32_t *row_slot = nullptr;
  float *x = nullptr, *qkv = nullptr, *q_rot = nullptr, *h = nullptr;
  int8_t *act_qs = nullptr;
  // the down projection's Q8_0 operand when gate+up quantizes in its epilogue
  // (it cannot overwrite act_qs while other workgroups still read gate+up's)
  int8_t *down_qs = nullptr;
  uint16_t *down_ds = nullptr;
  uint16_t *act_ds = nullptr, *act_f16 = nullptr;
  // Q8_K operands (K-quant weights): block scales and 16-value sums; f32 rows
  // staged for their quantizer (attention output)
  float *act_kd = nullptr;
  int16_t *act_ksum = nullptr;
  float *act_f32 = nullptr;
  float *scores = nullptr;  // [rows][kv_heads][kv_cap][8]: scores (head slot within the group)
  float *chunk_max = nullptr, *logits = nullptr;
  float *row_max = nullptr;  // [rows][heads] softmax maximum of each exact-pass row
  double *partial = nullptr;   // [rows][heads][max_chunks][head_dim] (chunk rows: f32 segment records)
  double *den_part = nullptr;  // [rows][heads][256-token chunks] softmax denominator partials
  // prefill chunks on the matrix cores: (16-row tile, key segment) work
  // items, per-row flags, and the list of rows left to the exact attention
  // passes (chunk rows' segment records live in `partial`)
  int4 *tiles = nullptr;
  uint32_t *row_skip = nullptr;
  uint32_t *row_map = nullptr;
  // the chunk lanes' key tiles as binary16 LDS images (rewritten every layer)
  // and the work items that make them
  int4 *stage = nullptr;
  uint4 *img = nullptr;
  unsigned long long *argmax = nullptr;  // final keys per lane, zeroed by the packer
  unsigned long long *argmax_part = nullptr;  // [lanes][head m-tiles]
  // capacities the buffers were laid out for
  uint32_t rows = 0, lanes = 0, kv_cap = 0, max_chunks = 0, max_tiles = 0, max_images = 0;
  bool logits_room = false;
};

// Pinned host staging of a context (uploads of the batch, read-back of results).
struct Staging {
  uint32_t *h_upload = nullptr;  // the workspace's upload region (lane_info, tokens, work list), same offsets
  uint32_t *h_row_err = nullptr;
  int4 *h_tiles = nullptr;        // tiles, row flags and the row list of the prefill regime
  int4 *h_stage = nullptr;        // the regime's tile image items
  uint32_t *h_row_skip = nullptr;
  uint32_t *h_row_map = nullptr;
  uint32_t *h_kv = nullptr;       // attended length of each exact-pass row (the work list's source)
  unsigned long long *h_argmax = nullptr;
};

// Bytes of a workspace for `rows` packed rows, `lanes` lanes and attention over
// at most kv_cap positions (logits: room for every lane's logits); with a
// non-null base, also fills `w` with buffers carved from it (256-byte aligned).
size_t layout_workspace(const cohx_model_desc &d, int nbp_h, int nbp_f, uint32_t rows, uint32_t lanes,
                        uint32_t kv_cap, bool logits, uint8_t *base, Workspace *w);
// 32-bit words of a workspace's upload region (lane_info, tokens, work list)
size_t upload_words(uint32_t rows, uint32_t lanes, uint32_t kv_cap);

enum ProfCat {
  kCatPack, kCatEmbed, kCatNorm, kCatMvQkv, kCatQkvPost, kCatAttnScores, kCatAttnSoftmax,
  kCatAttnPv, kCatAttnCombine, kCatMvO, kCatMvGateUp, kCatQuant, kCatMvDown, kCatMvHead,
  kCatAttnChunk, kCatAttnStage, kCatCount
};

struct Profiler {
  struct Launch {
    int cat;
    double bytes, flops;
    hipEvent_t a, b;
  };
  bool on = false;
  std::vector<hipEvent_t> pool;
  size_t next = 0;
  std::vector<Launch> pending;
  uint64_t launches[kCatCount] = {};
  double ms[kCatCount] = {}, bytes[kCatCount] = {}, flops[kCatCount] = {};
};

// A step's device work depends on these alone (pointers and model dimensions
// are fixed per context), so one captured graph serves every step with them.
struct StepKey {
  uint32_t rows, lanes, kv_grid;
  bool logits;
  bool operator<(const StepKey &o) const {
    return std::tie(rows, lanes, kv_grid, logits) < std::tie(o.rows, o.lanes, o.kv_grid, o.logits);
  }
};
constexpr size_t kMaxGraphs = 64;

struct Q35Model;  // Qwen3.5 hybrid model state (q35.cpp)

}  // namespace cohx

struct cohx_ctx {
  cohx_model_desc desc{};
  int device = 0;
  hipStream_t stream = nullptr;
  // steps with prefill chunks: the exact passes over the decode rows run on
  // `side` (default priority) beside the chunk attention, forked from and
  // joined back into `stream` by these events
  hipStream_t side = nullptr;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  std::string err;
  int nbp_h = 0, nbp_f = 0, nbp_max = 0;
  int max_pages = 0;  // pages per sequence
  int max_chunks = 0;
  size_t layer_stride = 0;  // floats per layer in each KV pool
  std::vector<cohx::Layer> layers;
  cohx::DeviceMatrix embd, output;
  float *output_norm = nullptr;
  float2 *rope = nullptr;
  float *kpool = nullptr, *vpool = nullptr;
  int32_t *page_table = nullptr;
  std::vector<int32_t> h_page_table;
  std::vector<uint8_t> pt_dirty;
  // pinned copy of the mirror's changed rows for one upload per step, and
  // the event after that upload (the staging rows are reused only once it
  // has completed)
  int32_t *h_pt_stage = nullptr;
  hipEvent_t pt_done = nullptr;
  bool pt_pending = false;
  std::vector<int32_t> free_pages;
  std::vector<int32_t> page_refs;
  std::vector<cohx::Sequence> seqs;
  std::vector<uint32_t> free_seqs;
  std::vector<std::string> uploaded;
  bool finalized = false;
  uint64_t matrix_bytes = 0;
  cohx::Workspace ws;      // laid out for max_rows / max_lanes / max_context
  uint8_t *ws_block = nullptr;
  cohx::Staging host;
  uint8_t *scratch = nullptr;  // this device's static scratch array (cohx_step_noalloc)
  cohx::Profiler prof;
  std::vector<void *> allocations;
  bool use_graphs = true;    // replay each step's launches as one captured graph
  bool prefill_mfma = true;  // packed-prefill regime (F16, Q8_0/Q5_0/Q4_0) on the matrix cores
  // every layer linear is a Q8/Q4 tile matrix the quantized GEMM takes (set at finalize)
  bool quant_gemm = false;
  std::map<cohx::StepKey, hipGraphExec_t> graphs;
  cohx::Q35Model *q35 = nullptr;  // set for Qwen3.5 contexts (cohx_create_qwen35)
  hipEvent_t done = nullptr;      // completion event of a hooked step (created on first use)
};

namespace cohx {
int fail(cohx_ctx *ctx, int code, const std::string &msg);
void drop_graphs(cohx_ctx *ctx);
// Qwen3.5 contexts: the C entry points hand over to these (q35.cpp).
void q35_free(cohx_ctx *ctx);
int q35_upload(cohx_ctx *ctx, const char *name, uint32_t dtype, uint64_t ne0, uint64_t ne1,
               const void *data, size_t bytes);
int q35_finalize(cohx_ctx *ctx);
int q35_seq_reset(cohx_ctx *ctx, uint32_t seq);
int q35_seq_copy(cohx_ctx *ctx, uint32_t src, uint32_t dst, uint32_t rows);
int q35_read_state(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int which, float *out);
int q35_step(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out, const cohx_step_hooks *hooks);
// Waits for everything enqueued on `s`; with a yield hook, calls it between
// polls of a completion event instead of blocking.  Returns COHX_CANCELLED
// (after the device has finished) when the hook asked to stop.
int wait_step(cohx_ctx *ctx, hipStream_t s, const cohx_step_hooks *hooks);
}
