// Qwen3.5 hybrid text step: context, upload, sequence state and the step
// driver (crates/coheryn-engine/src/qwen35/execution.rs:168-608,
// qwen35/generation.rs:335-406 step_batch).  The weights stay in HBM as
// BF16 tiles; each sequence slot owns its K/V rows (full-attention layers),
// causal-conv ring and delta-rule memory (linear layers), the engine's
// Session states (execution.rs:44-47,758-780).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <set>
#include <string>
#include <vector>

#include "device.h"
#include "internal.h"
#include "q35.h"

using namespace cohx;

namespace {

int pad16(int n) { return (n + 15) / 16 * 16; }

// Packed batches at least this tall take the matrix-core GEMM (regime on).
constexpr uint32_t kQ35PrefillRows = 128;

#define Q35_TRY(expr)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(ctx, COHX_DEVICE, std::string(#expr ": ") + hipGetErrorString(e_)); \
  } while (0)

template <typename T>
int q35_alloc(cohx_ctx *ctx, T **p, size_t count) {
  *p = nullptr;
  if (count == 0) count = 1;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(p), count * sizeof(T));
  if (e != hipSuccess)
    return fail(ctx, COHX_RESOURCE,
                "device allocation of " + std::to_string(count * sizeof(T)) + " bytes failed");
  ctx->allocations.push_back(*p);
  e = hipMemset(*p, 0, count * sizeof(T));
  return e == hipSuccess ? COHX_OK : fail(ctx, COHX_DEVICE, hipGetErrorString(e));
}

}  // namespace

namespace cohx {

struct Q35Layer {
  bool full = false;
  int slot = 0;  // index among the full (or linear) layers
  float *input_norm = nullptr, *post_norm = nullptr;
  uint16_t *mix = nullptr;   // linear: [qkv | z | a | b]; full: [q | k | v] (16-row padded parts)
  uint16_t *out = nullptr;   // out_proj / o_proj
  uint16_t *gu = nullptr;    // [gate | up]
  uint16_t *down = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr;                      // full
  float *conv = nullptr, *a_log = nullptr, *dt = nullptr, *norm = nullptr;  // linear
};

struct Q35Model {
  cohx_qwen35_desc d{};
  int H = 0, F = 0, V = 0, NH = 0, NKV = 0, D = 0, KH = 0, VH = 0, KD = 0, VD = 0, K = 0, ROT = 0;
  int keys = 0, vals = 0, C = 0, qw = 0, kvw = 0, n_full = 0, n_lin = 0;
  int lin_z = 0, lin_a = 0, lin_b = 0, lin_rows = 0;  // row offsets in [qkv | z | a | b]
  int full_k = 0, full_v = 0, full_rows = 0;           // row offsets in [q | k | v]
  int gu_up = 0, gu_rows = 0, h_rows = 0, head_rows = 0;
  std::vector<Q35Layer> layers;
  uint16_t *embed = nullptr, *head = nullptr;
  float *final_norm = nullptr;
  float2 *rope = nullptr;
  float *kc = nullptr, *vc = nullptr, *conv_state = nullptr, *delta_state = nullptr;
  size_t kv_layer = 0, kv_seq = 0, conv_seq = 0, delta_seq = 0;
  // step workspace
  int max_rows = 0, max_lanes = 0, ld_mix = 0, ld_att = 0;
  float *x = nullptr, *nrm = nullptr, *mix_out = nullptr, *cv = nullptr, *tgt = nullptr,
        *q = nullptr, *z = nullptr, *att = nullptr, *gu_out = nullptr, *hb = nullptr,
        *fin = nullptr, *logits = nullptr;
  float4 *gates = nullptr;  // [rows][value_heads]: q_scale, k_scale, decay, beta
  float *scores = nullptr;  // [rows][heads][max_context] attention scores
  unsigned long long *part = nullptr, *argmax = nullptr;
  uint32_t *row_err = nullptr, *tables = nullptr;
  uint32_t *h_tables = nullptr, *h_row_err = nullptr;
  unsigned long long *h_argmax = nullptr;
  bool split_linear = false;  // COHX_Q35_SPLIT_LINEAR=1: the four-kernel mixer (tests)
  // packed-prefill regime: steps of kQ35PrefillRows+ rows run their linears
  // on the matrix-core GEMM (f32 sums, within tolerance); a_hi/a_lo
  // [rows][kmax] hold the activations' bfloat16 parts
  bool mfma = false;
  int kmax = 0;
  uint16_t *a_hi = nullptr, *a_lo = nullptr;
  std::set<std::string> uploaded;
  size_t expected = 0;
  uint64_t matrix_bytes = 0;
};

}  // namespace cohx

namespace {

// Upload one BF16 matrix [rows][K] into rows [off, off + rows) of a tiled
// buffer (the part padded to 16 rows with zeros).
int put_matrix(cohx_ctx *ctx, uint16_t *dst, int off, int rows, int K, const uint16_t *src) {
  const int rp = pad16(rows);
  std::vector<uint16_t> tiled((size_t)rp * K, 0);
  for (int r = 0; r < rows; r++)
    for (int k = 0; k < K; k++) tiled[q35_tiled_index(r, k, K)] = src[(size_t)r * K + k];
  Q35_TRY(hipMemcpy(dst + (size_t)off * K, tiled.data(), tiled.size() * 2, hipMemcpyHostToDevice));
  return COHX_OK;
}

bool finite_bf16(const uint16_t *p, size_t n) {
  for (size_t i = 0; i < n; i++)
    if ((p[i] & 0x7f80u) == 0x7f80u) return false;
  return true;
}

int put_vector(cohx_ctx *ctx, float *dst, uint32_t dtype, size_t n, const void *data,
               size_t bytes) {
  std::vector<float> v(n);
  if (dtype == COHX_F32 && bytes == n * 4) {
    std::memcpy(v.data(), data, bytes);
  } else if (dtype == COHX_BF16 && bytes == n * 2) {
    for (size_t i = 0; i < n; i++) {
      const uint32_t b = (uint32_t)static_cast<const uint16_t *>(data)[i] << 16;
      std::memcpy(&v[i], &b, 4);
    }
  } else {
    return fail(ctx, COHX_INVALID_GGUF, "vector payload size or dtype mismatch");
  }
  for (float f : v)
    if (!std::isfinite(f)) return fail(ctx, COHX_INVALID_GGUF, "non-finite weight");
  Q35_TRY(hipMemcpy(dst, v.data(), n * 4, hipMemcpyHostToDevice));
  return COHX_OK;
}

}  // namespace

extern "C" {

// qwen35/config.rs:6-25,37-192 (shape checks) and execution.rs:758-780 (state sizes).
int cohx_create_qwen35(const cohx_qwen35_desc *dd, int device, cohx_ctx **out) {
  if (!dd || !out) return COHX_INVALID_REQUEST;
  *out = nullptr;
  const cohx_qwen35_desc &d = *dd;
  if (!d.layers || d.layers > 128 || !d.hidden || !d.heads || !d.kv_heads || d.heads % d.kv_heads ||
      !d.head_dim || !d.linear_key_heads ||
      d.linear_value_heads % d.linear_key_heads || !d.rotary_dim || d.rotary_dim % 2 ||
      d.rotary_dim > d.head_dim || !d.conv_kernel || !d.vocabulary || !d.intermediate ||
      !(d.epsilon > 0.0f) || !(d.rope_base > 1.0f))
    return COHX_INVALID_GGUF;
  const uint32_t group = d.heads / d.kv_heads;
  if (d.head_dim > (uint32_t)kQ35MaxHeadDim || d.head_dim % 4 || group > (uint32_t)kQ35MaxGroup ||
      (group & (group - 1)))
    return COHX_UNSUPPORTED;
  if (d.hidden % 8 || d.intermediate % 8 || (d.heads * d.head_dim) % 8 ||
      (d.linear_value_heads * d.linear_value_dim) % 8 || d.hidden > (uint32_t)kQ35MaxHidden ||
      d.conv_kernel > 8 || !q35_delta_supported((int)d.linear_key_dim, (int)d.linear_value_dim))
    return COHX_UNSUPPORTED;
  if (!d.max_lanes || d.max_lanes > 1024 || !d.max_rows || d.max_rows < d.max_lanes ||
      !d.max_seqs || !d.max_context || d.max_context > d.context ||
      d.max_context > (uint32_t)kQ35MaxContext ||
      d.n_eog > 4)
    return COHX_INVALID_REQUEST;
  cohx_ctx *ctx = new cohx_ctx();
  ctx->device = device;
  ctx->use_graphs = false;
  // COHX_PREFILL_MFMA=0 keeps tall packed steps on the exact (f64-sum)
  // matvecs
  if (const char *g = std::getenv("COHX_PREFILL_MFMA")) ctx->prefill_mfma = std::strcmp(g, "0") != 0;
  cohx_model_desc &m = ctx->desc;
  m.layers = d.layers;
  m.hidden = d.hidden;
  m.intermediate = d.intermediate;
  m.heads = d.heads;
  m.kv_heads = d.kv_heads;
  m.head_dim = d.head_dim;
  m.vocabulary = d.vocabulary;
  m.context = d.context;
  m.rope_base = d.rope_base;
  m.norm_epsilon = d.epsilon;
  m.weight_dtype = COHX_BF16;
  m.tied = d.tied;
  m.max_lanes = d.max_lanes;
  m.max_rows = d.max_rows;
  m.max_seqs = d.max_seqs;
  m.max_context = d.max_context;
  m.n_eog = d.n_eog;
  for (int i = 0; i < 4; i++) m.eog[i] = d.eog[i];
  auto *q = new Q35Model();
  ctx->q35 = q;
  q->d = d;
  q->H = (int)d.hidden;
  q->F = (int)d.intermediate;
  q->V = (int)d.vocabulary;
  q->NH = (int)d.heads;
  q->NKV = (int)d.kv_heads;
  q->D = (int)d.head_dim;
  q->KH = (int)d.linear_key_heads;
  q->VH = (int)d.linear_value_heads;
  q->KD = (int)d.linear_key_dim;
  q->VD = (int)d.linear_value_dim;
  q->K = (int)d.conv_kernel;
  q->ROT = (int)d.rotary_dim;
  q->keys = q->KH * q->KD;
  q->vals = q->VH * q->VD;
  q->C = 2 * q->keys + q->vals;
  q->qw = q->NH * q->D;
  q->kvw = q->NKV * q->D;
  q->lin_z = pad16(q->C);
  q->lin_a = q->lin_z + pad16(q->vals);
  q->lin_b = q->lin_a + pad16(q->VH);
  q->lin_rows = q->lin_b + pad16(q->VH);
  q->full_k = pad16(2 * q->qw);
  q->full_v = q->full_k + pad16(q->kvw);
  q->full_rows = q->full_v + pad16(q->kvw);
  q->gu_up = pad16(q->F);
  q->gu_rows = 2 * q->gu_up;
  q->h_rows = pad16(q->H);
  q->head_rows = pad16(q->V);
  q->max_rows = (int)d.max_rows;
  q->max_lanes = (int)d.max_lanes;
  if (const char *e = std::getenv("COHX_Q35_SPLIT_LINEAR")) q->split_linear = std::atoi(e) != 0;
  q->mfma = ctx->prefill_mfma && d.max_rows >= kQ35PrefillRows;
  q->kmax = std::max(std::max(q->H, q->F), std::max(q->qw, q->vals));
  int rc = 0;
  const hipError_t e0 = hipSetDevice(device);
  if (e0 == hipSuccess) {
    const hipError_t e1 = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e1 != hipSuccess) rc = fail(ctx, COHX_DEVICE, hipGetErrorString(e1));
  } else {
    rc = fail(ctx, COHX_DEVICE, hipGetErrorString(e0));
  }
  const int H = q->H;
  q->layers.resize(d.layers);
  for (uint32_t l = 0; l < d.layers && !rc; l++) {
    Q35Layer &L = q->layers[l];
    L.full = d.full_attention[l] != 0;
    L.slot = L.full ? q->n_full++ : q->n_lin++;
    rc = q35_alloc(ctx, &L.input_norm, H);
    if (!rc) rc = q35_alloc(ctx, &L.post_norm, H);
    if (!rc) rc = q35_alloc(ctx, &L.gu, (size_t)q->gu_rows * H);
    if (!rc) rc = q35_alloc(ctx, &L.down, (size_t)q->h_rows * q->F);
    if (rc) break;
    if (L.full) {
      rc = q35_alloc(ctx, &L.mix, (size_t)q->full_rows * H);
      if (!rc) rc = q35_alloc(ctx, &L.out, (size_t)q->h_rows * q->qw);
      if (!rc) rc = q35_alloc(ctx, &L.q_norm, q->D);
      if (!rc) rc = q35_alloc(ctx, &L.k_norm, q->D);
      q->expected += 11;
    } else {
      rc = q35_alloc(ctx, &L.mix, (size_t)q->lin_rows * H);
      if (!rc) rc = q35_alloc(ctx, &L.out, (size_t)q->h_rows * q->vals);
      if (!rc) rc = q35_alloc(ctx, &L.conv, (size_t)q->C * q->K);
      if (!rc) rc = q35_alloc(ctx, &L.a_log, q->VH);
      if (!rc) rc = q35_alloc(ctx, &L.dt, q->VH);
      if (!rc) rc = q35_alloc(ctx, &L.norm, q->VD);
      q->expected += 14;
    }
  }
  q->expected += d.tied ? 2 : 3;
  if (!rc) rc = q35_alloc(ctx, &q->embed, (size_t)q->V * H);
  if (!rc) rc = q35_alloc(ctx, &q->head, (size_t)q->head_rows * H);
  if (!rc) rc = q35_alloc(ctx, &q->final_norm, H);
  // rotary table (cos, sin) of angle pos * base^(-2i/rotary) (kernels.rs:252-254)
  if (!rc) {
    const int half = q->ROT / 2;
    std::vector<float2> tab((size_t)d.max_context * half);
    for (uint32_t p = 0; p < d.max_context; p++)
      for (int i = 0; i < half; i++) {
        const float angle = (float)p * powf(d.rope_base, -(float)(2 * i) / (float)q->ROT);
        tab[(size_t)p * half + i] = make_float2(cosf(angle), sinf(angle));
      }
    rc = q35_alloc(ctx, &q->rope, tab.size());
    if (!rc) {
      const hipError_t e = hipMemcpy(q->rope, tab.data(), tab.size() * sizeof(float2),
                                     hipMemcpyHostToDevice);
      if (e != hipSuccess) rc = fail(ctx, COHX_DEVICE, hipGetErrorString(e));
    }
  }
  // sequence state slabs
  const size_t S = d.max_seqs;
  q->kv_layer = (size_t)d.max_context * q->kvw;
  q->kv_seq = (size_t)std::max(q->n_full, 1) * q->kv_layer;
  q->conv_seq = (size_t)std::max(q->n_lin, 1) * q->C * q->K;
  q->delta_seq = (size_t)std::max(q->n_lin, 1) * q->VH * q->KD * q->VD;
  if (!rc) rc = q35_alloc(ctx, &q->kc, S * q->kv_seq);
  if (!rc) rc = q35_alloc(ctx, &q->vc, S * q->kv_seq);
  if (!rc) rc = q35_alloc(ctx, &q->conv_state, S * q->conv_seq);
  if (!rc) rc = q35_alloc(ctx, &q->delta_state, S * q->delta_seq);
  // workspace
  const size_t R = d.max_rows, NL = d.max_lanes;
  q->ld_mix = std::max(q->lin_rows, q->full_rows);
  q->ld_att = std::max(q->qw, q->vals);
  if (!rc) rc = q35_alloc(ctx, &q->x, R * H);
  if (!rc) rc = q35_alloc(ctx, &q->nrm, R * H);
  if (!rc) rc = q35_alloc(ctx, &q->mix_out, R * q->ld_mix);
  if (!rc) rc = q35_alloc(ctx, &q->cv, R * q->C);
  if (!rc) rc = q35_alloc(ctx, &q->tgt, R * q->ld_att);
  if (!rc) rc = q35_alloc(ctx, &q->q, R * q->qw);
  if (!rc) rc = q35_alloc(ctx, &q->z, R * q->qw);
  if (!rc) rc = q35_alloc(ctx, &q->att, R * q->ld_att);
  if (!rc) rc = q35_alloc(ctx, &q->gu_out, R * q->gu_rows);
  if (!rc) rc = q35_alloc(ctx, &q->hb, R * q->F);
  if (!rc) rc = q35_alloc(ctx, &q->fin, NL * H);
  if (!rc) rc = q35_alloc(ctx, &q->gates, R * q->VH);
  if (!rc && q->n_full) rc = q35_alloc(ctx, &q->scores, R * q->NH * (size_t)d.max_context);
  if (!rc) rc = q35_alloc(ctx, &q->logits, NL * q->V);
  if (!rc) rc = q35_alloc(ctx, &q->part, NL * q35_matvec_blocks(q->head_rows));
  if (!rc) rc = q35_alloc(ctx, &q->argmax, NL);
  if (!rc) rc = q35_alloc(ctx, &q->row_err, R);
  if (!rc && q->mfma) rc = q35_alloc(ctx, &q->a_hi, R * q->kmax);
  if (!rc && q->mfma) rc = q35_alloc(ctx, &q->a_lo, R * q->kmax);
  const size_t ntab = 5 * NL + 4 * R;
  if (!rc) rc = q35_alloc(ctx, &q->tables, ntab);
  if (!rc) {
    hipError_t e = hipHostMalloc(reinterpret_cast<void **>(&q->h_tables), ntab * 4);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void **>(&q->h_row_err), R * 4);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void **>(&q->h_argmax), NL * 8);
    if (e != hipSuccess) rc = fail(ctx, COHX_RESOURCE, hipGetErrorString(e));
  }
  ctx->seqs.resize(S);
  for (size_t i = S; i-- > 0;) ctx->free_seqs.push_back((uint32_t)i);
  if (rc) {
    const std::string msg = ctx->err;
    cohx_destroy(ctx);
    (void)msg;
    return rc;
  }
  *out = ctx;
  return COHX_OK;
}

}  // extern "C"

namespace cohx {

void q35_free(cohx_ctx *ctx) {
  Q35Model *q = ctx->q35;
  if (!q) return;
  if (q->h_tables) (void)hipHostFree(q->h_tables);
  if (q->h_row_err) (void)hipHostFree(q->h_row_err);
  if (q->h_argmax) (void)hipHostFree(q->h_argmax);
  delete q;
  ctx->q35 = nullptr;
}

// Tensor names and shapes of qwen35/config.rs:193-309 (safetensors names).
int q35_upload(cohx_ctx *ctx, const char *name, uint32_t dtype, uint64_t ne0, uint64_t ne1,
               const void *data, size_t bytes) {
  Q35Model *q = ctx->q35;
  const std::string n(name);
  if (q->uploaded.count(n)) return fail(ctx, COHX_INVALID_GGUF, "tensor uploaded twice: " + n);
  const int H = q->H;
  auto matrix = [&](uint16_t *dst, int off, int rows, int K) -> int {
    if (dtype != COHX_BF16)
      return fail(ctx, COHX_UNSUPPORTED, "Qwen3.5 matrices must be BF16 on the GPU: " + n);
    if (ne0 != (uint64_t)K || ne1 != (uint64_t)rows || bytes != (size_t)rows * K * 2)
      return fail(ctx, COHX_UNSUPPORTED, "unsupported Qwen3.5 tensor shape " + n);
    if (!finite_bf16(static_cast<const uint16_t *>(data), (size_t)rows * K))
      return fail(ctx, COHX_INVALID_GGUF, "non-finite weight in " + n);
    q->matrix_bytes += (uint64_t)rows * K * 2;
    return put_matrix(ctx, dst, off, rows, K, static_cast<const uint16_t *>(data));
  };
  auto vector = [&](float *dst, size_t len) -> int {
    if (ne0 * std::max<uint64_t>(ne1, 1) != len)
      return fail(ctx, COHX_UNSUPPORTED, "unsupported Qwen3.5 tensor shape " + n);
    return put_vector(ctx, dst, dtype, len, data, bytes);
  };
  int rc;
  if (n == "model.language_model.embed_tokens.weight") {
    if (dtype != COHX_BF16 || ne0 != (uint64_t)H || ne1 != (uint64_t)q->V ||
        bytes != (size_t)q->V * H * 2)
      return fail(ctx, COHX_UNSUPPORTED, "unsupported Qwen3.5 embedding " + n);
    if (!finite_bf16(static_cast<const uint16_t *>(data), (size_t)q->V * H))
      return fail(ctx, COHX_INVALID_GGUF, "non-finite weight in " + n);
    Q35_TRY(hipMemcpy(q->embed, data, bytes, hipMemcpyHostToDevice));  // row gather
    rc = q->d.tied ? matrix(q->head, 0, q->V, H) : COHX_OK;             // tied head tiles
  } else if (n == "model.language_model.norm.weight") {
    rc = vector(q->final_norm, H);
  } else if (n == "lm_head.weight") {
    if (q->d.tied) return fail(ctx, COHX_UNSUPPORTED, "lm_head.weight with tied embeddings");
    rc = matrix(q->head, 0, q->V, H);
  } else {
    const std::string pre = "model.language_model.layers.";
    if (n.compare(0, pre.size(), pre) != 0)
      return fail(ctx, COHX_UNSUPPORTED, "unexpected Qwen3.5 tensor " + n);
    size_t dot = n.find('.', pre.size());
    const int l = std::atoi(n.substr(pre.size(), dot - pre.size()).c_str());
    if (dot == std::string::npos || l < 0 || l >= (int)q->layers.size())
      return fail(ctx, COHX_UNSUPPORTED, "unexpected Qwen3.5 tensor " + n);
    const std::string t = n.substr(dot + 1);
    Q35Layer &L = q->layers[l];
    if (t == "input_layernorm.weight") rc = vector(L.input_norm, H);
    else if (t == "post_attention_layernorm.weight") rc = vector(L.post_norm, H);
    else if (t == "mlp.gate_proj.weight") rc = matrix(L.gu, 0, q->F, H);
    else if (t == "mlp.up_proj.weight") rc = matrix(L.gu, q->gu_up, q->F, H);
    else if (t == "mlp.down_proj.weight") rc = matrix(L.down, 0, H, q->F);
    else if (L.full && t == "self_attn.q_proj.weight") rc = matrix(L.mix, 0, 2 * q->qw, H);
    else if (L.full && t == "self_attn.k_proj.weight") rc = matrix(L.mix, q->full_k, q->kvw, H);
    else if (L.full && t == "self_attn.v_proj.weight") rc = matrix(L.mix, q->full_v, q->kvw, H);
    else if (L.full && t == "self_attn.o_proj.weight") rc = matrix(L.out, 0, H, q->qw);
    else if (L.full && t == "self_attn.q_norm.weight") rc = vector(L.q_norm, q->D);
    else if (L.full && t == "self_attn.k_norm.weight") rc = vector(L.k_norm, q->D);
    else if (!L.full && t == "linear_attn.in_proj_qkv.weight") rc = matrix(L.mix, 0, q->C, H);
    else if (!L.full && t == "linear_attn.in_proj_z.weight") rc = matrix(L.mix, q->lin_z, q->vals, H);
    else if (!L.full && t == "linear_attn.in_proj_a.weight") rc = matrix(L.mix, q->lin_a, q->VH, H);
    else if (!L.full && t == "linear_attn.in_proj_b.weight") rc = matrix(L.mix, q->lin_b, q->VH, H);
    else if (!L.full && t == "linear_attn.out_proj.weight") rc = matrix(L.out, 0, H, q->vals);
    else if (!L.full && t == "linear_attn.conv1d.weight") rc = vector(L.conv, (size_t)q->C * q->K);
    else if (!L.full && t == "linear_attn.A_log") rc = vector(L.a_log, q->VH);
    else if (!L.full && t == "linear_attn.dt_bias") rc = vector(L.dt, q->VH);
    else if (!L.full && t == "linear_attn.norm.weight") rc = vector(L.norm, q->VD);
    else return fail(ctx, COHX_UNSUPPORTED, "unexpected Qwen3.5 tensor " + n);
  }
  if (!rc) q->uploaded.insert(n);
  return rc;
}

int q35_finalize(cohx_ctx *ctx) {
  Q35Model *q = ctx->q35;
  if (q->uploaded.size() != q->expected)
    return fail(ctx, COHX_UNSUPPORTED,
                "missing Qwen3.5 tensors: " + std::to_string(q->uploaded.size()) + " of " +
                    std::to_string(q->expected));
  ctx->finalized = true;
  ctx->matrix_bytes = q->matrix_bytes;
  return COHX_OK;
}

// A fresh slot starts from zero state (kernels.rs:72-80,139-150).
int q35_seq_reset(cohx_ctx *ctx, uint32_t seq) {
  Q35Model *q = ctx->q35;
  Q35_TRY(hipMemsetAsync(q->conv_state + seq * q->conv_seq, 0, q->conv_seq * 4, ctx->stream));
  Q35_TRY(hipMemsetAsync(q->delta_state + seq * q->delta_seq, 0, q->delta_seq * 4, ctx->stream));
  return COHX_OK;
}

// Snapshot copy (execution.rs:117-133 Snapshot::capture/restore): recurrent
// state cannot be shared, so a fork copies everything at the source length.
int q35_seq_copy(cohx_ctx *ctx, uint32_t src, uint32_t dst, uint32_t rows) {
  Q35Model *q = ctx->q35;
  for (int l = 0; l < q->n_full; l++) {
    const size_t off = l * q->kv_layer, n = (size_t)rows * q->kvw * 4;
    Q35_TRY(hipMemcpyAsync(q->kc + dst * q->kv_seq + off, q->kc + src * q->kv_seq + off, n,
                           hipMemcpyDeviceToDevice, ctx->stream));
    Q35_TRY(hipMemcpyAsync(q->vc + dst * q->kv_seq + off, q->vc + src * q->kv_seq + off, n,
                           hipMemcpyDeviceToDevice, ctx->stream));
  }
  Q35_TRY(hipMemcpyAsync(q->conv_state + dst * q->conv_seq, q->conv_state + src * q->conv_seq,
                         q->conv_seq * 4, hipMemcpyDeviceToDevice, ctx->stream));
  Q35_TRY(hipMemcpyAsync(q->delta_state + dst * q->delta_seq, q->delta_state + src * q->delta_seq,
                         q->delta_seq * 4, hipMemcpyDeviceToDevice, ctx->stream));
  Q35_TRY(hipStreamSynchronize(ctx->stream));
  return COHX_OK;
}

// which: 0/1 K/V rows [0, length) of a full-attention layer, 2 the conv ring
// [channels][kernel] (slot order), 3 the delta memory [heads][key][value].
int q35_read_state(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int which, float *out) {
  Q35Model *q = ctx->q35;
  const Q35Layer &L = q->layers[layer];
  const uint32_t len = ctx->seqs[seq].length;
  size_t n = 0;
  const float *src = nullptr;
  if (which == 0 || which == 1) {
    if (!L.full) return fail(ctx, COHX_INVALID_REQUEST, "not a full-attention layer");
    src = (which ? q->vc : q->kc) + seq * q->kv_seq + L.slot * q->kv_layer;
    n = (size_t)len * q->kvw;
  } else if (which == 2 || which == 3) {
    if (L.full) return fail(ctx, COHX_INVALID_REQUEST, "not a linear-attention layer");
    if (which == 2) {
      src = q->conv_state + seq * q->conv_seq + (size_t)L.slot * q->C * q->K;
      n = (size_t)q->C * q->K;
    } else {
      src = q->delta_state + seq * q->delta_seq + (size_t)L.slot * q->VH * q->KD * q->VD;
      n = (size_t)q->VH * q->KD * q->VD;
    }
  } else {
    return fail(ctx, COHX_INVALID_REQUEST, "unknown state kind");
  }
  Q35_TRY(hipStreamSynchronize(ctx->stream));
  Q35_TRY(hipMemcpy(out, src, n * 4, hipMemcpyDeviceToHost));
  return COHX_OK;
}

// Graph::forward_batch over a ragged batch (execution.rs:257-608): a lane may
// carry several consecutive tokens (a prompt chunk); the linears run over all
// packed rows, and the recurrences walk each lane's tokens in order, so the
// result equals stepping the tokens one at a time.
int q35_step(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out, const cohx_step_hooks *hooks) {
  const auto t_start = std::chrono::steady_clock::now();
  Q35Model *q = ctx->q35;
  const cohx_model_desc &d = ctx->desc;
  if (!batch || batch->n_lanes == 0 || batch->n_lanes > d.max_lanes || !batch->lanes)
    return fail(ctx, COHX_INVALID_REQUEST, "batch width must be in 1..=" + std::to_string(d.max_lanes));
  if (!ctx->finalized) return fail(ctx, COHX_INVALID_REQUEST, "model tensors not finalized");
  if (!out || !out->lanes) return fail(ctx, COHX_INVALID_REQUEST, "missing output lanes");
  for (uint32_t i = 0; i < batch->n_lanes; i++)
    for (uint32_t j = i + 1; j < batch->n_lanes; j++)
      if (batch->lanes[i].seq == batch->lanes[j].seq)
        return fail(ctx, COHX_INVALID_REQUEST, "a sequence appears twice in one batch");
  const int NLmax = q->max_lanes, Rmax = q->max_rows;
  uint32_t *lane_first = q->h_tables, *lane_n = lane_first + NLmax, *lane_seq = lane_n + NLmax,
           *lane_start = lane_seq + NLmax, *lane_last = lane_start + NLmax;
  uint32_t *row_lane = lane_last + NLmax, *row_pos = row_lane + Rmax, *row_seq = row_pos + Rmax,
           *tokens = row_seq + Rmax;
  std::vector<int> included, head_of;  // head_of: row of the lane in the head pass, or -1
  uint32_t R = 0, n_head = 0;
  for (uint32_t i = 0; i < batch->n_lanes; i++) {
    const cohx_lane &ln = batch->lanes[i];
    int32_t st = COHX_OK;
    const bool live = ln.seq < ctx->seqs.size() && ctx->seqs[ln.seq].live;
    const uint32_t len = live ? ctx->seqs[ln.seq].length : 0;
    const uint32_t start = (live && ln.start_position == COHX_AT_END) ? len : ln.start_position;
    if (hooks && hooks->cancel && hooks->cancel[i]) {
      st = COHX_CANCELLED;  // Cancellation::check before the forward
    } else if (!live || ln.n_tokens == 0 || !ln.tokens || start != len) {
      st = COHX_INVALID_REQUEST;
    } else {
      for (uint32_t j = 0; j < ln.n_tokens; j++)
        if (ln.tokens[j] >= d.vocabulary) st = COHX_INVALID_REQUEST;
      if (!st && (uint64_t)start + ln.n_tokens > ctx->seqs[ln.seq].capacity) st = COHX_INVALID_REQUEST;
      if (!st && R + ln.n_tokens > d.max_rows) st = COHX_RESOURCE;
    }
    out->lanes[i].status = st;
    out->lanes[i].argmax = COHX_NO_TOKEN;
    if (st) continue;
    const uint32_t k = (uint32_t)included.size();
    lane_first[k] = R;
    lane_n[k] = ln.n_tokens;
    lane_seq[k] = ln.seq;
    lane_start[k] = start;
    if (ln.want_logits != COHX_SKIP_HEAD) {
      lane_last[n_head] = R + ln.n_tokens - 1;
      head_of.push_back((int)n_head++);
    } else {
      head_of.push_back(-1);
    }
    for (uint32_t j = 0; j < ln.n_tokens; j++) {
      row_lane[R + j] = k;
      row_pos[R + j] = start + j;
      row_seq[R + j] = ln.seq;
      tokens[R + j] = ln.tokens[j];
    }
    R += ln.n_tokens;
    included.push_back((int)i);
  }
  out->rows = R;
  out->width = 0;
  out->matrix_bytes = 0;
  out->kv_bytes = 0;
  if (included.empty()) return COHX_OK;
  const int NL = (int)included.size();
  uint32_t max_lane_tokens = 0;
  for (int k = 0; k < NL; k++) max_lane_tokens = std::max(max_lane_tokens, lane_n[k]);
  Q35_TRY(hipSetDevice(ctx->device));
  hipStream_t s = ctx->stream;
  uint32_t *dt = q->tables;
  Q35_TRY(hipMemcpyAsync(dt, q->h_tables, (5 * NLmax + 4 * Rmax) * 4, hipMemcpyHostToDevice, s));
  const Q35Lanes L{dt, dt + NLmax, dt + 2 * NLmax, dt + 3 * NLmax};
  const uint32_t *d_last = dt + 4 * NLmax;
  const Q35Rows Rw{dt + 5 * NLmax, dt + 5 * NLmax + Rmax, dt + 5 * NLmax + 2 * Rmax};
  const uint32_t *d_tokens = dt + 5 * NLmax + 3 * Rmax;
  launch_fill_u32(s, q->row_err, R, 0);
  const int H = q->H;
  const float eps = q->d.epsilon;
  // packed-prefill regime: a step of kQ35PrefillRows+ rows runs its linears
  // on the matrix-core GEMM over the tiled matrices (the recurrences,
  // attention, norms and the head stay exact)
  const bool regime = q->mfma && R >= kQ35PrefillRows;
  // One linear layer, out (=, +=) x . W^T: in the regime the f32 rows enter
  // as their bfloat16 hi and lo parts, both multiplied into the same f32
  // sums (the residual taken in by the accumulate epilogue, non-finite
  // outputs flagged per row); else (or for K not a multiple of 64) the exact
  // matvec.
  auto linear = [&](int epi, const uint16_t *w, int rows_w, int valid, int K, const float *x, int ldx, float *o,
                    int ldo) -> int {
    if (regime && K % 64 == 0) {
      q35_split_bf16(s, (int)R, K, x, ldx, q->a_hi, q->a_lo);
      q35_gemm_split(s, epi == kQ35Residual, w, valid, K, q->a_hi, q->a_lo, (int)R, o, ldo, q->row_err);
      return COHX_OK;
    }
    q35_matvec(s, epi, w, rows_w, valid, K, x, ldx, (int)R, o, ldo, nullptr, q->row_err, nullptr);
    return COHX_OK;
  };
  int lrc = COHX_OK;
  q35_embed(s, (int)R, q->embed, d_tokens, H, q->x);
  for (const Q35Layer &Ly : q->layers) {
    q35_norm(s, (int)R, q->x, H, nullptr, Ly.input_norm, H, eps, 1, q->nrm, H, q->row_err, nullptr);
    if (!Ly.full) {
      if ((lrc = linear(kQ35Store, Ly.mix, q->lin_rows, q->lin_rows, H, q->nrm, H, q->mix_out,
                        q->ld_mix)))
        return lrc;
      // one launch for the mixer when every lane is a decode row or a short
      // chunk; long prompt chunks gain from forming conv and gates for all
      // rows in parallel
      if (q35_linear_fused(q->K, q->KH, q->VH) && !q->split_linear && max_lane_tokens <= 4) {
        q35_linear(s, NL, L, q->mix_out, q->ld_mix, q->keys, q->lin_z, q->lin_a, q->lin_b, Ly.conv,
                   q->K, q->conv_state + (size_t)Ly.slot * q->C * q->K, q->conv_seq, Ly.a_log,
                   Ly.dt, Ly.norm, q->KH, q->VH, q->KD, q->VD, eps,
                   q->delta_state + (size_t)Ly.slot * q->VH * q->KD * q->VD, q->delta_seq, q->tgt,
                   q->ld_att, q->row_err);
      } else {
        q35_conv(s, NL, L, q->mix_out, q->ld_mix, Ly.conv, q->C, q->K,
                 q->conv_state + (size_t)Ly.slot * q->C * q->K, q->conv_seq, q->cv, q->C,
                 q->row_err);
        q35_delta(s, (int)R, NL, L, q->cv, q->C, q->keys, q->mix_out, q->ld_mix, q->lin_z,
                  q->lin_a, q->lin_b, Ly.a_log, Ly.dt, Ly.norm, q->KH, q->VH, q->KD, q->VD, eps,
                  q->delta_state + (size_t)Ly.slot * q->VH * q->KD * q->VD, q->delta_seq,
                  q->gates, q->att, q->tgt, q->ld_att, q->row_err);
      }
      if ((lrc = linear(kQ35Residual, Ly.out, q->h_rows, H, q->vals, q->tgt, q->ld_att, q->x, H)))
        return lrc;
    } else {
      if ((lrc = linear(kQ35Store, Ly.mix, q->full_rows, q->full_rows, H, q->nrm, H, q->mix_out,
                        q->ld_mix)))
        return lrc;
      q35_qk(s, (int)R, Rw, q->mix_out, q->ld_mix, q->full_k, q->full_v, Ly.q_norm, Ly.k_norm,
             q->NH, q->NKV, q->D, q->ROT, eps, q->rope, q->q, q->z, q->qw,
             q->kc + Ly.slot * q->kv_layer, q->vc + Ly.slot * q->kv_layer, q->kv_seq, q->row_err);
      q35_attention(s, (int)R, Rw, q->q, q->z, q->qw, q->kc + Ly.slot * q->kv_layer,
                    q->vc + Ly.slot * q->kv_layer, q->kv_seq, q->NH, q->NKV, q->D,
                    (int)d.max_context, q->scores, q->att, q->ld_att);
      if ((lrc = linear(kQ35Residual, Ly.out, q->h_rows, H, q->qw, q->att, q->ld_att, q->x, H)))
        return lrc;
    }
    q35_norm(s, (int)R, q->x, H, nullptr, Ly.post_norm, H, eps, 1, q->nrm, H, q->row_err, nullptr);
    if (regime || !q35_matvec_swiglu(s, Ly.gu, q->gu_up, q->F, H, q->nrm, H, (int)R, q->hb, q->F,
                                     q->row_err)) {
      if ((lrc = linear(kQ35Store, Ly.gu, q->gu_rows, q->gu_rows, H, q->nrm, H, q->gu_out,
                        q->gu_rows)))
        return lrc;
      q35_swiglu(s, (int)R, q->gu_out, q->gu_rows, q->F, q->gu_up, q->hb, q->F);
    }
    if ((lrc = linear(kQ35Residual, Ly.down, q->h_rows, H, q->F, q->hb, q->F, q->x, H)))
      return lrc;
  }
  // final norm and head over the last row of each lane that needs them
  // (execution.rs:586-594); d_last lists those rows in head order
  bool any_logits = false;
  for (int k = 0; k < NL; k++) any_logits |= batch->lanes[included[k]].want_logits == 1u;
  const int NH = (int)n_head;
  if (NH) {
    q35_norm(s, NH, q->x, H, d_last, q->final_norm, H, eps, 1, q->fin, H, q->row_err, d_last);
    q35_matvec(s, kQ35Argmax, q->head, q->head_rows, q->V, H, q->fin, H, NH,
               any_logits ? q->logits : nullptr, q->V, q->part, q->row_err, d_last);
    launch_argmax_reduce(s, NH, q->part, q35_matvec_blocks(q->head_rows), q->argmax);
  }
  Q35_TRY(hipGetLastError());
  if (NH) Q35_TRY(hipMemcpyAsync(q->h_argmax, q->argmax, NH * 8, hipMemcpyDeviceToHost, s));
  Q35_TRY(hipMemcpyAsync(q->h_row_err, q->row_err, R * 4, hipMemcpyDeviceToHost, s));
  for (int k = 0; k < NL; k++) {
    const cohx_lane &ln = batch->lanes[included[k]];
    float *dst = out->lanes[included[k]].logits;
    if (ln.want_logits == 1u && dst && head_of[k] >= 0)
      Q35_TRY(hipMemcpyAsync(dst, q->logits + (size_t)head_of[k] * q->V, q->V * 4,
                             hipMemcpyDeviceToHost, s));
  }
  // the recurrent state was updated in place and cannot be rewound, so the
  // completed step stands; a stop request from the yield hook (or a lane's
  // cancellation) takes effect at the next step
  const int wrc = wait_step(ctx, s, hooks);
  if (wrc && wrc != COHX_CANCELLED) return wrc;
  uint32_t width = 0;
  uint64_t kv_rows = 0;
  for (int k = 0; k < NL; k++) {
    const int i = included[k];
    const cohx_lane &ln = batch->lanes[i];
    uint32_t bits = 0;
    for (uint32_t j = 0; j < ln.n_tokens; j++) bits |= q->h_row_err[lane_first[k] + j];
    cohx_lane_out &o = out->lanes[i];
    o.argmax = head_of[k] < 0 ? COHX_NO_TOKEN
                              : 0xffffffffu - (uint32_t)(q->h_argmax[head_of[k]] & 0xffffffffull);
    if (bits & kErrRequest)
      o.status = COHX_INVALID_REQUEST;
    else if (bits)
      o.status = COHX_INVALID_GGUF;
    else {
      ctx->seqs[ln.seq].length += ln.n_tokens;
      width++;
    }
    for (uint32_t j = 0; j < ln.n_tokens; j++) kv_rows += lane_start[k] + j + 1;
  }
  out->width = width;
  out->matrix_bytes = q->matrix_bytes;
  out->kv_bytes = kv_rows * (uint64_t)q->kvw * 4 * 2 * q->n_full +
                  (uint64_t)NL * (q->conv_seq + 2 * q->delta_seq) * 4;
  out->elapsed_ns = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                        std::chrono::steady_clock::now() - t_start)
                        .count();
  return COHX_OK;
}

}  // namespace cohx
