/*
 * CPU ORACLE — test infrastructure only (never linked by the product).
 *
 * Qwen2 graph restated from the reference Rust sources:
 *   crates/coheryn-engine/src/inference/batch.rs:117-273   Model::forward_batch
 *   crates/coheryn-engine/src/inference.rs:349-365         Model::vector (row decode)
 *   crates/coheryn-engine/src/inference.rs:403-561         Model::forward_row
 *   crates/coheryn-engine/src/inference.rs:983-1043        Scratch / Kv::append
 *   crates/coheryn-engine/src/tensor.rs:302-436            matmul_batch_cooperative
 *                                                          (per-lane operand rounding /
 *                                                          activation quantization, then
 *                                                          one dot per (lane,row))
 * Rows of a matrix are split over OpenMP threads; every (lane,row) dot is an
 * independent sequential reduction, so the thread count never changes a bit
 * (the reference's rayon row split has the same property, docs/QUANTIZATION.md:8).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

struct orc_model {
  orc_config c;
  orc_tensor g[3];
  orc_tensor *layers; /* [layers][ORC_LAYER_TENSORS] */
  int threads;
  float *f16_lut; /* 65536 entries: exact binary16 -> f32 */
};

struct orc_session {
  uint32_t position, context;
  float *keys, *values; /* [layers][context][kv_dim] */
  float *x, *norm_weight, *normalized, *q, *k, *v, *bias, *attention, *projection, *gate, *up,
      *logits;
};

static const orc_tensor *layer_tensor(const orc_model *m, uint32_t layer, int slot) {
  return &m->layers[(size_t)layer * ORC_LAYER_TENSORS + slot];
}

static int check_shape(const orc_tensor *t, uint64_t ne0, uint64_t ne1) {
  if (!t->data || t->ne0 != ne0 || t->ne1 != ne1) return ORC_INVALID_GGUF;
  size_t rb;
  if (orc_row_bytes(t->dtype, (size_t)ne0, &rb)) return ORC_UNSUPPORTED;
  if ((uint64_t)rb * ne1 != t->bytes) return ORC_INVALID_GGUF;
  return ORC_OK;
}

/* compat.rs:161-221 graph(): exact tensor set and shapes */
int orc_model_new(const orc_config *c, const orc_tensor *globals, const orc_tensor *layers,
                  int threads, orc_model **out) {
  if (!c->layers || !c->hidden || !c->heads || !c->kv_heads || c->hidden % c->heads ||
      c->heads % c->kv_heads || c->head_dim != c->hidden / c->heads || c->head_dim % 2)
    return ORC_INVALID_GGUF;
  uint32_t kvd = c->kv_heads * c->head_dim;
  int rc = check_shape(&globals[0], c->hidden, c->vocabulary);
  if (!rc) rc = check_shape(&globals[1], c->hidden, 1);
  if (!rc && globals[2].data) rc = check_shape(&globals[2], c->hidden, c->vocabulary);
  for (uint32_t l = 0; l < c->layers && !rc; l++) {
    const orc_tensor *t = layers + (size_t)l * ORC_LAYER_TENSORS;
    rc = check_shape(&t[ORC_ATTN_NORM], c->hidden, 1);
    if (!rc) rc = check_shape(&t[ORC_FFN_NORM], c->hidden, 1);
    if (!rc) rc = check_shape(&t[ORC_Q], c->hidden, c->hidden);
    if (!rc) rc = check_shape(&t[ORC_K], c->hidden, kvd);
    if (!rc) rc = check_shape(&t[ORC_V], c->hidden, kvd);
    if (!rc) rc = check_shape(&t[ORC_QB], c->hidden, 1);
    if (!rc) rc = check_shape(&t[ORC_KB], kvd, 1);
    if (!rc) rc = check_shape(&t[ORC_VB], kvd, 1);
    if (!rc) rc = check_shape(&t[ORC_O], c->hidden, c->hidden);
    if (!rc) rc = check_shape(&t[ORC_GATE], c->hidden, c->intermediate);
    if (!rc) rc = check_shape(&t[ORC_UP], c->hidden, c->intermediate);
    if (!rc) rc = check_shape(&t[ORC_DOWN], c->intermediate, c->hidden);
  }
  if (rc) return rc;
  orc_model *m = (orc_model *)calloc(1, sizeof(*m));
  if (!m) return ORC_RESOURCE;
  m->c = *c;
  memcpy(m->g, globals, sizeof(m->g));
  m->layers = (orc_tensor *)malloc(sizeof(orc_tensor) * ORC_LAYER_TENSORS * c->layers);
  m->f16_lut = (float *)malloc(sizeof(float) * 65536);
  if (!m->layers || !m->f16_lut) {
    orc_model_free(m);
    return ORC_RESOURCE;
  }
  memcpy(m->layers, layers, sizeof(orc_tensor) * ORC_LAYER_TENSORS * c->layers);
  for (uint32_t i = 0; i < 65536; i++) m->f16_lut[i] = orc_f16_to_f32((uint16_t)i);
  m->threads = threads > 0 ? threads : 1;
  *out = m;
  return ORC_OK;
}

void orc_model_free(orc_model *m) {
  if (!m) return;
  free(m->layers);
  free(m->f16_lut);
  free(m);
}

int orc_session_new(const orc_model *m, uint32_t context, orc_session **out) {
  if (context == 0 || context > m->c.context) return ORC_INVALID_REQUEST;
  const orc_config *c = &m->c;
  size_t kvd = (size_t)c->kv_heads * c->head_dim;
  orc_session *s = (orc_session *)calloc(1, sizeof(*s));
  if (!s) return ORC_RESOURCE;
  s->context = context;
  s->keys = (float *)calloc((size_t)c->layers * context * kvd, sizeof(float));
  s->values = (float *)calloc((size_t)c->layers * context * kvd, sizeof(float));
  s->x = (float *)calloc(c->hidden, 4);
  s->norm_weight = (float *)calloc(c->hidden, 4);
  s->normalized = (float *)calloc(c->hidden, 4);
  s->q = (float *)calloc(c->hidden, 4);
  s->k = (float *)calloc(kvd, 4);
  s->v = (float *)calloc(kvd, 4);
  s->bias = (float *)calloc(c->hidden, 4);
  s->attention = (float *)calloc(c->hidden, 4);
  s->projection = (float *)calloc(c->hidden, 4);
  s->gate = (float *)calloc(c->intermediate, 4);
  s->up = (float *)calloc(c->intermediate, 4);
  s->logits = (float *)calloc(c->vocabulary, 4);
  if (!s->keys || !s->values || !s->x || !s->logits || !s->gate || !s->up) {
    orc_session_free(s);
    return ORC_RESOURCE;
  }
  *out = s;
  return ORC_OK;
}

void orc_session_free(orc_session *s) {
  if (!s) return;
  free(s->keys);
  free(s->values);
  free(s->x);
  free(s->norm_weight);
  free(s->normalized);
  free(s->q);
  free(s->k);
  free(s->v);
  free(s->bias);
  free(s->attention);
  free(s->projection);
  free(s->gate);
  free(s->up);
  free(s->logits);
  free(s);
}

uint32_t orc_session_position(const orc_session *s) { return s->position; }
const float *orc_session_logits(const orc_session *s) { return s->logits; }

int orc_session_truncate(orc_session *s, uint32_t rows) {
  if (rows > s->position) return ORC_INVALID_REQUEST;
  s->position = rows;
  return ORC_OK;
}

/* Model::vector -> tensor::read_row (tensor.rs:81-105) */
static int read_row(const orc_tensor *t, uint64_t row, float *out) {
  size_t rb;
  int rc = orc_row_bytes(t->dtype, (size_t)t->ne0, &rb);
  if (rc) return rc;
  if ((row + 1) * rb > t->bytes) return ORC_INVALID_GGUF;
  return orc_decode(t->data + row * rb, rb, t->dtype, out, (size_t)t->ne0);
}

/* One lane's operand for a matrix: F16 rounding or packed activation blocks
 * (tensor.rs:325-345). */
typedef struct {
  const float *input;
  float *output;
  float *operand;   /* F16-rounded copy */
  uint8_t *packed;  /* Q8_0 / Q8_K blocks */
  uint32_t kind;
  int32_t *error;
} lane_vec;

/* tensor::matmul_batch_cooperative numerics (tensor.rs:302-436): per-lane
 * preparation, then every live lane's dot for every row. */
static void matrix_batch(const orc_model *m, const orc_tensor *t, lane_vec *lanes, size_t n) {
  size_t width = (size_t)t->ne0, rows = (size_t)t->ne1, rb;
  if (orc_row_bytes(t->dtype, width, &rb)) {
    for (size_t i = 0; i < n; i++)
      if (!*lanes[i].error) *lanes[i].error = ORC_UNSUPPORTED;
    return;
  }
  int packed = t->dtype == 2 || t->dtype == 6 || t->dtype == 8 || t->dtype == 12 || t->dtype == 14;
  for (size_t i = 0; i < n; i++) {
    if (*lanes[i].error) continue;
    int rc = ORC_OK;
    if (t->dtype == 1) {
      rc = orc_round_f16(lanes[i].input, lanes[i].operand, width);
    } else if (packed) {
      size_t used;
      rc = orc_prepare(lanes[i].input, width, t->dtype, lanes[i].packed, (width / 32 + 1) * 292,
                       &used, &lanes[i].kind);
    }
    if (rc) *lanes[i].error = rc;
  }
  long nrows = (long)rows;
#pragma omp parallel for schedule(static) num_threads(m->threads)
  for (long r = 0; r < nrows; r++) {
    const uint8_t *row = t->data + (size_t)r * rb;
    float *wrow = NULL;
    if (!packed) {
      wrow = (float *)malloc(width * sizeof(float));
      if (t->dtype == 1) {
        for (size_t k = 0; k < width; k++)
          wrow[k] = m->f16_lut[(uint16_t)(row[2 * k] | (row[2 * k + 1] << 8))];
      } else {
        orc_decode(row, rb, t->dtype, wrow, width);
      }
    }
    for (size_t i = 0; i < n; i++) {
      if (*lanes[i].error) continue;
      float value;
      if (packed) {
        if (orc_qdot(row, rb, t->dtype, lanes[i].packed, lanes[i].kind, width, &value)) {
#pragma omp atomic write
          *lanes[i].error = ORC_INVALID_GGUF;
          continue;
        }
      } else {
        const float *src = t->dtype == 1 ? lanes[i].operand : lanes[i].input;
        value = orc_dot_f32(wrow, src, width);
      }
      if (!isfinite(value)) {
#pragma omp atomic write
        *lanes[i].error = ORC_INVALID_GGUF;
        continue;
      }
      lanes[i].output[r] = value;
    }
    free(wrow);
  }
}

typedef struct {
  float *operand;
  uint8_t *packed;
} lane_work;

/* batch.rs:117-273 Model::forward_batch */
static int forward_batch_impl(const orc_model *m, orc_session **ss, const uint32_t *tokens,
                              size_t n, int32_t *errors, float *trace) {
  const orc_config *c = &m->c;
  size_t kvd = (size_t)c->kv_heads * c->head_dim;
  size_t maxw = c->intermediate > c->hidden ? c->intermediate : c->hidden;
  lane_work *work = (lane_work *)calloc(n, sizeof(lane_work));
  lane_vec *lv = (lane_vec *)calloc(n, sizeof(lane_vec));
  if (!work || !lv) {
    free(work);
    free(lv);
    return ORC_RESOURCE;
  }
  for (size_t i = 0; i < n; i++) {
    work[i].operand = (float *)malloc(maxw * sizeof(float));
    work[i].packed = (uint8_t *)malloc((maxw / 32 + 1) * 292);
  }
  /* embedding (batch.rs:119-132) */
  for (size_t i = 0; i < n; i++) {
    if (errors[i]) continue;
    if (tokens[i] >= c->vocabulary) {
      errors[i] = ORC_INVALID_REQUEST;
      continue;
    }
    if (ss[i]->position >= ss[i]->context) {
      errors[i] = ORC_RESOURCE;
      continue;
    }
    int rc = read_row(&m->g[0], tokens[i], ss[i]->x);
    if (rc) errors[i] = rc;
  }
#define MATRIX(tensor, IN, OUT)                                  \
  do {                                                           \
    for (size_t i = 0; i < n; i++) {                             \
      lv[i].input = ss[i]->IN;                                   \
      lv[i].output = ss[i]->OUT;                                 \
      lv[i].operand = work[i].operand;                           \
      lv[i].packed = work[i].packed;                             \
      lv[i].error = &errors[i];                                  \
    }                                                            \
    matrix_batch(m, (tensor), lv, n);                            \
  } while (0)
  for (uint32_t l = 0; l < c->layers; l++) {
    for (size_t i = 0; i < n; i++) {
      if (errors[i]) continue;
      orc_session *s = ss[i];
      int rc = read_row(layer_tensor(m, l, ORC_ATTN_NORM), 0, s->norm_weight);
      if (rc) {
        errors[i] = rc;
        continue;
      }
      orc_rms_norm(s->x, s->norm_weight, c->norm_epsilon, s->normalized, c->hidden);
    }
    MATRIX(layer_tensor(m, l, ORC_Q), normalized, q);
    MATRIX(layer_tensor(m, l, ORC_K), normalized, k);
    MATRIX(layer_tensor(m, l, ORC_V), normalized, v);
    for (size_t i = 0; i < n; i++) {
      if (errors[i]) continue;
      orc_session *s = ss[i];
      int rc = ORC_OK;
      float *outs[3] = {s->q, s->k, s->v};
      size_t lens[3] = {c->hidden, kvd, kvd};
      for (int j = 0; j < 3 && !rc; j++) {
        rc = read_row(layer_tensor(m, l, ORC_QB + j), 0, s->bias);
        if (!rc)
          for (size_t e = 0; e < lens[j]; e++) outs[j][e] += s->bias[e];
      }
      if (rc) {
        errors[i] = rc;
        continue;
      }
      orc_rope(s->q, c->hidden, c->head_dim, s->position, c->rope_base);
      orc_rope(s->k, kvd, c->head_dim, s->position, c->rope_base);
      if (s->position >= s->context) {
        errors[i] = ORC_RESOURCE;
        continue;
      }
      size_t base = ((size_t)l * s->context + s->position) * kvd;
      memcpy(s->keys + base, s->k, kvd * 4);
      memcpy(s->values + base, s->v, kvd * 4);
      rc = orc_attention_rows(s->q, c->hidden, s->keys + (size_t)l * s->context * kvd,
                              s->values + (size_t)l * s->context * kvd, s->position + 1,
                              c->kv_heads, c->head_dim, s->attention);
      if (rc) errors[i] = rc;
    }
    MATRIX(layer_tensor(m, l, ORC_O), attention, projection);
    for (size_t i = 0; i < n; i++) {
      if (errors[i]) continue;
      orc_session *s = ss[i];
      for (size_t e = 0; e < c->hidden; e++) s->x[e] += s->projection[e];
      int rc = read_row(layer_tensor(m, l, ORC_FFN_NORM), 0, s->norm_weight);
      if (rc) {
        errors[i] = rc;
        continue;
      }
      orc_rms_norm(s->x, s->norm_weight, c->norm_epsilon, s->normalized, c->hidden);
    }
    MATRIX(layer_tensor(m, l, ORC_GATE), normalized, gate);
    MATRIX(layer_tensor(m, l, ORC_UP), normalized, up);
    for (size_t i = 0; i < n; i++)
      if (!errors[i]) orc_swiglu(ss[i]->gate, ss[i]->up, c->intermediate);
    MATRIX(layer_tensor(m, l, ORC_DOWN), gate, projection);
    for (size_t i = 0; i < n; i++) {
      if (errors[i]) continue;
      for (size_t e = 0; e < c->hidden; e++) ss[i]->x[e] += ss[i]->projection[e];
      if (trace) memcpy(trace + ((size_t)i * c->layers + l) * c->hidden, ss[i]->x, c->hidden * 4);
    }
  }
  for (size_t i = 0; i < n; i++) {
    if (errors[i]) continue;
    orc_session *s = ss[i];
    int rc = read_row(&m->g[1], 0, s->norm_weight);
    if (rc) {
      errors[i] = rc;
      continue;
    }
    orc_rms_norm(s->x, s->norm_weight, c->norm_epsilon, s->normalized, c->hidden);
  }
  MATRIX(m->g[2].data ? &m->g[2] : &m->g[0], normalized, logits);
  for (size_t i = 0; i < n; i++)
    if (!errors[i]) ss[i]->position += 1;
#undef MATRIX
  for (size_t i = 0; i < n; i++) {
    free(work[i].operand);
    free(work[i].packed);
  }
  free(work);
  free(lv);
  return ORC_OK;
}

int orc_forward_batch(const orc_model *m, orc_session **ss, const uint32_t *tokens, size_t n,
                      int32_t *errors) {
  return forward_batch_impl(m, ss, tokens, n, errors, NULL);
}

int orc_forward_batch_trace(const orc_model *m, orc_session **ss, const uint32_t *tokens,
                            size_t n, int32_t *errors, float *trace) {
  return forward_batch_impl(m, ss, tokens, n, errors, trace);
}

/* inference.rs:403-561 forward_row (one lane).  The batched graph computes
 * the final layer's attention/FFN for prompt rows too; the K/V rows it appends
 * and the position it advances are the same, and a prompt row's logits are
 * never sampled (generation.rs:325), so one restatement serves both. */
int orc_forward_row(const orc_model *m, orc_session *s, uint32_t token, int logits) {
  int32_t err = 0;
  (void)logits;
  orc_forward_batch(m, &s, &token, 1, &err);
  return err;
}

int orc_session_kv(const orc_model *m, const orc_session *s, uint32_t layer, int values,
                   float *out) {
  if (layer >= m->c.layers) return ORC_INVALID_REQUEST;
  size_t kvd = (size_t)m->c.kv_heads * m->c.head_dim;
  const float *src = (values ? s->values : s->keys) + (size_t)layer * s->context * kvd;
  memcpy(out, src, (size_t)s->position * kvd * sizeof(float));
  return ORC_OK;
}

/* Seeded synthetic K/V rows (the benchmark's pre-filled contexts); the GPU
 * library's fill kernel uses the same integer hash, so both sides hold
 * bit-identical caches. */
static uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

float orc_synthetic_kv(uint64_t seed, uint32_t stream, uint32_t layer, uint32_t which,
                       uint32_t position, uint32_t element) {
  uint64_t h = mix64(seed ^ mix64(((uint64_t)stream << 32) | ((uint64_t)layer << 1) | which) ^
                     (((uint64_t)position << 16) | element));
  return (float)((int32_t)(h >> 40) - (1 << 23)) * 0x1p-23f;
}

int orc_session_fill_synthetic(const orc_model *m, orc_session *s, uint32_t rows, uint64_t seed,
                               uint32_t stream) {
  if (rows > s->context || rows < s->position) return ORC_RESOURCE;
  size_t kvd = (size_t)m->c.kv_heads * m->c.head_dim;
  for (uint32_t l = 0; l < m->c.layers; l++)
    for (uint32_t p = s->position; p < rows; p++)
      for (uint32_t e = 0; e < kvd; e++) {
        size_t at = ((size_t)l * s->context + p) * kvd + e;
        s->keys[at] = orc_synthetic_kv(seed, stream, l, 0, p, e);
        s->values[at] = orc_synthetic_kv(seed, stream, l, 1, p, e);
      }
  s->position = rows;
  return ORC_OK;
}

/* Packing contract of the GPU step: lanes' rows are laid out lane after lane;
 * row r of lane i sits at position start[i] + (r - cu[i]) and in KV slot
 * pages[i][pos / page_size] * page_size + pos % page_size. */
int orc_pack(size_t n, const uint32_t *n_tokens, const uint32_t *start, const int32_t *pages,
             uint32_t max_pages, uint32_t page_size, uint32_t *cu, uint32_t *row_position,
             int64_t *row_slot, uint32_t *row_lane) {
  cu[0] = 0;
  for (size_t i = 0; i < n; i++) {
    if (n_tokens[i] == 0) return ORC_INVALID_REQUEST;
    cu[i + 1] = cu[i] + n_tokens[i];
  }
  for (size_t i = 0; i < n; i++) {
    for (uint32_t j = 0; j < n_tokens[i]; j++) {
      uint32_t r = cu[i] + j, pos = start[i] + j, page = pos / page_size;
      if (page >= max_pages) return ORC_RESOURCE;
      int32_t phys = pages[i * max_pages + page];
      if (phys < 0) return ORC_RESOURCE;
      row_position[r] = pos;
      row_slot[r] = (int64_t)phys * page_size + pos % page_size;
      row_lane[r] = (uint32_t)i;
    }
  }
  return ORC_OK;
}
