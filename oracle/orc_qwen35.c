/*
 * CPU ORACLE — test infrastructure only (see orc.h).
 *
 * Restatement of the Coheryn engine's Qwen3.5 hybrid text step
 * (crates/coheryn-engine/src/qwen35/execution.rs:257-608 Graph::forward_batch,
 * qwen35/kernels.rs:11-269) with Rust's float semantics: no contraction, f64
 * sums in element order (Iterator::sum starts at -0.0; the delta rule's
 * explicit accumulators start at +0.0), glibc expf / log1pf / powf / sinf /
 * cosf.  One token per lane per call, as the reference steps lanes.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "orc.h"

static int all_finite(const float *v, size_t n) {
  for (size_t i = 0; i < n; i++)
    if (!isfinite(v[i])) return 0;
  return 1;
}

/* kernels.rs:11-17 */
float orc_q35_sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
  const float e = expf(x);
  return e / (1.0f + e);
}
/* kernels.rs:19-21 */
float orc_q35_silu(float x) { return x * orc_q35_sigmoid(x); }
/* kernels.rs:22-24: x.max(0) + ln_1p(exp(-|x|)) */
float orc_q35_softplus(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

/* kernels.rs:26-52: zero_centered scales by (w + 1). */
int orc_q35_norm(const float *in, const float *w, float eps, int zero_centered, float *out,
                 size_t n) {
  if (n == 0 || !isfinite(eps) || eps <= 0.0f) return ORC_INVALID_REQUEST;
  if (!all_finite(in, n) || !all_finite(w, n)) return ORC_INVALID_REQUEST;
  double sum = -0.0;
  for (size_t i = 0; i < n; i++) sum += (double)(in[i] * in[i]);
  const double mean = sum / (double)n;
  if (!isfinite(mean) || !isfinite((float)mean)) return ORC_INVALID_REQUEST;
  const float scale = 1.0f / sqrtf((float)mean + eps);
  const float add = zero_centered ? 1.0f : 0.0f;
  for (size_t i = 0; i < n; i++) out[i] = (in[i] * scale) * (w[i] + add);
  return all_finite(out, n) ? ORC_OK : ORC_INVALID_REQUEST;
}

/* kernels.rs:54-120 ConvState::step: the ring keeps raw inputs; slot order
 * (cursor + 1 + i) % kernel pairs the oldest input with weight 0. */
int orc_q35_conv_step(float *history, uint32_t *cursor, size_t channels, size_t kernel,
                      const float *in, const float *w, float *out) {
  if (!all_finite(in, channels) || !all_finite(w, channels * kernel)) return ORC_INVALID_REQUEST;
  for (size_t ch = 0; ch < channels; ch++) {
    const size_t start = ch * kernel;
    history[start + *cursor] = in[ch];
    double sum = -0.0;
    for (size_t i = 0; i < kernel; i++) {
      const size_t slot = (*cursor + 1 + i) % kernel;
      sum += (double)(history[start + slot] * w[start + i]);
    }
    out[ch] = orc_q35_silu((float)sum);
  }
  *cursor = (uint32_t)((*cursor + 1) % kernel);
  return all_finite(out, channels) ? ORC_OK : ORC_INVALID_REQUEST;
}

/* kernels.rs:122-214 DeltaState::step over memory[head][key][value]. */
int orc_q35_delta_step(float *memory, size_t heads, size_t key, size_t value, const float *q,
                       const float *k, const float *v, const float *log_decay,
                       const float *beta, float *out) {
  if (!all_finite(q, heads * key) || !all_finite(k, heads * key) ||
      !all_finite(v, heads * value) || !all_finite(log_decay, heads) || !all_finite(beta, heads))
    return ORC_INVALID_REQUEST;
  for (size_t h = 0; h < heads; h++)
    if (log_decay[h] > 0.0f || !(beta[h] >= 0.0f && beta[h] <= 1.0f)) return ORC_INVALID_REQUEST;
  for (size_t i = 0; i < heads * value; i++) out[i] = 0.0f;
  for (size_t h = 0; h < heads; h++) {
    const float *qh = q + h * key, *kh = k + h * key;
    const float q_norm = orc_dot_f32(qh, qh, key), k_norm = orc_dot_f32(kh, kh, key);
    if (!isfinite(q_norm) || !isfinite(k_norm)) return ORC_INVALID_REQUEST;
    const float q_scale = (1.0f / sqrtf(q_norm + 1e-6f)) / sqrtf((float)key);
    const float k_scale = 1.0f / sqrtf(k_norm + 1e-6f);
    const float decay = expf(log_decay[h]);
    float *head = memory + h * key * value;
    for (size_t j = 0; j < value; j++) {
      double prediction = 0.0;
      for (size_t i = 0; i < key; i++) {
        float *cell = head + i * value + j;
        *cell *= decay;
        prediction += (double)(*cell * (kh[i] * k_scale));
      }
      const float correction = (v[h * value + j] - (float)prediction) * beta[h];
      double read = 0.0;
      for (size_t i = 0; i < key; i++) {
        float *cell = head + i * value + j;
        *cell += (kh[i] * k_scale) * correction;
        read += (double)(*cell * (qh[i] * q_scale));
      }
      out[h * value + j] = (float)read;
    }
  }
  if (!all_finite(out, heads * value) || !all_finite(memory, heads * key * value))
    return ORC_INVALID_REQUEST;
  return ORC_OK;
}

/* kernels.rs:226-268 partial_mrope for text positions (all three axes equal):
 * angle = pos * base^(-(2i)/rotary) (powf per index), first `rotary` dims of
 * each head rotated in halves. */
int orc_q35_partial_rope(float *values, size_t n, size_t head, size_t rotary, size_t position,
                         float base) {
  if (head == 0 || n % head || rotary == 0 || rotary > head || rotary % 2 || !isfinite(base) ||
      base <= 0.0f)
    return ORC_INVALID_REQUEST;
  const size_t half = rotary / 2;
  for (float *row = values; row < values + n; row += head) {
    for (size_t i = 0; i < half; i++) {
      const float angle = (float)position * powf(base, -(float)(2 * i) / (float)rotary);
      const float s = sinf(angle), c = cosf(angle);
      const float a = row[i], b = row[i + half];
      row[i] = a * c - b * s;
      row[i + half] = b * c + a * s;
    }
  }
  return all_finite(values, n) ? ORC_OK : ORC_INVALID_REQUEST;
}

/* ---- the hybrid model ---------------------------------------------------- */

typedef struct {
  uint32_t dtype;  /* 0 = F32, 30 = BF16 */
  size_t rows, cols;
  const void *data;
} q35_matrix;

typedef struct {
  float *input_norm, *post_norm;
  q35_matrix gate, up, down;
  /* full attention */
  q35_matrix q, k, v, o;
  float *q_norm, *k_norm;
  /* linear attention */
  q35_matrix qkv, z, a, b, out;
  float *conv, *a_log, *dt, *norm;
} q35_layer;

struct orc_q35_model {
  orc_q35_config c;
  q35_matrix embed, head;
  float *final_norm;
  q35_layer *layer;
  int threads;
  void *owned;  /* copies of every tensor's bytes */
};

struct orc_q35_session {
  uint32_t position, capacity, layers;
  float **keys, **values;  /* full layers: [capacity][kv_heads * head_dim] */
  float **history;         /* linear layers: [channels][kernel] */
  uint32_t *cursor;
  float **memory;          /* linear layers: [value_heads][key_dim][value_dim] */
  float *logits;
};

static inline float q35_weight(const q35_matrix *m, size_t r, size_t k) {
  if (m->dtype == 0) return ((const float *)m->data)[r * m->cols + k];
  const uint32_t bits = (uint32_t)((const uint16_t *)m->data)[r * m->cols + k] << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* tensor.rs:380-406 for F32/BF16 weights: cpu::dot(weight row, input)
 * (f32 products summed in f64, element order), non-finite -> Error::invalid. */
static int q35_matvec(const orc_q35_model *m, const q35_matrix *w, const float *x, float *y) {
  int bad = 0;
#pragma omp parallel for num_threads(m->threads) schedule(static) reduction(| : bad)
  for (size_t r = 0; r < w->rows; r++) {
    double sum = -0.0;
    for (size_t k = 0; k < w->cols; k++) sum += (double)(q35_weight(w, r, k) * x[k]);
    y[r] = (float)sum;
    bad |= !isfinite(y[r]);
  }
  return bad ? ORC_INVALID_GGUF : ORC_OK;
}

static int take_matrix(const orc_tensor *t, size_t rows, size_t cols, q35_matrix *out,
                       char **cursor) {
  if (!t || (t->dtype != 0 && t->dtype != 30) || t->ne0 != cols || t->ne1 != rows)
    return ORC_UNSUPPORTED;
  const size_t bytes = rows * cols * (t->dtype == 0 ? 4 : 2);
  if (t->bytes != bytes || !t->data) return ORC_INVALID_GGUF;
  memcpy(*cursor, t->data, bytes);
  *out = (q35_matrix){t->dtype, rows, cols, *cursor};
  *cursor += (bytes + 63) / 64 * 64;
  return ORC_OK;
}

/* safetensors read_vector: F32 or BF16 widened to f32; non-finite rejected. */
static int take_vector(const orc_tensor *t, size_t n, float **out, char **cursor) {
  if (!t || (t->dtype != 0 && t->dtype != 30) || t->ne0 * (t->ne1 ? t->ne1 : 1) != n)
    return ORC_UNSUPPORTED;
  if (t->bytes != n * (t->dtype == 0 ? 4 : 2) || !t->data) return ORC_INVALID_GGUF;
  float *v = (float *)*cursor;
  for (size_t i = 0; i < n; i++) {
    if (t->dtype == 0) {
      memcpy(&v[i], (const char *)t->data + 4 * i, 4);
    } else {
      const uint32_t bits = (uint32_t)((const uint16_t *)t->data)[i] << 16;
      memcpy(&v[i], &bits, 4);
    }
    if (!isfinite(v[i])) return ORC_INVALID_GGUF;
  }
  *out = v;
  *cursor += (n * 4 + 63) / 64 * 64;
  return ORC_OK;
}

static size_t tensor_room(const orc_tensor *t) {
  if (!t || !t->data) return 0;
  const size_t n = t->ne0 * (t->ne1 ? t->ne1 : 1);
  return (t->bytes > n * 4 ? t->bytes : n * 4) + 64;
}

int orc_q35_model_new(const orc_q35_config *c, const orc_tensor *globals,
                      const orc_tensor *layers, int threads, orc_q35_model **out) {
  *out = NULL;
  if (!c->layers || c->layers > 128 || !c->heads || !c->kv_heads || c->heads % c->kv_heads ||
      !c->key_heads || c->value_heads % c->key_heads || !c->rotary_dim || c->rotary_dim % 2 ||
      c->rotary_dim > c->head_dim || !c->conv_kernel || c->conv_kernel > 32)
    return ORC_UNSUPPORTED;
  size_t room = 0;
  for (int g = 0; g < 3; g++) room += tensor_room(&globals[g]);
  for (size_t i = 0; i < (size_t)c->layers * ORC_Q35_LAYER_TENSORS; i++) room += tensor_room(&layers[i]);
  orc_q35_model *m = calloc(1, sizeof *m);
  m->c = *c;
  m->threads = threads > 0 ? threads : 1;
  m->owned = malloc(room);
  m->layer = calloc(c->layers, sizeof(q35_layer));
  char *cur = m->owned;
  const size_t H = c->hidden, F = c->intermediate, V = c->vocabulary;
  const size_t keys = (size_t)c->key_heads * c->key_dim, vals = (size_t)c->value_heads * c->value_dim;
  const size_t ch = 2 * keys + vals;
  int rc = take_matrix(&globals[0], V, H, &m->embed, &cur);
  if (!rc) rc = take_vector(&globals[1], H, &m->final_norm, &cur);
  if (!rc) {
    if (globals[2].data)
      rc = take_matrix(&globals[2], V, H, &m->head, &cur);
    else
      m->head = m->embed;  /* tied: embed_tokens (execution.rs:191-196) */
  }
  for (uint32_t l = 0; l < c->layers && !rc; l++) {
    const orc_tensor *t = layers + (size_t)l * ORC_Q35_LAYER_TENSORS;
    q35_layer *L = &m->layer[l];
    rc = take_vector(&t[ORC_Q35_INPUT_NORM], H, &L->input_norm, &cur);
    if (!rc) rc = take_vector(&t[ORC_Q35_POST_NORM], H, &L->post_norm, &cur);
    if (!rc) rc = take_matrix(&t[ORC_Q35_GATE], F, H, &L->gate, &cur);
    if (!rc) rc = take_matrix(&t[ORC_Q35_UP], F, H, &L->up, &cur);
    if (!rc) rc = take_matrix(&t[ORC_Q35_DOWN], H, F, &L->down, &cur);
    if (rc) break;
    if (c->full[l]) {
      const size_t qw = (size_t)c->heads * c->head_dim, kw = (size_t)c->kv_heads * c->head_dim;
      rc = take_matrix(&t[ORC_Q35_Q], 2 * qw, H, &L->q, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_K], kw, H, &L->k, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_V], kw, H, &L->v, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_O], H, qw, &L->o, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_QNORM], c->head_dim, &L->q_norm, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_KNORM], c->head_dim, &L->k_norm, &cur);
    } else {
      rc = take_matrix(&t[ORC_Q35_QKV], ch, H, &L->qkv, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_Z], vals, H, &L->z, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_A], c->value_heads, H, &L->a, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_B], c->value_heads, H, &L->b, &cur);
      if (!rc) rc = take_matrix(&t[ORC_Q35_OUT], H, vals, &L->out, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_CONV], ch * c->conv_kernel, &L->conv, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_ALOG], c->value_heads, &L->a_log, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_DT], c->value_heads, &L->dt, &cur);
      if (!rc) rc = take_vector(&t[ORC_Q35_NORM], c->value_dim, &L->norm, &cur);
    }
  }
  if (rc) {
    orc_q35_model_free(m);
    return rc;
  }
  *out = m;
  return ORC_OK;
}

void orc_q35_model_free(orc_q35_model *m) {
  if (!m) return;
  free(m->layer);
  free(m->owned);
  free(m);
}

int orc_q35_session_new(const orc_q35_model *m, uint32_t context, orc_q35_session **out) {
  const orc_q35_config *c = &m->c;
  if (!context || context > c->context) return ORC_RESOURCE;
  orc_q35_session *s = calloc(1, sizeof *s);
  s->capacity = context;
  s->layers = c->layers;
  s->keys = calloc(c->layers, sizeof(float *));
  s->values = calloc(c->layers, sizeof(float *));
  s->history = calloc(c->layers, sizeof(float *));
  s->memory = calloc(c->layers, sizeof(float *));
  s->cursor = calloc(c->layers, sizeof(uint32_t));
  const size_t kw = (size_t)c->kv_heads * c->head_dim;
  const size_t ch = 2 * (size_t)c->key_heads * c->key_dim + (size_t)c->value_heads * c->value_dim;
  for (uint32_t l = 0; l < c->layers; l++) {
    if (c->full[l]) {
      s->keys[l] = calloc((size_t)context * kw, 4);
      s->values[l] = calloc((size_t)context * kw, 4);
    } else {
      s->history[l] = calloc(ch * c->conv_kernel, 4);
      s->memory[l] = calloc((size_t)c->value_heads * c->key_dim * c->value_dim, 4);
    }
  }
  s->logits = calloc(c->vocabulary, 4);
  *out = s;
  return ORC_OK;
}

void orc_q35_session_free(orc_q35_session *s) {
  if (!s) return;
  for (uint32_t l = 0; l < s->layers; l++) {
    free(s->keys[l]);
    free(s->values[l]);
    free(s->history[l]);
    free(s->memory[l]);
  }
  free(s->keys);
  free(s->values);
  free(s->history);
  free(s->memory);
  free(s->cursor);
  free(s->logits);
  free(s);
}

uint32_t orc_q35_session_position(const orc_q35_session *s) { return s->position; }
const float *orc_q35_session_logits(const orc_q35_session *s) { return s->logits; }

/* which: 0 = K rows, 1 = V rows (full layers, [0, position)), 2 = conv ring
 * [channels][kernel], 3 = delta memory [heads][key][value], 4 = conv cursor */
int orc_q35_session_state(const orc_q35_model *m, const orc_q35_session *s, uint32_t layer,
                          int which, float *out) {
  const orc_q35_config *c = &m->c;
  if (layer >= c->layers) return ORC_INVALID_REQUEST;
  const size_t kw = (size_t)c->kv_heads * c->head_dim;
  const size_t ch = 2 * (size_t)c->key_heads * c->key_dim + (size_t)c->value_heads * c->value_dim;
  if (which <= 1) {
    if (!c->full[layer]) return ORC_INVALID_REQUEST;
    memcpy(out, which ? s->values[layer] : s->keys[layer], (size_t)s->position * kw * 4);
  } else if (which == 2) {
    if (c->full[layer]) return ORC_INVALID_REQUEST;
    memcpy(out, s->history[layer], ch * c->conv_kernel * 4);
  } else if (which == 3) {
    if (c->full[layer]) return ORC_INVALID_REQUEST;
    memcpy(out, s->memory[layer], (size_t)c->value_heads * c->key_dim * c->value_dim * 4);
  } else if (which == 4) {
    if (c->full[layer]) return ORC_INVALID_REQUEST;
    out[0] = (float)s->cursor[layer];
  } else {
    return ORC_INVALID_REQUEST;
  }
  return ORC_OK;
}

typedef struct {
  float *x, *nrm, *mixed, *conv_out, *z, *a, *b, *dq, *dk, *att, *tgt, *q, *k, *v, *proj, *gate,
      *up, *fin;
} q35_scratch;

/* One lane, one token: execution.rs:257-608 (Graph::forward_batch body). */
static int q35_forward_lane(const orc_q35_model *m, orc_q35_session *s, uint32_t token,
                            int logits, q35_scratch *w) {
  const orc_q35_config *c = &m->c;
  const size_t H = c->hidden, D = c->head_dim, NH = c->heads, NKV = c->kv_heads;
  const size_t KD = c->key_dim, VD = c->value_dim, KH = c->key_heads, VH = c->value_heads;
  const size_t keys = KH * KD, vals = VH * VD, width = 2 * keys + vals;
  const size_t qw = NH * D, kw = NKV * D;
  const float eps = c->epsilon;
  int rc;
  if (s->position >= s->capacity || token >= c->vocabulary) return ORC_INVALID_REQUEST;
  for (size_t i = 0; i < H; i++) w->x[i] = q35_weight(&m->embed, token, i);
  for (uint32_t l = 0; l < c->layers; l++) {
    const q35_layer *L = &m->layer[l];
    if ((rc = orc_q35_norm(w->x, L->input_norm, eps, 1, w->nrm, H))) return rc;
    if (!c->full[l]) {
      if ((rc = q35_matvec(m, &L->qkv, w->nrm, w->mixed))) return rc;
      if ((rc = q35_matvec(m, &L->z, w->nrm, w->z))) return rc;
      if ((rc = q35_matvec(m, &L->a, w->nrm, w->a))) return rc;
      if ((rc = q35_matvec(m, &L->b, w->nrm, w->b))) return rc;
      if ((rc = orc_q35_conv_step(s->history[l], &s->cursor[l], width, c->conv_kernel, w->mixed,
                                  L->conv, w->conv_out)))
        return rc;
      const size_t repeat = VH / KH;
      for (size_t h = 0; h < VH; h++) {
        const size_t src = (h / repeat) * KD, dst = h * KD;
        memcpy(w->dq + dst, w->conv_out + src, KD * 4);
        memcpy(w->dk + dst, w->conv_out + keys + src, KD * 4);
        w->a[h] = -expf(L->a_log[h]) * orc_q35_softplus(w->a[h] + L->dt[h]);
        w->b[h] = orc_q35_sigmoid(w->b[h]);
      }
      if ((rc = orc_q35_delta_step(s->memory[l], VH, KD, VD, w->dq, w->dk,
                                   w->conv_out + 2 * keys, w->a, w->b, w->att)))
        return rc;
      for (size_t h = 0; h < VH; h++) {
        if ((rc = orc_q35_norm(w->att + h * VD, L->norm, eps, 0, w->tgt + h * VD, VD))) return rc;
        for (size_t j = 0; j < VD; j++) w->tgt[h * VD + j] *= orc_q35_silu(w->z[h * VD + j]);
      }
      if ((rc = q35_matvec(m, &L->out, w->tgt, w->proj))) return rc;
    } else {
      if ((rc = q35_matvec(m, &L->q, w->nrm, w->mixed))) return rc;
      for (size_t h = 0; h < NH; h++) {
        const size_t base = h * 2 * D;
        if ((rc = orc_q35_norm(w->mixed + base, L->q_norm, eps, 1, w->q + h * D, D))) return rc;
        memcpy(w->z + h * D, w->mixed + base + D, D * 4);
      }
      if ((rc = q35_matvec(m, &L->k, w->nrm, w->k))) return rc;
      if ((rc = q35_matvec(m, &L->v, w->nrm, w->v))) return rc;
      for (size_t h = 0; h < NKV; h++) {
        if ((rc = orc_q35_norm(w->k + h * D, L->k_norm, eps, 1, w->tgt, D))) return rc;
        memcpy(w->k + h * D, w->tgt, D * 4);
      }
      if ((rc = orc_q35_partial_rope(w->q, qw, D, c->rotary_dim, s->position, c->rope_base)))
        return rc;
      if ((rc = orc_q35_partial_rope(w->k, kw, D, c->rotary_dim, s->position, c->rope_base)))
        return rc;
      memcpy(s->keys[l] + (size_t)s->position * kw, w->k, kw * 4);
      memcpy(s->values[l] + (size_t)s->position * kw, w->v, kw * 4);
      if ((rc = orc_attention(w->q, qw, s->keys[l], s->values[l], s->position + 1, NKV, D,
                              w->att)))
        return rc;
      for (size_t e = 0; e < qw; e++) w->att[e] *= orc_q35_sigmoid(w->z[e]);
      if ((rc = q35_matvec(m, &L->o, w->att, w->proj))) return rc;
    }
    for (size_t i = 0; i < H; i++) w->x[i] += w->proj[i];
    if ((rc = orc_q35_norm(w->x, L->post_norm, eps, 1, w->nrm, H))) return rc;
    if ((rc = q35_matvec(m, &L->gate, w->nrm, w->gate))) return rc;
    if ((rc = q35_matvec(m, &L->up, w->nrm, w->up))) return rc;
    orc_swiglu(w->gate, w->up, c->intermediate);
    if ((rc = q35_matvec(m, &L->down, w->gate, w->proj))) return rc;
    for (size_t i = 0; i < H; i++) w->x[i] += w->proj[i];
  }
  if ((rc = orc_q35_norm(w->x, m->final_norm, eps, 1, w->fin, H))) return rc;
  if (logits && (rc = q35_matvec(m, &m->head, w->fin, s->logits))) return rc;
  s->position += 1;
  return ORC_OK;
}

int orc_q35_forward_batch(const orc_q35_model *m, orc_q35_session **sessions,
                          const uint32_t *tokens, const uint8_t *logits, size_t n,
                          int32_t *errors) {
  const orc_q35_config *c = &m->c;
  const size_t keys = (size_t)c->key_heads * c->key_dim, vals = (size_t)c->value_heads * c->value_dim;
  const size_t width = 2 * keys + vals, qw = (size_t)c->heads * c->head_dim;
  size_t big = c->hidden;
  const size_t cand[] = {c->intermediate, width, 2 * qw, vals, qw, (size_t)c->value_heads * c->key_dim};
  for (size_t i = 0; i < sizeof cand / sizeof cand[0]; i++) big = cand[i] > big ? cand[i] : big;
  q35_scratch w;
  float **slots[] = {&w.x, &w.nrm, &w.mixed, &w.conv_out, &w.z, &w.a, &w.b, &w.dq, &w.dk,
                     &w.att, &w.tgt, &w.q, &w.k, &w.v, &w.proj, &w.gate, &w.up, &w.fin};
  for (size_t i = 0; i < sizeof slots / sizeof slots[0]; i++) *slots[i] = calloc(big, 4);
  for (size_t i = 0; i < n; i++) {
    if (errors[i]) continue;
    errors[i] = q35_forward_lane(m, sessions[i], tokens[i], logits ? logits[i] : 1, &w);
  }
  for (size_t i = 0; i < sizeof slots / sizeof slots[0]; i++) free(*slots[i]);
  return ORC_OK;
}
