/*
 * CPU ORACLE — test infrastructure only (never linked by the product).
 *
 * Scalar kernels restated from the reference Rust sources:
 *   crates/coheryn-engine/src/quant.rs  (row_bytes 13-35, decode 67-137,
 *                                        prepare 175-240, dot 245-349)
 *   crates/coheryn-engine/src/cpu.rs    (decode 5-30, dot 31-35, round_f16 37-48,
 *                                        rms_norm 49-57, rope 59-73, swiglu 74-78,
 *                                        attention 80-124, attention_rows 133-210)
 *   crates/coheryn-engine/src/sampling.rs (Sampler 57-223, SplitMix64 123-130)
 * Built with -ffp-contract=off so that every a*b+c rounds twice, as Rust does.
 */
#include "orc.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * binary16 conversions (the `half` crate 2.7.1 contract: exact widening,
 * round-to-nearest-even narrowing, overflow to infinity).
 * ------------------------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      int shifts = 0;
      while (!(mant & 0x400u)) {
        mant <<= 1;
        shifts++;
      }
      bits = sign | ((uint32_t)(127 - 14 - shifts) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (mant ? 0x400000u : 0u) | (mant << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu, mant = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t full = mant | 0x800000u;
    int shift = 14 - e;
    uint32_t m = full >> shift, rem = full & ((1u << shift) - 1), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)h;
}

static int finite(float v) { return isfinite(v); }

/* quant::half — f16 scale that must be finite. quant.rs:36-43 */
static int scale_f16(const uint8_t *b, float *out) {
  float v = orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
  if (!finite(v)) return ORC_INVALID_GGUF;
  *out = v;
  return ORC_OK;
}

/* quant.rs:7-12 */
static int is_packed(uint32_t dtype) {
  return dtype == 2 || dtype == 6 || dtype == 8 || dtype == 12 || dtype == 14;
}

/* quant.rs:13-35 */
int orc_row_bytes(uint32_t dtype, size_t width, size_t *out) {
  size_t block, bytes;
  switch (dtype) {
    case 0: block = 1; bytes = 4; break;
    case 1: case 30: block = 1; bytes = 2; break;
    case 2: block = 32; bytes = 18; break;
    case 6: block = 32; bytes = 22; break;
    case 8: block = 32; bytes = 34; break;
    case 12: block = 256; bytes = 144; break;
    case 14: block = 256; bytes = 210; break;
    default: return ORC_UNSUPPORTED;
  }
  if (width == 0 || width % block) return ORC_INVALID_GGUF;
  if ((width / block) > SIZE_MAX / bytes) return ORC_RESOURCE;
  *out = (width / block) * bytes;
  return ORC_OK;
}

/* quant.rs:44-56 */
static void k4_coefficients(const uint8_t *scales, int group, int32_t *scale, int32_t *minimum) {
  if (group < 4) {
    *scale = scales[group] & 63;
    *minimum = scales[group + 4] & 63;
  } else {
    *scale = (scales[group + 4] & 15) | ((scales[group - 4] >> 6) << 4);
    *minimum = (scales[group + 4] >> 4) | ((scales[group] >> 6) << 4);
  }
}

/* quant.rs:57-65 */
static int32_t q6_value(const uint8_t *block, int index) {
  int half = index / 128, group = (index % 128) / 32, lane = index % 32;
  uint8_t low = block[half * 64 + (group % 2) * 32 + lane];
  low = group < 2 ? (low & 15) : (low >> 4);
  uint8_t high = (block[128 + half * 32 + lane] >> (2 * group)) & 3;
  return (int32_t)(low | (high << 4)) - 32;
}

/* quant.rs:67-137 (packed) and cpu.rs:5-30 (F32/F16/BF16). */
int orc_decode(const uint8_t *bytes, size_t nbytes, uint32_t dtype, float *out, size_t n) {
  if (is_packed(dtype)) {
    size_t rb;
    int rc = orc_row_bytes(dtype, n, &rb);
    if (rc) return rc;
    if (rb != nbytes) return ORC_INVALID_GGUF;
    size_t width = (dtype == 2 || dtype == 6 || dtype == 8) ? 32 : 256;
    size_t size = dtype == 2 ? 18 : dtype == 6 ? 22 : dtype == 8 ? 34 : dtype == 12 ? 144 : 210;
    for (size_t b = 0; b < n / width; b++) {
      const uint8_t *block = bytes + b * size;
      float *dst = out + b * width;
      float d;
      if (dtype == 14) {
        if (scale_f16(block + 208, &d)) return ORC_INVALID_GGUF;
        for (int i = 0; i < 256; i++)
          dst[i] = (d * (float)(int8_t)block[192 + i / 16]) * (float)q6_value(block, i);
        continue;
      }
      if (scale_f16(block, &d)) return ORC_INVALID_GGUF;
      if (dtype == 8) {
        for (int i = 0; i < 32; i++) dst[i] = d * (float)(int8_t)block[2 + i];
      } else if (dtype == 2) {
        for (int j = 0; j < 16; j++) {
          dst[j] = d * (float)((int32_t)(block[j + 2] & 15) - 8);
          dst[j + 16] = d * (float)((int32_t)(block[j + 2] >> 4) - 8);
        }
      } else if (dtype == 6) {
        uint32_t high = (uint32_t)block[2] | ((uint32_t)block[3] << 8) |
                        ((uint32_t)block[4] << 16) | ((uint32_t)block[5] << 24);
        for (int j = 0; j < 16; j++) {
          dst[j] = d * (float)((int32_t)((block[6 + j] & 15u) | (((high >> j) & 1u) << 4)) - 16);
          dst[j + 16] =
              d * (float)((int32_t)((block[6 + j] >> 4) | (((high >> (j + 16)) & 1u) << 4)) - 16);
        }
      } else { /* 12: Q4_K */
        float min;
        if (scale_f16(block + 2, &min)) return ORC_INVALID_GGUF;
        for (int group = 0; group < 8; group++) {
          int32_t sc, mn;
          k4_coefficients(block + 4, group, &sc, &mn);
          float ds = d * (float)sc, dm = min * (float)mn;
          for (int j = 0; j < 32; j++) {
            uint8_t packed = block[16 + (group / 2) * 32 + j];
            uint8_t q = (group % 2 == 0) ? (packed & 15) : (packed >> 4);
            dst[group * 32 + j] = ds * (float)q - dm;
          }
        }
      }
    }
    return ORC_OK;
  }
  size_t size;
  if (dtype == 0) size = 4;
  else if (dtype == 1 || dtype == 30) size = 2;
  else return ORC_INVALID_GGUF;
  if (n > SIZE_MAX / size || nbytes != n * size) return ORC_INVALID_GGUF;
  for (size_t i = 0; i < n; i++) {
    const uint8_t *s = bytes + i * size;
    float v;
    if (size == 4) {
      memcpy(&v, s, 4);
    } else if (dtype == 30) {
      uint32_t bits = (uint32_t)(s[0] | (s[1] << 8)) << 16;
      memcpy(&v, &bits, 4);
    } else {
      v = orc_f16_to_f32((uint16_t)(s[0] | (s[1] << 8)));
    }
    if (!finite(v)) return ORC_INVALID_GGUF;
    out[i] = v;
  }
  return ORC_OK;
}

/* cpu.rs:31-35: F32 products, sequential f64 sum (Rust's Sum starts at -0.0). */
float orc_dot_f32(const float *a, const float *b, size_t n) {
  double sum = -0.0;
  for (size_t i = 0; i < n; i++) sum += (double)(a[i] * b[i]);
  return (float)sum;
}

/* cpu.rs:37-48 */
int orc_round_f16(const float *in, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) {
    out[i] = orc_f16_to_f32(orc_f32_to_f16(in[i]));
    if (!finite(out[i])) return ORC_INVALID_GGUF;
  }
  return ORC_OK;
}

/* cpu.rs:49-57 */
void orc_rms_norm(const float *x, const float *w, float eps, float *out, size_t n) {
  double sum = -0.0;
  for (size_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
  float mean = (float)(sum / (double)n);
  float scale = 1.0f / sqrtf(mean + eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* cpu.rs:59-73: NeoX halves; the angle advances by repeated multiplication. */
void orc_rope(float *x, size_t n, size_t head_dim, size_t position, float base) {
  float step = powf(base, -2.0f / (float)head_dim);
  size_t half = head_dim / 2;
  for (size_t h = 0; h + head_dim <= n; h += head_dim) {
    float *head = x + h;
    float angle = (float)position;
    for (size_t i = 0; i < half; i++) {
      float s = sinf(angle), c = cosf(angle);
      float a = head[i], b = head[i + half];
      head[i] = fmaf(a, c, -(b * s));
      head[i + half] = fmaf(a, s, b * c);
      angle *= step;
    }
  }
}

/* cpu.rs:74-78 */
void orc_swiglu(float *gate, const float *up, size_t n) {
  for (size_t i = 0; i < n; i++) gate[i] = (gate[i] / (1.0f + expf(-gate[i]))) * up[i];
}

/* Rust `f as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v;
}

/* quant.rs:175-240 QuantizedInput::prepare */
int orc_prepare(const float *in, size_t n, uint32_t weight_dtype, uint8_t *out, size_t cap,
                size_t *used, uint32_t *kind) {
  size_t width, size;
  uint32_t k;
  if (weight_dtype == 2 || weight_dtype == 6 || weight_dtype == 8) {
    width = 32; size = 34; k = 8;
  } else if (weight_dtype == 12 || weight_dtype == 14) {
    width = 256; size = 292; k = 15;
  } else {
    return ORC_INVALID_GGUF;
  }
  if (n == 0 || n % width) return ORC_INVALID_GGUF;
  for (size_t i = 0; i < n; i++)
    if (!finite(in[i])) return ORC_INVALID_GGUF;
  size_t total = (n / width) * size;
  if (total > cap) return ORC_RESOURCE;
  for (size_t b = 0; b < n / width; b++) {
    const float *src = in + b * width;
    uint8_t *dst = out + b * size;
    float maximum = 0.0f;
    for (size_t i = 0; i < width; i++)
      if (fabsf(src[i]) > fabsf(maximum)) maximum = src[i];
    if (k == 8) {
      float d = fabsf(maximum) / 127.0f;
      float inverse = d == 0.0f ? 0.0f : 1.0f / d;
      uint16_t stored = orc_f32_to_f16(d);
      if (!finite(orc_f16_to_f32(stored)) || !finite(inverse)) return ORC_INVALID_GGUF;
      dst[0] = (uint8_t)(stored & 0xff);
      dst[1] = (uint8_t)(stored >> 8);
      for (size_t i = 0; i < 32; i++) dst[2 + i] = (uint8_t)sat_i8(roundf(src[i] * inverse));
    } else {
      memset(dst, 0, size);
      if (maximum != 0.0f) {
        float inverse = -127.0f / maximum;
        float d = 1.0f / inverse;
        if (!finite(inverse) || !finite(d)) return ORC_INVALID_GGUF;
        memcpy(dst, &d, 4);
        for (size_t i = 0; i < 256; i++) {
          float r = rintf(src[i] * inverse);
          dst[4 + i] = (uint8_t)sat_i8(r < 127.0f ? r : 127.0f);
        }
        for (int g = 0; g < 16; g++) {
          int16_t sum = 0;
          for (int i = 0; i < 16; i++) sum = (int16_t)(sum + (int8_t)dst[4 + g * 16 + i]);
          dst[260 + g * 2] = (uint8_t)((uint16_t)sum & 0xff);
          dst[261 + g * 2] = (uint8_t)((uint16_t)sum >> 8);
        }
      }
    }
  }
  *used = total;
  *kind = k;
  return ORC_OK;
}

/* quant.rs:245-349 quant::dot */
int orc_qdot(const uint8_t *row, size_t row_len, uint32_t dtype, const uint8_t *act,
             uint32_t act_kind, size_t width, float *out) {
  size_t bw, size;
  uint32_t kind;
  switch (dtype) {
    case 2: bw = 32; size = 18; kind = 8; break;
    case 6: bw = 32; size = 22; kind = 8; break;
    case 8: bw = 32; size = 34; kind = 8; break;
    case 12: bw = 256; size = 144; kind = 15; break;
    case 14: bw = 256; size = 210; kind = 15; break;
    default: return ORC_INVALID_GGUF;
  }
  size_t rb;
  if (act_kind != kind || orc_row_bytes(dtype, width, &rb) || rb != row_len)
    return ORC_INVALID_GGUF;
  float sum = 0.0f;
  float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t asize = kind == 8 ? 34 : 292;
  for (size_t b = 0; b < width / bw; b++) {
    const uint8_t *w = row + b * size;
    const uint8_t *a = act + b * asize;
    if (bw == 32) {
      float dw, da;
      if (scale_f16(w, &dw) || scale_f16(a, &da)) return ORC_INVALID_GGUF;
      int32_t integer = 0;
      if (dtype == 8) {
        for (int i = 0; i < 32; i++) integer += (int32_t)(int8_t)w[2 + i] * (int32_t)(int8_t)a[2 + i];
        sum = fmaf((float)integer, dw * da, sum);
      } else if (dtype == 6) {
        uint32_t high = (uint32_t)w[2] | ((uint32_t)w[3] << 8) | ((uint32_t)w[4] << 16) |
                        ((uint32_t)w[5] << 24);
        for (int i = 0; i < 16; i++) {
          int32_t low = (int32_t)((w[6 + i] & 15u) | (((high >> i) & 1u) << 4)) - 16;
          int32_t upper = (int32_t)((w[6 + i] >> 4) | (((high >> (i + 16)) & 1u) << 4)) - 16;
          integer += low * (int32_t)(int8_t)a[2 + i] + upper * (int32_t)(int8_t)a[18 + i];
        }
        sum = fmaf(dw * da, (float)integer, sum);
      } else {
        for (int i = 0; i < 16; i++) {
          integer += ((int32_t)(w[i + 2] & 15) - 8) * (int32_t)(int8_t)a[2 + i];
          integer += ((int32_t)(w[i + 2] >> 4) - 8) * (int32_t)(int8_t)a[18 + i];
        }
        sum = fmaf((float)integer * dw, da, sum);
      }
    } else {
      float da;
      memcpy(&da, a, 4);
      int32_t integers[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (dtype == 12) {
        float dw, dm;
        if (scale_f16(w, &dw) || scale_f16(w + 2, &dm)) return ORC_INVALID_GGUF;
        int32_t minimum_sum = 0;
        for (int g = 0; g < 8; g++) {
          int32_t sc, mn;
          k4_coefficients(w + 4, g, &sc, &mn);
          int32_t gs = (int32_t)(int16_t)(a[260 + g * 4] | (a[261 + g * 4] << 8)) +
                       (int32_t)(int16_t)(a[262 + g * 4] | (a[263 + g * 4] << 8));
          minimum_sum += mn * gs;
          for (int i = 0; i < 32; i++) {
            uint8_t packed = w[16 + (g / 2) * 32 + i];
            uint8_t q = (g % 2 == 0) ? (packed & 15) : (packed >> 4);
            integers[i % 8] += sc * (int32_t)q * (int32_t)(int8_t)a[4 + g * 32 + i];
          }
        }
        for (int i = 0; i < 8; i++) lanes[i] = fmaf(dw * da, (float)integers[i], lanes[i]);
        sum = fmaf(-(dm * da), (float)minimum_sum, sum);
      } else {
        float dw;
        if (scale_f16(w + 208, &dw)) return ORC_INVALID_GGUF;
        for (int i = 0; i < 256; i++)
          integers[i % 8] += q6_value(w, i) * (int32_t)(int8_t)w[192 + i / 16] *
                             (int32_t)(int8_t)a[4 + i];
        for (int i = 0; i < 8; i++) lanes[i] = fmaf(dw * da, (float)integers[i], lanes[i]);
      }
    }
  }
  if (bw == 256)
    for (int i = 0; i < 8; i++) sum += lanes[i];
  if (!finite(sum)) return ORC_INVALID_GGUF;
  *out = sum;
  return ORC_OK;
}

/* cpu.rs:133-210 two-pass row attention with wide reductions. */
int orc_attention_rows(const float *q, size_t nq, const float *keys, const float *values,
                       size_t kv_rows, size_t kv_heads, size_t head_dim, float *out) {
  size_t stride = kv_heads * head_dim;
  if (stride == 0 || nq == 0 || nq % head_dim || (nq / head_dim) % kv_heads || kv_rows == 0)
    return ORC_INVALID_GGUF;
  size_t heads = nq / head_dim;
  float scale = 1.0f / sqrtf((float)head_dim);
  float *scores = (float *)malloc(kv_rows * sizeof(float));
  double *acc = (double *)malloc(head_dim * sizeof(double));
  if (!scores || !acc) {
    free(scores);
    free(acc);
    return ORC_RESOURCE;
  }
  int rc = ORC_OK;
  for (size_t h = 0; h < heads && rc == ORC_OK; h++) {
    size_t group = h / (heads / kv_heads);
    const float *query = q + h * head_dim;
    float maximum = -INFINITY;
    for (size_t t = 0; t < kv_rows; t++) {
      scores[t] = orc_dot_f32(query, keys + t * stride + group * head_dim, head_dim) * scale;
      if (!finite(scores[t])) {
        rc = ORC_INVALID_GGUF;
        break;
      }
      maximum = fmaxf(maximum, scores[t]);
    }
    if (rc) break;
    double denominator = 0.0;
    for (size_t t = 0; t < kv_rows; t++) {
      scores[t] = expf(scores[t] - maximum);
      denominator += (double)scores[t];
    }
    float inverse = (float)(1.0 / denominator);
    for (size_t t = 0; t < kv_rows; t++) scores[t] *= inverse;
    for (size_t j = 0; j < head_dim; j++) acc[j] = 0.0;
    for (size_t t = 0; t < kv_rows; t++) {
      const float *row = values + t * stride + group * head_dim;
      for (size_t j = 0; j < head_dim; j++) acc[j] += (double)(scores[t] * row[j]);
    }
    for (size_t j = 0; j < head_dim; j++) {
      out[h * head_dim + j] = (float)acc[j];
      if (!finite(out[h * head_dim + j])) rc = ORC_INVALID_GGUF;
    }
  }
  free(scores);
  free(acc);
  return rc;
}

/* cpu.rs:80-124 online-softmax attention (used by the hybrid graph). */
int orc_attention(const float *q, size_t nq, const float *keys, const float *values,
                  size_t kv_rows, size_t kv_heads, size_t head_dim, float *out) {
  size_t heads = nq / head_dim, stride = kv_heads * head_dim;
  for (size_t h = 0; h < heads; h++) {
    const float *query = q + h * head_dim;
    float *target = out + h * head_dim;
    for (size_t j = 0; j < head_dim; j++) target[j] = 0.0f;
    size_t kv = h / (heads / kv_heads);
    float maximum = -INFINITY, denominator = 0.0f;
    for (size_t i = 0; i < kv_rows; i++) {
      const float *k = keys + i * stride + kv * head_dim;
      const float *v = values + i * stride + kv * head_dim;
      float score = orc_dot_f32(query, k, head_dim) / sqrtf((float)head_dim);
      float next = fmaxf(maximum, score);
      float old = expf(maximum - next);
      float nw = expf(score - next);
      denominator = denominator * old + nw;
      for (size_t j = 0; j < head_dim; j++) target[j] = target[j] * old + nw * v[j];
      maximum = next;
    }
    for (size_t j = 0; j < head_dim; j++) target[j] /= denominator;
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------------------
 * Sampler (sampling.rs:57-223)
 * ------------------------------------------------------------------------- */
struct orc_sampler {
  float temperature, top_p;
  uint32_t top_k;
  uint64_t state;
  float rep, freq, pres;
  uint32_t *counts;
  size_t ncounts;
};

static int penalties_enabled(const orc_sampler *s) {
  return s->rep != 1.0f || s->freq != 0.0f || s->pres != 0.0f;
}

int orc_sampler_new(float temperature, uint32_t top_k, float top_p, uint64_t seed, float rep,
                    float freq, float pres, orc_sampler **out) {
  if (!finite(temperature) || !(temperature >= 0.0f && temperature <= 2.0f) || !finite(top_p) ||
      top_p <= 0.0f || top_p > 1.0f)
    return ORC_INVALID_REQUEST;
  if (!finite(rep) || !(rep >= 0.01f && rep <= 10.0f) || !finite(freq) ||
      !(freq >= -2.0f && freq <= 2.0f) || !finite(pres) || !(pres >= -2.0f && pres <= 2.0f))
    return ORC_INVALID_REQUEST;
  orc_sampler *s = (orc_sampler *)calloc(1, sizeof(*s));
  if (!s) return ORC_RESOURCE;
  s->temperature = temperature;
  s->top_k = top_k;
  s->top_p = top_p;
  s->state = seed;
  s->rep = rep;
  s->freq = freq;
  s->pres = pres;
  *out = s;
  return ORC_OK;
}

void orc_sampler_free(orc_sampler *s) {
  if (s) free(s->counts);
  free(s);
}

int orc_sampler_observe(orc_sampler *s, uint32_t token) {
  if (penalties_enabled(s)) {
    if (token >= s->ncounts) return ORC_INVALID_REQUEST;
    if (s->counts[token] == UINT32_MAX) return ORC_RESOURCE;
    s->counts[token]++;
  }
  return ORC_OK;
}

int orc_sampler_history(orc_sampler *s, size_t vocabulary, const uint32_t *tokens, size_t n) {
  if (s->top_k > vocabulary) return ORC_INVALID_REQUEST;
  if (penalties_enabled(s)) {
    free(s->counts);
    s->counts = (uint32_t *)calloc(vocabulary ? vocabulary : 1, sizeof(uint32_t));
    if (!s->counts) return ORC_RESOURCE;
    s->ncounts = vocabulary;
    for (size_t i = 0; i < n; i++) {
      int rc = orc_sampler_observe(s, tokens[i]);
      if (rc) return rc;
    }
  }
  return ORC_OK;
}

/* SplitMix64, sampling.rs:123-130 */
static double sampler_random(orc_sampler *s) {
  s->state += 0x9e3779b97f4a7c15ULL;
  uint64_t z = s->state;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return (double)((z ^ (z >> 31)) >> 11) / (double)(1ULL << 53);
}

/* sampling.rs:131-143 */
static double adjusted(const orc_sampler *s, size_t id, float logit) {
  uint32_t count = id < s->ncounts ? s->counts[id] : 0;
  double value = (double)logit;
  if (count != 0) {
    value = value < 0.0 ? value * (double)s->rep : value / (double)s->rep;
    value -= (double)s->pres + (double)count * (double)s->freq;
  }
  return value;
}

typedef struct {
  size_t id;
  double value;
} ranked;

/* f64::total_cmp ordering key */
static int64_t total_key(double v) {
  int64_t b;
  memcpy(&b, &v, 8);
  return b ^ (int64_t)((uint64_t)(b >> 63) >> 1);
}

/* value(b).total_cmp(value(a)).then(a.cmp(b)) */
static int compare_ranked(const void *pa, const void *pb) {
  const ranked *a = (const ranked *)pa, *b = (const ranked *)pb;
  int64_t ka = total_key(a->value), kb = total_key(b->value);
  if (kb != ka) return kb < ka ? -1 : 1;
  return a->id < b->id ? -1 : a->id > b->id ? 1 : 0;
}

int orc_sampler_sample(orc_sampler *s, const float *logits, size_t n, const uint8_t *allowed,
                       uint32_t *token) {
  if (n == 0) return ORC_INVALID_GGUF;
  for (size_t i = 0; i < n; i++)
    if (!finite(logits[i])) return ORC_INVALID_GGUF;
  if (s->top_k > n) return ORC_INVALID_REQUEST;
  if (s->temperature == 0.0f) {
    long best = -1;
    double best_value = 0.0;
    for (size_t id = 0; id < n; id++) {
      if (allowed && !allowed[id]) continue;
      double v = adjusted(s, id, logits[id]);
      if (best < 0 || v > best_value) {
        best = (long)id;
        best_value = v;
      }
    }
    if (best < 0) return ORC_DEAD_END;
    *token = (uint32_t)best;
    return ORC_OK;
  }
  ranked *ids = (ranked *)malloc(n * sizeof(ranked));
  double *prob = (double *)malloc(n * sizeof(double));
  if (!ids || !prob) {
    free(ids);
    free(prob);
    return ORC_RESOURCE;
  }
  size_t count = 0;
  for (size_t id = 0; id < n; id++)
    if (!allowed || allowed[id]) {
      ids[count].id = id;
      ids[count].value = adjusted(s, id, logits[id]);
      count++;
    }
  if (count == 0) {
    free(ids);
    free(prob);
    return ORC_DEAD_END;
  }
  /* select_nth + truncate + sort == the first top_k of the full comparator sort */
  qsort(ids, count, sizeof(ranked), compare_ranked);
  if (s->top_k > 0 && s->top_k < count) count = s->top_k;
  double maximum = ids[0].value, total = -0.0;
  for (size_t i = 0; i < count; i++) {
    prob[i] = exp((ids[i].value - maximum) / (double)s->temperature);
  }
  for (size_t i = 0; i < count; i++) total += prob[i];
  double cumulative = 0.0;
  size_t keep = 0;
  for (size_t i = 0; i < count; i++) {
    cumulative += prob[i] / total;
    keep++;
    if (cumulative >= (double)s->top_p) break;
  }
  double mass = -0.0;
  for (size_t i = 0; i < keep; i++) mass += prob[i];
  double threshold = sampler_random(s) * mass;
  cumulative = 0.0;
  uint32_t chosen = (uint32_t)ids[keep - 1].id;
  for (size_t i = 0; i < keep; i++) {
    cumulative += prob[i];
    if (threshold < cumulative) {
      chosen = (uint32_t)ids[i].id;
      break;
    }
  }
  *token = chosen;
  free(ids);
  free(prob);
  return ORC_OK;
}
