// cohx context: HBM-resident weights, paged KV pool and the ragged step driver.
//
// Host-side counterpart of Model::load / Model::forward_batch
// (crates/coheryn-engine/src/inference.rs:238-297, inference/batch.rs:117-273):
// weights are repacked once into the matrix-core tile layout and stay in HBM
// (the engine re-reads them from the file every step, README.md:77); each
// sequence owns a page table into one KV pool (the engine's per-session
// Vec<f32>, inference.rs:1019-1043).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "device.h"
#include "internal.h"

using namespace cohx;

namespace cohx {
int fail(cohx_ctx *ctx, int code, const std::string &msg) {
  if (ctx) ctx->err = msg;
  return code;
}
void drop_graphs(cohx_ctx *ctx) {
  for (auto &g : ctx->graphs) (void)hipGraphExecDestroy(g.second);
  ctx->graphs.clear();
}
}  // namespace cohx

#define HIP_TRY(expr)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(ctx, COHX_DEVICE, std::string(#expr ": ") + hipGetErrorString(e_)); \
  } while (0)

namespace {

int even(int n) { return (n + 1) & ~1; }

template <typename T>
int dalloc(cohx_ctx *ctx, T **p, size_t count) {
  *p = nullptr;
  if (count == 0) count = 1;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(p), count * sizeof(T));
  if (e != hipSuccess) {
    return fail(ctx, COHX_RESOURCE,
                "device allocation of " + std::to_string(count * sizeof(T)) + " bytes failed");
  }
  ctx->allocations.push_back(*p);
  e = hipMemset(*p, 0, count * sizeof(T));
  if (e != hipSuccess) return fail(ctx, COHX_DEVICE, hipGetErrorString(e));
  return COHX_OK;
}

template <typename T>
int halloc(cohx_ctx *ctx, T **p, size_t count) {
  hipError_t e = hipHostMalloc(reinterpret_cast<void **>(p), std::max<size_t>(count, 1) * sizeof(T),
                               hipHostMallocDefault);
  if (e != hipSuccess) return fail(ctx, COHX_RESOURCE, "pinned host allocation failed");
  return COHX_OK;
}

// Carves one workspace out of `base` (or only counts its bytes when base is
// null): every buffer starts on a 256-byte boundary.
struct Carver {
  uint8_t *base;
  size_t off = 0;
  template <typename T>
  void take(T *&p, size_t count) {
    off = (off + 255) & ~(size_t)255;
    p = base ? reinterpret_cast<T *>(base + off) : nullptr;
    off += std::max<size_t>(count, 1) * sizeof(T);
  }
};

// Matrix-core tile view of a Q8_0 matrix with `rows` rows of width K.
int make_q8(cohx_ctx *ctx, DeviceMatrix &m, int rows, int K, int mtiles) {
  m.view.dtype = 8;
  m.view.rows = rows;
  m.view.K = K;
  m.view.nb = K / 32;
  m.view.nbp = even(m.view.nb);
  m.view.mtiles = mtiles;
  const size_t tile_bytes = (size_t)m.view.nbp * 512;
  int rc = dalloc(ctx, &m.qs, (size_t)mtiles * tile_bytes);
  if (!rc) rc = dalloc(ctx, &m.ds, (size_t)mtiles * m.view.nbp * 16);
  m.view.qs = m.qs;
  m.view.ds = m.ds;
  return rc;
}

// Q4_0 tiles: 4 bits per value (q4_byte), scales as for Q8_0.
int make_q4(cohx_ctx *ctx, DeviceMatrix &m, int rows, int K, int mtiles) {
  m.view.dtype = 2;
  m.view.rows = rows;
  m.view.K = K;
  m.view.nb = K / 32;
  m.view.nbp = even(m.view.nb);
  m.view.mtiles = mtiles;
  const size_t tile_bytes = (size_t)m.view.nbp * 256;
  int rc = dalloc(ctx, &m.qs, (size_t)mtiles * tile_bytes);
  if (!rc) rc = dalloc(ctx, &m.ds, (size_t)mtiles * m.view.nbp * 16);
  m.view.qs = m.qs;
  m.view.ds = m.ds;
  return rc;
}

int make_f16(cohx_ctx *ctx, DeviceMatrix &m, int rows, int K) {
  m.view.dtype = 1;
  m.view.rows = rows;
  m.view.K = K;
  m.view.nb = K / 32;
  m.view.nbp = even(m.view.nb);
  m.view.mtiles = (rows + 15) / 16;
  int rc = dalloc(ctx, &m.f16, (size_t)rows * K);
  m.view.f16 = m.f16;
  return rc;
}

// K-quant tiles (device.h kq_*) of a matrix with `rows` rows of width K
// (K % 256 == 0).
int make_kq(cohx_ctx *ctx, DeviceMatrix &m, int rows, int K, int mtiles) {
  m.view.dtype = kFmtKQ;
  m.view.rows = rows;
  m.view.K = K;
  m.view.nb = K / 256;
  m.view.nbp = 0;
  m.view.mtiles = mtiles;
  const size_t tb = (size_t)mtiles * m.view.nb;  // (tile, block) pairs
  int rc = dalloc(ctx, &m.qs, tb * 4096);
  if (!rc) rc = dalloc(ctx, &m.ksc, tb * 64);
  if (!rc) rc = dalloc(ctx, &m.ds, tb * 16);
  if (!rc) rc = dalloc(ctx, &m.kdm, tb * 16);
  if (!rc) rc = dalloc(ctx, &m.kmin, tb * 128);
  m.view.qs = m.qs;
  m.view.ds = m.ds;
  m.view.ksc = m.ksc;
  m.view.kdm = m.kdm;
  m.view.kmin = m.kmin;
  return rc;
}

// Device format a GGUF matrix dtype is held in (0: unsupported).
int device_format(uint32_t dtype) {
  switch (dtype) {
    case COHX_F16: return kFmtF16;
    case COHX_Q8_0: case COHX_Q5_0: return kFmtQ8;
    case COHX_Q4_0: return kFmtQ4;
    case COHX_Q4_K: case COHX_Q6_K: return kFmtKQ;
    default: return 0;
  }
}

// Allocates m in the device format of `dtype` on its first part; later parts
// must share that format.  For the tiled formats mtiles counts 16-row tiles.
int ensure_matrix(cohx_ctx *ctx, DeviceMatrix &m, uint32_t dtype, int rows, int K, int mtiles) {
  const int fmt = device_format(dtype);
  if (m.view.dtype) {
    if (m.view.dtype != fmt)
      return fail(ctx, COHX_UNSUPPORTED,
                  "the parts of a fused matrix must share one family (Q8_0/Q5_0, Q4_0, F16 or Q4_K/Q6_K)");
    return COHX_OK;
  }
  switch (fmt) {
    case kFmtQ8: return make_q8(ctx, m, rows, K, mtiles);
    case kFmtQ4: return make_q4(ctx, m, rows, K, mtiles);
    case kFmtKQ: return make_kq(ctx, m, rows, K, mtiles);
    default: return make_f16(ctx, m, rows, K);
  }
}

// Device row of source row r when the rows are query or key heads of
// rope_d elements (0: identity): element i of a head lands on row 2i and
// element i + rope_d/2 on row 2i + 1, so the two halves NeoX RoPE rotates
// together are adjacent rows of one 16-row tile (the fused qkv epilogue
// reads them from one workgroup).  Each row's dot product is unchanged.
int rope_row(int r, int rope_d) {
  if (!rope_d) return r;
  const int head = r / rope_d, i = r % rope_d, half = rope_d / 2;
  return head * rope_d + (i < half ? 2 * i : 2 * (i - half) + 1);
}

// GGUF Q8_0 rows -> tiles [tile_first, ...) of the device layout, tile i of the
// source landing on tile tile_first + i*tile_step; rows reordered by rope_row.
int upload_q8(cohx_ctx *ctx, DeviceMatrix &m, const uint8_t *src, int rows, int tile_first,
              int tile_step, int rope_d) {
  const int nb = m.view.nb, nbp = m.view.nbp;
  const int tiles = (rows + 15) / 16;
  const size_t tile_bytes = (size_t)nbp * 512, tile_scales = (size_t)nbp * 16;
  std::vector<int8_t> qs(tiles * tile_bytes, 0);
  std::vector<uint16_t> ds(tiles * tile_scales, 0);
  for (int r = 0; r < rows; r++) {
    const int dr = rope_row(r, rope_d), t = dr / 16, c = dr % 16;
    for (int b = 0; b < nb; b++) {
      const uint8_t *blk = src + ((size_t)r * nb + b) * 34;
      ds[q8_scale(t, nbp, b, c)] = (uint16_t)(blk[0] | (blk[1] << 8));
      for (int g = 0; g < 4; g++)
        for (int j = 0; j < 8; j++)
          qs[q8_byte(t, nbp, b, g * 16 + c, j)] = (int8_t)blk[2 + g * 8 + j];
    }
  }
  HIP_TRY(hipMemcpy2D(m.qs + (size_t)tile_first * tile_bytes, tile_bytes * tile_step, qs.data(),
                      tile_bytes, tile_bytes, tiles, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D(m.ds + (size_t)tile_first * tile_scales, tile_scales * 2 * tile_step,
                      ds.data(), tile_scales * 2, tile_scales * 2, tiles, hipMemcpyHostToDevice));
  return COHX_OK;
}

// GGUF Q4_0 rows (quant.rs:97-101: value j = low nibble of byte j, value
// j+16 = high nibble) -> Q4 tiles, tile i of the source at tile_first + i*tile_step.
int upload_q4(cohx_ctx *ctx, DeviceMatrix &m, const uint8_t *src, int rows, int tile_first,
              int tile_step, int rope_d) {
  const int nb = m.view.nb, nbp = m.view.nbp;
  const int tiles = (rows + 15) / 16;
  const size_t tile_bytes = (size_t)nbp * 256, tile_scales = (size_t)nbp * 16;
  std::vector<uint8_t> qs(tiles * tile_bytes, 0);
  std::vector<uint16_t> ds(tiles * tile_scales, 0);
  for (int r = 0; r < rows; r++) {
    const int dr = rope_row(r, rope_d), t = dr / 16, c = dr % 16;
    for (int b = 0; b < nb; b++) {
      const uint8_t *blk = src + ((size_t)r * nb + b) * 18;
      ds[q8_scale(t, nbp, b, c)] = (uint16_t)(blk[0] | (blk[1] << 8));
      for (int e = 0; e < 32; e++) {
        const uint8_t nib = e < 16 ? (blk[2 + e] & 15) : (blk[2 + e - 16] >> 4);
        const int g = e / 8, k = e % 8;
        uint8_t &byte = qs[q4_byte(t, nbp, b, g * 16 + c, k)];
        byte |= k < 4 ? nib : (uint8_t)(nib << 4);
      }
    }
  }
  HIP_TRY(hipMemcpy2D(m.qs + (size_t)tile_first * tile_bytes, tile_bytes * tile_step, qs.data(),
                      tile_bytes, tile_bytes, tiles, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D(m.ds + (size_t)tile_first * tile_scales, tile_scales * 2 * tile_step,
                      ds.data(), tile_scales * 2, tile_scales * 2, tiles, hipMemcpyHostToDevice));
  return COHX_OK;
}

// GGUF Q5_0 rows (quant.rs:102-114: value j = low nibble of byte 6+j with
// bit j of the high word, value j+16 = high nibble with bit j+16; minus 16)
// as Q8_0 blocks with the same scale: the 5-bit values widen to int8 exactly,
// and the Q5_0 chain fmaf(dw*da, isum, sum) (quant.rs:273-285) is the Q8_0
// chain with its multiplicands swapped, so the same kernels give its bits.
std::vector<uint8_t> q5_as_q8(const uint8_t *src, size_t blocks) {
  std::vector<uint8_t> out(blocks * 34);
  for (size_t i = 0; i < blocks; i++) {
    const uint8_t *b = src + i * 22;
    uint8_t *o = out.data() + i * 34;
    o[0] = b[0];
    o[1] = b[1];
    const uint32_t high = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int j = 0; j < 16; j++) {
      o[2 + j] = (uint8_t)(int8_t)((int)((b[6 + j] & 15) | (((high >> j) & 1) << 4)) - 16);
      o[18 + j] = (uint8_t)(int8_t)((int)((b[6 + j] >> 4) | (((high >> (j + 16)) & 1) << 4)) - 16);
    }
  }
  return out;
}

// quant.rs:44-55: the 6-bit (scale, min) pair of Q4_K group g.
void k4_pair(const uint8_t *sc, int g, int &scale, int &minimum) {
  if (g < 4) {
    scale = sc[g] & 63;
    minimum = sc[g + 4] & 63;
  } else {
    scale = (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4);
    minimum = (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
  }
}

// GGUF Q4_K (144-byte) / Q6_K (210-byte) rows -> K-quant tiles, tile i of the
// source at tile_first + i*tile_step.  Per 256-element block: the values as
// int8 (Q4_K nibble 0..15, quant.rs:116-133; Q6_K q6_value - 32, quant.rs:56-64),
// the scale of each 16-element sub-group (Q4_K: its group's, Q6_K: the
// int8 at byte 192 + s), d, and for Q4_K dmin and the group mins.
int upload_kq(cohx_ctx *ctx, DeviceMatrix &m, uint32_t dtype, const uint8_t *src, int rows, int tile_first,
              int tile_step) {
  const int nb = m.view.nb, tiles = (rows + 15) / 16;
  const size_t bb = dtype == COHX_Q4_K ? 144 : 210;
  std::vector<int8_t> vals((size_t)tiles * nb * 4096, 0);
  std::vector<uint32_t> sc((size_t)tiles * nb * 64, 0);
  std::vector<uint16_t> dd((size_t)tiles * nb * 16, 0), dm((size_t)tiles * nb * 16, 0);
  std::vector<uint8_t> mins((size_t)tiles * nb * 128, 0);
  for (int r = 0; r < rows; r++) {
    const int t = r / 16, rr = r % 16;
    for (int b = 0; b < nb; b++) {
      const uint8_t *blk = src + ((size_t)r * nb + b) * bb;
      const size_t wr = kq_row(t, nb, b, rr);
      int subscale[16];
      if (dtype == COHX_Q4_K) {
        dd[wr] = (uint16_t)(blk[0] | (blk[1] << 8));
        dm[wr] = (uint16_t)(blk[2] | (blk[3] << 8));
        for (int g = 0; g < 8; g++) {
          int scale, minimum;
          k4_pair(blk + 4, g, scale, minimum);
          subscale[2 * g] = subscale[2 * g + 1] = scale;
          mins[wr * 8 + g] = (uint8_t)minimum;
        }
      } else {
        dd[wr] = (uint16_t)(blk[208] | (blk[209] << 8));
        for (int s2 = 0; s2 < 16; s2++) subscale[s2] = (int8_t)blk[192 + s2];
      }
      for (int i = 0; i < 256; i++) {
        int v;
        if (dtype == COHX_Q4_K) {
          const int g = i / 32;
          const uint8_t packed = blk[16 + (g / 2) * 32 + i % 32];
          v = g % 2 == 0 ? (packed & 15) : (packed >> 4);
        } else {
          const int half = i / 128, grp = (i % 128) / 32, ln = i % 32;
          const uint8_t low = blk[half * 64 + (grp % 2) * 32 + ln];
          const int lo4 = grp < 2 ? (low & 15) : (low >> 4);
          const int hi2 = (blk[128 + half * 32 + ln] >> (2 * grp)) & 3;
          v = (lo4 | (hi2 << 4)) - 32;
        }
        const int c = i % 8, mm = i / 8;
        vals[kq_byte(t, nb, b, c, (mm / 8) * 16 + rr, mm % 8)] = (int8_t)v;
      }
      for (int kg = 0; kg < 4; kg++) {
        uint32_t word = 0;
        for (int j = 0; j < 4; j++) word |= (uint32_t)(uint8_t)(int8_t)subscale[4 * kg + j] << (8 * j);
        sc[kq_row(t, nb, b, 0) * 4 + kg * 16 + rr] = word;
      }
    }
  }
  const size_t tv = (size_t)nb * 4096, ts = (size_t)nb * 64 * 4, th = (size_t)nb * 16 * 2,
               tm = (size_t)nb * 128;
  HIP_TRY(hipMemcpy2D(m.qs + (size_t)tile_first * tv, tv * tile_step, vals.data(), tv, tv, tiles,
                      hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D((uint8_t *)m.ksc + (size_t)tile_first * ts, ts * tile_step, sc.data(), ts, ts, tiles,
                      hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D((uint8_t *)m.ds + (size_t)tile_first * th, th * tile_step, dd.data(), th, th, tiles,
                      hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D((uint8_t *)m.kdm + (size_t)tile_first * th, th * tile_step, dm.data(), th, th, tiles,
                      hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy2D(m.kmin + (size_t)tile_first * tm, tm * tile_step, mins.data(), tm, tm, tiles,
                      hipMemcpyHostToDevice));
  if (dtype == COHX_Q4_K) m.view.has_min = 1;
  return COHX_OK;
}

int upload_f16(cohx_ctx *ctx, DeviceMatrix &m, const void *src, int rows, int row_first) {
  HIP_TRY(hipMemcpy(m.f16 + (size_t)row_first * m.view.K, src, (size_t)rows * m.view.K * 2,
                    hipMemcpyHostToDevice));
  return COHX_OK;
}

// Tiled formats: `first` and `step` count 16-row tiles and rope_d reorders
// the rows (rope_row; Q8/Q4 only); F16: `first` counts rows and the order is
// the source's.  The matrix is already allocated (ensure_matrix).
int upload_matrix(cohx_ctx *ctx, DeviceMatrix &m, uint32_t dtype, const void *data, int rows,
                  int first, int step, int rope_d = 0) {
  const uint8_t *src = (const uint8_t *)data;
  switch (dtype) {
    case COHX_Q8_0: return upload_q8(ctx, m, src, rows, first, step, rope_d);
    case COHX_Q5_0: {
      const std::vector<uint8_t> q8 = q5_as_q8(src, (size_t)rows * (m.view.K / 32));
      return upload_q8(ctx, m, q8.data(), rows, first, step, rope_d);
    }
    case COHX_Q4_0: return upload_q4(ctx, m, src, rows, first, step, rope_d);
    case COHX_Q4_K: case COHX_Q6_K: return upload_kq(ctx, m, dtype, src, rows, first, step);
    default: return upload_f16(ctx, m, data, rows, first);
  }
}

// quant.rs:13-35 row_bytes (0: unsupported dtype or width not block-aligned).
size_t row_bytes(uint32_t dtype, uint64_t width) {
  const uint64_t blk = dtype == COHX_Q4_K || dtype == COHX_Q6_K ? 256
                       : (dtype == COHX_Q4_0 || dtype == COHX_Q5_0 || dtype == COHX_Q8_0) ? 32 : 1;
  if (!width || width % blk) return 0;
  switch (dtype) {
    case COHX_F32: return width * 4;
    case COHX_F16: return width * 2;
    case COHX_Q4_0: return width / 32 * 18;
    case COHX_Q5_0: return width / 32 * 22;
    case COHX_Q8_0: return width / 32 * 34;
    case COHX_Q4_K: return width / 256 * 144;
    case COHX_Q6_K: return width / 256 * 210;
    default: return 0;
  }
}

}  // namespace

namespace cohx {
size_t upload_words(uint32_t rows, uint32_t lanes, uint32_t kv_cap) {
  return (size_t)lanes * 4 + rows + 1 + (size_t)rows * ((kv_cap + 255) / 256);
}

size_t layout_workspace(const cohx_model_desc &d, int nbp_h, int nbp_f, uint32_t R, uint32_t NL,
                        uint32_t kv_cap, bool logits, uint8_t *base, Workspace *out) {
  const size_t H = d.hidden, F = d.intermediate, V = d.vocabulary, NH = d.heads, NKV = d.kv_heads,
               D = d.head_dim, KVD = NKV * D;
  const bool packed = d.weight_dtype != COHX_F16;
  const bool kquant = d.weight_dtype == COHX_Q4_K || d.weight_dtype == COHX_Q6_K || d.weight_dtype == COHX_MIXED;
  const size_t rtiles = (R + 15) / 16, nbp_max = (size_t)std::max(nbp_h, nbp_f);
  const size_t nsc = (kv_cap + 255) / 256, chunks = (kv_cap + kChunk - 1) / kChunk;
  Workspace tmp;
  Workspace &w = out ? *out : tmp;
  w = Workspace();
  w.rows = R;
  w.lanes = NL;
  w.kv_cap = kv_cap;
  w.max_chunks = (uint32_t)chunks;
  // prefill-chunk attention work items: 16-row tiles x key segments; key
  // tile images of the chunk lanes (16+ rows each, so at most R / 16 of them)
  w.max_tiles = ((R + 15) / 16 + NL) * ((kv_cap + kChunkSegKeys - 1) / kChunkSegKeys);
  w.max_images = D == 64 ? (uint32_t)(std::min<size_t>(NL, R / 16) *
                                      ((kv_cap + kChunkTileKeys - 1) / kChunkTileKeys) * NKV)
                         : 0;
  w.logits_room = logits;
  Carver c{base};
  c.take(w.lane_info, upload_words(R, NL, kv_cap));
  if (base) {
    w.tokens = w.lane_info + (size_t)NL * 4;
    w.att_items = w.tokens + R;
  }
  c.take(w.cu, NL + 1);
  c.take(w.row_pos, R);
  c.take(w.row_slot, R);
  c.take(w.row_lane, R);
  c.take(w.row_token, R);
  c.take(w.row_seq, R);
  c.take(w.lane_last, NL);
  c.take(w.row_err, R);
  c.take(w.x, R * H);
  c.take(w.qkv, R * (H + 2 * KVD));
  c.take(w.q_rot, R * H);
  c.take(w.h, R * F);
  c.take(w.act_qs, rtiles * nbp_max * 512);
  c.take(w.act_ds, rtiles * nbp_max * 16);
  if (packed) {
    c.take(w.down_qs, rtiles * nbp_f * 512);
    c.take(w.down_ds, rtiles * nbp_f * 16);
  }
  c.take(w.act_f16, R * std::max(H, F));
  if (kquant) {
    const size_t nb256 = std::max(H, F) / 256;
    c.take(w.act_kd, rtiles * 16 * nb256);
    c.take(w.act_ksum, rtiles * 16 * nb256 * 16);
    c.take(w.act_f32, R * H);
  }
  c.take(w.scores, R * NKV * kv_cap * 8);
  c.take(w.chunk_max, R * NH * nsc);
  c.take(w.row_max, R * NH);
  c.take(w.den_part, R * NH * nsc);
  c.take(w.tiles, w.max_tiles);
  c.take(w.stage, w.max_images);
  c.take(w.img, (size_t)w.max_images * kChunkImgUnits);
  c.take(w.row_skip, R);
  c.take(w.row_map, R);
  c.take(w.partial, R * NH * chunks * D);
  if (logits) c.take(w.logits, (size_t)NL * V);
  c.take(w.argmax, NL);
  c.take(w.argmax_part, (size_t)NL * ((V + 15) / 16));
  return (c.off + 255) & ~(size_t)255;
}
}  // namespace cohx

// ---- device scratch of the allocation-free step ------------------------------
// cohx_step_noalloc carves its workspace from this array instead of the
// context's block.  Each device that loads the library holds its own copy
// until the process ends; host code uses only the address resolved per
// device below, never the array's name (a host-side stand-in).
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<uint8_t *> g_scratch_ptr;  // per device, resolved once with that device current

// Called by cohx_create with ctx->device current.
int resolve_scratch(cohx_ctx *ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((size_t)ctx->device >= g_scratch_ptr.size()) g_scratch_ptr.resize(ctx->device + 1, nullptr);
  uint8_t *&p = g_scratch_ptr[ctx->device];
  if (!p) {
    void *addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return fail(ctx, COHX_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    p = static_cast<uint8_t *>(addr);
  }
  ctx->scratch = p;
  return COHX_OK;
}
}  // namespace

extern "C" {

const char *cohx_last_error(const cohx_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int cohx_create(const cohx_model_desc *d, int device, cohx_ctx **out) {
  if (!d || !out) return COHX_INVALID_REQUEST;
  *out = nullptr;
  if (!d->layers || !d->hidden || !d->heads || !d->kv_heads || d->hidden % d->heads ||
      d->heads % d->kv_heads || d->head_dim != d->hidden / d->heads || d->head_dim % 32 ||
      d->head_dim > 128 || d->heads / d->kv_heads > (uint32_t)kMaxGroup || d->hidden % 32 ||
      d->intermediate % 32 || !d->vocabulary)
    return COHX_INVALID_GGUF;
  if (d->weight_dtype != COHX_MIXED && !device_format(d->weight_dtype)) return COHX_UNSUPPORTED;
  if (!attention_shape_supported((int)d->head_dim, (int)(d->heads / d->kv_heads)))
    return COHX_UNSUPPORTED;
  if (d->kv_dtype != 0) return COHX_UNSUPPORTED;
  if (!d->max_lanes || d->max_lanes > 1024 || !d->max_rows || d->max_rows < d->max_lanes ||
      !d->max_seqs || !d->max_context || d->max_context > d->context || d->n_eog > 4)
    return COHX_INVALID_REQUEST;
  cohx_ctx *ctx = new cohx_ctx();
  ctx->desc = *d;
  ctx->device = device;
  // COHX_GRAPHS=0 issues every launch directly (graphs are on by default)
  if (const char *g = std::getenv("COHX_GRAPHS")) ctx->use_graphs = std::strcmp(g, "0") != 0;
  // COHX_PREFILL_MFMA=0 keeps tall F16 batches on the exact (f64-sum) kernels
  if (const char *g = std::getenv("COHX_PREFILL_MFMA")) ctx->prefill_mfma = std::strcmp(g, "0") != 0;
  auto bail = [&](int rc) {
    cohx_destroy(ctx);
    return rc;
  };
  if (hipSetDevice(device) != hipSuccess) return bail(COHX_DEVICE);
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->join_ev, hipEventDisableTiming) != hipSuccess)
    return bail(COHX_DEVICE);
  if (int rc_s = resolve_scratch(ctx)) return bail(rc_s);
  const int H = d->hidden, F = d->intermediate, V = d->vocabulary, NH = d->heads,
            NKV = d->kv_heads, D = d->head_dim, KVD = NKV * D, L = d->layers;
  const int R = d->max_rows;
  ctx->nbp_h = even(H / 32);
  ctx->nbp_f = even(F / 32);
  ctx->nbp_max = std::max(ctx->nbp_h, ctx->nbp_f);
  ctx->max_pages = (int)((d->max_context + kPage - 1) / kPage);
  ctx->max_chunks = (int)((d->max_context + kChunk - 1) / kChunk);
  const uint32_t pages = d->kv_pages ? d->kv_pages : d->max_seqs * (uint32_t)ctx->max_pages;
  ctx->layer_stride = (size_t)pages * NKV * kPage * D;
  int rc = COHX_OK;
  // vectors; each matrix is allocated in its device format by its first
  // uploaded part (ensure_matrix)
  ctx->layers.resize(L);
  for (int l = 0; l < L && !rc; l++) {
    Layer &ly = ctx->layers[l];
    rc = dalloc(ctx, &ly.attn_norm, H);
    if (!rc) rc = dalloc(ctx, &ly.ffn_norm, H);
    if (!rc) rc = dalloc(ctx, &ly.bqkv, H + 2 * KVD);
  }
  if (H % 16 || KVD % 16) rc = rc ? rc : COHX_INVALID_GGUF;
  if (!rc) rc = dalloc(ctx, &ctx->output_norm, H);
  // RoPE table: (cos, sin) of the engine's iterative angle (cpu.rs:59-73).
  if (!rc) {
    std::vector<float2> tab((size_t)d->max_context * (D / 2));
    const float step = powf(d->rope_base, -2.0f / (float)D);
    for (uint32_t p = 0; p < d->max_context; p++) {
      float angle = (float)p;
      for (int i = 0; i < D / 2; i++) {
        tab[(size_t)p * (D / 2) + i] = make_float2(cosf(angle), sinf(angle));
        angle *= step;
      }
    }
    rc = dalloc(ctx, &ctx->rope, tab.size());
    if (!rc && hipMemcpy(ctx->rope, tab.data(), tab.size() * sizeof(float2),
                         hipMemcpyHostToDevice) != hipSuccess)
      rc = COHX_DEVICE;
  }
  // KV pool and page tables
  if (!rc) rc = dalloc(ctx, &ctx->kpool, ctx->layer_stride * L);
  if (!rc) rc = dalloc(ctx, &ctx->vpool, ctx->layer_stride * L);
  if (!rc) rc = dalloc(ctx, &ctx->page_table, (size_t)d->max_seqs * ctx->max_pages);
  ctx->h_page_table.assign((size_t)d->max_seqs * ctx->max_pages, -1);
  ctx->pt_dirty.assign(d->max_seqs, 1);
  ctx->page_refs.assign(pages, 0);
  for (int32_t p = (int32_t)pages - 1; p >= 0; p--) ctx->free_pages.push_back(p);
  ctx->seqs.resize(d->max_seqs);
  for (int32_t s = (int32_t)d->max_seqs - 1; s >= 0; s--) ctx->free_seqs.push_back((uint32_t)s);
  // step workspaces: one device block carved by layout_workspace, and pinned
  // host staging
  if (!rc) {
    const size_t bytes = layout_workspace(*d, ctx->nbp_h, ctx->nbp_f, R, d->max_lanes, d->max_context,
                                          true, nullptr, nullptr);
    rc = dalloc(ctx, &ctx->ws_block, bytes);
    if (!rc)
      layout_workspace(*d, ctx->nbp_h, ctx->nbp_f, R, d->max_lanes, d->max_context, true, ctx->ws_block,
                       &ctx->ws);
  }
  Staging &h = ctx->host;
  const uint32_t NL = d->max_lanes;
  if (!rc) rc = halloc(ctx, &h.h_tiles, (size_t)ctx->ws.max_tiles);
  if (!rc) rc = halloc(ctx, &h.h_stage, (size_t)std::max(ctx->ws.max_images, 1u));
  if (!rc) rc = halloc(ctx, &h.h_row_skip, (size_t)R);
  if (!rc) rc = halloc(ctx, &h.h_row_map, (size_t)R);
  if (!rc) rc = halloc(ctx, &h.h_kv, (size_t)R);
  if (!rc) rc = halloc(ctx, &h.h_upload, upload_words(R, NL, d->max_context));
  if (!rc) rc = halloc(ctx, &h.h_row_err, R);
  if (!rc) rc = halloc(ctx, &h.h_argmax, NL);
  if (!rc) rc = halloc(ctx, &ctx->h_pt_stage, ctx->h_page_table.size());
  if (!rc && hipEventCreateWithFlags(&ctx->pt_done, hipEventDisableTiming) != hipSuccess) rc = COHX_DEVICE;
  if (rc) return bail(rc);
  *out = ctx;
  return COHX_OK;
}

void cohx_destroy(cohx_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  drop_graphs(ctx);
  for (void *p : ctx->allocations) (void)hipFree(p);
  for (void *p : {(void *)ctx->host.h_upload, (void *)ctx->host.h_row_err, (void *)ctx->host.h_argmax,
                  (void *)ctx->host.h_tiles, (void *)ctx->host.h_stage, (void *)ctx->host.h_row_skip, (void *)ctx->host.h_row_map,
                  (void *)ctx->host.h_kv, (void *)ctx->h_pt_stage})
    if (p) (void)hipHostFree(p);
  q35_free(ctx);
  if (ctx->done) (void)hipEventDestroy(ctx->done);
  if (ctx->pt_done) (void)hipEventDestroy(ctx->pt_done);
  if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
  if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
  if (ctx->side) (void)hipStreamDestroy(ctx->side);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

// compat.rs:161-221: names and shapes of the Qwen2 graph.
int cohx_upload_tensor(cohx_ctx *ctx, const char *name, uint32_t dtype, uint64_t ne0,
                       uint64_t ne1, const void *data, size_t bytes) {
  if (ctx && ctx->q35 && name && data) {
    if (ctx->finalized) return fail(ctx, COHX_INVALID_REQUEST, "context already finalized");
    (void)hipSetDevice(ctx->device);
    return q35_upload(ctx, name, dtype, ne0, ne1, data, bytes);
  }
  if (!ctx || !name || !data) return COHX_INVALID_REQUEST;
  if (hipSetDevice(ctx->device) != hipSuccess) return fail(ctx, COHX_DEVICE, "hipSetDevice");
  const cohx_model_desc &d = ctx->desc;
  const uint64_t H = d.hidden, F = d.intermediate, V = d.vocabulary,
                 KVD = (uint64_t)d.kv_heads * d.head_dim;
  const size_t rb = row_bytes(dtype, ne0);
  if (!rb) return fail(ctx, COHX_UNSUPPORTED, std::string("unsupported dtype for ") + name);
  if (rb * ne1 != bytes) return fail(ctx, COHX_INVALID_GGUF, std::string("size mismatch: ") + name);
  const std::string n(name);
  auto expect = [&](uint64_t e0, uint64_t e1) { return ne0 == e0 && ne1 == e1; };
  auto vec_f32 = [&](float *dst, uint64_t len, uint64_t offset) -> int {
    if (dtype != 0 || !expect(len, 1))
      return fail(ctx, COHX_INVALID_GGUF, "incorrect shape or dtype for " + n);
    HIP_TRY(hipMemcpy(dst + offset, data, len * 4, hipMemcpyHostToDevice));
    return COHX_OK;
  };
  // a matrix: the context's dtype, or any supported one for COHX_MIXED
  auto matrix_dtype_ok = [&]() -> int {
    if (!device_format(dtype) || (d.weight_dtype != COHX_MIXED && dtype != d.weight_dtype))
      return fail(ctx, COHX_UNSUPPORTED, "matrix dtype " + std::to_string(dtype) + " of " + n +
                                             " is not the context's weight dtype");
    return COHX_OK;
  };
  const int fmt = device_format(dtype);
  const bool tiled = fmt == kFmtQ8 || fmt == kFmtQ4 || fmt == kFmtKQ;
  int rc = COHX_OK;
  if (n == "token_embd.weight") {
    if (!expect(H, V)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
    rc = matrix_dtype_ok();
    if (!rc) rc = ensure_matrix(ctx, ctx->embd, dtype, (int)V, (int)H, (int)((V + 15) / 16));
    if (!rc) rc = upload_matrix(ctx, ctx->embd, dtype, data, (int)V, 0, 1);
    ctx->embd.gguf_bytes = bytes;
  } else if (n == "output.weight") {
    if (d.tied) return fail(ctx, COHX_INVALID_REQUEST, "context was created with a tied head");
    if (!expect(H, V)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
    rc = matrix_dtype_ok();
    if (!rc) rc = ensure_matrix(ctx, ctx->output, dtype, (int)V, (int)H, (int)((V + 15) / 16));
    if (!rc) rc = upload_matrix(ctx, ctx->output, dtype, data, (int)V, 0, 1);
    ctx->output.gguf_bytes = bytes;
  } else if (n == "output_norm.weight") {
    rc = vec_f32(ctx->output_norm, H, 0);
  } else {
    unsigned layer = 0;
    char suffix[64] = {0};
    if (std::sscanf(name, "blk.%u.%63s", &layer, suffix) != 2 || layer >= d.layers)
      return fail(ctx, COHX_INVALID_GGUF, "unexpected tensor " + n);
    Layer &ly = ctx->layers[layer];
    const std::string s(suffix);
    if (s == "attn_norm.weight") rc = vec_f32(ly.attn_norm, H, 0);
    else if (s == "ffn_norm.weight") rc = vec_f32(ly.ffn_norm, H, 0);
    else if (s == "attn_q.bias") rc = vec_f32(ly.bqkv, H, 0);
    else if (s == "attn_k.bias") rc = vec_f32(ly.bqkv, KVD, H);
    else if (s == "attn_v.bias") rc = vec_f32(ly.bqkv, KVD, H + KVD);
    else if (s == "attn_q.weight" || s == "attn_k.weight" || s == "attn_v.weight") {
      const uint64_t rows = s == "attn_q.weight" ? H : KVD;
      const uint64_t first = s == "attn_q.weight" ? 0 : s == "attn_k.weight" ? H : H + KVD;
      if (!expect(H, rows)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
      rc = matrix_dtype_ok();
      if (!rc)
        rc = ensure_matrix(ctx, ly.qkv, dtype, (int)(H + 2 * KVD), (int)H, (int)(H / 16 + 2 * ((KVD + 15) / 16)));
      // Q8/Q4 query and key rows pair each head's RoPE halves (rope_row) for
      // the fused epilogue; K-quant and F16 rows keep the source order
      if (!rc)
        rc = upload_matrix(ctx, ly.qkv, dtype, data, (int)rows, (int)(tiled ? first / 16 : first), 1,
                           s == "attn_v.weight" || fmt == kFmtKQ ? 0 : (int)d.head_dim);
      ly.qkv.gguf_bytes += bytes;
    } else if (s == "attn_output.weight") {
      if (!expect(H, H)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
      rc = matrix_dtype_ok();
      if (!rc) rc = ensure_matrix(ctx, ly.o, dtype, (int)H, (int)H, (int)((H + 15) / 16));
      if (!rc) rc = upload_matrix(ctx, ly.o, dtype, data, (int)H, 0, 1);
      ly.o.gguf_bytes = bytes;
    } else if (s == "ffn_gate.weight" || s == "ffn_up.weight") {
      if (!expect(H, F)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
      const bool up = s == "ffn_up.weight";
      rc = matrix_dtype_ok();
      if (!rc) rc = ensure_matrix(ctx, ly.gu, dtype, (int)(2 * F), (int)H, (int)(2 * ((F + 15) / 16)));
      // tiled: gate tile i -> tile 2i, up tile i -> tile 2i+1; F16: gate rows then up rows.
      if (!rc)
        rc = tiled ? upload_matrix(ctx, ly.gu, dtype, data, (int)F, up ? 1 : 0, 2)
                   : upload_matrix(ctx, ly.gu, dtype, data, (int)F, up ? (int)F : 0, 1);
      ly.gu.gguf_bytes += bytes;
    } else if (s == "ffn_down.weight") {
      if (!expect(F, H)) return fail(ctx, COHX_INVALID_GGUF, "incorrect shape for " + n);
      rc = matrix_dtype_ok();
      if (!rc) rc = ensure_matrix(ctx, ly.down, dtype, (int)H, (int)F, (int)((H + 15) / 16));
      if (!rc) rc = upload_matrix(ctx, ly.down, dtype, data, (int)H, 0, 1);
      ly.down.gguf_bytes = bytes;
    } else {
      return fail(ctx, COHX_UNSUPPORTED, "unexpected tensor in Qwen2 graph: " + n);
    }
  }
  if (!rc && std::find(ctx->uploaded.begin(), ctx->uploaded.end(), n) == ctx->uploaded.end())
    ctx->uploaded.push_back(n);
  return rc;
}

int cohx_finalize(cohx_ctx *ctx) {
  if (ctx && ctx->q35) return q35_finalize(ctx);
  if (!ctx) return COHX_INVALID_REQUEST;
  const cohx_model_desc &d = ctx->desc;
  std::vector<std::string> need = {"token_embd.weight", "output_norm.weight"};
  if (!d.tied) need.push_back("output.weight");
  const char *per[] = {"attn_norm.weight", "ffn_norm.weight", "attn_q.weight", "attn_k.weight",
                       "attn_v.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias",
                       "attn_output.weight", "ffn_gate.weight", "ffn_up.weight",
                       "ffn_down.weight"};
  for (uint32_t l = 0; l < d.layers; l++)
    for (const char *s : per) need.push_back("blk." + std::to_string(l) + "." + s);
  for (const auto &n : need)
    if (std::find(ctx->uploaded.begin(), ctx->uploaded.end(), n) == ctx->uploaded.end())
      return fail(ctx, COHX_INVALID_GGUF, "missing required tensor " + n);
  if (ctx->uploaded.size() != need.size())
    return fail(ctx, COHX_UNSUPPORTED, "unexpected tensors in Qwen2 graph");
  uint64_t total = ctx->embd.gguf_bytes + (d.tied ? 0 : ctx->output.gguf_bytes);
  for (auto &ly : ctx->layers)
    total += ly.qkv.gguf_bytes + ly.o.gguf_bytes + ly.gu.gguf_bytes + ly.down.gguf_bytes;
  // the embedding is read as a matrix only as the tied head
  ctx->matrix_bytes = d.tied ? total : total - ctx->embd.gguf_bytes;
  // the packed-prefill regime's quantized GEMM covers Q8/Q4 tiles with whole
  // block pairs per ring stage (K a multiple of 128)
  ctx->quant_gemm = true;
  for (auto &ly : ctx->layers)
    for (const DeviceMatrix *m : {&ly.qkv, &ly.o, &ly.gu, &ly.down})
      ctx->quant_gemm &= (m->view.dtype == kFmtQ8 || m->view.dtype == kFmtQ4) && m->view.K % 128 == 0;
  ctx->finalized = true;
  return COHX_OK;
}

// ---- sequences -------------------------------------------------------------

static int take_page(cohx_ctx *ctx, int32_t *page) {
  if (ctx->free_pages.empty()) return fail(ctx, COHX_RESOURCE, "KV pool exhausted");
  *page = ctx->free_pages.back();
  ctx->free_pages.pop_back();
  ctx->page_refs[*page] = 1;
  return COHX_OK;
}

static void drop_page(cohx_ctx *ctx, int32_t page) {
  if (page < 0) return;
  if (--ctx->page_refs[page] == 0) ctx->free_pages.push_back(page);
}

static void set_table(cohx_ctx *ctx, uint32_t seq, size_t idx, int32_t page) {
  ctx->h_page_table[(size_t)seq * ctx->max_pages + idx] = page;
  ctx->pt_dirty[seq] = 1;
}

static bool valid_seq(const cohx_ctx *ctx, uint32_t seq) {
  return seq < ctx->seqs.size() && ctx->seqs[seq].live;
}

// Pages for positions [0, rows) present and writable from `from` on.
static int ensure_pages(cohx_ctx *ctx, uint32_t seq, uint32_t from, uint32_t rows) {
  Sequence &s = ctx->seqs[seq];
  const size_t need = (rows + kPage - 1) / kPage;
  for (size_t i = from / kPage; i < need; i++) {
    if (i >= s.pages.size()) s.pages.resize(i + 1, -1);
    int32_t p = s.pages[i];
    if (p < 0) {
      int rc = take_page(ctx, &p);
      if (rc) return rc;
      s.pages[i] = p;
      set_table(ctx, seq, i, p);
    } else if (ctx->page_refs[p] > 1) {  // copy on write of a shared page
      int32_t q;
      int rc = take_page(ctx, &q);
      if (rc) return rc;
      launch_copy_page(ctx->stream, ctx->kpool, ctx->vpool, ctx->layer_stride,
                       (int)ctx->desc.layers, (int)(ctx->desc.kv_heads * kPage * ctx->desc.head_dim),
                       p, q);
      drop_page(ctx, p);
      s.pages[i] = q;
      set_table(ctx, seq, i, q);
    }
  }
  return COHX_OK;
}

// Uploads the page-table rows changed since the last upload: the range from
// the first to the last changed sequence (rows between them are unchanged,
// so equal on both sides) goes through pinned staging in one copy, and the
// mirror may change again as soon as this returns.
static int sync_page_table(cohx_ctx *ctx) {
  size_t lo = ctx->pt_dirty.size(), hi = 0;
  for (size_t s = 0; s < ctx->pt_dirty.size(); s++)
    if (ctx->pt_dirty[s]) {
      lo = std::min(lo, s);
      hi = s;
    }
  if (lo > hi) return COHX_OK;
  if (ctx->pt_pending) HIP_TRY(hipEventSynchronize(ctx->pt_done));  // the staging rows are free again
  const size_t first = lo * ctx->max_pages, count = (hi - lo + 1) * ctx->max_pages;
  std::memcpy(ctx->h_pt_stage + first, ctx->h_page_table.data() + first, count * sizeof(int32_t));
  HIP_TRY(hipMemcpyAsync(ctx->page_table + first, ctx->h_pt_stage + first, count * sizeof(int32_t),
                         hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipEventRecord(ctx->pt_done, ctx->stream));
  ctx->pt_pending = true;
  std::fill(ctx->pt_dirty.begin() + lo, ctx->pt_dirty.begin() + hi + 1, (uint8_t)0);
  return COHX_OK;
}

int cohx_seq_alloc(cohx_ctx *ctx, uint32_t capacity, uint32_t *seq) {
  if (!ctx || !seq) return COHX_INVALID_REQUEST;
  if (capacity == 0 || capacity > ctx->desc.max_context)
    return fail(ctx, COHX_INVALID_REQUEST, "sequence capacity outside 1..=max_context");
  if (ctx->free_seqs.empty()) return fail(ctx, COHX_RESOURCE, "no free sequence slots");
  const uint32_t s = ctx->free_seqs.back();
  ctx->free_seqs.pop_back();
  Sequence &q = ctx->seqs[s];
  q.live = true;
  q.length = 0;
  q.capacity = capacity;
  q.pages.clear();
  *seq = s;
  if (ctx->q35) {
    (void)hipSetDevice(ctx->device);
    return q35_seq_reset(ctx, s);
  }
  return COHX_OK;
}

int cohx_seq_free(cohx_ctx *ctx, uint32_t seq) {
  if (!ctx || !valid_seq(ctx, seq)) return COHX_INVALID_REQUEST;
  Sequence &q = ctx->seqs[seq];
  for (size_t i = 0; i < q.pages.size(); i++) {
    drop_page(ctx, q.pages[i]);
    set_table(ctx, seq, i, -1);
  }
  q = Sequence();
  ctx->free_seqs.push_back(seq);
  return COHX_OK;
}

int cohx_seq_fork(cohx_ctx *ctx, uint32_t src, uint32_t rows, uint32_t capacity, uint32_t *seq) {
  if (!ctx || !valid_seq(ctx, src) || !seq) return COHX_INVALID_REQUEST;
  if (rows > ctx->seqs[src].length || rows > capacity)
    return fail(ctx, COHX_INVALID_REQUEST, "fork longer than the source or the capacity");
  if (ctx->q35 && rows != ctx->seqs[src].length)
    return fail(ctx, COHX_UNSUPPORTED, "recurrent state forks only at the source length");
  int rc = cohx_seq_alloc(ctx, capacity, seq);
  if (rc) return rc;
  if (ctx->q35) {
    rc = q35_seq_copy(ctx, src, *seq, rows);
    if (rc) return rc;
    ctx->seqs[*seq].length = rows;
    return COHX_OK;
  }
  Sequence &d = ctx->seqs[*seq];
  const Sequence &s = ctx->seqs[src];
  const size_t pages = (rows + kPage - 1) / kPage;
  d.pages.assign(pages, -1);
  for (size_t i = 0; i < pages; i++) {
    d.pages[i] = s.pages[i];
    ctx->page_refs[s.pages[i]]++;
    set_table(ctx, *seq, i, s.pages[i]);
  }
  d.length = rows;
  return COHX_OK;
}

int cohx_seq_truncate(cohx_ctx *ctx, uint32_t seq, uint32_t rows) {
  if (!ctx || !valid_seq(ctx, seq)) return COHX_INVALID_REQUEST;
  Sequence &q = ctx->seqs[seq];
  if (rows > q.length) return fail(ctx, COHX_INVALID_REQUEST, "truncate beyond length");
  if (ctx->q35 && rows != q.length)
    return fail(ctx, COHX_UNSUPPORTED, "recurrent state cannot be rewound");
  const size_t keep = (rows + kPage - 1) / kPage;
  for (size_t i = keep; i < q.pages.size(); i++) {
    drop_page(ctx, q.pages[i]);
    set_table(ctx, seq, i, -1);
  }
  if (q.pages.size() > keep) q.pages.resize(keep);
  q.length = rows;
  return COHX_OK;
}

int cohx_seq_length(const cohx_ctx *ctx, uint32_t seq, uint32_t *rows) {
  if (!ctx || !valid_seq(ctx, seq) || !rows) return COHX_INVALID_REQUEST;
  *rows = ctx->seqs[seq].length;
  return COHX_OK;
}

uint32_t cohx_seq_pages(const cohx_ctx *ctx, uint32_t seq, int32_t *out, uint32_t cap) {
  if (ctx && ctx->q35) return 0;  // no KV pages: contiguous per-sequence state
  if (!ctx || !valid_seq(ctx, seq)) return 0;
  const Sequence &q = ctx->seqs[seq];
  const uint32_t n = (uint32_t)q.pages.size();
  if (out) std::memcpy(out, q.pages.data(), std::min(n, cap) * sizeof(int32_t));
  return n;
}

int cohx_seq_read_kv_rows(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int values, uint32_t first,
                          uint32_t count, float *out) {
  if (ctx && ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "row ranges are for paged Qwen2 contexts");
  if (!ctx || !valid_seq(ctx, seq) || layer >= ctx->desc.layers || (!out && count))
    return COHX_INVALID_REQUEST;
  const Sequence &q = ctx->seqs[seq];
  if ((uint64_t)first + count > q.length) return fail(ctx, COHX_INVALID_REQUEST, "rows beyond the length");
  HIP_TRY(hipSetDevice(ctx->device));
  const int NKV = ctx->desc.kv_heads, D = ctx->desc.head_dim;
  const float *pool = (values ? ctx->vpool : ctx->kpool) + (size_t)layer * ctx->layer_stride;
  std::vector<float> page((size_t)NKV * kPage * D);
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  const uint32_t end = first + count;
  for (uint32_t i = first / kPage; i * kPage < end; i++) {
    HIP_TRY(hipMemcpy(page.data(), pool + (size_t)q.pages[i] * page.size(),
                      page.size() * sizeof(float), hipMemcpyDeviceToHost));
    for (uint32_t o = 0; o < (uint32_t)kPage; o++) {
      const uint32_t pos = i * kPage + o;
      if (pos < first || pos >= end) continue;
      for (int g = 0; g < NKV; g++)
        for (int j = 0; j < D; j++)
          out[((size_t)(pos - first) * NKV + g) * D + j] =
              page[values ? v_at(0, g, NKV, (int)o, j, D) : k_at(0, i, g, NKV, (int)o, j, D)];
    }
  }
  return COHX_OK;
}

int cohx_seq_read_kv(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int values, float *out) {
  if (!ctx || !valid_seq(ctx, seq) || layer >= ctx->desc.layers || !out)
    return COHX_INVALID_REQUEST;
  if (ctx->q35) {
    (void)hipSetDevice(ctx->device);
    return q35_read_state(ctx, seq, layer, values, out);
  }
  return cohx_seq_read_kv_rows(ctx, seq, layer, values, 0, ctx->seqs[seq].length, out);
}

int cohx_seq_fill_synthetic(cohx_ctx *ctx, uint32_t seq, uint32_t rows, uint64_t seed,
                            uint32_t stream) {
  if (ctx && ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "no synthetic fill for Qwen3.5");
  if (!ctx || !valid_seq(ctx, seq)) return COHX_INVALID_REQUEST;
  Sequence &q = ctx->seqs[seq];
  if (rows > q.capacity) return fail(ctx, COHX_RESOURCE, "rows exceed the sequence capacity");
  if (rows < q.length) return fail(ctx, COHX_INVALID_REQUEST, "rows below the sequence length");
  HIP_TRY(hipSetDevice(ctx->device));
  const uint32_t from = q.length;
  int rc = ensure_pages(ctx, seq, from, rows);
  if (rc) return rc;
  if (rows > from) {
    int32_t *pages = nullptr;
    HIP_TRY(hipMalloc(&pages, q.pages.size() * sizeof(int32_t)));
    hipError_t e = hipMemcpy(pages, q.pages.data(), q.pages.size() * sizeof(int32_t),
                             hipMemcpyHostToDevice);
    if (e == hipSuccess) {
      launch_fill_synthetic(ctx->stream, ctx->kpool, ctx->vpool, ctx->layer_stride,
                            (int)ctx->desc.layers, pages, (int)from, (int)rows,
                            (int)ctx->desc.kv_heads,
                            (int)ctx->desc.head_dim, seed, stream);
      e = hipStreamSynchronize(ctx->stream);
    }
    (void)hipFree(pages);
    if (e != hipSuccess) return fail(ctx, COHX_DEVICE, hipGetErrorString(e));
  }
  q.length = rows;
  return COHX_OK;
}

}  // extern "C"

// ---- the step ----------------------------------------------------------------

namespace {

struct Prepared {
  std::vector<int> included;  // batch lane index of each device lane
  uint32_t rows = 0;
  uint32_t max_kv = 0;
  uint64_t kv_rows_read = 0;
  int n_tiles = 0;            // prefill-chunk attention tiles on the matrix cores
  uint32_t n_images = 0;      // key tile images of the chunk lanes (per layer)
  uint32_t n_exact = 0;       // rows left to the exact attention passes
  uint64_t kv_rows_chunk = 0; // attended positions of the tiles' rows
  uint64_t kv_chunk_lanes = 0;// KV rows of the lanes the tiles belong to
  uint32_t max_kv_exact = 0;  // longest attended length among the exact passes' rows
  bool single_token = true;   // every lane carries one token (a pure decode step)
  bool quant_gemm = false;    // Q8/Q4 linears of this step on the quantized GEMM (binary16 operands)
};

// Host validation (batch.rs:119-131) and upload of the device batch into w.
int prepare_batch(cohx_ctx *ctx, const cohx_batch *batch, cohx_lane_out *outs, Prepared &p,
                  Workspace &w, const volatile uint32_t *cancel = nullptr) {
  const cohx_model_desc &d = ctx->desc;
  if (!batch || batch->n_lanes == 0 || batch->n_lanes > d.max_lanes || !batch->lanes)
    return fail(ctx, COHX_INVALID_REQUEST,
                "batch width must be in 1..=" + std::to_string(d.max_lanes));
  if (!ctx->finalized) return fail(ctx, COHX_INVALID_REQUEST, "model tensors not finalized");
  Staging &hs = ctx->host;
  // the staging mirrors the workspace's upload region (same offsets)
  uint32_t *info = hs.h_upload;
  uint32_t *toks = info + (size_t)w.lanes * 4;
  // duplicate sequences within one step are a shared failure
  for (uint32_t i = 0; i < batch->n_lanes; i++)
    for (uint32_t j = i + 1; j < batch->n_lanes; j++)
      if (batch->lanes[i].seq == batch->lanes[j].seq)
        return fail(ctx, COHX_INVALID_REQUEST, "a sequence appears twice in one batch");
  for (uint32_t i = 0; i < batch->n_lanes; i++) {
    const cohx_lane &ln = batch->lanes[i];
    int32_t status = COHX_OK;
    const bool live = valid_seq(ctx, ln.seq);
    const uint32_t start =
        (live && ln.start_position == COHX_AT_END) ? ctx->seqs[ln.seq].length : ln.start_position;
    if (cancel && cancel[i]) {
      status = COHX_CANCELLED;  // Cancellation::check before the forward
    } else if (!live || ln.n_tokens == 0 || !ln.tokens || start != ctx->seqs[ln.seq].length) {
      status = COHX_INVALID_REQUEST;
    } else {
      for (uint32_t j = 0; j < ln.n_tokens; j++)
        if (ln.tokens[j] >= d.vocabulary) status = COHX_INVALID_REQUEST;  // token outside vocabulary
      if (!status && (uint64_t)start + ln.n_tokens > ctx->seqs[ln.seq].capacity)
        status = COHX_RESOURCE;  // context capacity exhausted
      if (!status && p.rows + ln.n_tokens > d.max_rows) status = COHX_RESOURCE;
      if (!status) status = ensure_pages(ctx, ln.seq, start, start + ln.n_tokens);
    }
    if (outs) {
      outs[i].status = status;
      outs[i].argmax = 0;
    }
    if (status) continue;
    const uint32_t k = (uint32_t)p.included.size();
    info[k * 4 + 0] = ln.n_tokens;
    info[k * 4 + 1] = start;
    info[k * 4 + 2] = ln.seq;
    info[k * 4 + 3] = p.rows;
    std::memcpy(toks + p.rows, ln.tokens, ln.n_tokens * sizeof(uint32_t));
    for (uint32_t j = 0; j < ln.n_tokens; j++)
      p.kv_rows_read += (uint64_t)start + j + 1;
    p.rows += ln.n_tokens;
    if (ln.n_tokens != 1) p.single_token = false;
    p.max_kv = std::max(p.max_kv, start + ln.n_tokens);
    p.included.push_back((int)i);
  }
  if (p.included.empty()) return COHX_OK;
  int rc = sync_page_table(ctx);
  if (rc) return rc;
  const size_t n = p.included.size();
  // packed-prefill regime (a step of 128+ rows carrying prompt rows, F16 or
  // Q8_0/Q5_0/Q4_0 weights): linears on the matrix cores, and lanes of 16+
  // tokens take the matrix-core chunk attention (both held to a tolerance)
  const int G = (int)(d.heads / d.kv_heads);
  const bool wide = ctx->prefill_mfma && p.rows >= 128;
  p.quant_gemm = wide && ctx->quant_gemm && !p.single_token;
  const bool regime = wide && (d.weight_dtype == COHX_F16 || ctx->quant_gemm) &&
                      attention_chunk_supported((int)d.head_dim, G);
  p.n_tiles = 0;
  p.n_images = 0;
  p.n_exact = p.rows;
  p.max_kv_exact = p.max_kv;
  if (regime) {
    std::memset(hs.h_row_skip, 0, p.rows * sizeof(uint32_t));
    for (size_t k = 0; k < n; k++) {
      const uint32_t nt = info[k * 4 + 0], start = info[k * 4 + 1], seq = info[k * 4 + 2],
                     row0 = info[k * 4 + 3];
      if (nt < 16) {
        p.max_kv_exact = std::max(p.max_kv_exact, start + nt);
        continue;
      }
      p.kv_chunk_lanes += start + nt;
      // the lane's key tile images: tile-major, KV head minor
      const uint32_t lane_end = start + nt, img0 = p.n_images,
                     n_img = (lane_end + kChunkTileKeys - 1) / kChunkTileKeys * d.kv_heads;
      if (img0 + n_img > w.max_images) return fail(ctx, COHX_RESOURCE, "chunk tile images exceed the workspace");
      for (uint32_t i = 0; i < n_img; i++)
        hs.h_stage[img0 + i] = int4{(int)seq, (int)lane_end, (int)(i / d.kv_heads * kChunkTileKeys),
                                    (int)(i % d.kv_heads)};
      p.n_images += n_img;
      for (uint32_t t = 0; t < nt; t += 16) {
        const uint32_t rows_t = std::min(16u, nt - t), kv_end = start + t + rows_t;
        for (uint32_t sg = 0; sg * kChunkSegKeys < kv_end; sg++)
          hs.h_tiles[p.n_tiles++] = int4{(int)(row0 + t), (int)(rows_t | (sg << 8)), (int)img0, (int)(start + t)};
        for (uint32_t j = t; j < std::min(nt, t + 16); j++) {
          hs.h_row_skip[row0 + j] = 1;
          p.kv_rows_chunk += (uint64_t)start + j + 1;
        }
      }
    }
    if (!p.n_tiles) p.max_kv_exact = p.max_kv;
    if (p.n_tiles) {
      // longest KV first, so the short tiles fill in behind the long ones
      // (a work item's keys: to the end of its segment or of its rows)
      auto keys = [](const int4 &a) {
        const int seg = a.y >> 8, end = a.w + (a.y & 0xff);
        return std::min(end, (seg + 1) * kChunkSegKeys) - seg * kChunkSegKeys;
      };
      std::stable_sort(hs.h_tiles, hs.h_tiles + p.n_tiles,
                       [&](const int4 &a, const int4 &b) { return keys(a) > keys(b); });
      p.n_exact = 0;
      for (uint32_t r = 0; r < p.rows; r++)
        if (!hs.h_row_skip[r]) hs.h_row_map[p.n_exact++] = r;
      HIP_TRY(hipMemcpyAsync(w.tiles, hs.h_tiles, p.n_tiles * sizeof(int4), hipMemcpyHostToDevice,
                             ctx->stream));
      HIP_TRY(hipMemcpyAsync(w.stage, hs.h_stage, p.n_images * sizeof(int4), hipMemcpyHostToDevice,
                             ctx->stream));
      HIP_TRY(hipMemcpyAsync(w.row_skip, hs.h_row_skip, p.rows * sizeof(uint32_t),
                             hipMemcpyHostToDevice, ctx->stream));
      if (p.n_exact)
        HIP_TRY(hipMemcpyAsync(w.row_map, hs.h_row_map, p.n_exact * sizeof(uint32_t),
                               hipMemcpyHostToDevice, ctx->stream));
    }
  }
  // the exact passes' work list: (256-key chunk, row) pairs of the rows they
  // attend for, chunks descending, rows ascending (x indexes row_map in a
  // step with prefill chunks, else the packed rows)
  {
    uint32_t *items = toks + w.rows, *kvx = hs.h_kv;
    uint32_t nx = 0;
    for (size_t k = 0; k < n; k++) {
      const uint32_t nt = info[k * 4 + 0], start = info[k * 4 + 1], row0 = info[k * 4 + 3];
      for (uint32_t j = 0; j < nt; j++)
        if (!p.n_tiles || !hs.h_row_skip[row0 + j]) kvx[nx++] = start + j + 1;
    }
    if (nx != p.n_exact) return fail(ctx, COHX_DEVICE, "exact attention rows do not match the row list");
    uint32_t ni = 0, top = 0;
    for (uint32_t x = 0; x < nx; x++) top = std::max(top, (kvx[x] + 255) / 256);
    // room: rows x chunks of the workspace (the kernels' grids never exceed it)
    if (nx > w.rows || nx > 65536 || top > (w.kv_cap + 255) / 256)
      return fail(ctx, COHX_DEVICE, "the attention work list exceeds its room");
    for (uint32_t c = top; c-- > 0;)
      for (uint32_t x = 0; x < nx; x++)
        if (c * 256 < kvx[x]) items[1 + ni++] = c << 16 | x;
    items[0] = ni;
    const size_t words = (size_t)w.lanes * 4 + w.rows + 1 + ni;
    HIP_TRY(hipMemcpyAsync(w.lane_info, info, words * sizeof(uint32_t), hipMemcpyHostToDevice, ctx->stream));
  }
  return COHX_OK;
}

// The device packer over the uploaded lanes (ragged rows, positions, slots).
void enqueue_pack(cohx_ctx *ctx, const Workspace &w, int n_lanes) {
  launch_pack(ctx->stream, n_lanes, w.lane_info, w.tokens, ctx->page_table, ctx->max_pages, w.cu,
              w.row_pos, w.row_slot, w.row_lane, w.row_token, w.row_seq, w.lane_last, w.row_err, w.argmax,
              n_lanes);
}

ActView act_view(const Workspace &w) {
  return ActView{w.act_qs, w.act_ds, w.act_f16, w.act_kd, w.act_ksum, w.act_f32};
}

// Operand kind of a matrix's input and the block count its preparation takes
// (Q8_0: 32-element block pairs; Q8_K: 256-element blocks).
int act_of(const DeviceMatrix &m) { return act_kind(m.view.dtype); }
int act_blocks(int kind, int K) { return kind == kActQ8K ? K / 256 : even(K / 32); }
// Algorithmic bytes of one prepared operand row of width K.
double act_row_bytes(int kind, int K) {
  return kind == kActQ8 ? (double)K / 32 * 34 : kind == kActQ8K ? (double)K / 256 * 292 : (double)K * 2;
}

}  // namespace

extern "C" int cohx_pack(cohx_ctx *ctx, const cohx_batch *batch, uint32_t *cu, uint32_t *positions,
                         int64_t *slots, uint32_t *lanes) {
  if (ctx && ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "no paged packer for Qwen3.5");
  if (!ctx) return COHX_INVALID_REQUEST;
  HIP_TRY(hipSetDevice(ctx->device));
  Prepared p;
  std::vector<cohx_lane_out> outs(batch ? batch->n_lanes : 0);
  Workspace &w = ctx->ws;
  int rc = prepare_batch(ctx, batch, outs.data(), p, w);
  if (rc) return rc;
  if (p.included.size() != batch->n_lanes)
    return fail(ctx, COHX_INVALID_REQUEST, "a lane failed validation");
  enqueue_pack(ctx, w, (int)p.included.size());
  HIP_TRY(hipGetLastError());
  std::vector<int32_t> slot32(p.rows);
  HIP_TRY(hipMemcpyAsync(cu, w.cu, (batch->n_lanes + 1) * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(positions, w.row_pos, p.rows * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(slot32.data(), w.row_slot, p.rows * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(lanes, w.row_lane, p.rows * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  for (uint32_t r = 0; r < p.rows; r++) slots[r] = slot32[r];
  return COHX_OK;
}

// ---- one matrix on its own (test utility) -----------------------------------------

extern "C" int cohx_matvec(cohx_ctx *ctx, uint32_t dtype, uint32_t rows, uint32_t K, const void *weights,
                           size_t bytes, uint32_t n, const float *inputs, float *out, uint8_t *act_bytes,
                           float *decoded, int32_t *status) {
  if (ctx && ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "cohx_matvec takes a Qwen2 context");
  if (!ctx || !weights || !rows || !K || !n || !inputs || !out) return COHX_INVALID_REQUEST;
  const int fmt = device_format(dtype);
  const size_t rb = row_bytes(dtype, K);
  if (!fmt || !rb) return fail(ctx, COHX_UNSUPPORTED, "unsupported matrix dtype or width");
  if (fmt != kFmtF16 && K % 32) return fail(ctx, COHX_INVALID_GGUF, "width not block aligned");
  if (rb * rows != bytes) return fail(ctx, COHX_INVALID_GGUF, "payload size mismatch");
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  // everything allocated here is released before returning
  const size_t keep = ctx->allocations.size();
  auto release = [&](int rc) {
    (void)hipStreamSynchronize(ctx->stream);
    for (size_t i = keep; i < ctx->allocations.size(); i++) (void)hipFree(ctx->allocations[i]);
    ctx->allocations.resize(keep);
    return rc;
  };
  DeviceMatrix m;
  int rc = ensure_matrix(ctx, m, dtype, (int)rows, (int)K, (int)((rows + 15) / 16));
  if (!rc) rc = upload_matrix(ctx, m, dtype, weights, (int)rows, 0, 1);
  if (rc) return release(rc);
  const int kind = act_kind(fmt), blocks = act_blocks(kind, (int)K);
  const size_t ntiles = (n + 15) / 16, npad = ntiles * 16;
  float *d_in = nullptr, *d_out = nullptr, *d_dec = nullptr;
  uint32_t *d_err = nullptr, *d_tok = nullptr;
  ActView act{};
  rc = dalloc(ctx, &d_in, (size_t)n * K);
  if (!rc) rc = dalloc(ctx, &d_out, (size_t)n * rows);
  if (!rc) rc = dalloc(ctx, &d_err, n);
  if (!rc) rc = dalloc(ctx, &act.qs, npad * (size_t)std::max<int>(K, blocks * 32));
  if (!rc) rc = dalloc(ctx, &act.ds, ntiles * (size_t)blocks * 16);
  if (!rc) rc = dalloc(ctx, &act.f16, (size_t)n * K);
  if (!rc) rc = dalloc(ctx, &act.kd, npad * (K / 256 + 1));
  if (!rc) rc = dalloc(ctx, &act.ksum, npad * (K / 256 + 1) * 16);
  if (decoded && !rc) rc = dalloc(ctx, &d_dec, (size_t)rows * K);
  if (decoded && !rc) rc = dalloc(ctx, &d_tok, rows);
  if (rc) return release(rc);
  hipStream_t s = ctx->stream;
  if (hipMemcpyAsync(d_in, inputs, (size_t)n * K * 4, hipMemcpyHostToDevice, s) != hipSuccess)
    return release(fail(ctx, COHX_DEVICE, "input upload"));
  set_prefill_mfma(false);  // exact kernels only
  launch_quant_act(s, (int)n, d_in, (int)K, kind, blocks, act, d_err);
  launch_matvec(s, kEpiStore, m.view, act, (int)n, MatvecOut{d_out, (int)rows, nullptr, nullptr, d_err, nullptr});
  if (decoded) {
    std::vector<uint32_t> tok(rows);
    for (uint32_t r = 0; r < rows; r++) tok[r] = r;
    if (hipMemcpyAsync(d_tok, tok.data(), rows * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return release(fail(ctx, COHX_DEVICE, "token upload"));
    uint32_t *d_derr = nullptr;
    if ((rc = dalloc(ctx, &d_derr, rows))) return release(rc);
    launch_embed(s, (int)rows, m.view, d_tok, d_dec, (int)K, d_derr);
  }
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return release(fail(ctx, COHX_DEVICE, "matvec launch"));
  std::vector<uint32_t> err(n);
  if (hipMemcpy(out, d_out, (size_t)n * rows * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(err.data(), d_err, n * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      (decoded && hipMemcpy(decoded, d_dec, (size_t)rows * K * 4, hipMemcpyDeviceToHost) != hipSuccess))
    return release(fail(ctx, COHX_DEVICE, "read back"));
  if (status)
    for (uint32_t i = 0; i < n; i++)
      status[i] = err[i] & kErrPage ? COHX_RESOURCE : err[i] ? COHX_INVALID_GGUF : COHX_OK;
  if (act_bytes) {  // each prepared input in the engine's byte form
    const size_t qbytes = npad * (size_t)std::max<int>(K, blocks * 32);
    std::vector<int8_t> qs(qbytes);
    if (hipMemcpy(qs.data(), act.qs, qbytes, hipMemcpyDeviceToHost) != hipSuccess)
      return release(fail(ctx, COHX_DEVICE, "read back"));
    if (kind == kActQ8) {
      std::vector<uint16_t> ds(ntiles * (size_t)blocks * 16);
      if (hipMemcpy(ds.data(), act.ds, ds.size() * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return release(fail(ctx, COHX_DEVICE, "read back"));
      for (uint32_t i = 0; i < n; i++)
        for (uint32_t b = 0; b < K / 32; b++) {
          uint8_t *o = act_bytes + ((size_t)i * (K / 32) + b) * 34;
          const uint16_t d = ds[q8_scale(i / 16, blocks, (int)b, i % 16)];
          o[0] = (uint8_t)d;
          o[1] = (uint8_t)(d >> 8);
          for (int e = 0; e < 32; e++) o[2 + e] = (uint8_t)qs[q8_byte(i / 16, blocks, (int)b, (e / 8) * 16 + i % 16, e % 8)];
        }
    } else if (kind == kActQ8K) {
      std::vector<float> kd(npad * (K / 256 + 1));
      std::vector<int16_t> ks(kd.size() * 16);
      if (hipMemcpy(kd.data(), act.kd, kd.size() * 4, hipMemcpyDeviceToHost) != hipSuccess ||
          hipMemcpy(ks.data(), act.ksum, ks.size() * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return release(fail(ctx, COHX_DEVICE, "read back"));
      for (uint32_t i = 0; i < n; i++)
        for (int b = 0; b < blocks; b++) {
          uint8_t *o = act_bytes + ((size_t)i * blocks + b) * 292;
          const size_t ar = kq_row(i / 16, blocks, b, i % 16);
          std::memcpy(o, &kd[ar], 4);
          for (int e = 0; e < 256; e++)
            o[4 + e] = (uint8_t)qs[kq_byte(i / 16, blocks, b, e % 8, ((e / 8) / 8) * 16 + i % 16, (e / 8) % 8)];
          std::memcpy(o + 260, &ks[ar * 16], 32);
        }
    } else {
      std::vector<uint16_t> h((size_t)n * K);
      if (hipMemcpy(h.data(), act.f16, h.size() * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return release(fail(ctx, COHX_DEVICE, "read back"));
      std::memcpy(act_bytes, h.data(), h.size() * 2);
    }
  }
  return release(COHX_OK);
}

// ---- profiling -----------------------------------------------------------------

namespace {

const char *kCatNames[kCatCount] = {
    "pack", "embed", "rmsnorm_act", "matvec_qkv", "qkv_rope_append", "attn_scores",
    "attn_softmax_stats", "attn_pv", "attn_combine_act", "matvec_o_residual", "matvec_gate_up_swiglu",
    "swiglu_act", "matvec_down_residual", "matvec_head_argmax", "attn_chunk_mfma", "attn_chunk_stage"};

int prof_begin(cohx_ctx *ctx, int cat, double bytes, double flops) {
  Profiler &p = ctx->prof;
  if (!p.on) return -1;
  while (p.pool.size() < p.next + 2) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -1;
    p.pool.push_back(e);
  }
  Profiler::Launch l{cat, bytes, flops, p.pool[p.next], p.pool[p.next + 1]};
  p.next += 2;
  // the category's first kernel records a at its start, every kernel records b at its end
  set_launch_events(l.a, l.b);
  p.pending.push_back(l);
  return (int)p.pending.size() - 1;
}

void prof_end(cohx_ctx *ctx, int idx) {
  (void)ctx;
  if (idx >= 0) set_launch_events(nullptr, nullptr);
}

// After the stream has synchronized.
void prof_collect(cohx_ctx *ctx) {
  Profiler &p = ctx->prof;
  for (const auto &l : p.pending) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, l.a, l.b) == hipSuccess) {
      p.launches[l.cat]++;
      p.ms[l.cat] += ms;
      p.bytes[l.cat] += l.bytes;
      p.flops[l.cat] += l.flops;
    } else {
      // an interval whose launcher launched nothing (a fused path that
      // declined the shape): its events were never recorded; clear the error
      // so the step's next status check does not report it
      (void)hipGetLastError();
    }
  }
  p.pending.clear();
  p.next = 0;
}

// Algorithmic bytes of one matrix pass over rows_b activation rows: the GGUF
// payload(s) it holds, the prepared operand rows and the f32 outputs.
double matrix_pass_bytes(const DeviceMatrix &m, int rows_b, int out_rows, bool residual) {
  const double abytes = rows_b * act_row_bytes(act_of(m), m.view.K);
  return (double)m.gguf_bytes + abytes + (double)rows_b * out_rows * 4 * (residual ? 2 : 1);
}

}  // namespace

extern "C" int cohx_profile(cohx_ctx *ctx, int enable) {
  if (ctx && ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "no kernel profile for Qwen3.5");
  if (!ctx) return COHX_INVALID_REQUEST;
  Profiler &p = ctx->prof;
  if (enable) {
    std::fill(std::begin(p.launches), std::end(p.launches), 0);
    std::fill(std::begin(p.ms), std::end(p.ms), 0.0);
    std::fill(std::begin(p.bytes), std::end(p.bytes), 0.0);
    std::fill(std::begin(p.flops), std::end(p.flops), 0.0);
  }
  p.on = enable != 0;
  return COHX_OK;
}

extern "C" uint32_t cohx_profile_read(const cohx_ctx *ctx, cohx_kernel_stat *out, uint32_t cap) {
  if (!ctx) return 0;
  const Profiler &p = ctx->prof;
  for (uint32_t i = 0; i < (uint32_t)kCatCount && out && i < cap; i++)
    out[i] = cohx_kernel_stat{kCatNames[i], p.launches[i], p.ms[i], p.bytes[i], p.flops[i]};
  return kCatCount;
}

// Everything one step runs on the device, in stream order: packer, embedding,
// the layers, final norm, LM head and argmax.  Launch-only (no host waits), so
// it can be captured into a graph.  kv_grid (>= the longest attended length)
// sizes the attention grids; blocks past a row's length exit at once.
int enqueue_device_step(cohx_ctx *ctx, Workspace &w, const Prepared &p, int kv_grid, bool any_logits) {
  const cohx_model_desc &d = ctx->desc;
  // the packed-prefill regime (F16 linears on the matrix cores) is for
  // steps that carry prompt rows; decode-only steps stay exact at any width
  set_prefill_mfma(ctx->prefill_mfma && !p.single_token);
  const int pk = prof_begin(ctx, kCatPack, 0.0, 0.0);
  enqueue_pack(ctx, w, (int)p.included.size());
  prof_end(ctx, pk);
  const int R = (int)p.rows, NL = (int)p.included.size();
  const int H = d.hidden, F = d.intermediate, NH = d.heads, NKV = d.kv_heads, D = d.head_dim,
            KVD = NKV * D;
  // each matrix's input is prepared in the form its dtype takes: Q8_0 blocks
  // for Q4_0/Q5_0/Q8_0, Q8_K blocks for Q4_K/Q6_K (quant.rs:181-187),
  // binary16 rounding for F16 (cpu.rs:37-48)
  const int act_head = act_of(d.tied ? ctx->embd : ctx->output);
  const double act_row = act_row_bytes(act_of(ctx->layers[0].qkv), H);
  hipStream_t s = ctx->stream;
  StepDims sd{H, F, (int)d.vocabulary, NH, NKV, D, KVD, NH / NKV, d.norm_epsilon,
              1.0f / sqrtf((float)D), ctx->max_pages, (int)w.kv_cap, (int)w.max_chunks,
              p.n_tiles ? w.row_skip : nullptr, p.n_tiles ? w.row_map : nullptr, w.att_items};
  const int RX = (int)p.n_exact;  // rows of the exact attention passes
  if (p.n_tiles) kv_grid = (int)((p.max_kv_exact + 255) / 256 * 256);
  const ActView act = act_view(w);
  // attended positions summed over the exact passes' rows and the tiles' rows
  const double kv_rows = (double)(p.kv_rows_read - p.kv_rows_chunk);
  const double kv_chunk = (double)p.kv_rows_chunk;
  int e;
  // per-launch algorithmic bytes
  const double b_norm = (double)R * H * 4 + H * 4 + R * act_row;
  // algorithmic bytes of the exact attention passes: the K rows attended
  // (and the queries) for the scores, the V rows for the values; the score,
  // exponent and partial-sum buffers between the passes are intermediates
  // and count nothing, nor does the exponent pass
  const double b_scores = kv_rows * KVD * 4 + (double)RX * H * 4;
  const double b_softmax = 0.0;
  const double b_pv = kv_rows * KVD * 4;
  const double f_attn = kv_rows * NH * D * 2;
  // chunk tiles: each lane's K and V once (read by the staging pass, whose
  // binary16 images are intermediates), Q in and O out; QK^T and PV flops
  const double b_stage = (double)p.kv_chunk_lanes * KVD * 4 * 2;
  const double b_chunk = (R - RX) * (double)H * 4 * 2;
  const double f_chunk = kv_chunk * NH * D * 4;
  const double b_combine = (double)R * H * 4 + R * act_row;
  const double b_post = (double)R * (H + 2 * KVD) * 4 * 2 + (H + 2 * KVD) * 4;
  e = prof_begin(ctx, kCatEmbed, (double)R * act_row + (double)R * H * 4, 0);
  launch_embed(s, R, ctx->embd.view, w.row_token, w.x, H, w.row_err);
  prof_end(ctx, e);
  for (uint32_t l = 0; l < d.layers; l++) {
    Layer &ly = ctx->layers[l];
    float *kp = ctx->kpool + (size_t)l * ctx->layer_stride;
    float *vp = ctx->vpool + (size_t)l * ctx->layer_stride;
    // the quantized GEMM of the packed-prefill regime takes the reference's
    // Q8_0 operand values as binary16 rows
    const bool qg = p.quant_gemm;
    const int a_qkv = qg ? kActQ8H : act_of(ly.qkv), a_o = qg ? kActQ8H : act_of(ly.o),
              a_gu = qg ? kActQ8H : act_of(ly.gu), a_down = qg ? kActQ8H : act_of(ly.down);
    e = prof_begin(ctx, kCatNorm, b_norm, 0);
    launch_norm_act(s, R, w.x, nullptr, ly.attn_norm, H, d.norm_epsilon, a_qkv, act_blocks(a_qkv, H), act,
                    w.row_err);
    prof_end(ctx, e);
    // the regime's GEMMs take the qkv projection with its bias, RoPE and K/V
    // append in their epilogue
    const QkvEpi qe{ly.bqkv, ctx->rope, w.row_pos, w.row_slot, w.q_rot, kp, vp, H, KVD, D, NKV};
    const bool f16_gemm = ly.qkv.view.dtype == kFmtF16 && ctx->prefill_mfma && !p.single_token && R >= 128;
    const double b_qkv_fused =
        matrix_pass_bytes(ly.qkv, R, 0, false) + (double)R * (H + 2 * KVD) * 4 + (H + 2 * KVD) * 4;
    bool fused = false;
    if (qg || f16_gemm) {
      e = prof_begin(ctx, kCatMvQkv, b_qkv_fused, 2.0 * R * (H + 2 * KVD) * H);
      fused = launch_gemm_qkv(s, ly.qkv.view, act.f16, R, w.row_err, qe);
      prof_end(ctx, e);
    }
    if (fused) {
      // done
    } else if (qg) {
      // quantized GEMM into f32 rows (query/key features back in source
      // order), then the bias, RoPE and K/V append pass
      e = prof_begin(ctx, kCatMvQkv, matrix_pass_bytes(ly.qkv, R, H + 2 * KVD, false),
                     2.0 * R * (H + 2 * KVD) * H);
      if (!launch_gemm_q(s, kEpiStore, ly.qkv.view, act.f16, R,
                        MatvecOut{w.qkv, H + 2 * KVD, nullptr, nullptr, w.row_err, nullptr}, nullptr, D, H + KVD))
        return fail(ctx, COHX_UNSUPPORTED, "matrix outside the quantized GEMM's shapes");
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatQkvPost, b_post, 0);
      launch_qkv_post(s, R, sd, w.qkv, ly.bqkv, ctx->rope, w.row_pos, w.row_slot, w.q_rot, kp, vp,
                      w.row_err);
      prof_end(ctx, e);
    } else if (ly.qkv.view.dtype != kFmtQ8 && ly.qkv.view.dtype != kFmtQ4) {
      e = prof_begin(ctx, kCatMvQkv, matrix_pass_bytes(ly.qkv, R, H + 2 * KVD, false),
                     2.0 * R * (H + 2 * KVD) * H);
      launch_matvec(s, kEpiStore, ly.qkv.view, act, R,
                    MatvecOut{w.qkv, H + 2 * KVD, nullptr, nullptr, w.row_err, nullptr});
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatQkvPost, b_post, 0);
      launch_qkv_post(s, R, sd, w.qkv, ly.bqkv, ctx->rope, w.row_pos, w.row_slot, w.q_rot, kp, vp,
                      w.row_err);
      prof_end(ctx, e);
    } else {
      // Q8_0/Q4_0: bias, RoPE and the K/V append run in the matvec's epilogue
      // (rows uploaded in rope_row order); the bytes are the matrix pass plus
      // the post pass's writes
      e = prof_begin(ctx, kCatMvQkv, b_qkv_fused, 2.0 * R * (H + 2 * KVD) * H);
      launch_matvec_qkv(s, ly.qkv.view, act, R, MatvecOut{nullptr, 0, nullptr, nullptr, w.row_err, nullptr}, qe);
      prof_end(ctx, e);
    }
    // with prefill chunks the decode rows' exact passes (VALU and f64
    // chains) run on the side stream beside the chunk attention (matrix
    // cores); they touch disjoint rows of every buffer they write.  Timed
    // runs keep one stream, so each launch is measured alone.
    const bool fork = p.n_tiles && RX && !ctx->prof.on;
    hipStream_t sx = s;
    if (fork) {
      HIP_TRY(hipEventRecord(ctx->fork_ev, s));
      HIP_TRY(hipStreamWaitEvent(ctx->side, ctx->fork_ev, 0));
      sx = ctx->side;
    }
    if (RX) {
      e = prof_begin(ctx, kCatAttnScores, b_scores, f_attn);
      launch_attn_scores(sx, RX, kv_grid, sd, w.q_rot, kp, w.row_pos, w.row_seq,
                         ctx->page_table, w.scores, w.chunk_max, w.row_err);
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatAttnSoftmax, b_softmax, 0);
      launch_attn_exp(sx, RX, kv_grid, sd, w.row_pos, w.scores, w.chunk_max, w.den_part, w.row_max);
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatAttnPv, b_pv, f_attn);
      launch_attn_pv(sx, RX, kv_grid, sd, vp, w.row_pos, w.row_seq, ctx->page_table, w.scores,
                     w.den_part, w.row_max, w.partial);
      prof_end(ctx, e);
    }
    if (p.n_tiles) {
      e = prof_begin(ctx, kCatAttnStage, b_stage, 0);
      launch_attn_stage(s, (int)p.n_images, sd, w.stage, kp, vp, ctx->page_table, w.img);
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatAttnChunk, b_chunk, f_chunk);
      launch_attn_chunk(s, p.n_tiles, sd, w.tiles, w.q_rot, w.img, w.partial);
      prof_end(ctx, e);
    }
    if (fork) {
      HIP_TRY(hipEventRecord(ctx->join_ev, ctx->side));
      HIP_TRY(hipStreamWaitEvent(s, ctx->join_ev, 0));
    }
    // Q8_K operands: the combine writes f32 rows, then their blocks
    const int a_comb = a_o == kActQ8K ? kActF32 : a_o;
    e = prof_begin(ctx, kCatAttnCombine, b_combine, 0);
    launch_attn_combine(s, R, sd, w.row_pos, w.partial, a_comb, act_blocks(a_comb, H), act, w.row_err);
    prof_end(ctx, e);
    if (a_o == kActQ8K) {
      e = prof_begin(ctx, kCatQuant, (double)R * H * 4 + R * act_row_bytes(kActQ8K, H), 0);
      launch_quant_act(s, R, w.act_f32, H, kActQ8K, act_blocks(kActQ8K, H), act, w.row_err);
      prof_end(ctx, e);
    }
    e = prof_begin(ctx, kCatMvO, matrix_pass_bytes(ly.o, R, H, true), 2.0 * R * H * H);
    if (qg) {
      if (!launch_gemm_q(s, kEpiResidual, ly.o.view, act.f16, R,
                        MatvecOut{w.x, H, nullptr, nullptr, w.row_err, nullptr}, nullptr, 0, 0))
        return fail(ctx, COHX_UNSUPPORTED, "matrix outside the quantized GEMM's shapes");
    } else {
      launch_matvec(s, kEpiResidual, ly.o.view, act, R,
                    MatvecOut{w.x, H, nullptr, nullptr, w.row_err, nullptr});
    }
    prof_end(ctx, e);
    e = prof_begin(ctx, kCatNorm, b_norm, 0);
    launch_norm_act(s, R, w.x, nullptr, ly.ffn_norm, H, d.norm_epsilon, a_gu, act_blocks(a_gu, H), act,
                    w.row_err);
    prof_end(ctx, e);
    // Q8_0/Q4_0 gate+up at K <= 1024 feeding a Q8_0-operand down projection:
    // the SwiGLU quantizer runs in gate+up's epilogue into the down operand
    // buffer; otherwise its own pass
    const ActView down_act{w.down_qs, w.down_ds, nullptr, nullptr, nullptr, nullptr};
    if (qg) {
      // quantized GEMMs: gate+up with SwiGLU and its Q8_0 rounding in the
      // epilogue writes the down projection's binary16 rows into w.h
      // (act.f16 holds gate+up's own operand, still being read), then down
      // accumulates into x
      uint16_t *down16 = reinterpret_cast<uint16_t *>(w.h);
      e = prof_begin(ctx, kCatMvGateUp, matrix_pass_bytes(ly.gu, R, 0, false) + (double)R * F * 2,
                     2.0 * R * 2 * F * H);
      if (!launch_gemm_q(s, kEpiSwiglu, ly.gu.view, act.f16, R,
                        MatvecOut{nullptr, 0, nullptr, nullptr, w.row_err, nullptr}, down16, 0, 0))
        return fail(ctx, COHX_UNSUPPORTED, "matrix outside the quantized GEMM's shapes");
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatMvDown, matrix_pass_bytes(ly.down, R, H, true), 2.0 * R * H * F);
      if (!launch_gemm_q(s, kEpiResidual, ly.down.view, down16, R,
                        MatvecOut{w.x, H, nullptr, nullptr, w.row_err, nullptr}, nullptr, 0, 0))
        return fail(ctx, COHX_UNSUPPORTED, "matrix outside the quantized GEMM's shapes");
      prof_end(ctx, e);
      continue;
    }
    bool fused_quant = false;
    if (w.down_qs && a_down == kActQ8) {
      e = prof_begin(ctx, kCatMvGateUp,
                     matrix_pass_bytes(ly.gu, R, 0, false) + (double)R * F / 32 * 34, 2.0 * R * 2 * F * H);
      // false (nothing launched) for shapes the fused quantizer does not cover
      fused_quant = launch_matvec_swiglu_q8(s, ly.gu.view, act, R,
                                            MatvecOut{nullptr, 0, nullptr, nullptr, w.row_err, nullptr},
                                            down_act, ly.down.view.nbp);
      prof_end(ctx, e);
    }
    if (!fused_quant && a_down == kActF16) {
      // F16 in the packed-prefill regime: gate+up on the matrix cores with
      // SwiGLU in the epilogue, writing the down projection's binary16
      // operand into the f32 SwiGLU rows' space, w.h (act.f16 holds gate+up's
      // own operand, which other workgroups are still reading); false:
      // nothing launched
      uint16_t *down16 = reinterpret_cast<uint16_t *>(w.h);
      e = prof_begin(ctx, kCatMvGateUp, matrix_pass_bytes(ly.gu, R, 0, false) + (double)R * F * 2,
                     2.0 * R * 2 * F * H);
      fused_quant = launch_matvec_swiglu_f16(s, ly.gu.view, act, R,
                                             MatvecOut{nullptr, 0, nullptr, nullptr, w.row_err, nullptr},
                                             down16);
      prof_end(ctx, e);
      if (fused_quant) {
        ActView down_f16 = act;
        down_f16.f16 = down16;
        e = prof_begin(ctx, kCatMvDown, matrix_pass_bytes(ly.down, R, H, true), 2.0 * R * H * F);
        launch_matvec(s, kEpiResidual, ly.down.view, down_f16, R,
                      MatvecOut{w.x, H, nullptr, nullptr, w.row_err, nullptr});
        prof_end(ctx, e);
        continue;
      }
    }
    if (!fused_quant) {
      e = prof_begin(ctx, kCatMvGateUp, matrix_pass_bytes(ly.gu, R, F, false), 2.0 * R * 2 * F * H);
      launch_matvec(s, kEpiSwiglu, ly.gu.view, act, R,
                    MatvecOut{w.h, F, nullptr, nullptr, w.row_err, nullptr});
      prof_end(ctx, e);
      e = prof_begin(ctx, kCatQuant, (double)R * F * 4 + R * act_row_bytes(a_down, F), 0);
      launch_quant_act(s, R, w.h, F, a_down, act_blocks(a_down, F), act, w.row_err);
      prof_end(ctx, e);
    }
    e = prof_begin(ctx, kCatMvDown, matrix_pass_bytes(ly.down, R, H, true), 2.0 * R * H * F);
    launch_matvec(s, kEpiResidual, ly.down.view, fused_quant ? down_act : act, R,
                  MatvecOut{w.x, H, nullptr, nullptr, w.row_err, nullptr});
    prof_end(ctx, e);
  }
  // final norm and head over the last row of every lane (batch.rs:250-266)
  e = prof_begin(ctx, kCatNorm, (double)NL * H * 4 + H * 4 + NL * act_row_bytes(act_head, H), 0);
  launch_norm_act(s, NL, w.x, w.lane_last, ctx->output_norm, H, d.norm_epsilon, act_head,
                  act_blocks(act_head, H), act, w.row_err);
  prof_end(ctx, e);
  const DeviceMatrix &head = d.tied ? ctx->embd : ctx->output;
  // a step in the packed-prefill regime (its linears on the matrix cores)
  // takes the F16 head there too; otherwise the head stays exact
  set_head_mfma(p.n_tiles > 0 ||
                (ctx->prefill_mfma && !p.single_token && head.view.dtype == kFmtF16 && R >= 128));
  e = prof_begin(ctx, kCatMvHead,
                 matrix_pass_bytes(head, NL, 0, false) + (any_logits ? (double)NL * d.vocabulary * 4 : 0.0) + NL * 8.0,
                 2.0 * NL * d.vocabulary * H);
  // the final keys start at zero (the packer clears them); a head kernel that
  // raises them itself needs no reduce over per-tile partials
  if (!launch_matvec(s, kEpiArgmax, head.view, act, NL,
                     MatvecOut{nullptr, 0, w.argmax_part, any_logits ? w.logits : nullptr, w.row_err,
                               w.lane_last, w.argmax}))
    launch_argmax_reduce(s, NL, w.argmax_part, head.view.mtiles, w.argmax);
  set_head_mfma(false);
  prof_end(ctx, e);
  HIP_TRY(hipGetLastError());
  return COHX_OK;
}

namespace {

// One ragged step over `batch` with its device scratch in w.  graphs: decode
// steps may replay a captured graph (the buffers in w must then stay fixed).
int run_step(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out, Workspace &w, bool graphs,
             const cohx_step_hooks *hooks = nullptr) {
  const auto t_start = std::chrono::steady_clock::now();
  HIP_TRY(hipSetDevice(ctx->device));
  const cohx_model_desc &d = ctx->desc;
  Prepared p;
  int rc = prepare_batch(ctx, batch, out->lanes, p, w, hooks ? hooks->cancel : nullptr);
  if (rc) {
    ctx->prof.pending.clear();
    ctx->prof.next = 0;
    return rc;
  }
  out->width = (uint32_t)p.included.size();
  out->rows = p.rows;
  out->matrix_bytes = 0;
  out->kv_bytes = 0;
  if (p.included.empty()) {
    ctx->prof.pending.clear();
    ctx->prof.next = 0;
    out->elapsed_ns = 0;
    return COHX_OK;
  }
  const int R = (int)p.rows, NL = (int)p.included.size();
  const int KVD = d.kv_heads * d.head_dim;
  hipStream_t s = ctx->stream;
  const Staging &hs = ctx->host;
  bool any_logits = false;
  for (int k = 0; k < NL; k++)
    if (batch->lanes[p.included[k]].want_logits == 1u && out->lanes[p.included[k]].logits)
      any_logits = true;
  if (any_logits && !w.logits) return fail(ctx, COHX_RESOURCE, "the workspace has no room for logits");
  const int kv_grid = (int)((p.max_kv + 255) / 256 * 256);
  if (ctx->prof.on || !graphs || !p.single_token) {
    rc = enqueue_device_step(ctx, w, p, kv_grid, any_logits);
    if (rc) return rc;
  } else {
    const StepKey key{(uint32_t)R, (uint32_t)NL, (uint32_t)kv_grid, any_logits};
    auto it = ctx->graphs.find(key);
    if (it == ctx->graphs.end()) {
      if (ctx->graphs.size() >= kMaxGraphs) drop_graphs(ctx);
      hipGraph_t g = nullptr;
      HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      rc = enqueue_device_step(ctx, w, p, kv_grid, any_logits);
      const hipError_t ec = hipStreamEndCapture(s, &g);
      if (rc || ec != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return rc ? rc : fail(ctx, COHX_DEVICE, std::string("step capture: ") + hipGetErrorString(ec));
      }
      hipGraphExec_t ex = nullptr;
      const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (ei != hipSuccess) return fail(ctx, COHX_DEVICE, std::string("step graph: ") + hipGetErrorString(ei));
      it = ctx->graphs.emplace(key, ex).first;
    }
    HIP_TRY(hipGraphLaunch(it->second, s));
  }
  HIP_TRY(hipMemcpyAsync(hs.h_argmax, w.argmax, NL * sizeof(unsigned long long),
                         hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(hs.h_row_err, w.row_err, R * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  for (int k = 0; k < NL; k++) {
    const cohx_lane &ln = batch->lanes[p.included[k]];
    float *dst = out->lanes[p.included[k]].logits;
    if (ln.want_logits == 1u && dst)
      HIP_TRY(hipMemcpyAsync(dst, w.logits + (size_t)k * d.vocabulary, d.vocabulary * sizeof(float),
                             hipMemcpyDeviceToHost, s));
  }
  const int wrc = wait_step(ctx, s, hooks);
  if (wrc && wrc != COHX_CANCELLED) return wrc;
  prof_collect(ctx);
  // lane statuses from row error bits; advance healthy sequences (none when
  // the yield hook asked to stop: a shared failure)
  uint32_t row = 0;
  for (int k = 0; k < NL; k++) {
    const int i = p.included[k];
    const cohx_lane &ln = batch->lanes[i];
    uint32_t bits = 0;
    for (uint32_t j = 0; j < ln.n_tokens; j++) bits |= hs.h_row_err[row + j];
    row += ln.n_tokens;
    cohx_lane_out &o = out->lanes[i];
    o.argmax = 0xffffffffu - (uint32_t)(hs.h_argmax[k] & 0xffffffffull);
    if (wrc || (hooks && hooks->cancel && hooks->cancel[i]))
      o.status = COHX_CANCELLED;
    else if (bits & kErrPage)
      o.status = COHX_RESOURCE;
    else if (bits)
      o.status = COHX_INVALID_GGUF;
    else
      ctx->seqs[ln.seq].length += ln.n_tokens;
  }
  if (wrc) {
    out->width = 0;
    return fail(ctx, COHX_CANCELLED, "shared batch compute cancelled");
  }
  uint32_t width = 0;
  for (uint32_t i = 0; i < batch->n_lanes; i++) width += out->lanes[i].status == COHX_OK;
  out->width = width;
  out->matrix_bytes = ctx->matrix_bytes;
  out->kv_bytes = p.kv_rows_read * (uint64_t)KVD * 4 * 2 * d.layers +
                  (uint64_t)R * KVD * 4 * 2 * d.layers;
  out->elapsed_ns = (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                        std::chrono::steady_clock::now() - t_start)
                        .count();
  return COHX_OK;
}

}  // namespace

extern "C" int cohx_step(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out) {
  if (ctx && ctx->q35) return q35_step(ctx, batch, out, nullptr);
  if (!ctx || !out || !out->lanes) return COHX_INVALID_REQUEST;
  return run_step(ctx, batch, out, ctx->ws, ctx->use_graphs);
}

extern "C" int cohx_step_hooked(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out,
                                const cohx_step_hooks *hooks) {
  if (ctx && ctx->q35) return q35_step(ctx, batch, out, hooks);
  if (!ctx || !out || !out->lanes) return COHX_INVALID_REQUEST;
  return run_step(ctx, batch, out, ctx->ws, ctx->use_graphs, hooks);
}

namespace cohx {
int wait_step(cohx_ctx *ctx, hipStream_t s, const cohx_step_hooks *hooks) {
  if (!hooks || !hooks->yield) {
    HIP_TRY(hipStreamSynchronize(s));
    return COHX_OK;
  }
  if (!ctx->done) HIP_TRY(hipEventCreateWithFlags(&ctx->done, hipEventDisableTiming));
  HIP_TRY(hipEventRecord(ctx->done, s));
  int stop = 0;
  for (;;) {
    const hipError_t q = hipEventQuery(ctx->done);
    if (q == hipSuccess) break;
    if (q != hipErrorNotReady) return fail(ctx, COHX_DEVICE, std::string("step: ") + hipGetErrorString(q));
    if (stop) {  // nothing more to offer the caller: wait for the device
      HIP_TRY(hipEventSynchronize(ctx->done));
      break;
    }
    stop = hooks->yield(hooks->user);
  }
  return stop ? COHX_CANCELLED : COHX_OK;
}
}  // namespace cohx

// The same step as cohx_step with every device buffer the step needs beyond
// the context's weights, KV pool and page tables carved from the static
// scratch array, sized for this batch; launches are issued directly (no
// graph instantiation).  No device allocation of any kind.
extern "C" int cohx_step_noalloc(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out) {
  if (!ctx || !out || !out->lanes) return COHX_INVALID_REQUEST;
  if (ctx->q35) return fail(ctx, COHX_UNSUPPORTED, "cohx_step_noalloc serves Qwen2 contexts");
  if (!batch || !batch->lanes || batch->n_lanes == 0 || batch->n_lanes > ctx->desc.max_lanes)
    return fail(ctx, COHX_INVALID_REQUEST,
                "batch width must be in 1..=" + std::to_string(ctx->desc.max_lanes));
  if (!ctx->scratch) return fail(ctx, COHX_DEVICE, "the scratch array was not resolved");
  // upper bounds of what the step packs, over the lanes that can pass
  // prepare_batch's checks (a live sequence, the start at its length, the
  // rows within its capacity): a lane that will be refused on its own must
  // not make the whole call fail for want of scratch
  uint64_t rows = 0;
  uint32_t kv = 1;
  bool logits = false;
  for (uint32_t i = 0; i < batch->n_lanes; i++) {
    const cohx_lane &ln = batch->lanes[i];
    if (!valid_seq(ctx, ln.seq) || ln.n_tokens == 0) continue;
    const Sequence &sq = ctx->seqs[ln.seq];
    const uint64_t start = ln.start_position == COHX_AT_END ? sq.length : ln.start_position;
    if (start != sq.length || start + ln.n_tokens > sq.capacity) continue;
    rows += ln.n_tokens;
    kv = (uint32_t)std::max<uint64_t>(kv, std::min<uint64_t>(start + ln.n_tokens, ctx->desc.max_context));
    logits |= ln.want_logits == 1u && out->lanes[i].logits;
  }
  rows = std::min<uint64_t>(std::max<uint64_t>(rows, 1), ctx->desc.max_rows);
  const size_t need = layout_workspace(ctx->desc, ctx->nbp_h, ctx->nbp_f, (uint32_t)rows, batch->n_lanes,
                                       kv, logits, nullptr, nullptr);
  if (need > kScratchBytes)
    return fail(ctx, COHX_RESOURCE,
                "cohx_step_noalloc: this step needs " + std::to_string(need) + " bytes of scratch, more than its " +
                    std::to_string(kScratchBytes) + " (fewer rows, lanes, logits or attended positions)");
  Workspace w;
  layout_workspace(ctx->desc, ctx->nbp_h, ctx->nbp_f, (uint32_t)rows, batch->n_lanes, kv, logits, ctx->scratch,
                   &w);
  // Every buffer of the step is written before it is read (the packer
  // clears the row error bits), so nothing left by an earlier call, of this
  // or another context on the device, needs clearing.  Calls that overlap on
  // one device race on the array.
  const bool prof = ctx->prof.on;  // the timing events would be created here
  ctx->prof.on = false;
  const int rc = run_step(ctx, batch, out, w, false);
  ctx->prof.on = prof;
  return rc;
}
