// Launch interface between the host step driver (cohx.cpp) and the kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cohx {

// Device view of one matrix.  Q8_0: tiled int8 + f16 block scales (device.h
// layout).  F16: row-major binary16 exactly as in the GGUF file.
// Device formats (MatrixView::dtype): 1 = F16; 8 = Q8 tiles (GGUF Q8_0, and
// Q5_0, whose 5-bit values widen to int8 losslessly and whose block chain is
// Q8_0's); 2 = Q4_0 tiles; 12 = K-quant tiles (GGUF Q4_K and Q6_K).
constexpr int kFmtF16 = 1, kFmtQ8 = 8, kFmtQ4 = 2, kFmtKQ = 12;
// Activation operand kinds: binary16-rounded rows, Q8_0 blocks, Q8_K blocks.
constexpr int kActF16 = 1, kActQ8 = 8, kActQ8K = 15;
// Q8_0 blocks written out as binary16 rows [rows][K] of the values the
// reference's dot multiplies (q * f16(d), one rounding): the operand of the
// packed-prefill regime's quantized GEMM.  Rows of nbp * 32 == K values.
constexpr int kActQ8H = 9;
// Producer-only kind: f32 rows into ActView::f32, quantized by a following
// launch_quant_act(kActQ8K).
constexpr int kActF32 = 32;

struct MatrixView {
  int dtype;     // device format (kFmt*)
  int rows;      // logical output rows
  int K;         // input width
  int nb, nbp;   // 32-element blocks, rounded up to even (K-quants: nb = 256-element blocks)
  int mtiles;    // ceil(rows/16)
  const int8_t *qs;
  const uint16_t *ds;  // Q8/Q4 block scales; K-quants: d per (tile, block, row)
  const uint16_t *f16;
  // K-quant side data (device.h kq_* layout)
  const uint32_t *ksc;  // sub-group scales
  const uint16_t *kdm;  // dmin
  const uint8_t *kmin;  // group mins
  int has_min;          // any Q4_K part (else the min chain is skipped: it stays +0)
};

// Activation operand buffers for the next matrix.
struct ActView {
  int8_t *qs;     // Q8 tiled (B operand); K-quant tiled for Q8_K
  uint16_t *ds;   // Q8 block scales
  uint16_t *f16;  // binary16-rounded activations, row-major [rows][K]
  float *kd;      // Q8_K block scales
  int16_t *ksum;  // Q8_K 16-value sums
  float *f32;     // f32 rows [rows][K] (kActF32 producers)
};

// Operand kind a matrix of device format `fmt` consumes.
inline int act_kind(int fmt) { return fmt == kFmtF16 ? kActF16 : fmt == kFmtKQ ? kActQ8K : kActQ8; }

struct StepDims {
  int H, F, V, NH, NKV, D, KVD, G;  // G = NH/NKV
  float eps, scale;                  // scale = 1/sqrt(D)
  int max_pages;                     // page-table row stride
  int kv_cap;                        // score row stride (>= max kv length this step)
  int max_chunks;                    // partial-sum stride
  // rows whose attention the matrix-core chunk kernel computes (nullptr: none);
  // the combine pass merges their key segments (chunk_seg_at), and the exact
  // passes run over row_map[0 .. n) only: block x takes row row_map[x]
  // (nullptr: row x)
  const uint32_t *row_skip;
  const uint32_t *row_map;
  // the exact passes' work list (nullptr: full grids over rows x chunks):
  // [0] = n, then n entries (chunk << 16) | x, one per live (row x, 256-key
  // chunk), chunks descending and rows ascending within a chunk.  The
  // scores, exponent and value passes then take 1-D grids over the list's
  // bound (rows x chunks of the grid's longest row), and their workgroups
  // past entry n exit at once
  const uint32_t *att_items;
};

enum Epilogue { kEpiStore = 0, kEpiResidual = 1, kEpiSwiglu = 2, kEpiArgmax = 3 };

struct MatvecOut {
  float *out;          // kEpiStore: [rows_b][ld]; kEpiResidual: x [rows_b][ld]; kEpiSwiglu: h
  int ld;
  unsigned long long *argmax;  // kEpiArgmax: per (batch row, 16-row tile) partial keys
                               // [rows_b][mtiles], reduced by launch_argmax_reduce
  float *logits;               // kEpiArgmax: optional [rows_b][V] (nullptr: none)
  uint32_t *row_err;           // per batch row error bits
  const uint32_t *err_rows;    // batch row -> packed row index for error bits (nullptr: same)
  // kEpiArgmax: the final key of each batch row (zero before the launch), which
  // kernels that see many tiles per workgroup raise with one atomic max per
  // row instead of writing partials; launch_matvec then returns true
  unsigned long long *argmax_final;
};

void launch_pack(hipStream_t s, int n_lanes, const uint32_t *lane_info, const uint32_t *tokens,
                 const int32_t *page_table, int max_pages, uint32_t *cu, uint32_t *row_pos,
                 int32_t *row_slot, uint32_t *row_lane, uint32_t *row_token, uint32_t *row_seq,
                 uint32_t *lane_last, uint32_t *row_err, unsigned long long *keys, int n_keys);
void launch_embed(hipStream_t s, int rows, const MatrixView &emb, const uint32_t *row_token,
                  float *x, int H, uint32_t *row_err);
// in_rows: optional map from output batch row to input row of x (final norm over logit rows).
void launch_norm_act(hipStream_t s, int rows, const float *x, const uint32_t *in_rows,
                     const float *weight, int H, float eps, int act_dtype, int nbp, ActView act,
                     uint32_t *row_err);
void launch_quant_act(hipStream_t s, int rows, const float *src, int K, int act_dtype, int nbp,
                      ActView act, uint32_t *row_err);
// Packed F16 batches of 128+ rows on the matrix cores (f32 sums, within tolerance
// of the reference's f64 sums) or always on the exact kernels.  The step
// driver turns it on for steps that carry prompt rows only.
void set_prefill_mfma(bool on);
// The F16 LM head of the next launches on the matrix cores too (f32 sums; a
// step in the packed-prefill regime, at 16 or more logit rows).
void set_head_mfma(bool on);
// Timing events for the next launches (see the launch helper); both null ends it.
void set_launch_events(hipEvent_t start, hipEvent_t stop);

// Returns true when a kEpiArgmax launch wrote o.argmax_final (no reduce needed).
bool launch_matvec(hipStream_t s, Epilogue epi, const MatrixView &w, const ActView &act,
                   int rows_b, const MatvecOut &o);
// Q8_0/Q4_0 gate+up with the SwiGLU quantizer in its epilogue: writes the
// down projection's Q8_0 operand to qout (which must not alias act; laid out
// with qout_nbp block pairs per row, the down projection's) instead of the
// f32 SwiGLU rows; the same bits as launch_matvec (kEpiSwiglu) then
// launch_quant_act.  Returns false (nothing launched) for shapes it does not
// cover: K > 1024, F not a multiple of 64, or qout_nbp not F/32 rounded up
// to even.
bool launch_matvec_swiglu_q8(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                             const MatvecOut &o, const ActView &qout, int qout_nbp);
// F16 gate+up of a step in the packed-prefill regime on the matrix-core GEMM
// (gemm.h) with SwiGLU in its epilogue, writing the down projection's
// binary16 operand rows out_f16[rows_b][F] directly (the rounding and
// non-finite checks of launch_quant_act(kActF16)).  Returns false (nothing
// launched) outside the regime (set_prefill_mfma off, under 128 rows, not
// F16) or when K is not a multiple of 64.
bool launch_matvec_swiglu_f16(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                              const MatvecOut &o, uint16_t *out_f16);
// Q8_0/Q4_0 linears of a step in the packed-prefill regime on the matrix
// cores (gemm.h k_gemm_q): binary16 operand rows x[rows_b][K], the weights
// dequantized to binary16 on their way into LDS, f32 sums.  kEpiStore into
// o.out (features [0, rope_rows) of a rope-ordered qkv matrix, heads of
// rope_d, back to their source columns; rope_d 0: none), kEpiResidual
// accumulates into o.out, kEpiSwiglu writes the down projection's binary16
// rows out16[rows_b][F] (gate/up tiles interleaved).  Returns false (nothing
// launched) for other formats or epilogues, or K not a multiple of 128.
bool launch_gemm_q(hipStream_t s, Epilogue epi, const MatrixView &w, const uint16_t *x, int rows_b,
                   const MatvecOut &o, uint16_t *out16, int rope_d, int rope_rows);

void launch_argmax_reduce(hipStream_t s, int rows, const unsigned long long *part, int units,
                          unsigned long long *out);
// The qkv projection's post work (bias, NeoX RoPE, K/V append into the paged
// pool), done by launch_qkv_post or inside the projection below.
struct QkvEpi {
  const float *bias;         // [H + 2 KVD], the source row order
  const float2 *rope;        // [position][D/2] (cos, sin)
  const uint32_t *row_pos;   // [rows_b]
  const int32_t *row_slot;   // [rows_b] KV slot (< 0: no append)
  float *q_rot;              // [rows_b][H]
  float *kpool, *vpool;      // the layer's pools
  int H, KVD, D, NKV;
};
// Q8_0/Q4_0 qkv projection with launch_qkv_post's work in its epilogue, for
// weights whose query and key rows were uploaded in rope_row order.  Gives
// the same bits as the matvec and launch_qkv_post in sequence; out.out is
// unused.
void launch_matvec_qkv(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                       const MatvecOut &o, const QkvEpi &q);
// The packed-prefill regime's qkv projection with the same work in the
// GEMM's epilogue (F16 rows in source order, Q8_0/Q4_0 tiles with the query
// and key rows in rope order): the same bits as the regime's GEMM and
// launch_qkv_post in sequence.  False (nothing launched) for shapes it does
// not take (D != 64, K not a multiple of 128).
bool launch_gemm_qkv(hipStream_t s, const MatrixView &w, const uint16_t *x, int rows_b, uint32_t *row_err,
                     const QkvEpi &q);
void launch_qkv_post(hipStream_t s, int rows, const StepDims &d, const float *qkv,
                     const float *bias, const float2 *rope, const uint32_t *row_pos,
                     const int32_t *row_slot, float *q_rot, float *kpool, float *vpool,
                     uint32_t *row_err);
// (head_dim, q heads per KV head) pairs the attention kernels are built for
bool attention_shape_supported(int D, int G);
void launch_attn_scores(hipStream_t s, int rows, int max_kv, const StepDims &d, const float *q_rot,
                        const float *kpool, const uint32_t *row_pos, const uint32_t *row_seq,
                        const int32_t *page_table, float *scores, float *chunk_max,
                        uint32_t *row_err);
// The f64 sums of e = exp(s - max) per 256-token chunk into
// den_part[row][head][chunk], and each row's maximum into row_max[row][head]
// (scores [row][kv_head][t][8] are only read).
void launch_attn_exp(hipStream_t s, int rows, int max_kv, const StepDims &d,
                     const uint32_t *row_pos, const float *scores, const float *chunk_max,
                     double *den_part, float *row_max);
// Values: e again from the scores and row_max, p = e / den, the f64 partial
// sums of p v per 128-token chunk into partial.
void launch_attn_pv(hipStream_t s, int rows, int max_kv, const StepDims &d, const float *vpool,
                    const uint32_t *row_pos, const uint32_t *row_seq, const int32_t *page_table,
                    const float *scores, const double *den_part, const float *row_max,
                    double *partial);
// Matrix-core attention for prefill chunks (tolerance regime): tiles[i] =
// {first packed row, rows (<= 16) | key segment << 8, index of the lane's
// first tile image, position of the first row}; a workgroup attends to keys
// [seg * kChunkSegKeys, + kChunkSegKeys) and writes the segment's row max,
// row sum and unnormalized output as f32 (chunk_seg_at) into the rows'
// partial-sum space, which the combine pass merges in segment order.
constexpr int kChunkSegKeys = 1024;
constexpr int kChunkSegFloats = 2 + 64;  // m, l, o[64] (head_dim 64)
// The chunk kernel's key tiles (64 keys of one lane and KV head, head_dim
// 64) as binary16 LDS images of kChunkImgUnits 16-byte units, written by
// launch_attn_stage once per layer: items[i] = {sequence, end of the lane's
// keys, first key of the tile, KV head} makes image i; a lane's images run
// tile-major from its first (image = first + tile * kv_heads + head).
constexpr int kChunkTileKeys = 64, kChunkImgUnits = 3 * 64 * 8;
bool attention_chunk_supported(int D, int G);
void launch_attn_stage(hipStream_t s, int n_images, const StepDims &d, const int4 *items, const float *kpool,
                       const float *vpool, const int32_t *page_table, uint4 *img);
void launch_attn_chunk(hipStream_t s, int n_tiles, const StepDims &d, const int4 *tiles, const float *q_rot,
                       const uint4 *img, double *partial);
void launch_attn_combine(hipStream_t s, int rows, const StepDims &d, const uint32_t *row_pos,
                         const double *partial, int act_dtype, int nbp, ActView act,
                         uint32_t *row_err);
void launch_fill_synthetic(hipStream_t s, float *kpool, float *vpool, size_t layer_stride,
                           int layers, const int32_t *pages, int from, int rows, int NKV, int D,
                           uint64_t seed, uint32_t stream);
void launch_copy_page(hipStream_t s, float *kpool, float *vpool, size_t layer_stride, int layers,
                      int page_floats, int src_page, int dst_page);
void launch_fill_u64(hipStream_t s, unsigned long long *p, size_t n, unsigned long long v);
void launch_fill_u32(hipStream_t s, uint32_t *p, size_t n, uint32_t v);

}  // namespace cohx
