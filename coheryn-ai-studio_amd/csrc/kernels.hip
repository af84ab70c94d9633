// HIP kernels of the ragged continuous-batching step (gfx950, wave64).
//
// Numerics follow the engine's CPU path bit for bit wherever the reference
// fixes an order (crates/coheryn-engine/src/cpu.rs, quant.rs):
//  * Q8_0 matvec: exact int32 block dot on the matrix cores
//    (v_mfma_i32_16x16x32_i8, one 32-element block per MFMA), then the
//    reference's per-block chain sum = fmaf(float(isum), dw*da, sum) in block
//    order for every (row, lane) — quant.rs:265-272.
//  * attention scores: q.k summed in f64 in element order, as cpu.rs:31-35.
//  * f64 sums over many elements (RMSNorm, softmax denominator, P.V) use a
//    fixed tree / chunk order; they equal the sequential sum whenever no
//    partial sum rounds, and otherwise differ below 2^-52 relative before the
//    final rounding to f32.
#include <hip/hip_runtime.h>

#include "device.h"
#include "kernels.h"

namespace cohx {

// ---------------------------------------------------------------------------
// Packer: cu_seqlens (exclusive scan of lane token counts), per-row position,
// KV slot (page_table[seq][pos/16]*16 + pos%16), lane, token and sequence.
// lane_info: [n_tokens, start_position, seq, token_offset] per lane.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_pack(int n, const uint32_t *__restrict__ info,
                                               const uint32_t *__restrict__ tokens,
                                               const int32_t *__restrict__ pt, int max_pages,
                                               uint32_t *cu, uint32_t *row_pos, int32_t *row_slot,
                                               uint32_t *row_lane, uint32_t *row_token,
                                               uint32_t *row_seq, uint32_t *lane_last,
                                               uint32_t *row_err) {
  __shared__ uint32_t scan[1024];
  const int i = threadIdx.x;
  const uint32_t nt = i < n ? info[i * 4] : 0u;
  scan[i] = nt;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    uint32_t v = i >= off ? scan[i - off] : 0u;
    __syncthreads();
    scan[i] += v;
    __syncthreads();
  }
  if (i == 0) cu[0] = 0;
  if (i < n) {
    const uint32_t end = scan[i], base = end - nt;
    const uint32_t start = info[i * 4 + 1], seq = info[i * 4 + 2], toff = info[i * 4 + 3];
    cu[i + 1] = end;
    for (uint32_t j = 0; j < nt; j++) {
      const uint32_t r = base + j, pos = start + j, pidx = pos / kPage;
      const int32_t phys = pidx < (uint32_t)max_pages ? pt[(size_t)seq * max_pages + pidx] : -1;
      row_pos[r] = pos;
      row_lane[r] = (uint32_t)i;
      row_token[r] = tokens[toff + j];
      row_seq[r] = seq;
      row_slot[r] = phys < 0 ? -1 : phys * kPage + (int32_t)(pos % kPage);
      row_err[r] = phys < 0 ? kErrPage : 0u;
    }
    lane_last[i] = end - 1;
  }
}

// ---------------------------------------------------------------------------
// Token embedding row gather (Model::vector -> read_row -> decode,
// inference.rs:349-365, quant.rs:92-96: value = d * q).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed(MatrixView e, const uint32_t *__restrict__ row_token,
                                               float *__restrict__ x, int H, uint32_t *row_err) {
  const int r = blockIdx.x;
  const uint32_t tok = row_token[r];
  bool bad = false;
  for (int k = threadIdx.x; k < H; k += blockDim.x) {
    float v;
    if (e.dtype == 8) {
      const int mt = tok / 16, c = tok % 16, b = k / 32, g = (k % 32) / 8, j = k % 8;
      const int8_t q = e.qs[q8_byte(mt, e.nbp, b, g * 16 + c, j)];
      const float d = h2f(e.ds[q8_scale(mt, e.nbp, b, c)]);
      bad |= !finitef(d);
      v = d * (float)q;
    } else {
      v = h2f(e.f16[(size_t)tok * H + k]);
      bad |= !finitef(v);
    }
    x[(size_t)r * H + k] = v;
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Q8_0 activation blocks (QuantizedInput::prepare, quant.rs:193-213) for one
// 32-element block held by 32 consecutive lanes: d = max|x|/127, inv = 1/d
// (0 when d == 0), stored scale f16(d), q = round-half-away(x*inv) as i8.
// Writes the B-operand tile layout. Returns true if the block is invalid.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool quant_block_q8(float v, bool active, int row, int b, int t, int nbp,
                                               ActView act) {
  bool bad = active && !finitef(v);
  const float amax = half_max_f32(active ? fabsf(v) : 0.0f);
  const float d = amax / 127.0f;
  const float inv = d == 0.0f ? 0.0f : 1.0f / d;
  const uint16_t hd = f2h(d);
  if (active) {
    bad |= !finitef(h2f(hd)) || !finitef(inv);
    act.qs[q8_byte(row / 16, nbp, b, (t / 8) * 16 + row % 16, t % 8)] = sat_i8(roundf(v * inv));
    if (t == 0) act.ds[q8_scale(row / 16, nbp, b, row % 16)] = hd;
  }
  return bad;
}

// ---------------------------------------------------------------------------
// RMSNorm (cpu.rs:49-57) fused with the operand preparation of the next
// matrix: Q8_0 activation blocks, or binary16 rounding for F16 weights
// (cpu.rs:37-48).  One workgroup per row.
// ---------------------------------------------------------------------------
template <int kAct>
__global__ __launch_bounds__(256) void k_norm_act(const float *__restrict__ x,
                                                  const uint32_t *__restrict__ in_rows,
                                                  const float *__restrict__ w, int H, float eps,
                                                  int nbp, ActView act, uint32_t *row_err) {
  extern __shared__ float y[];
  __shared__ double red[4];
  const int ob = blockIdx.x;
  const int ib = in_rows ? (int)in_rows[ob] : ob;
  const float *xr = x + (size_t)ib * H;
  double ss = -0.0;
  for (int k = threadIdx.x; k < H; k += 256) {
    const float v = xr[k];
    ss += (double)(v * v);
  }
  const double total = block_sum_f64<256>(ss, red);
  const float mean = (float)(total / (double)H);
  const float scale = 1.0f / sqrtf(mean + eps);
  for (int k = threadIdx.x; k < H; k += 256) y[k] = xr[k] * scale * w[k];
  __syncthreads();
  bool bad = false;
  if (kAct == 8) {
    const int hw = threadIdx.x / 32, t = threadIdx.x % 32;
    for (int base = 0; base < nbp; base += 8) {
      const int b = base + hw, k = b * 32 + t;
      const bool active = b < nbp;
      const float v = (active && k < H) ? y[k] : 0.0f;
      bad |= quant_block_q8(v, active, ob, b, t, nbp, act);
    }
  } else {
    for (int k = threadIdx.x; k < H; k += 256) {
      const uint16_t h = f2h(y[k]);
      bad |= !finitef(h2f(h));
      act.f16[(size_t)ob * H + k] = h;
    }
  }
  if (bad) atomicOr(&row_err[ib], kErrNonFinite);
}

// Operand preparation of an f32 row (SwiGLU output before ffn_down).
template <int kAct>
__global__ __launch_bounds__(256) void k_quant_act(const float *__restrict__ src, int K, int nbp,
                                                   ActView act, uint32_t *row_err) {
  const int r = blockIdx.x;
  const float *s = src + (size_t)r * K;
  bool bad = false;
  if (kAct == 8) {
    const int hw = threadIdx.x / 32, t = threadIdx.x % 32;
    for (int base = 0; base < nbp; base += 8) {
      const int b = base + hw, k = b * 32 + t;
      const bool active = b < nbp;
      const float v = (active && k < K) ? s[k] : 0.0f;
      bad |= quant_block_q8(v, active, r, b, t, nbp, act);
    }
  } else {
    for (int k = threadIdx.x; k < K; k += 256) {
      const uint16_t h = f2h(s[k]);
      bad |= !finitef(h2f(h));
      act.f16[(size_t)r * K + k] = h;
    }
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Epilogues
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
  if (v == 0.0f) v = 0.0f;  // -0 ties +0 (sampling.rs:163 compares with >)
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)row);
}

// Best (value, lowest row) of one batch column over the four lanes that hold
// it (lanes c, c+16, c+32, c+48), then one atomic per column.
__device__ __forceinline__ void argmax_commit(float best, int best_row, bool valid, int r,
                                              unsigned long long *out) {
  unsigned long long key = valid ? argmax_key(best, best_row) : 0ull;
  unsigned long long o = __shfl_xor(key, 16, kWave);
  key = o > key ? o : key;
  o = __shfl_xor(key, 32, kWave);
  key = o > key ? o : key;
  if ((threadIdx.x % kWave) < 16 && valid) atomicMax(out + r, key);
}

// ---------------------------------------------------------------------------
// Q8_0 matvec on the matrix cores.  One wave owns kNM m-tiles (16 matrix rows
// each; kNM = 2 pairs a gate tile with its up tile) and kNT n-tiles (16 batch
// rows each).  Per 32-element block: int32 isum of the 16x16 tile from one
// MFMA, then acc = fmaf(float(isum), dw*da, acc) — the reference chain, block
// by block, for each of the lane's 4 (row, batch-row) outputs.
// ---------------------------------------------------------------------------
template <int kEpi, int kNT, int kNM>
__global__ __launch_bounds__(256) void k_mv_q8(MatrixView w, ActView act, int rows_b,
                                               MatvecOut o) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int unit = blockIdx.x * 4 + wave;
  if (unit * kNM >= w.mtiles) return;
  const int nt0 = blockIdx.y * kNT;
  const int n_tiles = (rows_b + 15) / 16;
  const int nbp = w.nbp;
  float acc[kNM][kNT][4];
#pragma unroll
  for (int m = 0; m < kNM; m++)
#pragma unroll
    for (int n = 0; n < kNT; n++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][n][i] = 0.0f;
  const v4i zero = {0, 0, 0, 0};
  const int rsub = 4 * (lane / 16);
  for (int bp = 0; bp < nbp / 2; bp++) {
    uint4 a[kNM], bq[kNT];
#pragma unroll
    for (int m = 0; m < kNM; m++)
      a[m] = *reinterpret_cast<const uint4 *>(w.qs + q8_byte(unit * kNM + m, nbp, bp * 2, lane, 0));
#pragma unroll
    for (int n = 0; n < kNT; n++)
      if (nt0 + n < n_tiles)
        bq[n] = *reinterpret_cast<const uint4 *>(act.qs + q8_byte(nt0 + n, nbp, bp * 2, lane, 0));
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int b = bp * 2 + h;
      float dw[kNM][4];
#pragma unroll
      for (int m = 0; m < kNM; m++) {
        const uint2 s2 =
            *reinterpret_cast<const uint2 *>(w.ds + q8_scale(unit * kNM + m, nbp, b, rsub));
        dw[m][0] = h2f((uint16_t)(s2.x & 0xffffu));
        dw[m][1] = h2f((uint16_t)(s2.x >> 16));
        dw[m][2] = h2f((uint16_t)(s2.y & 0xffffu));
        dw[m][3] = h2f((uint16_t)(s2.y >> 16));
      }
#pragma unroll
      for (int n = 0; n < kNT; n++) {
        if (nt0 + n >= n_tiles) continue;
        const float da = h2f(act.ds[q8_scale(nt0 + n, nbp, b, lane % 16)]);
        const long bop = h ? (long)(((unsigned long)bq[n].w << 32) | bq[n].z)
                           : (long)(((unsigned long)bq[n].y << 32) | bq[n].x);
#pragma unroll
        for (int m = 0; m < kNM; m++) {
          const long aop = h ? (long)(((unsigned long)a[m].w << 32) | a[m].z)
                             : (long)(((unsigned long)a[m].y << 32) | a[m].x);
          const v4i s = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, zero, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[m][n][i] = fmaf((float)s[i], dw[m][i] * da, acc[m][n][i]);
        }
      }
    }
  }
  // ---- epilogue
#pragma unroll
  for (int n = 0; n < kNT; n++) {
    const int r = (nt0 + n) * 16 + lane % 16;
    const bool rvalid = (nt0 + n < n_tiles) && r < rows_b;
    const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
    bool bad = false;
    if (kEpi == kEpiArgmax) {
      float best = 0.0f;
      int best_row = 0;
      bool have = false;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = unit * 16 + rsub + i;
        if (!rvalid || row >= w.rows) continue;
        const float v = acc[0][n][i];
        bad |= !finitef(v);
        if (o.logits) o.logits[(size_t)r * w.rows + row] = v;
        if (!have || v > best) {
          best = v;
          best_row = row;
          have = true;
        }
      }
      argmax_commit(best, best_row, rvalid && have, r, o.argmax);
    } else if (kEpi == kEpiSwiglu) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = unit * 16 + rsub + i;
        if (!rvalid || row >= w.rows / 2) continue;
        const float g = acc[0][n][i], u = acc[1][n][i];
        bad |= !finitef(g) || !finitef(u);
        o.out[(size_t)r * o.ld + row] = (g / (1.0f + exp_f32(-g))) * u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = unit * 16 + rsub + i;
        if (!rvalid || row >= w.rows) continue;
        const float v = acc[0][n][i];
        bad |= !finitef(v);
        float *p = o.out + (size_t)r * o.ld + row;
        if (kEpi == kEpiResidual)
          *p = *p + v;
        else
          *p = v;
      }
    }
    if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
  }
}

// ---------------------------------------------------------------------------
// F16 matvec with the reference's wide reduction (cpu.rs:31-35 over
// round_f16 operands): f32 products of binary16 values are exact, summed in
// f64 per lane in element order, then across lanes in a fixed butterfly.
// One wave per output row; kEpiSwiglu pairs row i with row i + F.
// ---------------------------------------------------------------------------
template <int kEpi>
__global__ __launch_bounds__(256) void k_mv_f16(MatrixView w, ActView act, int rows_b,
                                                MatvecOut o) {
  const int lane = threadIdx.x % kWave;
  const int row = blockIdx.x * 4 + threadIdx.x / kWave;
  const int out_rows = kEpi == kEpiSwiglu ? w.rows / 2 : w.rows;
  if (row >= out_rows) return;
  const int K = w.K;
  const uint16_t *wr = w.f16 + (size_t)row * K;
  const uint16_t *wu = kEpi == kEpiSwiglu ? w.f16 + (size_t)(row + out_rows) * K : nullptr;
  for (int r = 0; r < rows_b; r++) {
    const uint16_t *ar = act.f16 + (size_t)r * K;
    double s = -0.0, su = -0.0;
    for (int k = lane; k < K; k += kWave) {
      const float a = h2f(ar[k]);
      s += (double)(h2f(wr[k]) * a);
      if (kEpi == kEpiSwiglu) su += (double)(h2f(wu[k]) * a);
    }
    s = wave_sum_f64(s);
    if (kEpi == kEpiSwiglu) su = wave_sum_f64(su);
    const float v = (float)s;
    const int er = o.err_rows ? (int)o.err_rows[r] : r;
    if (kEpi == kEpiArgmax) {
      if (o.logits && lane == 0) o.logits[(size_t)r * w.rows + row] = v;
      if (lane == 0) {
        if (!finitef(v)) atomicOr(&o.row_err[er], kErrNonFinite);
        atomicMax(o.argmax + r, argmax_key(v, row));
      }
    } else if (kEpi == kEpiSwiglu) {
      const float u = (float)su;
      if (lane == 0) {
        if (!finitef(v) || !finitef(u)) atomicOr(&o.row_err[er], kErrNonFinite);
        o.out[(size_t)r * o.ld + row] = (v / (1.0f + exp_f32(-v))) * u;
      }
    } else if (lane == 0) {
      if (!finitef(v)) atomicOr(&o.row_err[er], kErrNonFinite);
      float *p = o.out + (size_t)r * o.ld + row;
      if (kEpi == kEpiResidual)
        *p = *p + v;
      else
        *p = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Bias add, NeoX RoPE from the host-built table (cos, sin of the engine's
// iterative angle, cpu.rs:59-73), K/V append into the paged pool
// (Kv::append, inference.rs:1019-1043; batch.rs:164-184).
// Pool layout per layer: [page][kv_head][16][head_dim] f32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_qkv_post(StepDims d, const float *__restrict__ qkv,
                                                  const float *__restrict__ bias,
                                                  const float2 *__restrict__ rope,
                                                  const uint32_t *__restrict__ row_pos,
                                                  const int32_t *__restrict__ row_slot,
                                                  float *__restrict__ q_rot, float *kpool,
                                                  float *vpool) {
  const int r = blockIdx.x;
  const uint32_t pos = row_pos[r];
  const int32_t slot = row_slot[r];
  const int half = d.D / 2, width = d.H + 2 * d.KVD;
  const float *src = qkv + (size_t)r * width;
  const float2 *rp = rope + (size_t)pos * half;
  for (int p = threadIdx.x; p < d.NH * half; p += 256) {
    const int h = p / half, i = p % half, e = h * d.D + i;
    const float a = src[e] + bias[e], b = src[e + half] + bias[e + half];
    const float2 cs = rp[i];
    q_rot[(size_t)r * d.H + e] = fmaf(a, cs.x, -(b * cs.y));
    q_rot[(size_t)r * d.H + e + half] = fmaf(a, cs.y, b * cs.x);
  }
  if (slot < 0) return;
  const int page = slot / kPage, off = slot % kPage;
  for (int p = threadIdx.x; p < d.NKV * half; p += 256) {
    const int g = p / half, i = p % half, e = d.H + g * d.D + i;
    const float a = src[e] + bias[e], b = src[e + half] + bias[e + half];
    const float2 cs = rp[i];
    float *dst = kpool + ((size_t)(page * d.NKV + g) * kPage + off) * d.D;
    dst[i] = fmaf(a, cs.x, -(b * cs.y));
    dst[i + half] = fmaf(a, cs.y, b * cs.x);
  }
  for (int e = threadIdx.x; e < d.KVD; e += 256) {
    const int g = e / d.D, j = e % d.D, s = d.H + d.KVD + e;
    vpool[((size_t)(page * d.NKV + g) * kPage + off) * d.D + j] = src[s] + bias[s];
  }
}

// ---------------------------------------------------------------------------
// Attention (cpu.rs:133-210 attention_rows), split over 128-token chunks.
// Pass 1: scores s = f32(sum_j f64(q_j*k_j)) * scale for the G query heads
// sharing a KV head, plus per-chunk maxima.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(128) void k_attn_scores(StepDims d, const float *__restrict__ q_rot,
                                                     const float *__restrict__ kpool,
                                                     const uint32_t *__restrict__ row_pos,
                                                     const uint32_t *__restrict__ row_seq,
                                                     const int32_t *__restrict__ pt,
                                                     float *__restrict__ scores,
                                                     float *__restrict__ chunk_max,
                                                     uint32_t *row_err) {
  const int r = blockIdx.x, g = blockIdx.y, c = blockIdx.z;
  const int kv = (int)row_pos[r] + 1;
  const int t0 = c * kChunk;
  if (t0 >= kv) return;
  __shared__ float qs[kMaxGroup * 128];
  __shared__ float red[2];
  for (int e = threadIdx.x; e < d.G * d.D; e += 128)
    qs[e] = q_rot[(size_t)r * d.H + (size_t)g * d.G * d.D + e];
  __syncthreads();
  const int t = t0 + threadIdx.x;
  const bool valid = t < kv;
  double acc[kMaxGroup];
#pragma unroll
  for (int hh = 0; hh < kMaxGroup; hh++) acc[hh] = -0.0;
  if (valid) {
    const int32_t phys = pt[(size_t)row_seq[r] * d.max_pages + t / kPage];
    const float *krow = kpool + ((size_t)(phys * d.NKV + g) * kPage + t % kPage) * d.D;
    for (int j = 0; j < d.D; j += 4) {
      const float4 k4 = *reinterpret_cast<const float4 *>(krow + j);
#pragma unroll
      for (int hh = 0; hh < kMaxGroup; hh++) {
        if (hh < d.G) {
          const float *q = qs + hh * d.D + j;
          acc[hh] += (double)(q[0] * k4.x);
          acc[hh] += (double)(q[1] * k4.y);
          acc[hh] += (double)(q[2] * k4.z);
          acc[hh] += (double)(q[3] * k4.w);
        }
      }
    }
  }
  bool bad = false;
#pragma unroll
  for (int hh = 0; hh < kMaxGroup; hh++) {
    if (hh >= d.G) break;
    const int head = g * d.G + hh;
    const float s = valid ? (float)acc[hh] * d.scale : -__builtin_inff();
    if (valid) {
      bad |= !finitef(s);
      scores[((size_t)r * d.NH + head) * d.kv_cap + t] = s;
    }
    const float m = block_max_f32<128>(s, red);
    if (threadIdx.x == 0) chunk_max[((size_t)r * d.NH + head) * d.max_chunks + c] = m;
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// Pass 2: p = exp(s - max) (f32), denominator in f64, p *= f32(1/den).
__global__ __launch_bounds__(256) void k_attn_softmax(StepDims d,
                                                      const uint32_t *__restrict__ row_pos,
                                                      float *__restrict__ scores,
                                                      const float *__restrict__ chunk_max) {
  __shared__ float redf[4];
  __shared__ double redd[4];
  const int r = blockIdx.x, h = blockIdx.y;
  const int kv = (int)row_pos[r] + 1, nch = (kv + kChunk - 1) / kChunk;
  float *s = scores + ((size_t)r * d.NH + h) * d.kv_cap;
  float m = -__builtin_inff();
  for (int c = threadIdx.x; c < nch; c += 256)
    m = fmaxf(m, chunk_max[((size_t)r * d.NH + h) * d.max_chunks + c]);
  m = block_max_f32<256>(m, redf);
  double den = 0.0;
  for (int t = threadIdx.x; t < kv; t += 256) {
    const float p = exp_f32(s[t] - m);
    s[t] = p;
    den += (double)p;
  }
  den = block_sum_f64<256>(den, redd);
  const float inv = (float)(1.0 / den);
  for (int t = threadIdx.x; t < kv; t += 256) s[t] = s[t] * inv;
}

// Pass 3: per-chunk f64 partials of sum_t f64(p_t * v_t[j]) in token order.
__global__ __launch_bounds__(1024) void k_attn_pv(StepDims d, const float *__restrict__ vpool,
                                                  const uint32_t *__restrict__ row_pos,
                                                  const uint32_t *__restrict__ row_seq,
                                                  const int32_t *__restrict__ pt,
                                                  const float *__restrict__ scores,
                                                  double *__restrict__ partial) {
  const int r = blockIdx.x, g = blockIdx.y, c = blockIdx.z;
  const int kv = (int)row_pos[r] + 1, t0 = c * kChunk;
  if (t0 >= kv) return;
  const int t1 = min(t0 + kChunk, kv);
  __shared__ int32_t slots[kChunk];
  for (int i = threadIdx.x; i < t1 - t0; i += blockDim.x) {
    const int t = t0 + i;
    slots[i] = pt[(size_t)row_seq[r] * d.max_pages + t / kPage] * kPage + t % kPage;
  }
  __syncthreads();
  const int hh = threadIdx.x / d.D, j = threadIdx.x % d.D;
  if (hh >= d.G) return;
  const int head = g * d.G + hh;
  const float *p = scores + ((size_t)r * d.NH + head) * d.kv_cap;
  double acc = 0.0;
  for (int t = t0; t < t1; t++) {
    const int32_t sl = slots[t - t0];
    const float v = vpool[((size_t)((sl / kPage) * d.NKV + g) * kPage + sl % kPage) * d.D + j];
    acc += (double)(p[t] * v);
  }
  partial[(((size_t)r * d.NH + head) * d.max_chunks + c) * d.D + j] = acc;
}

// Pass 4: chunks combined in order, rounded to f32, and prepared as the
// operand of attn_output (each head's D elements hold whole Q8_0 blocks).
template <int kAct>
__global__ __launch_bounds__(128) void k_attn_combine(StepDims d,
                                                      const uint32_t *__restrict__ row_pos,
                                                      const double *__restrict__ partial, int nbp,
                                                      ActView act, uint32_t *row_err) {
  const int r = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const int kv = (int)row_pos[r] + 1, nch = (kv + kChunk - 1) / kChunk;
  const double *pp = partial + ((size_t)r * d.NH + h) * d.max_chunks * d.D;
  const bool active = j < d.D;
  double acc = 0.0;
  if (active) {
    acc = pp[j];
    for (int c = 1; c < nch; c++) acc += pp[(size_t)c * d.D + j];
  }
  const float o = (float)acc;
  const int e = h * d.D + j;
  bool bad = active && !finitef(o);
  if (kAct == 8) {
    bad |= quant_block_q8(o, active, r, e / 32, e % 32, nbp, act);
  } else if (active) {
    const uint16_t hv = f2h(o);
    bad |= !finitef(h2f(hv));
    act.f16[(size_t)r * d.H + e] = hv;
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Utilities
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ULL;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float synthetic_kv(uint64_t seed, uint32_t stream, uint32_t layer,
                                              uint32_t which, uint32_t pos, uint32_t e) {
  const uint64_t h = mix64(seed ^ mix64(((uint64_t)stream << 32) | ((uint64_t)layer << 1) | which) ^
                           (((uint64_t)pos << 16) | e));
  return (float)((int32_t)(h >> 40) - (1 << 23)) * 0x1p-23f;
}

__global__ void k_fill_synthetic(float *kpool, float *vpool, size_t layer_stride,
                                 const int32_t *__restrict__ pages, int rows, int NKV, int D,
                                 uint64_t seed, uint32_t stream) {
  const int layer = blockIdx.y;
  const size_t total = (size_t)rows * NKV * D;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int pos = (int)(idx / ((size_t)NKV * D));
    const int e = (int)(idx % ((size_t)NKV * D));
    const int g = e / D, j = e % D;
    const size_t at = (size_t)layer * layer_stride +
                      ((size_t)(pages[pos / kPage] * NKV + g) * kPage + pos % kPage) * D + j;
    kpool[at] = synthetic_kv(seed, stream, layer, 0, pos, e);
    vpool[at] = synthetic_kv(seed, stream, layer, 1, pos, e);
  }
}

__global__ void k_copy_page(float *kpool, float *vpool, size_t layer_stride, int page_floats,
                            int src, int dst) {
  const int layer = blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < page_floats; i += gridDim.x * blockDim.x) {
    const size_t s = (size_t)layer * layer_stride + (size_t)src * page_floats + i;
    const size_t t = (size_t)layer * layer_stride + (size_t)dst * page_floats + i;
    kpool[t] = kpool[s];
    vpool[t] = vpool[s];
  }
}

__global__ void k_fill_u64(unsigned long long *p, size_t n, unsigned long long v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}
__global__ void k_fill_u32(uint32_t *p, size_t n, uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// ---------------------------------------------------------------------------
// Launch wrappers
// ---------------------------------------------------------------------------
void launch_pack(hipStream_t s, int n_lanes, const uint32_t *lane_info, const uint32_t *tokens,
                 const int32_t *page_table, int max_pages, uint32_t *cu, uint32_t *row_pos,
                 int32_t *row_slot, uint32_t *row_lane, uint32_t *row_token, uint32_t *row_seq,
                 uint32_t *lane_last, uint32_t *row_err) {
  hipLaunchKernelGGL(k_pack, dim3(1), dim3(1024), 0, s, n_lanes, lane_info, tokens, page_table,
                     max_pages, cu, row_pos, row_slot, row_lane, row_token, row_seq, lane_last,
                     row_err);
}

void launch_embed(hipStream_t s, int rows, const MatrixView &emb, const uint32_t *row_token,
                  float *x, int H, uint32_t *row_err) {
  hipLaunchKernelGGL(k_embed, dim3(rows), dim3(256), 0, s, emb, row_token, x, H, row_err);
}

void launch_norm_act(hipStream_t s, int rows, const float *x, const uint32_t *in_rows,
                     const float *weight, int H, float eps, int act_dtype, int nbp, ActView act,
                     uint32_t *row_err) {
  const size_t lds = (size_t)H * sizeof(float);
  if (act_dtype == 8)
    hipLaunchKernelGGL(k_norm_act<8>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
  else
    hipLaunchKernelGGL(k_norm_act<1>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
}

void launch_quant_act(hipStream_t s, int rows, const float *src, int K, int act_dtype, int nbp,
                      ActView act, uint32_t *row_err) {
  if (act_dtype == 8)
    hipLaunchKernelGGL(k_quant_act<8>, dim3(rows), dim3(256), 0, s, src, K, nbp, act, row_err);
  else
    hipLaunchKernelGGL(k_quant_act<1>, dim3(rows), dim3(256), 0, s, src, K, nbp, act, row_err);
}

template <int kEpi, int kNM>
static void mv_q8(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                  const MatvecOut &o) {
  constexpr int kNT = 2;
  const int units = w.mtiles / kNM;
  const int n_tiles = (rows_b + 15) / 16;
  dim3 grid((units + 3) / 4, (n_tiles + kNT - 1) / kNT);
  hipLaunchKernelGGL((k_mv_q8<kEpi, kNT, kNM>), grid, dim3(256), 0, s, w, act, rows_b, o);
}

template <int kEpi>
static void mv_f16(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                   const MatvecOut &o) {
  const int out_rows = kEpi == kEpiSwiglu ? w.rows / 2 : w.rows;
  hipLaunchKernelGGL(k_mv_f16<kEpi>, dim3((out_rows + 3) / 4), dim3(256), 0, s, w, act, rows_b, o);
}

void launch_matvec(hipStream_t s, Epilogue epi, const MatrixView &w, const ActView &act,
                   int rows_b, const MatvecOut &o) {
  if (w.dtype == 8) {
    switch (epi) {
      case kEpiStore: mv_q8<kEpiStore, 1>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_q8<kEpiResidual, 1>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_q8<kEpiSwiglu, 2>(s, w, act, rows_b, o); break;
      case kEpiArgmax: mv_q8<kEpiArgmax, 1>(s, w, act, rows_b, o); break;
    }
  } else {
    switch (epi) {
      case kEpiStore: mv_f16<kEpiStore>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_f16<kEpiResidual>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_f16<kEpiSwiglu>(s, w, act, rows_b, o); break;
      case kEpiArgmax: mv_f16<kEpiArgmax>(s, w, act, rows_b, o); break;
    }
  }
}

void launch_qkv_post(hipStream_t s, int rows, const StepDims &d, const float *qkv,
                     const float *bias, const float2 *rope, const uint32_t *row_pos,
                     const int32_t *row_slot, float *q_rot, float *kpool, float *vpool,
                     uint32_t *row_err) {
  (void)row_err;
  hipLaunchKernelGGL(k_qkv_post, dim3(rows), dim3(256), 0, s, d, qkv, bias, rope, row_pos,
                     row_slot, q_rot, kpool, vpool);
}

void launch_attn_scores(hipStream_t s, int rows, int chunks, const StepDims &d, const float *q_rot,
                        const float *kpool, const uint32_t *row_pos, const uint32_t *row_seq,
                        const int32_t *page_table, float *scores, float *chunk_max,
                        uint32_t *row_err) {
  hipLaunchKernelGGL(k_attn_scores, dim3(rows, d.NKV, chunks), dim3(128), 0, s, d, q_rot, kpool,
                     row_pos, row_seq, page_table, scores, chunk_max, row_err);
}

void launch_attn_softmax(hipStream_t s, int rows, const StepDims &d, const uint32_t *row_pos,
                         float *scores, const float *chunk_max) {
  hipLaunchKernelGGL(k_attn_softmax, dim3(rows, d.NH), dim3(256), 0, s, d, row_pos, scores,
                     chunk_max);
}

void launch_attn_pv(hipStream_t s, int rows, int chunks, const StepDims &d, const float *vpool,
                    const uint32_t *row_pos, const uint32_t *row_seq, const int32_t *page_table,
                    const float *scores, double *partial) {
  const int threads = ((d.G * d.D + kWave - 1) / kWave) * kWave;
  hipLaunchKernelGGL(k_attn_pv, dim3(rows, d.NKV, chunks), dim3(threads), 0, s, d, vpool, row_pos,
                     row_seq, page_table, scores, partial);
}

void launch_attn_combine(hipStream_t s, int rows, const StepDims &d, const uint32_t *row_pos,
                         const double *partial, int act_dtype, int nbp, ActView act,
                         uint32_t *row_err) {
  const int threads = ((d.D + kWave - 1) / kWave) * kWave;
  if (act_dtype == 8)
    hipLaunchKernelGGL(k_attn_combine<8>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
  else
    hipLaunchKernelGGL(k_attn_combine<1>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
}

void launch_fill_synthetic(hipStream_t s, float *kpool, float *vpool, size_t layer_stride,
                           int layers, const int32_t *pages, int rows, int NKV, int D,
                           uint64_t seed, uint32_t stream) {
  const size_t total = (size_t)rows * NKV * D;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_fill_synthetic, dim3(blocks, layers), dim3(256), 0, s, kpool, vpool,
                     layer_stride, pages, rows, NKV, D, seed, stream);
}

void launch_copy_page(hipStream_t s, float *kpool, float *vpool, size_t layer_stride, int layers,
                      int page_floats, int src_page, int dst_page) {
  hipLaunchKernelGGL(k_copy_page, dim3((page_floats + 255) / 256, layers), dim3(256), 0, s, kpool,
                     vpool, layer_stride, page_floats, src_page, dst_page);
}

void launch_fill_u64(hipStream_t s, unsigned long long *p, size_t n, unsigned long long v) {
  int blocks = (int)((n + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_fill_u64, dim3(blocks), dim3(256), 0, s, p, n, v);
}

void launch_fill_u32(hipStream_t s, uint32_t *p, size_t n, uint32_t v) {
  int blocks = (int)((n + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_fill_u32, dim3(blocks), dim3(256), 0, s, p, n, v);
}

}  // namespace cohx
