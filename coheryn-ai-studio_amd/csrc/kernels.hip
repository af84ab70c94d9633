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
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "device.h"
#include "gemm.h"
#include "kernels.h"

namespace cohx {

// ---------------------------------------------------------------------------
// Launch helper.  While timing events are set, the next launch carries the
// start event in its own dispatch packet and every launch carries the stop
// event, so the interval is the kernels' execution (the same quantity
// rocprofv3's kernel trace reports) rather than marker-to-marker time.
// ---------------------------------------------------------------------------
namespace {
thread_local hipEvent_t t_ev_start = nullptr, t_ev_stop = nullptr;
thread_local bool g_prefill_mfma = true;  // set per step from the context
thread_local bool g_head_mfma = false;    // this step's F16 head on the matrix cores

template <typename F, typename... Args>
void launch_k(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
  if (t_ev_start || t_ev_stop) {
    hipExtLaunchKernelGGL(kernel, grid, block, shm, s, t_ev_start, t_ev_stop, 0u, args...);
    t_ev_start = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, s, args...);
  }
}
}  // namespace

void set_prefill_mfma(bool on) { g_prefill_mfma = on; }
void set_head_mfma(bool on) { g_head_mfma = on; }

void set_launch_events(hipEvent_t start, hipEvent_t stop) {
  t_ev_start = start;
  t_ev_stop = stop;
}

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
                                               uint32_t *row_err, unsigned long long *keys,
                                               int n_keys) {
  __shared__ uint32_t scan[1024];
  __shared__ uint32_t s_start[1024], s_seq[1024], s_toff[1024];
  const int i = threadIdx.x;
  // the step's final argmax keys start at zero (the head raises them)
  for (int k = i; k < n_keys; k += 1024) keys[k] = 0ull;
  const uint32_t nt = i < n ? info[i * 4] : 0u;
  scan[i] = nt;
  if (i < n) {
    s_start[i] = info[i * 4 + 1];
    s_seq[i] = info[i * 4 + 2];
    s_toff[i] = info[i * 4 + 3];
  }
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    uint32_t v = i >= off ? scan[i - off] : 0u;
    __syncthreads();
    scan[i] += v;
    __syncthreads();
  }
  if (i == 0) cu[0] = 0;
  if (i < n) {
    cu[i + 1] = scan[i];
    lane_last[i] = scan[i] - 1;
  }
  // rows r = i, i + 1024, ...: the lane is the first whose inclusive end
  // exceeds r (lanes with no rows never match)
  const uint32_t rows = n > 0 ? scan[n - 1] : 0u;
  for (uint32_t r = i; r < rows; r += 1024) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (scan[mid] > r) hi = mid; else lo = mid + 1;
    }
    const uint32_t base = lo > 0 ? scan[lo - 1] : 0u, j = r - base;
    const uint32_t pos = s_start[lo] + j, seq = s_seq[lo], pidx = pos / kPage;
    const int32_t phys = pidx < (uint32_t)max_pages ? pt[(size_t)seq * max_pages + pidx] : -1;
    row_pos[r] = pos;
    row_lane[r] = (uint32_t)lo;
    row_token[r] = tokens[s_toff[lo] + j];
    row_seq[r] = seq;
    row_slot[r] = phys < 0 ? -1 : phys * kPage + (int32_t)(pos % kPage);
    row_err[r] = phys < 0 ? kErrPage : 0u;
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
    } else if (e.dtype == 2) {  // Q4_0: d * (nibble - 8) (quant.rs:97-101)
      const int mt = tok / 16, c = tok % 16, b = k / 32, g = (k % 32) / 8, j = k % 8;
      const uint8_t byte = (uint8_t)e.qs[q4_byte(mt, e.nbp, b, g * 16 + c, j)];
      const int q = (j < 4 ? (byte & 15) : (byte >> 4)) - 8;
      const float d = h2f(e.ds[q8_scale(mt, e.nbp, b, c)]);
      bad |= !finitef(d);
      v = d * (float)q;
    } else if (e.dtype == kFmtKQ) {
      // Q4_K: (d*scale)*q - dmin*min; Q6_K: (d*scale)*q, stored with dmin = +0
      // and min = 0, so the same expression gives the same value (quant.rs:83-86,122-135)
      const int mt = tok / 16, rr = tok % 16, b = k / 256, i = k % 256, m = i / 8;
      const int q = e.qs[kq_byte(mt, e.nb, b, i % 8, (m / 8) * 16 + rr, m % 8)];
      const int sub = i / 16;
      const int sc = (int)(int8_t)(e.ksc[kq_row(mt, e.nb, b, 0) * 4 + (sub / 4) * 16 + rr] >> (8 * (sub % 4)));
      const size_t wr = kq_row(mt, e.nb, b, rr);
      const float dw = h2f(e.ds[wr]), dm = h2f(e.kdm[wr]);
      bad |= !finitef(dw) || !finitef(dm);
      v = (dw * (float)sc) * (float)q - dm * (float)e.kmin[wr * 8 + i / 32];
    } else {
      v = h2f(e.f16[(size_t)tok * H + k]);
      bad |= !finitef(v);
    }
    x[(size_t)r * H + k] = v;
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Q8_0 activation blocks (QuantizedInput::prepare, quant.rs:193-213):
// d = max|x|/127 over the 32-element block, inv = 1/d (0 when d == 0), stored
// scale f16(d), q = round-half-away(x*inv) as i8, in the B-operand tile layout.
// One thread quantizes an 8-element group (a quarter of a block); the four
// groups of a block sit in lanes kStride apart (kStride 1: four consecutive
// aligned lanes; 16: lanes l, l+16, l+32, l+48), combine their maxima with
// two shuffles, and each writes its 8 quantized values as one 8-byte store
// into the B-operand tile layout.  kRows (kActQ8H): the 8 values q * f16(d)
// as binary16 into act.f16 row `row` (stride nbp * 32) instead.
template <int kStride = 1, bool kRows = false>
__device__ __forceinline__ bool quant_group_q8(const float (&v)[8], bool active, int row, int kg,
                                               int nbp, ActView act) {
  float m = 0.0f;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    bad |= active && !finitef(v[i]);
    m = fmaxf(m, active ? fabsf(v[i]) : 0.0f);
  }
  m = fmaxf(m, __shfl_xor(m, kStride, kWave));
  m = fmaxf(m, __shfl_xor(m, 2 * kStride, kWave));
  const Q8Scale sc = q8_scale_of(m);
  if (active) {
    bad |= !finitef(h2f(sc.hd)) || !finitef(sc.inv);
    if constexpr (kRows) {
      const float dh = h2f(sc.hd);
      uint32_t p[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint16_t a = q8_value_h(q8_round(v[2 * i], sc.inv), dh);
        const uint16_t b = q8_value_h(q8_round(v[2 * i + 1], sc.inv), dh);
        bad |= !finitef(h2f(a)) || !finitef(h2f(b));
        p[i] = a | (uint32_t)b << 16;
      }
      *reinterpret_cast<uint4 *>(act.f16 + (size_t)row * nbp * 32 + kg * 8) = make_uint4(p[0], p[1], p[2], p[3]);
    } else {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        lo |= (uint32_t)(uint8_t)q8_round(v[i], sc.inv) << (8 * i);
        hi |= (uint32_t)(uint8_t)q8_round(v[i + 4], sc.inv) << (8 * i);
      }
      const int b = kg / 4, g = kg % 4;
      *reinterpret_cast<uint2 *>(act.qs + q8_byte(row / 16, nbp, b, g * 16 + row % 16, 0)) =
          make_uint2(lo, hi);
      if (g == 0) act.ds[q8_scale(row / 16, nbp, b, row % 16)] = sc.hd;
    }
  }
  return bad;
}

// ---------------------------------------------------------------------------
// Q8_K activation block (QuantizedInput::prepare for Q4_K/Q6_K weights,
// quant.rs:214-233), one wave per 256-element block; lane l brings elements
// 4l .. 4l+3 in v.  m = the first element of largest magnitude (signed);
// all-zero blocks stay zero (d = 0, sums 0); else inv = -127/m, d = 1/inv
// and q = min(round_ties_even(x*inv), 127) as i8, plus the sums of each 16
// consecutive q.  Writes the K-quant B-operand tiles (device.h kq_*).
// Returns the row's error bits (non-finite input; scale overflow).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t quant_block_q8k(const float (&v)[4], int row, int b, int nb, ActView act) {
  const int lane = threadIdx.x % kWave;
  bool bad = false;
  // (|x|, lowest index) key; |x| of a finite float orders as its bits
  unsigned long long key = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    bad |= !finitef(v[e]);
    const unsigned long long k = ((unsigned long long)__float_as_uint(fabsf(v[e])) << 32) |
                                 (unsigned long long)(0xffffffffu - (uint32_t)(4 * lane + e));
    key = k > key ? k : key;
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const unsigned long long o = __shfl_xor(key, m, kWave);
    key = o > key ? o : key;
  }
  const int idx = (int)(0xffffffffu - (uint32_t)key);
  const float cand = v[idx & 3];
  const float maximum = __shfl(cand, idx >> 2, kWave);
  uint32_t err = bad ? kErrNonFinite : 0u;
  uint32_t qw = 0;
  float d = 0.0f;
  if (maximum != 0.0f) {
    const float inv = -127.0f / maximum;
    d = 1.0f / inv;
    if (!finitef(inv) || !finitef(d)) err |= kErrScale;
#pragma unroll
    for (int e = 0; e < 4; e++)
      qw |= (uint32_t)(uint8_t)sat_i8(fminf(rintf(v[e] * inv), 127.0f)) << (8 * e);
  }
  // 16-value sums: lanes 4s .. 4s+3 hold sub-group s
  int sum = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) sum += (int)(int8_t)(qw >> (8 * e));
  sum += __shfl_xor(sum, 1, kWave);
  sum += __shfl_xor(sum, 2, kWave);
  const size_t tile = (size_t)(row / 16);
  const size_t rb = kq_row(tile, nb, b, row % 16);
  if (lane % 4 == 0) act.ksum[rb * 16 + lane / 4] = (int16_t)sum;
  if (lane == 0) act.kd[rb] = d;
  // lane T < 32 writes class c = T % 8, k-group kg = T / 8: values j = 0..7
  // are elements c + 64 kg + 8 j, byte c % 4 of lane 16 kg + 2 j + c / 4
  const int c = lane % 8, kg = (lane / 8) % 4;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t w = (uint32_t)__shfl((int)qw, 16 * kg + 2 * j + c / 4, kWave);
    const uint32_t byte = (w >> (8 * (c % 4))) & 0xffu;
    if (j < 4)
      lo |= byte << (8 * j);
    else
      hi |= byte << (8 * (j - 4));
  }
  if (lane < 32)
    *reinterpret_cast<uint2 *>(act.qs + kq_byte(tile, nb, b, c, kg * 16 + row % 16, 0)) = make_uint2(lo, hi);
  return err;
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
  // the thread's first kPer elements of x and of the weight are requested at
  // once and held (H <= 1024 needs no more); the per-thread sum of squares
  // runs in element order as before
  constexpr int kPer = 4;
  float xv[kPer], wv[kPer];
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int k = min((int)threadIdx.x + i * 256, H - 1);
    xv[i] = xr[k];
    wv[i] = w[k];
  }
  double ss = -0.0;
#pragma unroll
  for (int i = 0; i < kPer; i++)
    if ((int)threadIdx.x + i * 256 < H) ss += (double)(xv[i] * xv[i]);
  for (int k = threadIdx.x + kPer * 256; k < H; k += 256) {
    const float v = xr[k];
    ss += (double)(v * v);
  }
  const double total = block_sum_f64<256>(ss, red);
  const float mean = (float)(total / (double)H);
  const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int k = (int)threadIdx.x + i * 256;
    if (k < H) y[k] = xv[i] * scale * wv[i];
  }
  for (int k = threadIdx.x + kPer * 256; k < H; k += 256) y[k] = xr[k] * scale * w[k];
  __syncthreads();
  bool bad = false;
  if (kAct == 8 || kAct == kActQ8H) {
    for (int base = 0; base < nbp * 4; base += 256) {
      const int kg = base + threadIdx.x;
      const bool active = kg < nbp * 4;
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = (active && kg * 8 + i < H) ? y[kg * 8 + i] : 0.0f;
      bad |= quant_group_q8<1, kAct == kActQ8H>(v, active, ob, kg, nbp, act);
    }
  } else if (kAct == kActQ8K) {
    // one wave per 256-element block (H % 256 == 0; nbp = H / 256)
    uint32_t err = 0;
    const int lane = threadIdx.x % kWave;
    for (int b = threadIdx.x / kWave; b < nbp; b += 4) {
      const float v[4] = {y[b * 256 + 4 * lane], y[b * 256 + 4 * lane + 1], y[b * 256 + 4 * lane + 2],
                          y[b * 256 + 4 * lane + 3]};
      err |= quant_block_q8k(v, ob, b, nbp, act);
    }
    if (err) atomicOr(&row_err[ib], err);
  } else {
    for (int k = threadIdx.x; k < H; k += 256) {
      const uint16_t h = f2h(y[k]);
      bad |= !finitef(h2f(h));
      act.f16[(size_t)ob * H + k] = h;
    }
  }
  if (bad) atomicOr(&row_err[ib], kErrNonFinite);
}

// RMSNorm + Q8_0 operands for rows of at most 2048 elements: thread t owns
// the 8-element group t (elements 8t .. 8t+7; groups past the row are the
// zero padding of the last block pair).  It loads its x and weight values at
// once, sums its squares in element order, and after the workgroup's f64 tree
// normalizes and quantizes its group in registers: no LDS staging of the row
// and one barrier pair fewer than k_norm_act.
template <bool kRows>
__global__ __launch_bounds__(256) void k_norm_q8(const float *__restrict__ x,
                                                 const uint32_t *__restrict__ in_rows,
                                                 const float *__restrict__ w, int H, float eps, int nbp,
                                                 ActView act, uint32_t *row_err) {
  __shared__ double red[4];
  const int ob = blockIdx.x;
  const int ib = in_rows ? (int)in_rows[ob] : ob;
  const int kg = threadIdx.x;
  const bool active = kg < nbp * 4, inrow = kg * 8 < H;  // H % 8 == 0
  const int k0 = inrow ? kg * 8 : 0;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)ib * H + k0);
  const float4 *wr = reinterpret_cast<const float4 *>(w + k0);
  const float4 xa = xr[0], xb = xr[1], wa = wr[0], wb = wr[1];
  const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
  double ss = -0.0;
  if (inrow) {
#pragma unroll
    for (int i = 0; i < 8; i++) ss += (double)(xv[i] * xv[i]);
  }
  const double total = block_sum_f64<256>(ss, red);
  const float mean = (float)(total / (double)H);
  const float scale = 1.0f / sqrtf(mean + eps);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = inrow ? xv[i] * scale * wv[i] : 0.0f;
  if (quant_group_q8<1, kRows>(v, active, ob, kg, nbp, act)) atomicOr(&row_err[ib], kErrNonFinite);
}

// Operand preparation of an f32 row (SwiGLU output before ffn_down).
template <int kAct>
__global__ __launch_bounds__(256) void k_quant_act(const float *__restrict__ src, int K, int nbp,
                                                   ActView act, uint32_t *row_err) {
  const int r = blockIdx.x;
  const float *s = src + (size_t)r * K;
  bool bad = false;
  if (kAct == 8) {
    // block y takes groups [256 y, 256 y + 256) of the row: one group of 8
    // values per thread, 64 whole 32-element blocks per workgroup
    const int kg = blockIdx.y * 256 + threadIdx.x;
    const bool active = kg < nbp * 4;
    float v[8];
    if (active && kg * 8 + 8 <= K) {
      const float4 a = reinterpret_cast<const float4 *>(s)[kg * 2];
      const float4 c = reinterpret_cast<const float4 *>(s)[kg * 2 + 1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = (active && kg * 8 + i < K) ? s[kg * 8 + i] : 0.0f;
    }
    bad |= quant_group_q8(v, active, r, kg, nbp, act);
  } else if (kAct == kActQ8K) {
    // block y takes 256-element blocks [4 y, 4 y + 4): one per wave (nbp = K / 256)
    const int b = blockIdx.y * 4 + (int)threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (b < nbp) {
      const float4 a = reinterpret_cast<const float4 *>(s + (size_t)b * 256)[lane];
      const float v[4] = {a.x, a.y, a.z, a.w};
      const uint32_t err = quant_block_q8k(v, r, b, nbp, act);
      if (err) atomicOr(&row_err[r], err);
    }
  } else {
    for (int k = blockIdx.y * 256 + threadIdx.x; k < K; k += 256 * gridDim.y) {
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
// Split-K Q8_0 matvec.  A workgroup of 8 waves owns one output tile: kNM
// m-tiles (16 matrix rows each; 2 = a gate tile and its up tile) x one n-tile
// (16 batch rows).  K is walked in chunks of 16*kP blocks; in each chunk every
// wave takes kP block pairs, computes the exact int32 block sums on the matrix
// cores and parks them (as f32, exact below 2^24) in LDS with the block scales;
// then 256 threads, one per (row, batch row), run the reference chain
// acc = fmaf(isum, dw*da, acc) over the chunk's blocks in order.  The next
// chunk's operands are loaded before the current chunk is consumed.
// Block -> (tile, n-tile) mapping keeps all n-tiles of a weight tile on one
// XCD (blockIdx % 8), so the tile is fetched into that XCD's L2 once.
// ---------------------------------------------------------------------------
// The scales of a block pair: kNM weight tiles x 2 blocks x 16 rows, then
// 2 blocks x 16 batch rows, (kNM + 1) * 32 values spread over the wave's
// lanes, one 16-bit load per lane per 64 values.  Slot s = v * 64 + lane:
// s < kNM * 32 is weight tile s / 32, block 2p + (s % 32) / 16, row s % 16;
// the next 32 are the batch tile's, block 2p + (s % 32) / 16, batch row s % 16.
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

template <int kNM>
struct Q8Regs {
  static constexpr int kSV = (kNM + 2) / 2;  // scale values per lane
  u32x4v a[kNM];
  u32x4v b;
  uint16_t sc[kSV];
};

// Branch-free, so the compiler can count the loads in flight and wait only
// for the ones it needs: the caller clamps `pair` to the last valid pair and
// ignores what a clamped load returns.  Each scale stays in its own register
// until phase 1 stores it: combining two right after the load would make the
// wave wait for every load in flight (vmcnt counts in order).
template <int kNM, int kFmt>
__device__ __forceinline__ void q8_load(Q8Regs<kNM> &r, const MatrixView &w, const ActView &act,
                                        int unit, int nt, int pair, int lane) {
  const int nbp = w.nbp;
#pragma unroll
  for (int m = 0; m < kNM; m++) {
    if constexpr (kFmt == 8) {
      r.a[m] = *reinterpret_cast<const u32x4v *>(w.qs + q8_byte(unit * kNM + m, nbp, pair * 2, lane, 0));
    } else {
      const uint2 v = *reinterpret_cast<const uint2 *>(w.qs + q4_byte(unit * kNM + m, nbp, pair * 2, lane, 0));
      r.a[m] = u32x4v{v.x, v.y, 0u, 0u};
    }
  }
  r.b = *reinterpret_cast<const u32x4v *>(act.qs + q8_byte(nt, nbp, pair * 2, lane, 0));
#pragma unroll
  for (int v = 0; v < Q8Regs<kNM>::kSV; v++) {
    const int sl = v * 64 + lane;
    const int blk = pair * 2 + (sl % 32) / 16, row = sl % 16;
    const uint16_t *src = sl < kNM * 32 ? w.ds + q8_scale(unit * kNM + min(sl / 32, kNM - 1), nbp, blk, row)
                                        : act.ds + q8_scale(nt, nbp, blk, row);
    r.sc[v] = *src;
  }
}

__device__ __forceinline__ long lo64(u32x4v v) {
  return (long)(((unsigned long)v[1] << 32) | v[0]);
}
__device__ __forceinline__ long hi64(u32x4v v) {
  return (long)(((unsigned long)v[3] << 32) | v[2]);
}
__device__ __forceinline__ long lo64(uint4 v) {
  return (long)(((unsigned long)v.y << 32) | v.x);
}
__device__ __forceinline__ long hi64(uint4 v) {
  return (long)(((unsigned long)v.w << 32) | v.z);
}

// Epilogue of the fused qkv projection (launch_matvec_qkv); the generic
// launch_matvec never selects it.
constexpr int kEpiQkv = 4;

template <int kEpi, int kNM, int kD, int kFmt, int kW = 8>
__global__ __launch_bounds__(64 * kW) void k_mv_q8s(MatrixView w, ActView act, int rows_b,
                                                    int n_tiles, MatvecOut o, QkvEpi qe) {
  static_assert(kD >= 2, "at least the next chunk in flight");
  constexpr int kCB = 2 * kW;  // blocks per chunk: one pair per wave
  __shared__ float s_isum[kCB][kNM * 256];
  __shared__ float s_dw[kCB][kNM * 16];
  __shared__ float s_da[kCB][16];
  __shared__ unsigned long long s_key[4][16];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int units = w.mtiles / kNM;
  const int group = blockIdx.x / (8 * n_tiles), rem = blockIdx.x % (8 * n_tiles);
  const int nt = rem / 8, unit = group * 8 + rem % 8;
  if (unit >= units) return;
  const int nbp = w.nbp, npairs = nbp / 2, nchunks = (nbp + kCB - 1) / kCB;
  const v4i zero = {0, 0, 0, 0};
  // phase-2 ownership: thread t < 256 owns the output the matrix-core layout
  // puts in lane t%64, slot t/64: row 4*((t%64)/16) + t/64, batch column t%16.
  // The block sums are parked as [slot][lane], so the MFMA lanes' writes and
  // the owners' reads are both consecutive (no bank conflicts).
  const int t = threadIdx.x, prow = 4 * ((t % 64) / 16) + t / 64, pcol = t % 16;
  float acc[kNM];
#pragma unroll
  for (int m = 0; m < kNM; m++) acc[m] = 0.0f;
  // kD - 1 chunks in flight ahead of the one consumed (a ring of registers)
  Q8Regs<kNM> ring[kD];
#pragma unroll
  for (int i = 0; i < kD - 1; i++)
    q8_load<kNM, kFmt>(ring[i], w, act, unit, nt, min(i * kW + wave, npairs - 1), lane);
  for (int c0 = 0; c0 < nchunks; c0 += kD) {
#pragma unroll
    for (int u = 0; u < kD; u++) {
      const int c = c0 + u;
      // chunks past the last prefetch a clamped (valid, unused) pair rather
      // than branch, and the prefetch is issued on every path, also for a
      // chunk past the end: a path without it would make the compiler wait
      // for every load in flight where the paths meet (the loop head),
      // including the prefetch of the next chunk
      q8_load<kNM, kFmt>(ring[(u + kD - 1) % kD], w, act, unit, nt, min((c + kD - 1) * kW + wave, npairs - 1),
                         lane);
      if (c < nchunks) {
        const Q8Regs<kNM> &cur = ring[u];
        if (c * kW + wave < npairs) {
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const int blk = 2 * wave + h;
            const long bop = h ? hi64(cur.b) : lo64(cur.b);
#pragma unroll
            for (int m = 0; m < kNM; m++) {
              long aop;
              if constexpr (kFmt == 8)
                aop = h ? hi64(cur.a[m]) : lo64(cur.a[m]);
              else
                aop = q4_operand(h ? cur.a[m][1] : cur.a[m][0]);
              const v4i s4 = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, zero, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; i++)
                s_isum[blk][m * 256 + i * 64 + lane] = (float)s4[i];
            }
          }
#pragma unroll
          for (int v = 0; v < Q8Regs<kNM>::kSV; v++) {
            const int sl = v * 64 + lane, blk = 2 * wave + (sl % 32) / 16;
            if (sl < kNM * 32)
              s_dw[blk][(sl / 32) * 16 + sl % 16] = h2f(cur.sc[v]);
            else if (sl < kNM * 32 + 32)
              s_da[blk][sl % 16] = h2f(cur.sc[v]);
          }
        }
        __syncthreads();
        if (t < 256) {
          const int nblk = min(kCB, nbp - c * kCB);
#pragma unroll 8
          for (int blk = 0; blk < nblk; blk++) {
            const float da = s_da[blk][pcol];
#pragma unroll
            for (int m = 0; m < kNM; m++) {
              if constexpr (kFmt == 8)
                acc[m] = fmaf(s_isum[blk][m * 256 + t], s_dw[blk][m * 16 + prow] * da, acc[m]);
              else
                acc[m] = fmaf(s_isum[blk][m * 256 + t] * s_dw[blk][m * 16 + prow], da, acc[m]);
            }
          }
        }
        __syncthreads();
      }
    }
  }
  // ---- epilogue
  const int r = nt * 16 + pcol;
  const bool rvalid = t < 256 && r < rows_b;
  const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
  bool bad = false;
  if constexpr (kEpi == kEpiQkv) {
    // The tile's 16 x 16 outputs meet in LDS (the block sums' space is free
    // after the chain's last barrier), so that one thread holds both rows of
    // a RoPE pair: with rows in rope_row order, rows 2i and 2i + 1 of a query
    // or key head are its elements i and i + D/2.  Then k_qkv_post's
    // arithmetic, operation for operation.
    float *s_out = &s_isum[0][0];
    if (t < 256) {
      const float v = acc[0];
      s_out[prow * 16 + pcol] = v;
      bad = rvalid && unit * 16 + prow < w.rows && !finitef(v);
    }
    __syncthreads();
    const int pi = t / 16, c = t % 16, rb = nt * 16 + c, row0 = unit * 16 + 2 * pi;
    if (t < 128 && rb < rows_b && row0 + 1 < w.rows) {
      const float va = s_out[2 * pi * 16 + c], vb = s_out[(2 * pi + 1) * 16 + c];
      const uint32_t pos = qe.row_pos[rb];
      const int32_t slot = qe.row_slot[rb];
      const int half = qe.D / 2, page = slot / kPage, off = slot % kPage;
      if (row0 < qe.H + qe.KVD) {
        const bool isq = row0 < qe.H;
        const int e0 = isq ? row0 : row0 - qe.H;
        const int head = e0 / qe.D, i = (e0 % qe.D) / 2;
        const int e = (isq ? 0 : qe.H) + head * qe.D + i;  // source row of element i
        const float a = va + qe.bias[e], b = vb + qe.bias[e + half];
        const float2 cs = qe.rope[(size_t)pos * half + i];
        const float ya = fmaf(a, cs.x, -(b * cs.y)), yb = fmaf(a, cs.y, b * cs.x);
        if (isq) {
          float *q = qe.q_rot + (size_t)rb * qe.H + head * qe.D + i;
          q[0] = ya;
          q[half] = yb;
        } else if (slot >= 0) {
          qe.kpool[k_at(page, pos / kPage, head, qe.NKV, off, i, qe.D)] = ya;
          qe.kpool[k_at(page, pos / kPage, head, qe.NKV, off, i + half, qe.D)] = yb;
        }
      } else if (slot >= 0) {
        const int e0 = row0 - qe.H - qe.KVD, g = e0 / qe.D, j = e0 % qe.D;
        const float *bv = qe.bias + qe.H + qe.KVD + e0;
        qe.vpool[v_at(page, g, qe.NKV, off, j, qe.D)] = va + bv[0];
        qe.vpool[v_at(page, g, qe.NKV, off, j + 1, qe.D)] = vb + bv[1];
      }
    }
  } else if (kEpi == kEpiArgmax) {
    const int row = unit * 16 + prow;
    const bool valid = rvalid && row < w.rows;
    const float v = acc[0];
    if (valid) {
      bad = !finitef(v);
      if (o.logits) o.logits[(size_t)r * w.rows + row] = v;
    }
    unsigned long long key = valid ? argmax_key(v, row) : 0ull;
    unsigned long long x = __shfl_xor(key, 16, kWave);
    key = x > key ? x : key;
    x = __shfl_xor(key, 32, kWave);
    key = x > key ? x : key;
    if (t < 256 && lane < 16) s_key[wave][lane] = key;
    __syncthreads();
    if (t < 16) {
      unsigned long long best = s_key[0][t];
#pragma unroll
      for (int i = 1; i < 4; i++) best = s_key[i][t] > best ? s_key[i][t] : best;
      // per-(batch row, tile) partial; reduced by k_argmax_reduce
      if (nt * 16 + t < rows_b) o.argmax[(size_t)(nt * 16 + t) * units + unit] = best;
    }
  } else if (rvalid) {
    if (kEpi == kEpiSwiglu) {
      const int row = unit * 16 + prow;
      if (row < w.rows / 2) {
        const float g = acc[0], u = acc[kNM - 1];
        bad = !finitef(g) || !finitef(u);
        o.out[(size_t)r * o.ld + row] = (g / (1.0f + exp_f32(-g))) * u;
      }
    } else {
      const int row = unit * 16 + prow;
      if (row < w.rows) {
        const float v = acc[0];
        bad = !finitef(v);
        float *p = o.out + (size_t)r * o.ld + row;
        if (kEpi == kEpiResidual)
          *p = *p + v;
        else
          *p = v;
      }
    }
  }
  if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// K-quant matvec (Q4_K / Q6_K weights, Q8_K activations; quant.rs:294-341).
// A workgroup of 8 waves owns kNM weight tiles x one batch tile, and wave c
// owns lane-class c (device.h kq_*), i.e. the engine's integers[c] and
// lanes[c].  Per block, in block order, the wave multiplies each weight value
// by its sub-group scale (|w| <= 4096), splits it as 128*hi + lo with hi and
// lo int8, and two int8 MFMAs give the exact class sum 128*(hi.a) + lo.a for
// every (row, batch row) of the tile; then
// lanes[c] = fmaf(dw*da, f32(integers[c]), lanes[c]).  Lanes 0-31 of each
// wave also run the Q4_K min chain of one (row, batch row) pair:
// sum = fmaf(-(dmin*da), f32(sum_g min_g * (s_2g + s_2g+1)), sum).  After the
// last block the chains meet in LDS and sum + lanes[0] + ... + lanes[7] is
// added in that order.  Q6_K has no min chain; its sum starts at +0 too.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void kq_split(uint2 q, uint32_t sc, long &hi, long &lo) {
  uint32_t h[2] = {0u, 0u}, l[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t word = j < 4 ? q.x : q.y;
    const int v = (int)(int8_t)(word >> (8 * (j % 4)));
    const int s = (int)(int8_t)(sc >> (8 * (j / 2)));
    const int p = v * s;
    h[j / 4] |= (uint32_t)((p >> 7) & 0xff) << (8 * (j % 4));
    l[j / 4] |= (uint32_t)(p & 0x7f) << (8 * (j % 4));
  }
  hi = (long)(((unsigned long)h[1] << 32) | h[0]);
  lo = (long)(((unsigned long)l[1] << 32) | l[0]);
}

template <int kEpi, int kNM>
__global__ __launch_bounds__(512) void k_mv_kq(MatrixView w, ActView act, int rows_b, int n_tiles,
                                               MatvecOut o) {
  __shared__ float s_lane[8][kNM][256];
  __shared__ float s_min[kNM][256];
  __shared__ unsigned long long s_key[4][16];
  const int lane = threadIdx.x % kWave, c = threadIdx.x / kWave;
  const int units = w.mtiles / kNM;
  const int group = blockIdx.x / (8 * n_tiles), rem = blockIdx.x % (8 * n_tiles);
  const int nt = rem / 8, unit = group * 8 + rem % 8;
  if (unit >= units) return;
  const int nb = w.nb;
  const v4i zero = {0, 0, 0, 0};
  // the (row, batch row) pair of this lane's min chain: slot p of the MFMA
  // output layout, row 4*((p%64)/16) + p/64, batch row p%16
  const int p = c * 32 + (lane % 32);
  const int mrow = 4 * ((p % 64) / 16) + p / 64, mcol = p % 16;
  const bool mown = w.has_min && lane < 32;
  float L[kNM][4], S[kNM];
#pragma unroll
  for (int m = 0; m < kNM; m++) {
    S[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) L[m][i] = 0.0f;
  }
  for (int b = 0; b < nb; b++) {
    const uint2 av = *reinterpret_cast<const uint2 *>(act.qs + kq_byte(nt, nb, b, c, lane, 0));
    const long bop = (long)(((unsigned long)av.y << 32) | av.x);
    const float da = act.kd[kq_row(nt, nb, b, lane % 16)];
#pragma unroll
    for (int m = 0; m < kNM; m++) {
      const size_t tile = (size_t)unit * kNM + m;
      const uint2 qv = *reinterpret_cast<const uint2 *>(w.qs + kq_byte(tile, nb, b, c, lane, 0));
      const uint32_t sc = w.ksc[kq_row(tile, nb, b, 0) * 4 + lane];
      const uint2 dw4 = *reinterpret_cast<const uint2 *>(w.ds + kq_row(tile, nb, b, 4 * (lane / 16)));
      long hi, lo;
      kq_split(qv, sc, hi, lo);
      v4i ih = __builtin_amdgcn_mfma_i32_16x16x32_i8(hi, bop, zero, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) ih[i] *= 128;
      const v4i is = __builtin_amdgcn_mfma_i32_16x16x32_i8(lo, bop, ih, 0, 0, 0);
      const uint16_t dws[4] = {(uint16_t)dw4.x, (uint16_t)(dw4.x >> 16), (uint16_t)dw4.y,
                               (uint16_t)(dw4.y >> 16)};
#pragma unroll
      for (int i = 0; i < 4; i++) L[m][i] = fmaf(h2f(dws[i]) * da, (float)is[i], L[m][i]);
    }
    if (mown) {
      const size_t ar = kq_row(nt, nb, b, mcol);
      const float dam = act.kd[ar];
      const uint4 g0 = *reinterpret_cast<const uint4 *>(act.ksum + ar * 16);
      const uint4 g1 = *reinterpret_cast<const uint4 *>(act.ksum + ar * 16 + 8);
      const uint32_t gw[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int m = 0; m < kNM; m++) {
        const size_t wr = kq_row((size_t)unit * kNM + m, nb, b, mrow);
        const uint2 mn = *reinterpret_cast<const uint2 *>(w.kmin + wr * 8);
        int ms = 0;
#pragma unroll
        for (int g = 0; g < 8; g++) {
          const int mg = (int)(((g < 4 ? mn.x : mn.y) >> (8 * (g % 4))) & 0xffu);
          const int gsum = (int)(int16_t)(gw[g] & 0xffffu) + (int)(int16_t)(gw[g] >> 16);
          ms += mg * gsum;
        }
        S[m] = fmaf(-(h2f(w.kdm[wr]) * dam), (float)ms, S[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kNM; m++) {
#pragma unroll
    for (int i = 0; i < 4; i++) s_lane[c][m][i * 64 + lane] = L[m][i];
    if (lane < 32) s_min[m][p] = S[m];
  }
  __syncthreads();
  // ---- the chains meet; then the epilogue (as k_mv_q8s)
  const int t = threadIdx.x, prow = 4 * ((t % 64) / 16) + t / 64, pcol = t % 16;
  float acc[kNM];
#pragma unroll
  for (int m = 0; m < kNM; m++) {
    acc[m] = 0.0f;
    if (t < 256) {
      float v = s_min[m][t];
#pragma unroll
      for (int cc = 0; cc < 8; cc++) v = v + s_lane[cc][m][t];
      acc[m] = v;
    }
  }
  const int r = nt * 16 + pcol;
  const bool rvalid = t < 256 && r < rows_b;
  const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
  bool bad = false;
  if constexpr (kEpi == kEpiArgmax) {
    const int row = unit * 16 + prow;
    const bool valid = rvalid && row < w.rows;
    const float v = acc[0];
    if (valid) {
      bad = !finitef(v);
      if (o.logits) o.logits[(size_t)r * w.rows + row] = v;
    }
    unsigned long long key = valid ? argmax_key(v, row) : 0ull;
    unsigned long long x = __shfl_xor(key, 16, kWave);
    key = x > key ? x : key;
    x = __shfl_xor(key, 32, kWave);
    key = x > key ? x : key;
    if (t < 256 && lane < 16) s_key[c][lane] = key;
    __syncthreads();
    if (t < 16) {
      unsigned long long best = s_key[0][t];
#pragma unroll
      for (int i = 1; i < 4; i++) best = s_key[i][t] > best ? s_key[i][t] : best;
      if (nt * 16 + t < rows_b) o.argmax[(size_t)(nt * 16 + t) * units + unit] = best;
    }
  } else if (rvalid) {
    const int row = unit * 16 + prow;
    if (kEpi == kEpiSwiglu) {
      if (row < w.rows / 2) {
        const float g = acc[0], u = acc[kNM - 1];
        bad = !finitef(g) || !finitef(u);
        o.out[(size_t)r * o.ld + row] = (g / (1.0f + exp_f32(-g))) * u;
      }
    } else if (row < w.rows) {
      const float v = acc[0];
      bad = !finitef(v);
      float *q = o.out + (size_t)r * o.ld + row;
      if (kEpi == kEpiResidual)
        *q = *q + v;
      else
        *q = v;
    }
  }
  if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Register-chain Q8_0 matvec for short K.  A wave owns kNM weight tiles x kNN
// batch tiles and walks the blocks in order, as the reference chain does
// (quant.rs:265-272): per block one int8 MFMA gives the exact isum of every
// (row, batch row) pair, then acc = fmaf((float)isum, dw*da, acc).  dw*da is
// one v_fma_mix_f32 of the two binary16 scales with a +0 addend: the product
// of two binary16 values is exact in f32, and the accumulator, starting at
// +0, is never -0, so the sign of a zero product cannot reach the result.
// Operands come through buffer resources (scalar base, per-lane offset); a
// batch tile past the last one gets an empty resource and reads zeros.
// ---------------------------------------------------------------------------
template <int WH, int AH>
__device__ __forceinline__ float scale_mul(uint32_t w, uint32_t a) {
  float r;
  if constexpr (WH == 0 && AH == 0)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(w), "v"(a));
  else if constexpr (WH == 1 && AH == 0)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(w), "v"(a));
  else if constexpr (WH == 0 && AH == 1)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(w), "v"(a));
  else
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(w), "v"(a));
  return r;
}

// Q4_0 chain (quant.rs:286-292): t = f32(isum) * dw rounded once, then
// acc = fmaf(t, da, acc); the binary16 scale is read from the low (H=0) or
// high (H=1) half of a packed register by the mixed-precision FMA.
template <int WH>
__device__ __forceinline__ float mul_half(float a, uint32_t w) {
  float r;
  if constexpr (WH == 0)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w));
  else
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(a), "v"(w));
  return r;
}
__device__ __forceinline__ float fma_half(float t, uint32_t a, float acc) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(t), "v"(a), "v"(acc));
  return r;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

template <int kNM, int kNN>
struct ChainPair {
  uint4 a[kNM];        // weight tiles, blocks 2p and 2p+1
  uint4 b[kNN];        // batch tiles, blocks 2p and 2p+1
  uint2 dw[kNM][2];    // the lane's 4 rows' scales, block 2p / 2p+1
  uint32_t da[kNN][2]; // the lane's batch row scale, block 2p / 2p+1
};

constexpr int kChainWaves = 4;  // batch groups per workgroup

template <int kEpi, int kNM, int kNN, int kDepth, int kFmt>
__global__ __launch_bounds__(64 * kChainWaves) void k_mv_q8c(MatrixView w, ActView act, int rows_b,
                                                            int n_tiles, MatvecOut o) {
  constexpr uint32_t kPairBytes = kFmt == 8 ? 1024 : 512;  // weight bytes per tile per block pair
  const int lane = threadIdx.x % kWave;
  const int ng = blockIdx.y * (int)(blockDim.x / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int unit = blockIdx.x;
  if (ng * kNN >= n_tiles) return;
  const int npairs = w.nbp / 2, nbp = w.nbp, rsub = 4 * (lane / 16), col = lane % 16;
  __amdgpu_buffer_rsrc_t ra[kNM], rw[kNM], rb[kNN], rd[kNN];
#pragma unroll
  for (int m = 0; m < kNM; m++) {
    const int tile = unit * kNM + m;
    ra[m] = buffer_rsrc(w.qs + (size_t)tile * npairs * kPairBytes, (uint32_t)npairs * kPairBytes);
    rw[m] = buffer_rsrc(w.ds + (size_t)tile * nbp * 16, (uint32_t)nbp * 32);
  }
#pragma unroll
  for (int n = 0; n < kNN; n++) {
    const int nt = ng * kNN + n;
    const bool live = nt < n_tiles;
    rb[n] = buffer_rsrc(act.qs + (size_t)(live ? nt : 0) * npairs * 1024, live ? (uint32_t)npairs * 1024 : 0u);
    rd[n] = buffer_rsrc(act.ds + (size_t)(live ? nt : 0) * nbp * 16, live ? (uint32_t)nbp * 32 : 0u);
  }
  const int voff = lane * 16, woff = rsub * 2, doff = col * 2;
  auto load = [&](ChainPair<kNM, kNN> &r, int p) {
#pragma unroll
    for (int m = 0; m < kNM; m++) {
      if constexpr (kFmt == 8) {
        r.a[m] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra[m], voff, p * 1024, 0));
      } else {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ra[m], lane * 8, p * 512, 0));
        r.a[m] = make_uint4(v.x, v.y, 0u, 0u);
      }
      r.dw[m][0] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw[m], woff, p * 64, 0));
      r.dw[m][1] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw[m], woff + 32, p * 64, 0));
    }
#pragma unroll
    for (int n = 0; n < kNN; n++) {
      r.b[n] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb[n], voff, p * 1024, 0));
      r.da[n][0] = __builtin_amdgcn_raw_buffer_load_b16(rd[n], doff, p * 64, 0);
      r.da[n][1] = __builtin_amdgcn_raw_buffer_load_b16(rd[n], doff + 32, p * 64, 0);
    }
  };
  float acc[kNM][kNN][4];
#pragma unroll
  for (int m = 0; m < kNM; m++)
#pragma unroll
    for (int n = 0; n < kNN; n++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[m][n][i] = 0.0f;
  const v4i zero = {0, 0, 0, 0};
  ChainPair<kNM, kNN> ring[kDepth];
#pragma unroll
  for (int i = 0; i < kDepth; i++)
    if (i < npairs) load(ring[i], i);
  for (int p0 = 0; p0 < npairs; p0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; u++) {
      const int pr = p0 + u;
      if (pr < npairs) {
        const ChainPair<kNM, kNN> &r = ring[u];
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
          for (int m = 0; m < kNM; m++) {
            long aop;
            if constexpr (kFmt == 8)
              aop = h ? hi64(r.a[m]) : lo64(r.a[m]);
            else
              aop = q4_operand(h ? r.a[m].y : r.a[m].x);
#pragma unroll
            for (int n = 0; n < kNN; n++) {
              const v4i sum = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, h ? hi64(r.b[n]) : lo64(r.b[n]),
                                                                    zero, 0, 0, 0);
              const uint2 s2 = r.dw[m][h];
              if constexpr (kFmt == 8) {
                const float sc[4] = {scale_mul<0, 0>(s2.x, r.da[n][h]), scale_mul<1, 0>(s2.x, r.da[n][h]),
                                     scale_mul<0, 0>(s2.y, r.da[n][h]), scale_mul<1, 0>(s2.y, r.da[n][h])};
#pragma unroll
                for (int i = 0; i < 4; i++) acc[m][n][i] = fmaf((float)sum[i], sc[i], acc[m][n][i]);
              } else {
                const float t[4] = {mul_half<0>((float)sum[0], s2.x), mul_half<1>((float)sum[1], s2.x),
                                    mul_half<0>((float)sum[2], s2.y), mul_half<1>((float)sum[3], s2.y)};
#pragma unroll
                for (int i = 0; i < 4; i++) acc[m][n][i] = fma_half(t[i], r.da[n][h], acc[m][n][i]);
              }
            }
          }
        }
        if (pr + kDepth < npairs) load(ring[u], pr + kDepth);
      }
    }
  }
  // ---- epilogue: lane holds rows (unit*kNM + m)*16 + rsub + i of batch row (ng*kNN + n)*16 + col
  const int units = w.mtiles / kNM;
#pragma unroll
  for (int n = 0; n < kNN; n++) {
    const int r = (ng * kNN + n) * 16 + col;
    const bool rvalid = r < rows_b;
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
      unsigned long long key = have ? argmax_key(best, best_row) : 0ull;
      unsigned long long x = __shfl_xor(key, 16, kWave);
      key = x > key ? x : key;
      x = __shfl_xor(key, 32, kWave);
      key = x > key ? x : key;
      if (lane < 16 && rvalid) o.argmax[(size_t)r * units + unit] = key;
    } else if (kEpi == kEpiSwiglu) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = unit * 16 + rsub + i;
        if (!rvalid || row >= w.rows / 2) continue;
        const float g = acc[0][n][i], u = acc[kNM - 1][n][i];
        bad |= !finitef(g) || !finitef(u);
        o.out[(size_t)r * o.ld + row] = (g / (1.0f + exp_f32(-g))) * u;
      }
    } else {
#pragma unroll
      for (int m = 0; m < kNM; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int row = (unit * kNM + m) * 16 + rsub + i;
          if (!rvalid || row >= w.rows) continue;
          const float v = acc[m][n][i];
          bad |= !finitef(v);
          float *q = o.out + (size_t)r * o.ld + row;
          if (kEpi == kEpiResidual)
            *q = *q + v;
          else
            *q = v;
        }
    }
    if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
  }
}

// ---------------------------------------------------------------------------
// Short-K Q8_0/Q4_0 matvec with the weight unit in LDS.  A workgroup owns one
// unit (kNM weight tiles of 16 rows; 2 = a gate tile and its up tile) and up
// to 8 batch tiles, one per wave.  At the start every thread issues its share
// of one cooperative copy into LDS (the unit's quantized tiles, their block
// scales and the batch tiles' block scales), and each wave issues the loads
// of its batch tile's whole B operand into registers, so the kernel waits on
// memory once.  Then every wave walks the blocks in order, as the reference
// chain does (quant.rs:265-292): per block one int8 MFMA gives the exact isum
// of every (row, batch row) pair, then acc = fmaf((float)isum, dw*da, acc)
// for Q8_0 (dw*da exact in f32, formed by v_fma_mix_f32 with a +0 addend) or
// acc = fmaf((float)isum*dw, da, acc) for Q4_0.  K is limited to
// 64 * kMaxPairs inputs (the B operand lives in registers).
// ---------------------------------------------------------------------------
template <int kEpi, int kNM, int kFmt, int kMaxPairs, int kU, bool kExact = false>
__global__ __launch_bounds__(512 * kU) void k_mv_q8w(MatrixView w, ActView act, int rows_b, int n_tiles,
                                                     MatvecOut o, ActView qout, int qout_nbp) {
  static_assert(kU == 1 || (kU == 2 && kEpi == kEpiSwiglu), "two units per workgroup: the fused quantizer");
  constexpr int kPairBytes = kFmt == 8 ? 1024 : 512;  // weight bytes per tile per block pair
  constexpr int kCopy = 8;                            // 16-byte copy items per thread (<= 64 KB)
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nthreads = blockDim.x;
  // kU units per workgroup of kU * W waves (W = min(n_tiles, 8) for every
  // workgroup): wave w takes unit kU * blockIdx.x + w / W and batch tile
  // tile0 + w % W (past n_tiles in a last, partial row of tiles: not live)
  const int W = nthreads / (kWave * kU);
  const int tile0 = blockIdx.y * W, nbt = min(W, n_tiles - tile0);
  const int uw = wave / W, bt = wave % W;
  const int unit = blockIdx.x * kU + uw, nt = tile0 + bt;
  // kExact: K is exactly kMaxPairs block pairs (checked by the launch), so
  // the block loop below is straight-line code the compiler can schedule
  // across pairs (MFMAs of later pairs issued under earlier chains)
  const int npairs = kExact ? kMaxPairs : w.nbp / 2, nbp = kExact ? 2 * kMaxPairs : w.nbp;
  const int nw = kU * kNM * npairs * kPairBytes / 16;  // copy items: weights, weight scales, batch scales
  const int ns = kU * kNM * nbp * 32 / 16;
  const int nd = nbt * nbp * 32 / 16;
  const uint4 *gw = reinterpret_cast<const uint4 *>(w.qs + (size_t)blockIdx.x * kU * kNM * npairs * kPairBytes);
  const uint4 *gs = reinterpret_cast<const uint4 *>(w.ds + (size_t)blockIdx.x * kU * kNM * nbp * 16);
  const uint4 *gd = reinterpret_cast<const uint4 *>(act.ds + (size_t)tile0 * nbp * 16);
  const bool live = nt < n_tiles;
  uint4 b[kMaxPairs];
#pragma unroll
  for (int p = 0; p < kMaxPairs; p++)
    if (live && p < npairs) b[p] = *reinterpret_cast<const uint4 *>(act.qs + q8_byte(nt, nbp, 2 * p, lane, 0));
  // one round covers 64 KB with 8 waves; fewer waves (few batch rows) take more
  const int total = nw + ns + nd;
  for (int base = 0; base < total; base += kCopy * nthreads) {
    uint4 cp[kCopy];
#pragma unroll
    for (int k = 0; k < kCopy; k++) {  // past the end: reload the last item, not stored
      const int i = min(base + (int)threadIdx.x + k * nthreads, total - 1);
      const uint4 *src = i < nw ? gw + i : i < nw + ns ? gs + (i - nw) : gd + (i - nw - ns);
      cp[k] = *src;
    }
#pragma unroll
    for (int k = 0; k < kCopy; k++) {
      const int i = base + (int)threadIdx.x + k * nthreads;
      if (i < total) smem[i] = cp[k];
    }
  }
  __shared__ uint64_t s_tab[32];  // expf's table for the SwiGLU epilogue
  if (kEpi == kEpiSwiglu && threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  if (kU == 1 && !live) return;
  // this wave's unit: its kNM tiles and their scales
  const uint8_t *sw = reinterpret_cast<const uint8_t *>(smem) + (size_t)uw * kNM * npairs * kPairBytes;
  const uint16_t *ssc = reinterpret_cast<const uint16_t *>(smem + nw) + uw * kNM * nbp * 16;  // [m][block][16]
  const uint16_t *sda = reinterpret_cast<const uint16_t *>(smem + nw) + kU * kNM * nbp * 16;  // [tile][block][16]
  const int rsub = 4 * (lane / 16), col = lane % 16;
  const v4i zero = {0, 0, 0, 0};
  float acc[kNM][4];
#pragma unroll
  for (int m = 0; m < kNM; m++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[m][i] = 0.0f;
  // one block pair of the chain: the unit's tiles from LDS, an MFMA per
  // (block, tile), then acc = fmaf(isum, scale product, acc) in block order
  auto pair = [&](int p) __attribute__((always_inline)) {
    uint4 a[kNM];
#pragma unroll
    for (int m = 0; m < kNM; m++) {
      if constexpr (kFmt == 8) {
        a[m] = *reinterpret_cast<const uint4 *>(sw + (m * npairs + p) * kPairBytes + lane * 16);
      } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(sw + (m * npairs + p) * kPairBytes + lane * 8);
        a[m] = make_uint4(v.x, v.y, 0u, 0u);
      }
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int blk = 2 * p + h;
      const long bop = h ? hi64(b[p]) : lo64(b[p]);
      const uint32_t da = sda[(bt * nbp + blk) * 16 + col];
#pragma unroll
      for (int m = 0; m < kNM; m++) {
        long aop;
        if constexpr (kFmt == 8)
          aop = h ? hi64(a[m]) : lo64(a[m]);
        else
          aop = q4_operand(h ? a[m].y : a[m].x);
        const v4i sum = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, zero, 0, 0, 0);
        const uint2 s2 = *reinterpret_cast<const uint2 *>(ssc + (m * nbp + blk) * 16 + rsub);
        if constexpr (kFmt == 8) {
          const float sc[4] = {scale_mul<0, 0>(s2.x, da), scale_mul<1, 0>(s2.x, da), scale_mul<0, 0>(s2.y, da),
                               scale_mul<1, 0>(s2.y, da)};
#pragma unroll
          for (int i = 0; i < 4; i++) acc[m][i] = fmaf((float)sum[i], sc[i], acc[m][i]);
        } else {
          const float t[4] = {mul_half<0>((float)sum[0], s2.x), mul_half<1>((float)sum[1], s2.x),
                              mul_half<0>((float)sum[2], s2.y), mul_half<1>((float)sum[3], s2.y)};
#pragma unroll
          for (int i = 0; i < 4; i++) acc[m][i] = fma_half(t[i], da, acc[m][i]);
        }
      }
    }
  };
  if constexpr (kExact) {
    if (live) {
#pragma unroll
      for (int p = 0; p < kMaxPairs; p++) pair(p);
    }
  } else {
#pragma unroll
    for (int p = 0; p < kMaxPairs; p++)
      if (p < npairs && live) pair(p);
  }
  // ---- epilogue: lane holds rows (unit*kNM + m)*16 + rsub + i of batch row nt*16 + col
  const int r = nt * 16 + col;
  const bool rvalid = r < rows_b;
  const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
  bool bad = false;
  if constexpr (kU == 2) {
    // Fused SwiGLU quantizer: the two units' 32 outputs are one Q8_0 block
    // (block blockIdx.x) of each batch row.  Each wave parks its 16 x 16
    // SwiGLU values in LDS; then the
    // first unit's wave of each batch tile gives lane l the block's elements
    // 8 (l / 16) .. + 7 of batch row l % 16 and runs k_quant_act's arithmetic.
    // (over the weight tiles: every wave is past its MFMAs at the barrier;
    // the launch allocates at least the 16 KB this needs)
    float *s_h = reinterpret_cast<float *>(smem);  // [uw][bt][16 rows][16 batch rows]
    __syncthreads();
    if (live) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float g = acc[0][i], u = acc[kNM - 1][i];
        bad |= rvalid && (!finitef(g) || !finitef(u));
        s_h[((uw * 8 + bt) * 16 + rsub + i) * 16 + col] = (g / (1.0f + exp_f32_tab(-g, s_tab))) * u;
      }
    }
    __syncthreads();
    if (live && uw == 0) {
      const int k = lane / 16;  // elements 8k .. 8k + 7 of the block
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int el = 8 * k + e;
        v[e] = s_h[(((el / 16) * 8 + bt) * 16 + el % 16) * 16 + col];
      }
      bad |= quant_group_q8<16>(v, rvalid, r, blockIdx.x * 4 + k, qout_nbp, qout);
    }
  } else if (kEpi == kEpiSwiglu) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = unit * 16 + rsub + i;
      if (!rvalid || row >= w.rows / 2) continue;
      const float g = acc[0][i], u = acc[kNM - 1][i];
      bad |= !finitef(g) || !finitef(u);
      o.out[(size_t)r * o.ld + row] = (g / (1.0f + exp_f32_tab(-g, s_tab))) * u;
    }
  } else {
#pragma unroll
    for (int m = 0; m < kNM; m++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = (unit * kNM + m) * 16 + rsub + i;
        if (!rvalid || row >= w.rows) continue;
        const float v = acc[m][i];
        bad |= !finitef(v);
        float *q = o.out + (size_t)r * o.ld + row;
        if (kEpi == kEpiResidual)
          *q = *q + v;
        else
          *q = v;
      }
  }
  if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// Gate+up projection with SwiGLU and the down projection's Q8_0 quantizer in
// the epilogue (Q8_0/Q4_0 weights, K <= 64 * kMaxPairs).  A workgroup owns one
// Q8_0 block of the SwiGLU output (two 16-row units: gate and up tiles
// 4q .. 4q+3) for kNB batch tiles; wave w multiplies weight tile 4q + w % 4
// with batch tile w / 4, the whole K in block order, so each (row, batch row)
// chain is the reference's (quant.rs:265-292) as in k_mv_q8w.  The wave's
// weight tile goes straight to registers; the batch tiles' B operand and all
// block scales are copied to LDS once per workgroup, in the same memory round
// trip.  Workgroups of one block q sit on one XCD (blockIdx % 8), so the
// weight tiles shared by its batch groups are fetched into that L2 once.
// ---------------------------------------------------------------------------
template <int kFmt, int kNB, int kNN, int kMaxPairs, bool kExact = false>
__global__ __launch_bounds__(256 * kNB) void k_mv_gu(MatrixView w, ActView act, int rows_b, int n_tiles,
                                                     uint32_t *row_err, const uint32_t *err_rows,
                                                     ActView qout, int qout_nbp) {
  constexpr int kBT = kNB * kNN;  // batch tiles per workgroup
  extern __shared__ uint4 smem[];
  __shared__ uint64_t s_tab[32];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nq = w.mtiles / 4, nbg = (n_tiles + kBT - 1) / kBT;
  const int g8 = blockIdx.x / (8 * nbg), rem = blockIdx.x % (8 * nbg);
  const int bg = rem / 8, q = g8 * 8 + rem % 8;
  if (q >= nq) return;  // whole workgroup, before any barrier
  // kExact: K is exactly kMaxPairs block pairs (checked by the launch): the
  // block loop is straight-line code, scheduled across pairs
  const int npairs = kExact ? kMaxPairs : w.nbp / 2, nbp = kExact ? 2 * kMaxPairs : w.nbp;
  const int tw = wave % 4, tile = 4 * q + tw;
  const int tile0 = bg * kBT, nbt = min(kBT, n_tiles - tile0);
  // LDS: [kBT][npairs][64] uint4 B operand, then [4][nbp][16] weight scales,
  // then [kBT][nbp][16] batch scales (u16)
  const int nb_items = nbt * npairs * 64, nw_items = 4 * nbp * 2, nd_items = nbt * nbp * 2;
  const uint4 *gb = reinterpret_cast<const uint4 *>(act.qs) + (size_t)tile0 * npairs * 64;
  const uint4 *gw = reinterpret_cast<const uint4 *>(w.ds + (size_t)4 * q * nbp * 16);
  const uint4 *gd = reinterpret_cast<const uint4 *>(act.ds + (size_t)tile0 * nbp * 16);
  const int total = nb_items + nw_items + nd_items;
  // the wave's weight tile into registers (branch-free: pairs past K reload the last)
  uint4 a[kMaxPairs];
#pragma unroll
  for (int p = 0; p < kMaxPairs; p++) {
    const int pp = min(p, npairs - 1);
    if constexpr (kFmt == 8) {
      a[p] = *reinterpret_cast<const uint4 *>(w.qs + q8_byte(tile, nbp, 2 * pp, lane, 0));
    } else {
      const uint2 v = *reinterpret_cast<const uint2 *>(w.qs + q4_byte(tile, nbp, 2 * pp, lane, 0));
      a[p] = make_uint4(v.x, v.y, 0u, 0u);
    }
  }
  constexpr int kCopy = 8;
  for (int base = 0; base < total; base += kCopy * 256 * kNB) {
    uint4 cp[kCopy];
#pragma unroll
    for (int k = 0; k < kCopy; k++) {
      const int i = min(base + (int)threadIdx.x + k * 256 * kNB, total - 1);
      cp[k] = i < nb_items ? gb[i] : i < nb_items + nw_items ? gw[i - nb_items] : gd[i - nb_items - nw_items];
    }
#pragma unroll
    for (int k = 0; k < kCopy; k++) {
      const int i = base + (int)threadIdx.x + k * 256 * kNB;
      if (i < total) smem[i] = cp[k];
    }
  }
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  __syncthreads();
  // wave w: weight tile 4q + w % 4 against batch tiles (w / 4) * kNN + n
  const int bt0 = (wave / 4) * kNN;
  const uint16_t *sdw = reinterpret_cast<const uint16_t *>(smem + nb_items) + (size_t)tw * nbp * 16;
  const uint16_t *sda = reinterpret_cast<const uint16_t *>(smem + nb_items + nw_items);
  const int rsub = 4 * (lane / 16), col = lane % 16;
  const v4i zero = {0, 0, 0, 0};
  float acc[kNN][4];
#pragma unroll
  for (int n = 0; n < kNN; n++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[n][i] = 0.0f;
  // one block pair against batch tile bt0 + n: an MFMA per block, then
  // acc = fmaf(isum, scale product, acc) in block order
  auto pair = [&](int p, int n) __attribute__((always_inline)) {
    const int bt = bt0 + n;
    const uint4 b = smem[(bt * npairs + p) * 64 + lane];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int blk = 2 * p + h;
      long aop;
      if constexpr (kFmt == 8)
        aop = h ? hi64(a[p]) : lo64(a[p]);
      else
        aop = q4_operand(h ? a[p].y : a[p].x);
      const v4i sum = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, h ? hi64(b) : lo64(b), zero, 0, 0, 0);
      const uint2 s2 = *reinterpret_cast<const uint2 *>(sdw + blk * 16 + rsub);
      const uint32_t da = sda[(bt * nbp + blk) * 16 + col];
      if constexpr (kFmt == 8) {
        const float sc[4] = {scale_mul<0, 0>(s2.x, da), scale_mul<1, 0>(s2.x, da),
                             scale_mul<0, 0>(s2.y, da), scale_mul<1, 0>(s2.y, da)};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = fmaf((float)sum[i], sc[i], acc[n][i]);
      } else {
        const float t[4] = {mul_half<0>((float)sum[0], s2.x), mul_half<1>((float)sum[1], s2.x),
                            mul_half<0>((float)sum[2], s2.y), mul_half<1>((float)sum[3], s2.y)};
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = fma_half(t[i], da, acc[n][i]);
      }
    }
  };
  if (kExact && bt0 + kNN <= nbt) {  // every batch tile of the wave present
#pragma unroll
    for (int p = 0; p < kMaxPairs; p++)
#pragma unroll
      for (int n = 0; n < kNN; n++) pair(p, n);
  } else {
#pragma unroll
    for (int p = 0; p < kMaxPairs; p++) {
      if (p < npairs) {
#pragma unroll
        for (int n = 0; n < kNN; n++)
          if (bt0 + n < nbt) pair(p, n);
      }
    }
  }
  // ---- epilogue: the block's 4 x 16 x 16 chains per batch tile meet in LDS
  // (the B operand's space: every wave is past its last LDS read at the barrier)
  __syncthreads();
  float *s_o = reinterpret_cast<float *>(smem);  // [kBT][tw][16 rows][16 batch rows]
#pragma unroll
  for (int n = 0; n < kNN; n++) {
    const int bt = bt0 + n;
    if (bt < nbt) {
#pragma unroll
      for (int i = 0; i < 4; i++) s_o[((bt * 4 + tw) * 16 + rsub + i) * 16 + col] = acc[n][i];
    }
  }
  __syncthreads();
  // wave w quantizes batch tiles w, w + 4 kNB, ...: lane l takes elements
  // 8 (l / 16) .. + 7 of the block for batch row l % 16
  for (int bt = wave; bt < nbt; bt += 4 * kNB) {
    const int k = lane / 16, r = (tile0 + bt) * 16 + col;
    const bool rvalid = r < rows_b;
    bool bad = false;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int el = 8 * k + e, u = el / 16, row = el % 16;
      const float g = s_o[((bt * 4 + 2 * u) * 16 + row) * 16 + col];
      const float up = s_o[((bt * 4 + 2 * u + 1) * 16 + row) * 16 + col];
      bad |= rvalid && (!finitef(g) || !finitef(up));
      v[e] = (g / (1.0f + exp_f32_tab(-g, s_tab))) * up;
    }
    bad |= quant_group_q8<16>(v, rvalid, r, q * 4 + k, qout_nbp, qout);
    if (bad) atomicOr(&row_err[err_rows ? (int)err_rows[r] : r], kErrNonFinite);
  }
}

// ---------------------------------------------------------------------------
// LM head (Q8_0/Q4_0, many weight tiles, short K) with per-tile argmax keys.
// Persistent workgroups of up to 8 waves, wave w = batch tile w: each wave
// loads its batch tile's B operand into registers once, and the workgroup
// streams weight tiles unit = blockIdx.x, + gridDim.x, ... through two LDS
// buffers (the next tile's copy is requested before the current one is
// consumed; one barrier per tile), so a weight tile is read from memory once
// per workgroup and the activations once per wave, instead of once per
// (tile, wave).  The chain per (row, batch row) is the reference's
// (quant.rs:265-292), as in k_mv_q8w.  K <= 64 * kMaxPairs, n_tiles <= 8.
// ---------------------------------------------------------------------------
template <int kFmt, int kMaxPairs>
__global__ __launch_bounds__(512, 4) void k_mv_q8h(MatrixView w, ActView act, int rows_b, int n_tiles,
                                                   MatvecOut o) {
  constexpr int kPairBytes = kFmt == 8 ? 1024 : 512;
  constexpr int kCopy = 4;  // 16-byte items per thread per tile copy (<= 32 KB: 512 threads)
  static_assert(kCopy == 4, "the loop's copy registers are cp0..cp3");
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nthreads = blockDim.x;
  const int units = w.mtiles, npairs = w.nbp / 2, nbp = w.nbp;
  const int nw = npairs * kPairBytes / 16, ns = nbp * 32 / 16, nd = n_tiles * nbp * 32 / 16;
  const int tile_items = nw + ns;  // one weight tile and its scales, in 16-byte items (<= 2048)
  const uint16_t *sda = reinterpret_cast<const uint16_t *>(smem + 2 * tile_items);  // [tile][block][16]
  const int nt = wave;
  const bool live = nt < n_tiles;
  uint4 b[kMaxPairs];
#pragma unroll
  for (int p = 0; p < kMaxPairs; p++)
    if (live && p < npairs) b[p] = *reinterpret_cast<const uint4 *>(act.qs + q8_byte(nt, nbp, 2 * p, lane, 0));
  // batch scales (once) and the first weight tile
  const uint4 *gd = reinterpret_cast<const uint4 *>(act.ds);
  for (int i = threadIdx.x; i < nd; i += nthreads) smem[2 * tile_items + i] = gd[i];
  // tile item i: the tile's quantized pairs, then its block scales
  const uint4 *gq = reinterpret_cast<const uint4 *>(w.qs);
  const uint4 *gs = reinterpret_cast<const uint4 *>(w.ds);
  int unit = blockIdx.x;
  {
    uint4 c0[kCopy];
#pragma unroll
    for (int k = 0; k < kCopy; k++) {
      const int i = min((int)threadIdx.x + k * nthreads, tile_items - 1);
      c0[k] = i < nw ? gq[(size_t)unit * nw + i] : gs[(size_t)unit * ns + (i - nw)];
    }
#pragma unroll
    for (int k = 0; k < kCopy; k++)
      if ((int)threadIdx.x + k * nthreads < tile_items) smem[threadIdx.x + k * nthreads] = c0[k];
  }
  __syncthreads();
  const int rsub = 4 * (lane / 16), col = lane % 16;
  const v4i zero = {0, 0, 0, 0};
  const int r = nt * 16 + col;
  const bool rvalid = live && r < rows_b;
  const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
  bool bad = false;
  unsigned long long run = 0ull;  // the row's best key over this workgroup's tiles
  for (int it = 0; unit < units; it++, unit += gridDim.x) {
    const int next = unit + gridDim.x;
    // the next tile's share of this thread (kCopy == 4 items), requested now;
    // the last tile refetches itself (never stored) rather than branch
    const int nu = min(next, units - 1);
    auto item = [&](int k) {
      const int i = min((int)threadIdx.x + k * nthreads, tile_items - 1);
      return i < nw ? gq[(size_t)nu * nw + i] : gs[(size_t)nu * ns + (i - nw)];
    };
    const uint4 cp0 = item(0), cp1 = item(1), cp2 = item(2), cp3 = item(3);
    const uint4 *cur = smem + (it & 1) * tile_items;  // the two tile buffers alternate
    const uint8_t *sw = reinterpret_cast<const uint8_t *>(cur);
    const uint16_t *ssc = reinterpret_cast<const uint16_t *>(cur + nw);  // [block][16 rows]
    if (live) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int p = 0; p < kMaxPairs; p++) {
        if (p < npairs) {
          uint4 a;
          if constexpr (kFmt == 8) {
            a = *reinterpret_cast<const uint4 *>(sw + p * kPairBytes + lane * 16);
          } else {
            const uint2 v = *reinterpret_cast<const uint2 *>(sw + p * kPairBytes + lane * 8);
            a = make_uint4(v.x, v.y, 0u, 0u);
          }
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const int blk = 2 * p + h;
            long aop;
            if constexpr (kFmt == 8)
              aop = h ? hi64(a) : lo64(a);
            else
              aop = q4_operand(h ? a.y : a.x);
            const v4i sum = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, h ? hi64(b[p]) : lo64(b[p]), zero, 0, 0, 0);
            const uint32_t da = sda[(nt * nbp + blk) * 16 + col];
            const uint2 s2 = *reinterpret_cast<const uint2 *>(ssc + blk * 16 + rsub);
            if constexpr (kFmt == 8) {
              const float sc[4] = {scale_mul<0, 0>(s2.x, da), scale_mul<1, 0>(s2.x, da),
                                   scale_mul<0, 0>(s2.y, da), scale_mul<1, 0>(s2.y, da)};
#pragma unroll
              for (int i = 0; i < 4; i++) acc[i] = fmaf((float)sum[i], sc[i], acc[i]);
            } else {
              const float t[4] = {mul_half<0>((float)sum[0], s2.x), mul_half<1>((float)sum[1], s2.x),
                                  mul_half<0>((float)sum[2], s2.y), mul_half<1>((float)sum[3], s2.y)};
#pragma unroll
              for (int i = 0; i < 4; i++) acc[i] = fma_half(t[i], da, acc[i]);
            }
          }
        }
      }
      // per-tile argmax key of batch row r over the tile's rows (lowest row wins ties)
      float best = 0.0f;
      int best_row = 0;
      bool have = false;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = unit * 16 + rsub + i;
        if (!rvalid || row >= w.rows) continue;
        const float v = acc[i];
        bad |= !finitef(v);
        if (o.logits) o.logits[(size_t)r * w.rows + row] = v;
        if (!have || v > best) {
          best = v;
          best_row = row;
          have = true;
        }
      }
      unsigned long long key = have ? argmax_key(best, best_row) : 0ull;
      unsigned long long x = __shfl_xor(key, 16, kWave);
      key = x > key ? x : key;
      x = __shfl_xor(key, 32, kWave);
      key = x > key ? x : key;
      run = key > run ? key : run;
    }
    if (next < units) {
      uint4 *dst = smem + ((it + 1) & 1) * tile_items;
      const int i0 = threadIdx.x;
      if (i0 < tile_items) dst[i0] = cp0;
      if (i0 + nthreads < tile_items) dst[i0 + nthreads] = cp1;
      if (i0 + 2 * nthreads < tile_items) dst[i0 + 2 * nthreads] = cp2;
      if (i0 + 3 * nthreads < tile_items) dst[i0 + 3 * nthreads] = cp3;
    }
    __syncthreads();
  }
  if (lane < 16 && rvalid && run) atomicMax(o.argmax_final + r, run);
  if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
}

// Final argmax over the per-tile partial keys of each batch row.
__global__ __launch_bounds__(256) void k_argmax_reduce(const unsigned long long *__restrict__ part,
                                                       int units, unsigned long long *out) {
  __shared__ unsigned long long red[4];
  const int r = blockIdx.x;
  unsigned long long best = 0;
  for (int u = threadIdx.x; u < units; u += 256) {
    const unsigned long long k = part[(size_t)r * units + u];
    best = k > best ? k : best;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long x = __shfl_xor(best, m, kWave);
    best = x > best ? x : best;
  }
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; i++) best = red[i] > best ? red[i] : best;
    out[r] = red[0] > best ? red[0] : best;
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
// F16 matvec for batches of 16..127 rows, in the reference's exact order: lane
// = batch row, each dot one sequential f64 chain over k from -0.0
// (cpu.rs:31-35 over round_f16 operands), f32 result.  A wave owns 4 output
// rows (4 gate + 4 up rows for SwiGLU) and one pass of up to 64 batch rows;
// the weight rows are wave-uniform loads, the activation rows per lane.  The
// argmax epilogue leaves one key per (batch row, 16-row tile) for
// k_argmax_reduce.
// ---------------------------------------------------------------------------
template <int kEpi>
__global__ __launch_bounds__(256) void k_mv_f16s(MatrixView w, ActView act, int rows_b,
                                                 MatvecOut o) {
  constexpr int kQ = kEpi == kEpiSwiglu ? 8 : 4;
  __shared__ unsigned long long s_key[4][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int out_rows = kEpi == kEpiSwiglu ? w.rows / 2 : w.rows;
  const int o0 = (blockIdx.x * 4 + wave) * 4;
  const int r = blockIdx.y * kWave + lane;
  const int K = w.K;
  const int rr = min(r, rows_b - 1);
  const uint16_t *xr = act.f16 + (size_t)rr * K;
  const uint16_t *wq[kQ];
#pragma unroll
  for (int q = 0; q < kQ; q++) {
    int row = o0 + (q % 4);
    row = min(row, out_rows - 1);
    if (kEpi == kEpiSwiglu && q >= 4) row += out_rows;
    wq[q] = w.f16 + (size_t)row * K;
  }
  double acc[kQ];
#pragma unroll
  for (int q = 0; q < kQ; q++) acc[q] = -0.0;
  for (int k0 = 0; k0 < K; k0 += 8) {
    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + k0);
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    uint4 wv[kQ];
#pragma unroll
    for (int q = 0; q < kQ; q++) wv[q] = *reinterpret_cast<const uint4 *>(wq[q] + k0);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float a = h2f((uint16_t)(xw[e / 2] >> (16 * (e % 2))));
#pragma unroll
      for (int q = 0; q < kQ; q++) {
        const uint32_t ww[4] = {wv[q].x, wv[q].y, wv[q].z, wv[q].w};
        acc[q] += (double)(h2f((uint16_t)(ww[e / 2] >> (16 * (e % 2)))) * a);
      }
    }
  }
  const bool rvalid = r < rows_b;
  const int er = (rvalid && o.err_rows) ? (int)o.err_rows[r] : r;
  bool bad = false;
  if (kEpi == kEpiArgmax) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int row = o0 + q;
      if (!rvalid || row >= w.rows) continue;
      const float v = (float)acc[q];
      bad |= !finitef(v);
      if (o.logits) o.logits[(size_t)r * w.rows + row] = v;
      const unsigned long long key = argmax_key(v, row);
      best = key > best ? key : best;
    }
    s_key[wave][lane] = best;
    __syncthreads();
    if (wave == 0 && rvalid) {
      unsigned long long b = s_key[0][lane];
#pragma unroll
      for (int i = 1; i < 4; i++) b = s_key[i][lane] > b ? s_key[i][lane] : b;
      o.argmax[(size_t)r * w.mtiles + blockIdx.x] = b;
    }
  } else if (rvalid) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int row = o0 + q;
      if (row >= out_rows) continue;
      float v = (float)acc[q];
      float *p = o.out + (size_t)r * o.ld + row;
      if (kEpi == kEpiSwiglu) {
        const float u = (float)acc[q + 4];
        bad |= !finitef(v) || !finitef(u);
        *p = (v / (1.0f + exp_f32(-v))) * u;
      } else {
        bad |= !finitef(v);
        *p = kEpi == kEpiResidual ? *p + v : v;
      }
    }
  }
  if (bad) atomicOr(&o.row_err[er], kErrNonFinite);
}

// ---------------------------------------------------------------------------
// F16 LM head with argmax: the same per-output arithmetic as k_mv_f16 (f64
// per lane in element order, fixed butterfly), 16 vocabulary rows per
// workgroup (4 per wave); each batch row's best key over the 16 rows goes to
// part[r][tile] for k_argmax_reduce, so no output contends on an atomic.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_head_f16(MatrixView w, ActView act, int rows_b,
                                                  MatvecOut o) {
  __shared__ unsigned long long s_key[4];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * 16 + wave * 4;
  const int K = w.K, units = w.mtiles;
  for (int r = 0; r < rows_b; r++) {
    const uint16_t *ar = act.f16 + (size_t)r * K;
    double acc[4] = {-0.0, -0.0, -0.0, -0.0};
    for (int k = lane; k < K; k += kWave) {
      const float a = h2f(ar[k]);
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (row0 + q < w.rows) acc[q] += (double)(h2f(w.f16[(size_t)(row0 + q) * K + k]) * a);
    }
    const int er = o.err_rows ? (int)o.err_rows[r] : r;
    unsigned long long best = 0ull;
    bool bad = false;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float v = (float)wave_sum_f64(acc[q]);
      const int row = row0 + q;
      if (row >= w.rows) continue;
      bad |= !finitef(v);
      if (o.logits && lane == 0) o.logits[(size_t)r * w.rows + row] = v;
      const unsigned long long key = argmax_key(v, row);
      best = key > best ? key : best;
    }
    if (bad && lane == 0) atomicOr(&o.row_err[er], kErrNonFinite);
    if (lane == 0) s_key[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long b = s_key[0];
#pragma unroll
      for (int i = 1; i < 4; i++) b = s_key[i] > b ? s_key[i] : b;
      o.argmax[(size_t)r * units + blockIdx.x] = b;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Bias add, NeoX RoPE from the host-built table (cos, sin of the engine's
// iterative angle, cpu.rs:59-73), K/V append into the paged pool
// (Kv::append, inference.rs:1019-1043; batch.rs:164-184).
// Pool layout per layer: [page][kv_head][16 tokens x head_dim] f32, K rows
// through k_at (element-quad-major, rotated), V rows through v_at.
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
  // query pairs: kQ per thread requested at once, then rotated and stored
  constexpr int kQ = 2;
  for (int p0 = 0; p0 < d.NH * half; p0 += kQ * 256) {
    float qa[kQ], qb[kQ];
    float2 qcs[kQ];
#pragma unroll
    for (int u = 0; u < kQ; u++) {
      const int pc = min(p0 + u * 256 + (int)threadIdx.x, d.NH * half - 1);
      const int e = (pc / half) * d.D + pc % half;
      qa[u] = src[e] + bias[e];
      qb[u] = src[e + half] + bias[e + half];
      qcs[u] = rp[pc % half];
    }
#pragma unroll
    for (int u = 0; u < kQ; u++) {
      const int p = p0 + u * 256 + (int)threadIdx.x;
      if (p >= d.NH * half) continue;
      const int e = (p / half) * d.D + p % half;
      q_rot[(size_t)r * d.H + e] = fmaf(qa[u], qcs[u].x, -(qb[u] * qcs[u].y));
      q_rot[(size_t)r * d.H + e + half] = fmaf(qa[u], qcs[u].y, qb[u] * qcs[u].x);
    }
  }
  if (slot < 0) return;
  const int page = slot / kPage, off = slot % kPage;
  for (int p = threadIdx.x; p < d.NKV * half; p += 256) {
    const int g = p / half, i = p % half, e = d.H + g * d.D + i;
    const float a = src[e] + bias[e], b = src[e + half] + bias[e + half];
    const float2 cs = rp[i];
    kpool[k_at(page, pos / kPage, g, d.NKV, off, i, d.D)] = fmaf(a, cs.x, -(b * cs.y));
    kpool[k_at(page, pos / kPage, g, d.NKV, off, i + half, d.D)] = fmaf(a, cs.y, b * cs.x);
  }
  for (int e = threadIdx.x; e < d.KVD; e += 256) {
    const int g = e / d.D, j = e % d.D, s = d.H + d.KVD + e;
    vpool[v_at(page, g, d.NKV, off, j, d.D)] = src[s] + bias[s];
  }
}

// ---------------------------------------------------------------------------
// Attention (cpu.rs:133-210 attention_rows), exact form.
// Operands that are uniform across a wave (the query of a head in pass 1, the
// normalized score of a token in pass 3) are read with scalar loads and used
// as SGPR operands, so each (token, head, element) costs the reference's own
// three operations: f32 product, widening, f64 add.
//
// Pass 1 (scores): one thread per cached token; its K row sits in VGPRs; for
// each query head the dot is summed in f64 in element order (cpu.rs:31-35).
// The kG heads of a KV group are split over kS workgroups (part p takes heads
// p*kH ..), which read the same K rows (the second read hits the L2): twice
// the waves in flight, and fewer registers per wave (higher occupancy).  A
// part's heads advance together, kE elements at a time, issued as groups
// [products][widenings][adds]: a head's consecutive adds are kH instructions
// apart, so the f64 latency is covered inside the wave (the compiler would
// otherwise chain every triple through one temporary); the query values of
// the next group are requested while the current group computes.
// s = f32(dot) * scale, stored per token as 8 floats
// (scores[row][kv_head][t][8], slot = q head within the group, unused slots
// 0); per-256-token chunk maxima per head.  A wave's four page entries come
// through scalar loads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f4get(const float4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int kD, int kH, int kE>
__device__ __forceinline__ void qk_heads(const float4 (&k4)[kD / 4], const float *qbase, float (&sc)[kH],
                                         float scale) {
  double acc[kH];
#pragma unroll
  for (int h = 0; h < kH; h++) acc[h] = -0.0;
  float qc[kE * kH], qn[kE * kH];
#pragma unroll
  for (int i = 0; i < kE * kH; i++) qc[i] = qbase[(i % kH) * kD + i / kH];
#pragma unroll
  for (int j0 = 0; j0 < kD; j0 += kE) {
    if (j0 + kE < kD) {
#pragma unroll
      for (int i = 0; i < kE * kH; i++) qn[i] = qbase[(i % kH) * kD + j0 + kE + i / kH];
    }
    __builtin_amdgcn_sched_barrier(0);  // the next group's loads stay ahead of this group
    float pr[kE * kH];
#pragma unroll
    for (int e = 0; e < kE; e++) {
      const float kj = f4get(k4[(j0 + e) / 4], (j0 + e) % 4);
#pragma unroll
      for (int h = 0; h < kH; h++) pr[e * kH + h] = qc[e * kH + h] * kj;
    }
    pin_vgprs(pr);
    double w[kE * kH];
#pragma unroll
    for (int i = 0; i < kE * kH; i++) w[i] = (double)pr[i];
    pin_vgprs(w);
#pragma unroll
    for (int e = 0; e < kE; e++)
#pragma unroll
      for (int h = 0; h < kH; h++) acc[h] += w[e * kH + h];
    pin_vgprs(acc);
#pragma unroll
    for (int i = 0; i < kE * kH; i++) qc[i] = qn[i];
  }
#pragma unroll
  for (int h = 0; h < kH; h++) sc[h] = (float)acc[h] * scale;
}

template <int kD, int kH>
__device__ __forceinline__ void qk_finish(const float (&sc)[kH], bool valid, int h0, int r, int g, int t,
                                          int c, const StepDims &d, float *scores, float *chunk_max,
                                          float (*wmax)[8], uint32_t *row_err) {
  constexpr int kT = 256;
  bool bad = false;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (valid) {
    float *dst = scores + (((size_t)r * d.NKV + g) * d.kv_cap + t) * 8 + h0;
    if constexpr (kH == 4) {
      if (h0 % 4 == 0) {
        *reinterpret_cast<float4 *>(dst) = make_float4(sc[0], sc[1], sc[2], sc[3]);
      } else {
#pragma unroll
        for (int h = 0; h < kH; h++) dst[h] = sc[h];
      }
    } else {
#pragma unroll
      for (int h = 0; h < kH; h++) dst[h] = sc[h];
    }
    // head slots past the group (G < 8) read as zero
    if (h0 + kH == d.G) {
      for (int hh = d.G; hh < 8; hh++) dst[hh - h0] = 0.0f;
    }
#pragma unroll
    for (int h = 0; h < kH; h++) bad |= !finitef(sc[h]);
  }
#pragma unroll
  for (int h = 0; h < kH; h++) {
    const float m = wave_max_f32(valid ? sc[h] : -__builtin_inff());
    if (lane == 0) wmax[wave][h] = m;
  }
  __syncthreads();
  const int nsc = (d.kv_cap + kT - 1) / kT;
  if (threadIdx.x < kH) {
    float m = wmax[0][threadIdx.x];
#pragma unroll
    for (int w = 1; w < 4; w++) m = fmaxf(m, wmax[w][threadIdx.x]);
    chunk_max[((size_t)r * d.NH + g * d.G + h0 + threadIdx.x) * nsc + c] = m;
  }
  if (bad) atomicOr(&row_err[r], kErrNonFinite);
}

// Item (row, KV head, chunk) of a scores-pass workgroup, from its linear id in
// dispatch order.  Items run KV head fastest, then row, then chunk, so the two
// KV heads' halves of each page are requested together; with kS = 2 head
// parts per item, the parts of one item take ids 8 apart within each block of
// 16, which the dispatcher's round robin over the 8 XCDs places on the same
// XCD one round apart (ids past the last full block of 16 pair up adjacently).
// Measured at 128 decode rows over the default 256 steps: 27.7 -> 26.7 us per
// launch against row-fastest items with the parts a whole grid plane apart;
// the part pairing alone, or KV head fastest with adjacent parts, was slower.
template <int kS>
__device__ __forceinline__ void attn_item(int &row_x, int &g, int &crev, int &part) {
  static_assert(kS == 1 || kS == 2, "one or two head parts");
  const unsigned X = gridDim.x, Y = gridDim.y;
  const unsigned L = blockIdx.x + X * (blockIdx.y + Y * blockIdx.z);
  unsigned q = L;
  part = 0;
  if constexpr (kS == 2) {
    const unsigned full = (X * Y * gridDim.z) & ~15u;
    if (L < full) {
      q = (L / 16) * 8 + L % 8;
      part = (int)((L / 8) % 2);
    } else {
      q = full / 2 + (L - full) / 2;
      part = (int)((L - full) % 2);
    }
  }
  g = (int)(q % Y);
  row_x = (int)((q / Y) % X);
  crev = (int)(q / (X * Y));
}

// Item of a 1-D pass grid over the work list: the same pairing of head parts
// (ids 8 apart in each block of 16) over the grid's linear ids.
template <int kS>
__device__ __forceinline__ void list_item(int &q, int &part) {
  const unsigned L = blockIdx.x, total = gridDim.x;
  q = (int)L;
  part = 0;
  if constexpr (kS == 2) {
    const unsigned full = total & ~15u;
    if (L < full) {
      q = (int)((L / 16) * 8 + L % 8);
      part = (int)((L / 8) % 2);
    } else {
      q = (int)(full / 2 + (L - full) / 2);
      part = (int)((L - full) % 2);
    }
  }
}

template <int kD, int kG, int kS>
__global__ __launch_bounds__(256) void k_attn_scores(StepDims d, const float *__restrict__ q_rot,
                                                     const float *__restrict__ kpool,
                                                     const uint32_t *__restrict__ row_pos,
                                                     const uint32_t *__restrict__ row_seq,
                                                     const int32_t *__restrict__ pt, float *__restrict__ scores,
                                                     float *__restrict__ chunk_max, uint32_t *row_err) {
  constexpr int kT = 256;
  constexpr int kH = (kG + kS - 1) / kS;                               // heads of every part but the last
  constexpr int kHL = kG - (kS - 1) * kH > 0 ? kG - (kS - 1) * kH : 1;  // heads of the last part
  constexpr int kE = kD == 64 ? (kH > 4 ? 4 : 2) : 1;                  // elements per group (VGPR budget)
  int x, g, c, part;
  if (d.att_items) {
    // list entry i = q / NKV (the grid never exceeds the list's room); KV
    // head fastest, as below
    int q;
    list_item<kS>(q, part);
    g = q % d.NKV;
    const int i = q / d.NKV;
    const uint32_t n = d.att_items[0], e = d.att_items[1 + i];
    if ((uint32_t)i >= n) return;
    x = (int)(e & 0xffffu);
    c = (int)(e >> 16);
  } else {
    int crev;
    attn_item<kS>(x, g, crev, part);
    // chunks in reverse launch order: the high chunks only the longest rows
    // have are dispatched first, the dense low chunks fill in behind them
    c = (int)(gridDim.z / kS) - 1 - crev;
  }
  const int r = d.row_map ? (int)d.row_map[x] : x;
  const int kv = (int)row_pos[r] + 1;
  const int t0 = c * kT;
  if (t0 >= kv) return;
  __shared__ float wmax[4][8];
  const int t = t0 + threadIdx.x;
  const bool valid = t < kv;
  float4 k4[kD / 4];
  if (valid) {
    // the wave's four page entries (wave-uniform loads; entries past the table clamp to its last)
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int32_t *prow = pt + (size_t)row_seq[r] * d.max_pages;
    const int pb = t0 / kPage + 4 * wv, last = d.max_pages - 1;
    const int32_t p0 = prow[min(pb, last)], p1 = prow[min(pb + 1, last)], p2 = prow[min(pb + 2, last)],
                  p3 = prow[min(pb + 3, last)];
    const int li = (threadIdx.x % kWave) / kPage;
    const int32_t phys = li == 0 ? p0 : li == 1 ? p1 : li == 2 ? p2 : p3;
    const uint32_t rot = k_rot((uint32_t)t / kPage, g, d.NKV, kD);
    const float *kq = kpool + (size_t)(phys * d.NKV + g) * (kPage * kD) + (t % kPage) * 4;
#pragma unroll
    for (int j = 0; j < kD / 4; j++)
      k4[j] = *reinterpret_cast<const float4 *>(kq + ((j + rot) % (kD / 4)) * (kPage * 4));
  } else {
#pragma unroll
    for (int j = 0; j < kD / 4; j++) k4[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int h0 = part * kH;
  const float *qbase = q_rot + (size_t)r * d.H + (size_t)(g * kG + h0) * kD;
  if (kHL == kH || part < kS - 1) {
    float sc[kH];
    qk_heads<kD, kH, kE>(k4, qbase, sc, d.scale);
    qk_finish<kD, kH>(sc, valid, h0, r, g, t, c, d, scores, chunk_max, wmax, row_err);
  } else if constexpr (kHL != kH) {
    float sc[kHL];
    qk_heads<kD, kHL, kE>(k4, qbase, sc, d.scale);
    qk_finish<kD, kHL>(sc, valid, h0, r, g, t, c, d, scores, chunk_max, wmax, row_err);
  }
}

// Pass 2 (exponentials), one block per (row, KV head, 256-token chunk); a
// thread owns one head slot (tid % 8) of tokens tid/8 + 32k, k < 8, so the
// scores are read as consecutive floats.  M = max over the row's chunk
// maxima (chunk 0's block stores it in row_max[row][head]); the chunk's f64
// sum of e = f32(exp(s - M)) per head (token order within a thread, then a
// fixed tree) goes to den_part[row][head][chunk].  The exponentials are not
// stored: the value pass forms the same e from s and M.
template <int kG>
__global__ __launch_bounds__(256) void k_attn_exp(StepDims d, const uint32_t *__restrict__ row_pos,
                                                  const float *__restrict__ scores,
                                                  const float *__restrict__ chunk_max,
                                                  double *__restrict__ den_part,
                                                  float *__restrict__ row_max) {
  constexpr int kT = 256, kW = kT / kWave, kK = kT / 32;
  __shared__ float redf[kW][8];
  __shared__ double redd[kW][8];
  __shared__ uint64_t s_tab[32];  // expf's table, read per lane below
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  int x = (int)blockIdx.x, g = (int)blockIdx.y, c = (int)blockIdx.z;
  if (d.att_items) {  // 1-D grid over the work list, KV head fastest
    g = (int)(blockIdx.x % (unsigned)d.NKV);
    const int i = (int)(blockIdx.x / (unsigned)d.NKV);
    const uint32_t n = d.att_items[0], e = d.att_items[1 + i];
    if ((uint32_t)i >= n) return;
    x = (int)(e & 0xffffu);
    c = (int)(e >> 16);
  }
  const int r = d.row_map ? (int)d.row_map[x] : x;
  const int kv = (int)row_pos[r] + 1, t0 = c * kT;
  if (t0 >= kv) return;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int slot = threadIdx.x % 8, tok = threadIdx.x / 8;
  const int nch = (kv + kT - 1) / kT, nsc = (d.kv_cap + kT - 1) / kT;
  const bool live = slot < kG;
  const float *base = scores + (((size_t)r * d.NKV + g) * d.kv_cap + t0) * 8 + threadIdx.x;
  float sv[kK];
#pragma unroll
  for (int k = 0; k < kK; k++) {
    const int t = t0 + tok + 32 * k;
    sv[k] = (t < kv && live) ? base[k * kT] : 0.0f;
  }
  float m = -__builtin_inff();
  if (live) {
    const float *cm = chunk_max + ((size_t)r * d.NH + g * kG + slot) * nsc;
    for (int i = tok; i < nch; i += 32) m = fmaxf(m, cm[i]);
  }
  m = fmaxf(m, __shfl_xor(m, 8, kWave));
  m = fmaxf(m, __shfl_xor(m, 16, kWave));
  m = fmaxf(m, __shfl_xor(m, 32, kWave));
  if (lane < 8) redf[w][lane] = m;
  __syncthreads();
  m = fmaxf(fmaxf(redf[0][slot], redf[1][slot]), fmaxf(redf[2][slot], redf[3][slot]));
  if (c == 0 && threadIdx.x < kG) row_max[(size_t)r * d.NH + g * kG + threadIdx.x] = m;
  double den = 0.0;
#pragma unroll
  for (int k = 0; k < kK; k++) {
    const int t = t0 + tok + 32 * k;
    if (t < kv && live) den += (double)exp_f32_tab(sv[k] - m, s_tab);
  }
  den += __shfl_xor(den, 8, kWave);
  den += __shfl_xor(den, 16, kWave);
  den += __shfl_xor(den, 32, kWave);
  if (lane < 8) redd[w][lane] = den;
  __syncthreads();
  if (threadIdx.x < kG) {
    const double total = ((redd[0][threadIdx.x] + redd[1][threadIdx.x]) + redd[2][threadIdx.x]) +
                         redd[3][threadIdx.x];
    den_part[((size_t)r * d.NH + g * kG + threadIdx.x) * nsc + c] = total;
  }
}

// Pass 3 (values).  Prologue: den = the row's chunk partials summed in a
// fixed order (lane-strided, then butterfly), inv = f32(1/den), e =
// f32(exp(s - M)) again from the scores and the row maximum (the exponent
// pass's bits), and the block's 128 tokens of weights p = e * inv
// (cpu.rs:196-201) staged in LDS.
// Then wave w takes pages 2w and 2w+1 of the block's 128 tokens (16 tokens
// each), lane = element j: acc[h] += f64(p_t[h] * v_t[j]) in token order; the
// 4 waves' sums are combined in a fixed order into the chunk's f64 partial.
// Every global load the block needs (denominator partials, exponentials and
// the wave's 32 V rows) is issued before the first wait, so the prologue and
// the V stream share one memory latency.
template <int kD, int kG>
__global__ __launch_bounds__(256) void k_attn_pv(StepDims d, const float *__restrict__ vpool,
                                                 const uint32_t *__restrict__ row_pos,
                                                 const uint32_t *__restrict__ row_seq,
                                                 const int32_t *__restrict__ pt,
                                                 const float *__restrict__ scores,
                                                 const double *__restrict__ den_part,
                                                 const float *__restrict__ row_max,
                                                 double *__restrict__ partial) {
  constexpr int kE = (kD + kWave - 1) / kWave;  // elements per lane (lanes >= kD idle when kD < 64)
  static_assert(kChunk * 2 == 256, "one float4 of weights per thread");
  static_assert(kG <= 8, "a wave sums the denominators of at most two heads");
  // high chunks first, as in the scores pass; with the full grid rows run
  // fastest (the scores pass's KV-head-fastest order measured 25.3 -> 25.9 us
  // per launch at 128 decode rows over the default 256 steps); over the work
  // list, KV head fastest, then the upper and lower half of each 256-key chunk
  int x = (int)blockIdx.x, g = (int)blockIdx.y, c = (int)gridDim.z - 1 - (int)blockIdx.z;
  if (d.att_items) {
    g = (int)(blockIdx.x % (unsigned)d.NKV);
    const int j = (int)(blockIdx.x / (unsigned)d.NKV), i = j / 2;
    const uint32_t n = d.att_items[0], e = d.att_items[1 + i];
    if ((uint32_t)i >= n) return;
    x = (int)(e & 0xffffu);
    c = 2 * (int)(e >> 16) + 1 - j % 2;
  }
  const int r = d.row_map ? (int)d.row_map[x] : x;
  const int kv = (int)row_pos[r] + 1, t0 = c * kChunk;
  if (t0 >= kv) return;
  __shared__ double red[3][kG][kD];
  __shared__ float s_inv[8];
  __shared__ float4 s_p[kChunk * 2];
  __shared__ uint64_t s_tab[32];  // expf's table, read per lane below
  if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nch = (kv + 255) / 256, nsc = (d.kv_cap + 255) / 256;
  // (1) denominator partials of heads `wave` and `wave + 4`: the first 64
  // chunks now, any further ones in the loop below
  double dsum[2] = {0.0, 0.0};
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int hh = wave + 4 * i;
    if (hh < kG && lane < nch) dsum[i] = den_part[((size_t)r * d.NH + g * kG + hh) * nsc + lane];
  }
  // (2) this thread's 4 scores and their heads' row maxima
  const int et = t0 + threadIdx.x / 2, ehalf = threadIdx.x % 2;
  float4 e = make_float4(0.f, 0.f, 0.f, 0.f);
  if (et < kv)
    e = reinterpret_cast<const float4 *>(scores + (((size_t)r * d.NKV + g) * d.kv_cap + et) * 8)[ehalf];
  float mx[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int hh = ehalf * 4 + i;
    mx[i] = hh < kG ? row_max[(size_t)r * d.NH + g * kG + hh] : 0.0f;
  }
  // (3) the wave's two pages of V, zero past the sequence's end.  Addresses
  // are clamped into the last valid page so the loads need no branch.
  const int32_t *ptr = pt + (size_t)row_seq[r] * d.max_pages;
  float vr[2][kPage][kE];
#pragma unroll
  for (int pg = 0; pg < 2; pg++) {
    const int tp = t0 + (wave * 2 + pg) * kPage;  // first token of the page
    const int n = min(kPage, kv - tp);             // <= 0 when the page is past the end
    const float *vbase = vpool + (size_t)(ptr[min(tp, kv - 1) / kPage] * d.NKV + g) * kPage * kD;
#pragma unroll
    for (int i = 0; i < kPage; i++)
#pragma unroll
      for (int el = 0; el < kE; el++) {
        const int j = min(lane + el * kWave, kD - 1);
        const float x = vbase[max(min(i, n - 1), 0) * kD + j];
        vr[pg][i][el] = (i < n && lane + el * kWave < kD) ? x : 0.0f;
      }
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int hh = wave + 4 * i;
    if (hh < kG) {
      const double *dp = den_part + ((size_t)r * d.NH + g * kG + hh) * nsc;
      double v = dsum[i];
      for (int j = lane + kWave; j < nch; j += kWave) v += dp[j];
      v = wave_sum_f64(v);
      if (lane == 0) s_inv[hh] = (float)(1.0 / v);
    }
  }
  __syncthreads();
  {
    // tokens past the end keep p = 0 (their products must be +-0)
    const int b = ehalf * 4;
    const bool live = et < kv;
    e.x = live && b + 0 < kG ? exp_f32_tab(e.x - mx[0], s_tab) * s_inv[b + 0] : 0.0f;
    e.y = live && b + 1 < kG ? exp_f32_tab(e.y - mx[1], s_tab) * s_inv[b + 1] : 0.0f;
    e.z = live && b + 2 < kG ? exp_f32_tab(e.z - mx[2], s_tab) * s_inv[b + 2] : 0.0f;
    e.w = live && b + 3 < kG ? exp_f32_tab(e.w - mx[3], s_tab) * s_inv[b + 3] : 0.0f;
    s_p[threadIdx.x] = e;
  }
  __syncthreads();
  // Tokens past the end carry p = 0 and v = 0: their products are +-0, and
  // adding +-0 leaves the accumulator unchanged (it starts at +0 and a sum
  // that cancels rounds to +0, so it is never -0).  Both pages therefore run
  // in full, without branches.
  const float *pl = reinterpret_cast<const float *>(s_p);
  double acc[kG][kE];
#pragma unroll
  for (int hh = 0; hh < kG; hh++)
#pragma unroll
    for (int el = 0; el < kE; el++) acc[hh][el] = 0.0;
#pragma unroll
  for (int pg = 0; pg < 2; pg++) {
    const float *pbase = pl + (wave * 2 + pg) * kPage * 8;
#pragma unroll
    for (int i = 0; i < kPage; i++)
#pragma unroll
      for (int hh = 0; hh < kG; hh++) {
        const float ph = pbase[i * 8 + hh];
#pragma unroll
        for (int el = 0; el < kE; el++) acc[hh][el] += (double)(ph * vr[pg][i][el]);
      }
  }
  if (wave > 0) {
#pragma unroll
    for (int hh = 0; hh < kG; hh++)
#pragma unroll
      for (int e = 0; e < kE; e++)
        if (lane + e * kWave < kD) red[wave - 1][hh][lane + e * kWave] = acc[hh][e];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int hh = 0; hh < kG; hh++)
#pragma unroll
      for (int e = 0; e < kE; e++) {
        const int j = lane + e * kWave;
        if (j >= kD) continue;
        double sum = acc[hh][e];
#pragma unroll
        for (int w = 0; w < 3; w++) sum += red[w][hh][j];
        partial[(((size_t)r * d.NH + g * kG + hh) * d.max_chunks + c) * kD + j] = sum;
      }
  }
}

// ---------------------------------------------------------------------------
// Prefill chunks on the matrix cores (tolerance regime, used only with the
// matrix-core linears).  A workgroup takes up to 16 consecutive rows of one
// lane and one KV head; wave w is query head g*kG + w.  Key tiles of 64
// tokens enter in binary16: K as a hi/lo pair (k = hi + lo to about 2^-22
// relative), V rounded once; Q and P are rounded to binary16 (2^-12
// relative, the rounding the regime's linears already give their operands).
// S = (K_lo + K_hi) Q^T takes two v_mfma_f32_16x16x32_f16, O = V P one, all
// with f32 sums.  (A bfloat16 hi/lo split of every operand, three MFMAs per
// product, ran 2.46 against 1.83 ms/step at C3; with V split too, 2.22.)
//   S^T = K Q^T: lane (grp, c) ends up holding S[row c][key 16n + 4grp + i]
//     for n, i in 0..3, so one lane owns one query row: the row max and sum
//     need two cross-lane steps, and P never leaves registers.
//   O^T = V^T P^T: the lane's 16 probabilities are exactly its B operand when
//     the k-slots of each 32-key step are ordered 16*(j/4) + 4grp + j%4;
//     V^T is staged in that key order, so each A operand is one 16-byte read.
// Key tiles are converted once per layer and step (k_attn_stage) into the
// exact LDS image the chunk kernel multiplies from, which it copies with
// direct-to-LDS loads, one tile ahead; every row tile of a lane shares them.
// (Converting each tile from f32 in every workgroup cost about 0.45 of the
// kernel's 1.77 ms/step at C3.)
// Scores are taken in log2 units (Q pre-scaled by scale*log2(e)) and
// exponentiated with v_exp_f32; rows are normalized once at the end.  The
// reference computes the same attention with f64 dot products and sums
// (cpu.rs:133-210); rows handled here are flagged in row_skip so the exact
// passes leave them.  Tiles arrive sorted by KV length, longest first.
// ---------------------------------------------------------------------------
// 16 bytes per lane straight from global memory into LDS: lane l's bytes
// land at l * 16 past `lds` (the same for the whole wave).  Completion counts
// in vmcnt.
__device__ __forceinline__ void lds_load16(const void *global, void *lds) {
  __builtin_amdgcn_global_load_lds(global, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}
typedef float float4v __attribute__((ext_vector_type(4)));

// Segment record of a chunk row: in the row's own partial-sum space (the
// exact passes skip chunk rows), kChunkSegFloats floats per key segment.
__device__ __forceinline__ float *chunk_seg_at(double *partial, const StepDims &d, int row, int head, int seg) {
  return reinterpret_cast<float *>(partial + ((size_t)row * d.NH + head) * d.max_chunks * d.D) +
         seg * kChunkSegFloats;
}

typedef _Float16 f16x8c __attribute__((ext_vector_type(8)));

namespace chunk {
constexpr int kD = 64, kKT = 64;  // head dim, keys per tile
// A tile image: three blocks of 64 rows x 8 units of 16 bytes (K hi rows,
// K lo rows, V^T rows), unit u of row R stored at R * 8 + (u ^ swz(R)).  An
// MFMA operand read gives each eight lanes that one pass of a 16-byte LDS
// access serves the rows R..R+7 of one unit; swz(R) = R & 7 puts them at
// eight distinct positions modulo 128 bytes, which is free of bank conflicts.
constexpr int kRowUnits = 8, kBlock = kKT * kRowUnits;
static_assert(kChunkImgUnits == 3 * kBlock, "K hi, K lo and V^T blocks");
static_assert(kChunkTileKeys == kKT && kChunkSegKeys % kKT == 0, "segments of whole key tiles");
__device__ __forceinline__ int swz(int R) { return R & 7; }
__device__ __forceinline__ int unit_at(int R, int u) { return R * kRowUnits + (u ^ swz(R)); }

__device__ __forceinline__ void split(float x, _Float16 &hi, _Float16 &lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// Key of k-slot s (0..63 within a tile) in the V^T rows: the k-slot order
// of the P operand (see above): slot 32ks + 8grp + 4h + j holds key
// 32ks + 16h + 4grp + j.
__device__ __forceinline__ int vkey(int s) {
  const int ks = s / 32, r = s % 32, grp = r / 8, h = (r % 8) / 4, j = r % 4;
  return ks * 32 + h * 16 + grp * 4 + j;
}
}  // namespace chunk

// One tile image per workgroup: item = {sequence, end of the lane's keys,
// first key of the tile, KV head}; keys at or past the end are zero.
// Thread t converts K row t / 4, dims 16 (t % 4) .. + 15, and then V^T row
// (dim) t / 4, k-slots 16 (t % 4) .. + 15 from the tile's V staged in LDS.
__global__ __launch_bounds__(256) void k_attn_stage(StepDims d, const int4 *__restrict__ items,
                                                    const float *__restrict__ kpool,
                                                    const float *__restrict__ vpool,
                                                    const int32_t *__restrict__ pt, uint4 *__restrict__ img) {
  using namespace chunk;
  __shared__ float s_vr[kKT][kD + 1];  // the tile's V rows, f32
  const int4 it = items[blockIdx.x];
  const int tid = threadIdx.x, k = tid >> 2, q = tid & 3, t = it.z + k, g = it.w;
  float kx[16], vx[16];
  if (t < it.y) {
    const int32_t phys = pt[(size_t)it.x * d.max_pages + t / kPage];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 a = *reinterpret_cast<const float4 *>(
          kpool + k_at(phys, (uint32_t)(t / kPage), g, d.NKV, t % kPage, 16 * q + 4 * j, kD));
      const float4 b = *reinterpret_cast<const float4 *>(vpool + v_at(phys, g, d.NKV, t % kPage, 16 * q + 4 * j, kD));
      kx[4 * j] = a.x, kx[4 * j + 1] = a.y, kx[4 * j + 2] = a.z, kx[4 * j + 3] = a.w;
      vx[4 * j] = b.x, vx[4 * j + 1] = b.y, vx[4 * j + 2] = b.z, vx[4 * j + 3] = b.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) kx[j] = vx[j] = 0.0f;
  }
  uint4 *out = img + (size_t)blockIdx.x * kChunkImgUnits;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    f16x8c hi, lo;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      _Float16 a, b;
      split(kx[8 * h + e], a, b);
      hi[e] = a;
      lo[e] = b;
    }
    const int at = unit_at(k, 2 * q + h);
    out[at] = __builtin_bit_cast(uint4, hi);
    out[kBlock + at] = __builtin_bit_cast(uint4, lo);
  }
#pragma unroll
  for (int j = 0; j < 16; j++) s_vr[k][16 * q + j] = vx[j];
  __syncthreads();
  const int dim = k;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int u = 2 * q + h;
    f16x8c v;
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (_Float16)s_vr[vkey(8 * u + e)][dim];
    out[2 * kBlock + unit_at(dim, u)] = __builtin_bit_cast(uint4, v);
  }
}

template <int kG>
__global__ __launch_bounds__(64 * kG) void k_attn_chunk(StepDims d, const int4 *__restrict__ tiles,
                                                        const float *__restrict__ q_rot,
                                                        const uint4 *__restrict__ img,
                                                        double *__restrict__ partial) {
  using namespace chunk;
  constexpr int kThreads = 64 * kG;
  using E = _Float16;
  using E8 = f16x8c;
  auto mfma = [](E8 a, E8 b, float4v c) __attribute__((always_inline)) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  };
  __shared__ __align__(16) uint4 s_img[2][kChunkImgUnits];  // two tile images, one in flight
  // first row, rows | segment << 8, the lane's first tile image, position of first row
  const int4 tile = tiles[blockIdx.x / d.NKV];
  const int g = blockIdx.x % d.NKV, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int h = g * kG + wave, grp = lane / 16, c = lane % 16;
  const int nr = tile.y & 0xff, seg = tile.y >> 8, pos0 = tile.w, kv_end = pos0 + nr;
  const int t_begin = seg * kChunkSegKeys, t_end = min(t_begin + kChunkSegKeys, kv_end);
  const int prow = pos0 + min(c, nr - 1);  // rows past the tile repeat its last row
  // B operand of S^T: Q[row c][dims 32ks + 8grp .. +7] in log2 units
  E8 qh[2];
  {
    const float qs = d.scale * 1.4426950408889634f;
    const float *qrow = q_rot + (size_t)(tile.x + min(c, nr - 1)) * d.H + h * kD;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const float4 a = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * grp);
      const float4 b = *reinterpret_cast<const float4 *>(qrow + 32 * ks + 8 * grp + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; j++) qh[ks][j] = (E)(v[j] * qs);
    }
  }
  float4v o[4];
#pragma unroll
  for (int n = 0; n < 4; n++) o[n] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.0f;
  // image of key tile t0 / 64 into stage st: wave w copies 16-byte units
  // 64u + lane for u = w, w + kG, ...
  auto fetch = [&](int t0, int st) {
    const uint4 *src = img + ((size_t)tile.z + (size_t)(t0 / kKT) * d.NKV + g) * kChunkImgUnits;
    for (int u = wave; u < kChunkImgUnits / kWave; u += kG)
      lds_load16(src + u * kWave + lane, &s_img[st][u * kWave]);
  };
  fetch(t_begin, 0);
  for (int t0 = t_begin, st = 0; t0 < t_end; t0 += kKT, st ^= 1) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's units of the tile have landed
    __syncthreads();                     // every wave's units; every wave is done with the other stage
    if (t0 + kKT < t_end) fetch(t0 + kKT, st ^ 1);  // the next image lands while this one is multiplied
    const E8 *kh = reinterpret_cast<const E8 *>(s_img[st]);
    const E8 *kl = kh + kBlock, *vt = kh + 2 * kBlock;
    // S^T tile: s[n][i] = S[row c][key t0 + 16n + 4grp + i]
    float4v s[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      s[n] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const int at = unit_at(16 * n + c, 4 * ks + grp);
        s[n] = mfma(kl[at], qh[ks], s[n]);
        s[n] = mfma(kh[at], qh[ks], s[n]);
      }
    }
    if (t0 + kKT - 1 > pos0 || t0 + kKT > t_end) {  // causal mask key <= row; keys past the segment
#pragma unroll
      for (int n = 0; n < 4; n++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = t0 + 16 * n + 4 * grp + i;
          if (t > prow || t >= t_end) s[n][i] = -__builtin_inff();
        }
    }
    float mx = m;
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[n][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    // a row whose keys so far are all masked (a segment past its position)
    // keeps m = -inf and p = 0
    const float mref = mx == -__builtin_inff() ? 0.0f : mx;
    const float alpha = __builtin_amdgcn_exp2f(m - mref);  // 0 on the first live tile
    m = mx;
    // B operand of O^T: P[row c][k-slot j of step ks] (the f32 sum keeps
    // the unrounded p)
    E8 ph[2];
    float sum = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float p = __builtin_amdgcn_exp2f(s[2 * ks + j / 4][j % 4] - mref);
        sum += p;
        ph[ks][j] = (E)p;
      }
    l = l * alpha + sum;  // this lane's share of the row sum
#pragma unroll
    for (int n = 0; n < 4; n++) o[n] *= alpha;
    // O^T tile: o[n][i] += sum_k V[k][dim 16n + 4grp + i] P[row c][k]
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int ks = 0; ks < 2; ks++) o[n] = mfma(vt[unit_at(16 * n + c, 4 * ks + grp)], ph[ks], o[n]);
  }
  l += __shfl_xor(l, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  if (c >= nr) return;
  // the segment's (m, l, o) of row c, head h (log2 units, o unnormalized)
  float *out = chunk_seg_at(partial, d, tile.x + c, h, seg);
  if (grp == 0) {
    out[0] = m;
    out[1] = l;
  }
#pragma unroll
  for (int n = 0; n < 4; n++)
    *reinterpret_cast<float4 *>(out + 2 + 16 * n + 4 * grp) = make_float4(o[n][0], o[n][1], o[n][2], o[n][3]);
}

// Pass 4: chunks combined in order, rounded to f32, and prepared as the
// operand of attn_output (each head's D elements hold whole Q8_0 blocks).
template <int kAct>
__global__ __launch_bounds__(128) void k_attn_combine(StepDims d,
                                                      const uint32_t *__restrict__ row_pos,
                                                      const double *__restrict__ partial, int nbp,
                                                      ActView act, uint32_t *row_err) {
  __shared__ float o_s[128];
  const int r = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const int kv = (int)row_pos[r] + 1, nch = (kv + kChunk - 1) / kChunk;
  const double *pp = partial + ((size_t)r * d.NH + h) * d.max_chunks * d.D;
  const bool active = j < d.D;
  double acc = 0.0;
  const bool direct = d.row_skip && d.row_skip[r];
  if (active && !direct) {
    // chunk partials summed in chunk order; each batch of up to 16 is
    // requested at once (clamped into range, past-the-end values unused)
    constexpr int kB = 16;
    for (int c0 = 0; c0 < nch; c0 += kB) {
      double v[kB];
#pragma unroll
      for (int i = 0; i < kB; i++) v[i] = pp[(size_t)min(c0 + i, nch - 1) * d.D + j];
#pragma unroll
      for (int i = 0; i < kB; i++)
        if (c0 + i < nch) acc = (c0 + i == 0) ? v[i] : acc + v[i];
    }
  }
  float o = (float)acc;
  if (direct && active) {
    // the chunk kernel's key segments merged in order: M = max m_s,
    // o = sum 2^(m_s - M) o_s / sum 2^(m_s - M) l_s (log2 units)
    // (batches of 8 segments requested at once, clamped into range)
    const float *sg = chunk_seg_at(const_cast<double *>(partial), d, r, h, 0);
    const int nseg = (kv + kChunkSegKeys - 1) / kChunkSegKeys;
    constexpr int kB = 8;
    float M = -__builtin_inff(), L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < nseg; s0 += kB) {
      float mv[kB], lv[kB], ov[kB];
#pragma unroll
      for (int i = 0; i < kB; i++) {
        const float *rec = sg + min(s0 + i, nseg - 1) * kChunkSegFloats;
        mv[i] = rec[0];
        lv[i] = rec[1];
        ov[i] = rec[2 + j];
      }
      float Mb = M;
#pragma unroll
      for (int i = 0; i < kB; i++)
        if (s0 + i < nseg) Mb = fmaxf(Mb, mv[i]);
      const float rescale = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(M - Mb);
      L *= rescale;
      O *= rescale;
#pragma unroll
      for (int i = 0; i < kB; i++) {
        if (s0 + i < nseg) {
          const float a = mv[i] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mv[i] - Mb);
          L += a * lv[i];
          O += a * ov[i];
        }
      }
      M = Mb;
    }
    o = O / L;
  }
  bool bad = active && !finitef(o);
  if (kAct == 8 || kAct == kActQ8H) {
    if (active) o_s[j] = o;
    __syncthreads();
    // D/8 groups of this head: group kg of the row is h*D/8 + j
    const int ng = d.D / 8;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = j < ng ? o_s[j * 8 + i] : 0.0f;
    if (j < ((ng + 3) & ~3))
      bad |= quant_group_q8<1, kAct == kActQ8H>(v, j < ng, r, h * ng + j, nbp, act);
  } else if (kAct == kActF32) {  // f32 rows for a following Q8_K quantizer
    if (active) act.f32[(size_t)r * d.H + h * d.D + j] = o;
  } else if (active) {
    const uint16_t hv = f2h(o);
    bad |= !finitef(h2f(hv));
    act.f16[(size_t)r * d.H + h * d.D + j] = hv;
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
                                 const int32_t *__restrict__ pages, int from, int rows, int NKV,
                                 int D, uint64_t seed, uint32_t stream) {
  const int layer = blockIdx.y;
  const size_t total = (size_t)(rows - from) * NKV * D;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int pos = from + (int)(idx / ((size_t)NKV * D));
    const int e = (int)(idx % ((size_t)NKV * D));
    const int g = e / D, j = e % D;
    const size_t base = (size_t)layer * layer_stride;
    kpool[base + k_at(pages[pos / kPage], pos / kPage, g, NKV, pos % kPage, j, D)] = synthetic_kv(seed, stream, layer, 0, pos, e);
    vpool[base + v_at(pages[pos / kPage], g, NKV, pos % kPage, j, D)] = synthetic_kv(seed, stream, layer, 1, pos, e);
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
                 uint32_t *lane_last, uint32_t *row_err, unsigned long long *keys, int n_keys) {
  launch_k(k_pack, dim3(1), dim3(1024), 0, s, n_lanes, lane_info, tokens, page_table,
                     max_pages, cu, row_pos, row_slot, row_lane, row_token, row_seq, lane_last,
                     row_err, keys, n_keys);
}

void launch_embed(hipStream_t s, int rows, const MatrixView &emb, const uint32_t *row_token,
                  float *x, int H, uint32_t *row_err) {
  launch_k(k_embed, dim3(rows), dim3(256), 0, s, emb, row_token, x, H, row_err);
}

void launch_norm_act(hipStream_t s, int rows, const float *x, const uint32_t *in_rows,
                     const float *weight, int H, float eps, int act_dtype, int nbp, ActView act,
                     uint32_t *row_err) {
  const size_t lds = (size_t)H * sizeof(float);
  if (act_dtype == 8 && nbp * 4 <= 256 && H % 8 == 0)  // one 8-element group per thread
    launch_k(k_norm_q8<false>, dim3(rows), dim3(256), 0, s, x, in_rows, weight, H, eps, nbp, act, row_err);
  else if (act_dtype == kActQ8H && nbp * 4 <= 256 && H % 8 == 0)
    launch_k(k_norm_q8<true>, dim3(rows), dim3(256), 0, s, x, in_rows, weight, H, eps, nbp, act, row_err);
  else if (act_dtype == kActQ8H)
    launch_k(k_norm_act<kActQ8H>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
  else if (act_dtype == kActQ8K)  // nbp = H / 256 blocks
    launch_k(k_norm_act<kActQ8K>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
  else if (act_dtype == 8)
    launch_k(k_norm_act<8>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
  else
    launch_k(k_norm_act<1>, dim3(rows), dim3(256), lds, s, x, in_rows, weight, H, eps,
                       nbp, act, row_err);
}

void launch_quant_act(hipStream_t s, int rows, const float *src, int K, int act_dtype, int nbp,
                      ActView act, uint32_t *row_err) {
  if (act_dtype == kActQ8K) {  // nbp = K / 256 blocks, four per workgroup
    launch_k(k_quant_act<kActQ8K>, dim3(rows, (nbp + 3) / 4), dim3(256), 0, s, src, K, nbp, act, row_err);
    return;
  }
  const int splits = (nbp * 4 + 255) / 256;  // 256 groups of 8 values per workgroup
  if (act_dtype == 8)
    launch_k(k_quant_act<8>, dim3(rows, splits), dim3(256), 0, s, src, K, nbp, act, row_err);
  else
    launch_k(k_quant_act<1>, dim3(rows, splits), dim3(256), 0, s, src, K, nbp, act, row_err);
}

template <int kEpi, int kNM, int kFmt>
static bool mv_q8(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                  const MatvecOut &o) {
  const int units = w.mtiles / kNM;
  const int n_tiles = (rows_b + 15) / 16;
  constexpr int kWPairs = 16;  // k_mv_q8w: K <= 1024
  if (kEpi == kEpiSwiglu && w.nbp <= 2 * kWPairs) {
    // gate+up at short K: the unit's weights in LDS, B operands in registers
    const int by = (n_tiles + 7) / 8;
    const int nthreads = 64 * (n_tiles < 8 ? n_tiles : 8);
    const size_t lds = (size_t)kNM * (w.nbp / 2) * (kFmt == 8 ? 1024 : 512) + (size_t)kNM * w.nbp * 32 +
                       (size_t)8 * w.nbp * 32;
    launch_k((k_mv_q8w<kEpi, kNM, kFmt, kWPairs, 1>), dim3(units, by), dim3(nthreads), lds, s, w, act, rows_b,
             n_tiles, o, ActView{}, 0);
  } else if (kEpi == kEpiArgmax && kNM == 1 && n_tiles <= 8 && w.nbp <= 2 * kWPairs && o.argmax_final) {
    // LM head: persistent workgroups streaming weight tiles through LDS, two
    // per CU (4 waves per SIMD); always 8 waves, since the tile copy needs
    // them all (waves past the last batch tile only copy)
    const size_t tile = (size_t)(w.nbp / 2) * (kFmt == 8 ? 1024 : 512) + (size_t)w.nbp * 32;
    const size_t lds = 2 * tile + (size_t)n_tiles * w.nbp * 32;
    // up to 4 batch tiles: workgroups of 4 waves, four per CU (a Q8_0 tile
    // of K <= 896 is at most 952 copy items, four per thread), so that more
    // weight tiles are in flight per CU
    const int nthreads = n_tiles <= 4 && w.nbp <= 28 ? 256 : 512;
    const int max_blocks = nthreads == 256 ? 1024 : 512;
    const int blocks = units < max_blocks ? units : max_blocks;
    if (w.nbp <= 28)  // K <= 896: 14 register pairs of B operand
      launch_k((k_mv_q8h<kFmt, 14>), dim3(blocks), dim3(nthreads), lds, s, w, act, rows_b, n_tiles, o);
    else
      launch_k((k_mv_q8h<kFmt, kWPairs>), dim3(blocks), dim3(nthreads), lds, s, w, act, rows_b, n_tiles, o);
    return true;
  } else if ((kEpi == kEpiArgmax || kEpi == kEpiSwiglu) && w.nbp <= 64) {
    // short K, many weight tiles (the LM head, gate+up beyond k_mv_q8w's K):
    // register chains, 4 waves per workgroup; the head takes 4 batch tiles
    // per wave (each weight pair loaded once feeds 8 MFMAs)
    constexpr int kNN = kEpi == kEpiArgmax ? 4 : 2;
    const int groups = (n_tiles + kNN - 1) / kNN;
    const int waves = groups < kChainWaves ? groups : kChainWaves;
    launch_k((k_mv_q8c<kEpi, kNM, kNN, 4, kFmt>), dim3(units, (groups + kChainWaves - 1) / kChainWaves),
             dim3(64 * waves), 0, s, w, act, rows_b, n_tiles, o);
  } else {
    // chunks of 16 blocks: 18 KB of LDS per workgroup, so several workgroups
    // per CU overlap one's chain with another's loads (128-row down
    // projection 13.3 -> 11.6 us against chunks of 64; qkv and o 0.2 us
    // faster than one chunk of 32)
    const int groups = (units + 7) / 8;
    // few batch tiles: 16 waves, chunks of 32 blocks (half the chunk
    // barriers on the long-K down projection; the grid is small anyway)
    if (kNM == 1 && n_tiles <= 4)
      launch_k((k_mv_q8s<kEpi, kNM, 2, kFmt, 16>), dim3(groups * 8 * n_tiles), dim3(1024), 0, s, w, act,
               rows_b, n_tiles, o, QkvEpi{});
    else
      launch_k((k_mv_q8s<kEpi, kNM, 2, kFmt>), dim3(groups * 8 * n_tiles), dim3(512), 0, s, w, act,
               rows_b, n_tiles, o, QkvEpi{});
  }
  return false;
}

// Packed batches at least this tall take the matrix-core F16 linears.
constexpr int kPrefillRows = 128;

// The packed-prefill regime's F16 GEMM (gemm.h) for one projection; false
// (nothing launched) when K is not a multiple of 64.  Tiles measured on the
// C3 shapes (2,616 packed rows): 128 x 128 on eight waves of 64 features x 32
// rows with four K steps in flight for the plain and residual projections
// (qkv 15.8, o 15.8, down 49.0 us; on four waves of 64 x 64: 16.5, 18.4,
// 55.6), 256 x 128 on eight waves for gate+up with the SwiGLU epilogue (67
// us, which also replaces a separate SwiGLU-to-binary16 pass), 128 x 64 for
// the head's few logit rows.
static bool gemm_f16(hipStream_t s, Epilogue epi, const MatrixView &w, const uint16_t *x, int rows_b,
                     const MatvecOut &o, uint16_t *out16) {
  using namespace gemm;
  if (w.K % 64) return false;
  const bool four = w.K % 128 == 0;  // four K steps of 32 in flight divide K
  Args g{};
  g.w = w.f16;
  g.x = x;
  g.N = w.rows;
  g.K = w.K;
  g.M = rows_b;
  g.ldx = w.K;
  g.row_err = o.row_err;
  g.err_rows = o.err_rows;
  if (epi == kEpiSwiglu) {
    g.out16 = out16;
    const dim3 grid(tile_order(g, w.rows / 2, 128, 128));
    launch_k(k_gemm<kF16, false, 4, 2, 4, 4, 2, kSwigluF16>, grid, dim3(512),
             lds_bytes<4, 2, 4, 4, false, kSwigluF16>(), s, g);
  } else if (epi == kEpiArgmax) {
    g.keys = o.argmax;
    g.ktiles = w.mtiles;
    g.logits = o.logits;
    const dim3 grid(tile_order(g, w.rows, 128, 64));
    constexpr int lds = lds_bytes<2, 2, 4, 2, false, kArgmax>();
    if (four)
      launch_k(k_gemm<kF16, false, 2, 2, 4, 2, 4, kArgmax>, grid, dim3(256), lds, s, g);
    else
      launch_k(k_gemm<kF16, false, 2, 2, 4, 2, 2, kArgmax>, grid, dim3(256), lds, s, g);
  } else {
    g.out = o.out;
    g.ldo = o.ld;
    const dim3 grid(tile_order(g, w.rows, 128, 128));
    constexpr int lds = lds_bytes<2, 4, 4, 2, false, kStore>();
    if (epi == kEpiResidual) {
      if (four)
        launch_k(k_gemm<kF16, false, 2, 4, 4, 2, 4, kAccumulate>, grid, dim3(512), lds, s, g);
      else
        launch_k(k_gemm<kF16, false, 2, 4, 4, 2, 2, kAccumulate>, grid, dim3(512), lds, s, g);
    } else {
      if (four)
        launch_k(k_gemm<kF16, false, 2, 4, 4, 2, 4, kStore>, grid, dim3(512), lds, s, g);
      else
        launch_k(k_gemm<kF16, false, 2, 4, 4, 2, 2, kStore>, grid, dim3(512), lds, s, g);
    }
  }
  return true;
}

bool launch_gemm_q(hipStream_t s, Epilogue epi, const MatrixView &w, const uint16_t *x, int rows_b,
                   const MatvecOut &o, uint16_t *out16, int rope_d, int rope_rows) {
  using namespace gemm;
  if ((w.dtype != kFmtQ8 && w.dtype != kFmtQ4) || w.K % 128 || w.nbp * 32 != w.K) return false;
  if (epi != kEpiStore && epi != kEpiResidual && epi != kEpiSwiglu) return false;
  Args g{};
  g.qs = w.qs;
  g.ds = w.ds;
  g.nbp = w.nbp;
  g.x = x;
  g.N = w.rows;
  g.K = w.K;
  g.M = rows_b;
  g.ldx = w.K;
  g.row_err = o.row_err;
  g.err_rows = o.err_rows;
  const bool q8 = w.dtype == kFmtQ8;
  const double wb = q8 ? 34.0 / 32 : 18.0 / 32;
  // 128 x 128 tiles on eight waves of 64 features x 32 rows, two block pairs
  // in flight: on the C3 shapes (Q8_0) qkv 15.3, o 15.7, down 51.2, gate+up
  // 76.6 us against 17.0, 18.5, 64.8, 83.5 on four waves of 64 x 64
  if (epi == kEpiSwiglu) {
    g.out16 = out16;
    const dim3 grid(tile_order(g, w.rows / 2, 64, 128, wb));
    constexpr int lds = lds_bytes_q<2, 4, 4, 2, kSwigluQ8>();
    if (q8)
      launch_k(k_gemm_q<8, 2, 4, 4, 2, 2, kSwigluQ8>, grid, dim3(512), lds, s, g);
    else
      launch_k(k_gemm_q<4, 2, 4, 4, 2, 2, kSwigluQ8>, grid, dim3(512), lds, s, g);
    return true;
  }
  g.out = o.out;
  g.ldo = o.ld;
  g.rope_d = rope_d;
  g.rope_rows = rope_d ? rope_rows : 0;
  const dim3 grid(tile_order(g, w.rows, 128, 128, wb));
  constexpr int lds = lds_bytes_q<2, 4, 4, 2, kStore>();
  if (epi == kEpiResidual) {
    if (q8)
      launch_k(k_gemm_q<8, 2, 4, 4, 2, 2, kAccumulate>, grid, dim3(512), lds, s, g);
    else
      launch_k(k_gemm_q<4, 2, 4, 4, 2, 2, kAccumulate>, grid, dim3(512), lds, s, g);
  } else {
    if (q8)
      launch_k(k_gemm_q<8, 2, 4, 4, 2, 2, kStore>, grid, dim3(512), lds, s, g);
    else
      launch_k(k_gemm_q<4, 2, 4, 4, 2, 2, kStore>, grid, dim3(512), lds, s, g);
  }
  return true;
}

bool launch_gemm_qkv(hipStream_t s, const MatrixView &w, const uint16_t *x, int rows_b, uint32_t *row_err,
                     const QkvEpi &q) {
  using namespace gemm;
  const bool f16 = w.dtype == kFmtF16, quant = w.dtype == kFmtQ8 || w.dtype == kFmtQ4;
  if (!f16 && !quant) return false;
  if (q.D != 64 || q.H % 64 || q.KVD % 64 || w.rows != q.H + 2 * q.KVD || w.K % 128) return false;
  if (quant && w.nbp * 32 != w.K) return false;
  Args g{};
  g.x = x;
  g.N = w.rows;
  g.K = w.K;
  g.M = rows_b;
  g.ldx = w.K;
  g.row_err = row_err;
  g.qk_bias = q.bias;
  g.qk_rope = q.rope;
  g.qk_pos = q.row_pos;
  g.qk_slot = q.row_slot;
  g.qk_q = q.q_rot;
  g.qk_kpool = q.kpool;
  g.qk_vpool = q.vpool;
  g.qk_H = q.H;
  g.qk_KVD = q.KVD;
  g.qk_NKV = q.NKV;
  if (f16) {  // source row order
    g.w = w.f16;
    const dim3 grid(tile_order(g, w.rows, 128, 128));
    launch_k(k_gemm<kF16, false, 2, 4, 4, 2, 4, kQkvRope>, grid, dim3(512), lds_bytes<2, 4, 4, 2, false, kQkvRope>(),
             s, g);
    return true;
  }
  // the quantized tiles hold the query and key rows in rope order
  g.qs = w.qs;
  g.ds = w.ds;
  g.nbp = w.nbp;
  g.rope_d = q.D;
  g.rope_rows = q.H + q.KVD;
  const dim3 grid(tile_order(g, w.rows, 128, 128, w.dtype == kFmtQ8 ? 34.0 / 32 : 18.0 / 32));
  constexpr int lds = lds_bytes_q<2, 4, 4, 2, kQkvRope>();
  if (w.dtype == kFmtQ8)
    launch_k(k_gemm_q<8, 2, 4, 4, 2, 2, kQkvRope>, grid, dim3(512), lds, s, g);
  else
    launch_k(k_gemm_q<4, 2, 4, 4, 2, 2, kQkvRope>, grid, dim3(512), lds, s, g);
  return true;
}

bool launch_matvec_swiglu_f16(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                              const MatvecOut &o, uint16_t *out_f16) {
  if (!g_prefill_mfma || rows_b < kPrefillRows || w.dtype != kFmtF16) return false;
  return gemm_f16(s, kEpiSwiglu, w, act.f16, rows_b, o, out_f16);
}

template <int kEpi>
static void mv_f16(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                   const MatvecOut &o) {
  const int out_rows = kEpi == kEpiSwiglu ? w.rows / 2 : w.rows;
  // the head of a step in the packed-prefill regime (16+ logit rows): the
  // regime's GEMM with partial keys per 16-row tile
  if (kEpi == kEpiArgmax && g_head_mfma && rows_b >= 16 &&
      gemm_f16(s, kEpiArgmax, w, act.f16, rows_b, o, nullptr))
    return;
  // tall packed batches of a prefill step: matrix cores (f32 sums); gate+up
  // with SwiGLU goes through launch_matvec_swiglu_f16
  if ((kEpi == kEpiStore || kEpi == kEpiResidual) && g_prefill_mfma && rows_b >= kPrefillRows &&
      gemm_f16(s, (Epilogue)kEpi, w, act.f16, rows_b, o, nullptr))
    return;
  if (rows_b >= 16 && w.K % 8 == 0) {  // lane = batch row, sequential f64 chains
    launch_k(k_mv_f16s<kEpi>, dim3((out_rows + 15) / 16, (rows_b + kWave - 1) / kWave), dim3(256), 0,
             s, w, act, rows_b, o);
    return;
  }
  if (kEpi == kEpiArgmax) {  // partial keys per 16-row tile, then k_argmax_reduce
    launch_k(k_head_f16, dim3(w.mtiles), dim3(256), 0, s, w, act, rows_b, o);
    return;
  }
  launch_k(k_mv_f16<kEpi>, dim3((out_rows + 3) / 4), dim3(256), 0, s, w, act, rows_b, o);
}

template <int kEpi, int kNM>
static void mv_kq(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b, const MatvecOut &o) {
  const int units = w.mtiles / kNM, n_tiles = (rows_b + 15) / 16;
  launch_k((k_mv_kq<kEpi, kNM>), dim3((units + 7) / 8 * 8 * n_tiles), dim3(512), 0, s, w, act, rows_b,
           n_tiles, o);
}

bool launch_matvec(hipStream_t s, Epilogue epi, const MatrixView &w, const ActView &act,
                   int rows_b, const MatvecOut &o) {
  if (w.dtype == kFmtKQ) {
    switch (epi) {
      case kEpiStore: mv_kq<kEpiStore, 1>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_kq<kEpiResidual, 1>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_kq<kEpiSwiglu, 2>(s, w, act, rows_b, o); break;
      case kEpiArgmax: mv_kq<kEpiArgmax, 1>(s, w, act, rows_b, o); break;
    }
  } else if (w.dtype == 8) {
    switch (epi) {
      case kEpiStore: mv_q8<kEpiStore, 1, 8>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_q8<kEpiResidual, 1, 8>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_q8<kEpiSwiglu, 2, 8>(s, w, act, rows_b, o); break;
      case kEpiArgmax: return mv_q8<kEpiArgmax, 1, 8>(s, w, act, rows_b, o);
    }
  } else if (w.dtype == 2) {
    switch (epi) {
      case kEpiStore: mv_q8<kEpiStore, 1, 2>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_q8<kEpiResidual, 1, 2>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_q8<kEpiSwiglu, 2, 2>(s, w, act, rows_b, o); break;
      case kEpiArgmax: return mv_q8<kEpiArgmax, 1, 2>(s, w, act, rows_b, o);
    }
  } else {
    switch (epi) {
      case kEpiStore: mv_f16<kEpiStore>(s, w, act, rows_b, o); break;
      case kEpiResidual: mv_f16<kEpiResidual>(s, w, act, rows_b, o); break;
      case kEpiSwiglu: mv_f16<kEpiSwiglu>(s, w, act, rows_b, o); break;
      case kEpiArgmax: mv_f16<kEpiArgmax>(s, w, act, rows_b, o); break;
    }
  }
  return false;
}

void launch_matvec_qkv(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                       const MatvecOut &o, const QkvEpi &q) {
  const int n_tiles = (rows_b + 15) / 16, groups = (w.mtiles + 7) / 8;
  if (n_tiles <= 2 && w.dtype == 8)  // as for the residual projections, below 3 batch tiles
    launch_k((k_mv_q8s<kEpiQkv, 1, 2, 8, 16>), dim3(groups * 8 * n_tiles), dim3(1024), 0, s, w, act, rows_b,
             n_tiles, o, q);
  else if (w.dtype == 8)
    launch_k((k_mv_q8s<kEpiQkv, 1, 2, 8>), dim3(groups * 8 * n_tiles), dim3(512), 0, s, w, act, rows_b,
             n_tiles, o, q);
  else
    launch_k((k_mv_q8s<kEpiQkv, 1, 2, 2>), dim3(groups * 8 * n_tiles), dim3(512), 0, s, w, act, rows_b,
             n_tiles, o, q);
}

bool launch_matvec_swiglu_q8(hipStream_t s, const MatrixView &w, const ActView &act, int rows_b,
                             const MatvecOut &o, const ActView &qout, int qout_nbp) {
  constexpr int kWPairs = 16;
  // K = 896 (Qwen2.5-0.5B's hidden size) gets kernels built for exactly its
  // 14 block pairs (straight-line block loops)
  constexpr int kExactPairs = 14;
  const int F = w.rows / 2, n_tiles = (rows_b + 15) / 16;
  if ((w.dtype != 8 && w.dtype != 2) || w.nbp > 2 * kWPairs || F % 64 != 0) return false;
  // the epilogue writes whole block pairs of the down projection's operand
  if (qout_nbp != ((F / 32 + 1) & ~1)) return false;
  if (n_tiles < 8) {
    // few batch tiles: one wave per (weight tile, batch tile), every CU busy
    const int nq = w.mtiles / 4, npairs = w.nbp / 2;
    const size_t items = (size_t)npairs * 64 + 4 * (size_t)w.nbp * 2 + (size_t)w.nbp * 2;
    const size_t lds = items * 16 > 4096 ? items * 16 : 4096;
    const dim3 grid((nq + 7) / 8 * 8 * n_tiles);
    if (w.dtype == 8 && npairs == kExactPairs)
      launch_k((k_mv_gu<8, 1, 1, kExactPairs, true>), grid, dim3(256), lds, s, w, act, rows_b, n_tiles, o.row_err,
               o.err_rows, qout, qout_nbp);
    else if (w.dtype == 8)
      launch_k((k_mv_gu<8, 1, 1, kWPairs>), grid, dim3(256), lds, s, w, act, rows_b, n_tiles, o.row_err, o.err_rows,
               qout, qout_nbp);
    else
      launch_k((k_mv_gu<2, 1, 1, kWPairs>), grid, dim3(256), lds, s, w, act, rows_b, n_tiles, o.row_err, o.err_rows,
               qout, qout_nbp);
    return true;
  }
  // eight batch tiles and more: the unit pair's weights shared through LDS
  const int groups = w.mtiles / 4;  // pairs of (gate, up) tile units: one Q8_0 block each
  const int by = (n_tiles + 7) / 8, nthreads = 2 * 64 * (n_tiles < 8 ? n_tiles : 8);
  const size_t pair_bytes = w.dtype == 8 ? 1024 : 512;
  // LDS: the two units' tiles and scales and the batch scales, and at least
  // the epilogue's exchange of 2 units x 8 batch tiles x 16 x 16 floats
  const size_t copy = 2 * 2 * (size_t)(w.nbp / 2) * pair_bytes + 2 * 2 * (size_t)w.nbp * 32 + 8 * (size_t)w.nbp * 32;
  const size_t lds = copy > 2 * 8 * 256 * 4 ? copy : 2 * 8 * 256 * 4;
  if (w.dtype == 8 && w.nbp == 2 * kExactPairs)
    launch_k((k_mv_q8w<kEpiSwiglu, 2, 8, kExactPairs, 2, true>), dim3(groups, by), dim3(nthreads), lds, s, w, act,
             rows_b, n_tiles, o, qout, qout_nbp);
  else if (w.dtype == 8)
    launch_k((k_mv_q8w<kEpiSwiglu, 2, 8, kWPairs, 2>), dim3(groups, by), dim3(nthreads), lds, s, w, act, rows_b,
             n_tiles, o, qout, qout_nbp);
  else
    launch_k((k_mv_q8w<kEpiSwiglu, 2, 2, kWPairs, 2>), dim3(groups, by), dim3(nthreads), lds, s, w, act, rows_b,
             n_tiles, o, qout, qout_nbp);
  return true;
}

void launch_argmax_reduce(hipStream_t s, int rows, const unsigned long long *part, int units,
                          unsigned long long *out) {
  launch_k(k_argmax_reduce, dim3(rows), dim3(256), 0, s, part, units, out);
}

void launch_qkv_post(hipStream_t s, int rows, const StepDims &d, const float *qkv,
                     const float *bias, const float2 *rope, const uint32_t *row_pos,
                     const int32_t *row_slot, float *q_rot, float *kpool, float *vpool,
                     uint32_t *row_err) {
  (void)row_err;
  launch_k(k_qkv_post, dim3(rows), dim3(256), 0, s, d, qkv, bias, rope, row_pos,
                     row_slot, q_rot, kpool, vpool);
}

#define COHX_DG_DISPATCH(D, G, LAUNCH)                                                    \
  do {                                                                                     \
    switch ((D) * 16 + (G)) {                                                              \
      case 64 * 16 + 7: LAUNCH(64, 7); break;                                              \
      case 64 * 16 + 8: LAUNCH(64, 8); break;                                              \
      case 64 * 16 + 4: LAUNCH(64, 4); break;                                              \
      case 64 * 16 + 2: LAUNCH(64, 2); break;                                              \
      case 64 * 16 + 1: LAUNCH(64, 1); break;                                              \
      case 128 * 16 + 6: LAUNCH(128, 6); break;                                            \
      case 128 * 16 + 7: LAUNCH(128, 7); break;                                            \
      case 128 * 16 + 8: LAUNCH(128, 8); break;                                            \
      case 128 * 16 + 4: LAUNCH(128, 4); break;                                            \
      case 128 * 16 + 2: LAUNCH(128, 2); break;                                            \
      case 128 * 16 + 1: LAUNCH(128, 1); break;                                            \
      case 32 * 16 + 2: LAUNCH(32, 2); break;                                              \
      case 32 * 16 + 4: LAUNCH(32, 4); break;                                              \
      case 32 * 16 + 1: LAUNCH(32, 1); break;                                              \
      default: ok = false;                                                                 \
    }                                                                                      \
  } while (0)

bool attention_shape_supported(int D, int G) {
  bool ok = true;
#define NOOP(a, b) (void)0
  COHX_DG_DISPATCH(D, G, NOOP);
#undef NOOP
  return ok;
}

void launch_attn_scores(hipStream_t s, int rows, int max_kv, const StepDims &d, const float *q_rot,
                        const float *kpool, const uint32_t *row_pos, const uint32_t *row_seq,
                        const int32_t *page_table, float *scores, float *chunk_max,
                        uint32_t *row_err) {
  // groups of 4+ heads in two workgroups (measured at 128 decode rows, G = 7:
  // 26.7 us against 28.3 us in one)
  const int ks = d.G >= 4 ? 2 : 1;
  const dim3 grid = d.att_items ? dim3(rows * d.NKV * ((max_kv + 255) / 256) * ks)
                                : dim3(rows, d.NKV, (max_kv + 255) / 256 * ks);
  bool ok = true;
#define L(DD, GG)                                                                                       \
  if (ks == 2)                                                                                          \
    launch_k((k_attn_scores<DD, GG, (GG >= 4 ? 2 : 1)>), grid, dim3(256), 0, s, d, q_rot, kpool, row_pos, \
             row_seq, page_table, scores, chunk_max, row_err);                                          \
  else                                                                                                  \
    launch_k((k_attn_scores<DD, GG, 1>), grid, dim3(256), 0, s, d, q_rot, kpool, row_pos, row_seq,      \
             page_table, scores, chunk_max, row_err)
  COHX_DG_DISPATCH(d.D, d.G, L);
#undef L
  (void)ok;
}

void launch_attn_exp(hipStream_t s, int rows, int max_kv, const StepDims &d,
                     const uint32_t *row_pos, const float *scores, const float *chunk_max,
                     double *den_part, float *row_max) {
  const dim3 grid = d.att_items ? dim3(rows * d.NKV * ((max_kv + 255) / 256)) : dim3(rows, d.NKV, (max_kv + 255) / 256);
  switch (d.G) {
#define L(GG)                                                                               \
  case GG:                                                                                  \
    launch_k(k_attn_exp<GG>, grid, dim3(256), 0, s, d, row_pos, scores, chunk_max, \
                       den_part, row_max);                                                  \
    break;
    L(1) L(2) L(4) L(6) L(7) L(8)
#undef L
    default: break;
  }
}

void launch_attn_pv(hipStream_t s, int rows, int max_kv, const StepDims &d, const float *vpool,
                    const uint32_t *row_pos, const uint32_t *row_seq, const int32_t *page_table,
                    const float *scores, const double *den_part, const float *row_max,
                    double *partial) {
  const dim3 grid = d.att_items ? dim3(rows * d.NKV * ((max_kv + 255) / 256) * 2)
                                : dim3(rows, d.NKV, (max_kv + kChunk - 1) / kChunk);
  bool ok = true;
#define L(DD, GG)                                                                          \
  launch_k((k_attn_pv<DD, GG>), grid, dim3(256), 0, s, d, vpool, row_pos, row_seq, \
                     page_table, scores, den_part, row_max, partial)
  COHX_DG_DISPATCH(d.D, d.G, L);
#undef L
  (void)ok;
}

bool attention_chunk_supported(int D, int G) {
  return D == 64 && (G == 1 || G == 2 || G == 4 || G == 6 || G == 7 || G == 8);
}

void launch_attn_stage(hipStream_t s, int n_images, const StepDims &d, const int4 *items, const float *kpool,
                       const float *vpool, const int32_t *page_table, uint4 *img) {
  if (n_images <= 0) return;
  launch_k(k_attn_stage, dim3(n_images), dim3(256), 0, s, d, items, kpool, vpool, page_table, img);
}

void launch_attn_chunk(hipStream_t s, int n_tiles, const StepDims &d, const int4 *tiles, const float *q_rot,
                       const uint4 *img, double *partial) {
  if (n_tiles <= 0) return;
  const dim3 grid(n_tiles * d.NKV);  // tile-major: the longest tiles of every KV head first
  switch (d.G) {
#define L(GG)                                                                        \
  case GG:                                                                           \
    launch_k(k_attn_chunk<GG>, grid, dim3(64 * GG), 0, s, d, tiles, q_rot, img, partial); \
    break;
    L(1) L(2) L(4) L(6) L(7) L(8)
#undef L
    default: break;
  }
}

void launch_attn_combine(hipStream_t s, int rows, const StepDims &d, const uint32_t *row_pos,
                         const double *partial, int act_dtype, int nbp, ActView act,
                         uint32_t *row_err) {
  const int threads = ((d.D + kWave - 1) / kWave) * kWave;
  if (act_dtype == kActQ8)
    launch_k(k_attn_combine<kActQ8>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
  else if (act_dtype == kActQ8H)
    launch_k(k_attn_combine<kActQ8H>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
  else if (act_dtype == kActF32)
    launch_k(k_attn_combine<kActF32>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
  else
    launch_k(k_attn_combine<1>, dim3(rows, d.NH), dim3(threads), 0, s, d, row_pos,
                       partial, nbp, act, row_err);
}

void launch_fill_synthetic(hipStream_t s, float *kpool, float *vpool, size_t layer_stride,
                           int layers, const int32_t *pages, int from, int rows, int NKV, int D,
                           uint64_t seed, uint32_t stream) {
  const size_t total = (size_t)(rows - from) * NKV * D;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  launch_k(k_fill_synthetic, dim3(blocks, layers), dim3(256), 0, s, kpool, vpool,
                     layer_stride, pages, from, rows, NKV, D, seed, stream);
}

void launch_copy_page(hipStream_t s, float *kpool, float *vpool, size_t layer_stride, int layers,
                      int page_floats, int src_page, int dst_page) {
  launch_k(k_copy_page, dim3((page_floats + 255) / 256, layers), dim3(256), 0, s, kpool,
                     vpool, layer_stride, page_floats, src_page, dst_page);
}

void launch_fill_u64(hipStream_t s, unsigned long long *p, size_t n, unsigned long long v) {
  int blocks = (int)((n + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  launch_k(k_fill_u64, dim3(blocks), dim3(256), 0, s, p, n, v);
}

void launch_fill_u32(hipStream_t s, uint32_t *p, size_t n, uint32_t v) {
  int blocks = (int)((n + 255) / 256);
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  launch_k(k_fill_u32, dim3(blocks), dim3(256), 0, s, p, n, v);
}

}  // namespace cohx
