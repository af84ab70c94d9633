// Qwen3.5 hybrid text step on the GPU, exact: every kernel reproduces the
// engine's float arithmetic (crates/coheryn-engine/src/qwen35/execution.rs:
// 257-608, qwen35/kernels.rs:11-269, cpu.rs:31-35,74-124) bit for bit:
// f32 products, f64 sums in the reference's element order, glibc expf and
// log1pf restated (exp_f32, log1p_f32), no contraction.
//
// Layout: activations are row-major f32 per packed row; matrices are BF16
// tiles of 16 outputs (q35_tiled_index); the sequence state lives in slabs
// indexed by sequence slot: K/V rows of the full-attention layers, the
// causal-conv ring and the delta-rule memory of the linear layers.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device.h"
#include "gemm.h"
#include "log1pf.h"
#include "q35.h"

namespace cohx {
namespace {

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// kernels.rs:11-24
__device__ __forceinline__ float sigmoid_f32(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + exp_f32(-x));
  const float e = exp_f32(x);
  return e / (1.0f + e);
}
__device__ __forceinline__ float silu_f32(float x) { return x * sigmoid_f32(x); }
__device__ __forceinline__ float softplus_f32(float x) {
  return fmaxf(x, 0.0f) + log1p_f32(exp_f32(-fabsf(x)));
}

// ---------------------------------------------------------------------------
// Token embedding (tensor.rs read_row over BF16: exact widening).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q35_embed(const uint16_t *__restrict__ embed,
                                                   const uint32_t *__restrict__ tokens, int H,
                                                   float *__restrict__ x) {
  const int r = blockIdx.x;
  const uint16_t *src = embed + (size_t)tokens[r] * H;
  for (int i = threadIdx.x; i < H; i += 256) x[(size_t)r * H + i] = bf_lo(src[i]);
}

// Sum of v[0..n) in f64, in index order from `init`, by one lane: the
// terms stream from LDS in batches of 16, the next batch loading while the
// current one is added, so the dependent add chain sets the pace.
__device__ __forceinline__ double ordered_sum_f64(const double *v, int n, double init) {
  double sum = init;
  const int n16 = n / 16;
  double cur[16], nxt[16];
  if (n16) {
#pragma unroll
    for (int j = 0; j < 16; j++) cur[j] = v[j];
  }
  for (int b = 0; b < n16; b++) {
    const int nb = min(b + 1, n16 - 1) * 16;
#pragma unroll
    for (int j = 0; j < 16; j++) nxt[j] = v[nb + j];
#pragma unroll
    for (int j = 0; j < 16; j++) sum += cur[j];
#pragma unroll
    for (int j = 0; j < 16; j++) cur[j] = nxt[j];
  }
  for (int i = n16 * 16; i < n; i++) sum += v[i];
  return sum;
}

// ---------------------------------------------------------------------------
// Norm (kernels.rs:26-52): mean of f32 squares summed in f64 in element
// order, scale = 1/sqrt(f32(mean) + eps), y = (x*scale)*(w + zc).  The
// squares are formed and widened in parallel; one lane runs the ordered sum.
// ---------------------------------------------------------------------------
constexpr int kNormMax = kQ35MaxHidden;
__global__ __launch_bounds__(256) void k_q35_norm(const float *__restrict__ x, int ldx,
                                                  const uint32_t *__restrict__ src,
                                                  const float *__restrict__ w, int n, float eps,
                                                  int zc, float *__restrict__ out, int ldo,
                                                  uint32_t *row_err,
                                                  const uint32_t *__restrict__ err_row) {
  __shared__ double sq[kNormMax];
  __shared__ float s_scale;
  __shared__ int s_bad;
  const int r = blockIdx.x;
  const float *xr = x + (size_t)(src ? src[r] : r) * ldx;
  bool bad = false;
  // the first kHeld elements per thread (n <= 1024) keep x and the weight in
  // registers across the ordered sum, so the scaling pass issues no loads
  constexpr int kHeld = 4;
  float xv[kHeld], wv[kHeld];
#pragma unroll
  for (int c = 0; c < kHeld; c++) {
    const int i = threadIdx.x + c * 256;
    xv[c] = i < n ? xr[i] : 0.0f;
    wv[c] = i < n ? w[i] : 0.0f;
  }
#pragma unroll
  for (int c = 0; c < kHeld; c++) {
    const int i = threadIdx.x + c * 256;
    if (i < n) {
      sq[i] = (double)(xv[c] * xv[c]);
      bad |= !finitef(xv[c]);
    }
  }
  for (int i = threadIdx.x + kHeld * 256; i < n; i += 256) {
    const float v = xr[i];
    sq[i] = (double)(v * v);
    bad |= !finitef(v);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const double sum = ordered_sum_f64(sq, n, -0.0);
    const double mean = sum / (double)n;
    s_bad = !(__builtin_isfinite(mean) && finitef((float)mean));
    s_scale = 1.0f / sqrtf((float)mean + eps);
  }
  __syncthreads();
  const float scale = s_scale, add = zc ? 1.0f : 0.0f;
#pragma unroll
  for (int c = 0; c < kHeld; c++) {
    const int i = threadIdx.x + c * 256;
    if (i < n) {
      const float y = (xv[c] * scale) * (wv[c] + add);
      out[(size_t)r * ldo + i] = y;
      bad |= !finitef(y);
    }
  }
  for (int i = threadIdx.x + kHeld * 256; i < n; i += 256) {
    const float y = (xr[i] * scale) * (w[i] + add);
    out[(size_t)r * ldo + i] = y;
    bad |= !finitef(y);
  }
  if (bad || (threadIdx.x == 0 && s_bad)) atomicOr(&row_err[err_row ? err_row[r] : r], kErrRequest);
}

// ---------------------------------------------------------------------------
// BF16 matvec (tensor.rs:380-406 -> cpu::dot): out[r][o] = f32(sum_k
// f64(w[o][k] * x[r][k])), k in order from -0.0.  A workgroup owns 64
// outputs (4 tiles of 16, one per wave) x 16 batch rows staged in LDS; lane
// (o16, g) runs rows 4g..4g+3 of output o16 as four chains, issued as pinned
// groups of products, widenings and adds.
// ---------------------------------------------------------------------------
constexpr int kMvRows = 16, kMvKC = 256;
template <int kEpi>
__global__ __launch_bounds__(256) void k_q35_mv(const uint16_t *__restrict__ w, int rows_w,
                                                int valid_rows, int K,
                                                const float *__restrict__ x, int ldx, int R,
                                                float *out, int ldo,
                                                unsigned long long *__restrict__ part,
                                                uint32_t *row_err,
                                                const uint32_t *__restrict__ err_row) {
  // rows padded by 4 floats: the four row groups of a wave read different banks
  __shared__ __align__(16) float xs[kMvRows][kMvKC + 4];
  __shared__ unsigned long long keys[kMvRows][64];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int o16 = lane % 16, g = lane / 16;
  const int tile = blockIdx.x * 4 + wave, r0 = blockIdx.y * kMvRows;
  const int o = tile * 16 + o16;
  const bool live_tile = tile * 16 < rows_w;
  const uint4 *wt = reinterpret_cast<const uint4 *>(w) + (size_t)tile * (K / 8) * 16 + o16;
  double acc[4] = {-0.0, -0.0, -0.0, -0.0};
  for (int k0 = 0; k0 < K; k0 += kMvKC) {
    const int kc = min(kMvKC, K - k0);
    __syncthreads();
    for (int i = threadIdx.x; i < kMvRows * (kMvKC / 4); i += 256) {
      const int rr = i / (kMvKC / 4), c4 = (i % (kMvKC / 4)) * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (r0 + rr < R && c4 < kc)
        v = *reinterpret_cast<const float4 *>(x + (size_t)(r0 + rr) * ldx + k0 + c4);
      *reinterpret_cast<float4 *>(&xs[rr][c4]) = v;
    }
    __syncthreads();
    if (!live_tile) continue;
    for (int kk = 0; kk < kc; kk += 8) {
      const uint4 wv = wt[(size_t)((k0 + kk) / 8) * 16];
      const float wf[8] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y),
                           bf_lo(wv.z), bf_hi(wv.z), bf_lo(wv.w), bf_hi(wv.w)};
      float xv[4][8];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const float4 lo = *reinterpret_cast<const float4 *>(&xs[g * 4 + rr][kk]);
        const float4 hi = *reinterpret_cast<const float4 *>(&xs[g * 4 + rr][kk + 4]);
        xv[rr][0] = lo.x; xv[rr][1] = lo.y; xv[rr][2] = lo.z; xv[rr][3] = lo.w;
        xv[rr][4] = hi.x; xv[rr][5] = hi.y; xv[rr][6] = hi.z; xv[rr][7] = hi.w;
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float pr[4];
#pragma unroll
        for (int rr = 0; rr < 4; rr++) pr[rr] = wf[e] * xv[rr][e];
        pin_vgprs(pr);
        double wd[4];
#pragma unroll
        for (int rr = 0; rr < 4; rr++) wd[rr] = (double)pr[rr];
        pin_vgprs(wd);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) acc[rr] += wd[rr];
        pin_vgprs(acc);
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < 4; rr++) {
    const int br = g * 4 + rr, r = r0 + br;
    const float v = (float)acc[rr];
    const bool ok = live_tile && r < R && o < valid_rows;
    if (kEpi == kQ35Argmax) {
      keys[br][wave * 16 + o16] = ok ? argmax_key(v, o) : 0ull;
      if (ok && out) out[(size_t)r * ldo + o] = v;
    } else if (ok) {
      float *p = out + (size_t)r * ldo + o;
      *p = kEpi == kQ35Residual ? *p + v : v;
    }
    if (ok && !finitef(v)) atomicOr(&row_err[err_row ? err_row[r] : r], kErrNonFinite);
  }
  if (kEpi == kQ35Argmax) {
    __syncthreads();
    if (threadIdx.x < kMvRows && r0 + (int)threadIdx.x < R) {
      unsigned long long best = 0;
      for (int i = 0; i < 64; i++) best = keys[threadIdx.x][i] > best ? keys[threadIdx.x][i] : best;
      part[(size_t)(r0 + threadIdx.x) * gridDim.x + blockIdx.x] = best;
    }
  }
}

// The same product for a few rows (decode steps): a workgroup of kWaves
// waves owns one tile of 16 outputs x 4*kWaves rows, a wave 4 rows, a lane
// one (output, row) chain, so a 1024-output matrix still spreads over 256
// waves.  The tile's weights and the rows' activations pass through LDS in
// chunks of kChunk inputs, double buffered: each thread holds its share of
// the next chunk in registers while the current chunk is summed, so a whole
// chunk of work covers the memory latency.  The weights are widened to f32
// once, when stored to LDS, rather than by each of the 16 lanes that use
// them.  The k order of each chain is the reference's.
// kEpi == kQ35Swiglu: eight waves over the same 16 rows, waves 0-3 on gate
// tile blockIdx.x and waves 4-7 on up tile blockIdx.x + up_off / 16 (up_off
// passed in valid_rows, F in ldo's place as the output count); the up waves
// hand their sums to the gate waves through LDS, which write
// h = (g / (1 + exp(-g))) * u (the SwiGLU pass's expression) to out [R][F].
template <int kEpi, int kChunk, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void k_q35_mvd(
    const uint16_t *__restrict__ w, int valid_rows, int K, const float *__restrict__ x, int ldx,
    int R, float *out, int ldo, unsigned long long *__restrict__ part, uint32_t *row_err,
    const uint32_t *__restrict__ err_row) {
  constexpr bool kGlu = kEpi == kQ35Swiglu;
  constexpr int kTiles = kGlu ? 2 : 1;          // weight tiles per workgroup
  constexpr int kT = kWaves * 64, kRows = 4 * kWaves / kTiles;
  constexpr int kXld = kChunk + 4;            // padded LDS row (floats)
  constexpr int kW4 = kChunk / 8 * 16;        // uint4 words of one tile's weight chunk
  constexpr int kX4 = kRows * kChunk / 4;     // float4 words of an activation chunk
  static_assert((kTiles * kW4) % kT == 0 && kX4 % kT == 0, "chunk must split evenly over the threads");
  __shared__ __align__(16) float4 ws[2][kTiles * 2 * kW4];  // f32 weights [tile][k8][half][output]
  __shared__ __align__(16) float xs[2][kRows * kXld];
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int sel = wave / (kWaves / kTiles), wv = wave % (kWaves / kTiles);
  const int o16 = lane % 16, tile = blockIdx.x, r0 = blockIdx.y * kRows;
  const int br = wv * 4 + lane / 16, r = r0 + br;
  const int o = tile * 16 + o16;
  const bool live = r < R;
  const int nk8 = K / 8;
  const uint4 *wt = reinterpret_cast<const uint4 *>(w) + (size_t)tile * nk8 * 16;
  const uint4 *wt_up = reinterpret_cast<const uint4 *>(w) + (size_t)(tile + (kGlu ? valid_rows / 16 : 0)) * nk8 * 16;
  uint4 wr[kTiles * kW4 / kT];
  float4 xr[kX4 / kT];
  auto fetch = [&](int k0) {
    const int kc = min(kChunk, K - k0);
    const int n4 = kc / 8 * 16;  // weight words in this chunk
#pragma unroll
    for (int i = 0; i < kTiles * kW4 / kT; i++) {
      const int idx = (tid + kT * i) % kW4;
      const uint4 *src = (tid + kT * i) < kW4 ? wt : wt_up;
      wr[i] = idx < n4 ? src[(size_t)k0 / 8 * 16 + idx] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kX4 / kT; i++) {
      const int idx = tid + kT * i, row = idx / (kChunk / 4), c = (idx % (kChunk / 4)) * 4;
      xr[i] = (r0 + row < R && c < kc)
                  ? *reinterpret_cast<const float4 *>(x + (size_t)(r0 + row) * ldx + k0 + c)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kTiles * kW4 / kT; i++) {
      const int idx = tid + kT * i, t2 = idx / kW4, k8 = idx % kW4 / 16, oo = idx % 16;
      const uint4 v = wr[i];
      float4 *dst = ws[buf] + t2 * 2 * kW4;
      dst[(2 * k8) * 16 + oo] = make_float4(bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y));
      dst[(2 * k8 + 1) * 16 + oo] = make_float4(bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w));
    }
#pragma unroll
    for (int i = 0; i < kX4 / kT; i++) {
      const int idx = tid + kT * i, row = idx / (kChunk / 4), c = (idx % (kChunk / 4)) * 4;
      *reinterpret_cast<float4 *>(&xs[buf][row * kXld + c]) = xr[i];
    }
  };
  fetch(0);
  stash(0);
  __syncthreads();
  double acc = -0.0;
  int buf = 0;
  for (int k0 = 0; k0 < K; k0 += kChunk) {
    const bool more = k0 + kChunk < K;
    if (more) fetch(k0 + kChunk);
    const int n8 = min(kChunk, K - k0) / 8;
    const float4 *wl = ws[buf] + sel * 2 * kW4 + o16;
    const float *xl = xs[buf] + br * kXld;
    for (int k8 = 0; k8 < n8; k8++) {
      const float4 a = wl[(2 * k8) * 16], b = wl[(2 * k8 + 1) * 16];
      const float4 p = *reinterpret_cast<const float4 *>(xl + k8 * 8);
      const float4 q = *reinterpret_cast<const float4 *>(xl + k8 * 8 + 4);
      acc += (double)(a.x * p.x);
      acc += (double)(a.y * p.y);
      acc += (double)(a.z * p.z);
      acc += (double)(a.w * p.w);
      acc += (double)(b.x * q.x);
      acc += (double)(b.y * q.y);
      acc += (double)(b.z * q.z);
      acc += (double)(b.w * q.w);
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  const float v = (float)acc;
  if constexpr (kGlu) {
    __shared__ float s_up[kRows][16];
    const bool ok = live && o < ldo;  // ldo: the output count F
    if (sel == 1) s_up[br][o16] = v;
    __syncthreads();
    if (sel == 0 && ok) {
      const float u = s_up[br][o16];
      out[(size_t)r * ldo + o] = (v / (1.0f + exp_f32(-v))) * u;
    }
    if (ok && !finitef(v)) atomicOr(&row_err[r], kErrNonFinite);
    return;
  }
  const bool ok = live && o < valid_rows;
  if (kEpi == kQ35Argmax) {
    unsigned long long key = ok ? argmax_key(v, o) : 0ull;
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
      const unsigned long long other = __shfl_xor(key, m, 16);
      key = other > key ? other : key;
    }
    if (ok && out) out[(size_t)r * ldo + o] = v;
    if (live && o16 == 0) part[(size_t)r * gridDim.x + tile] = key;
  } else if (ok) {
    float *p = out + (size_t)r * ldo + o;
    *p = kEpi == kQ35Residual ? *p + v : v;
  }
  if (ok && !finitef(v)) atomicOr(&row_err[err_row ? err_row[r] : r], kErrNonFinite);
}

// Broadcast lane J of each 16-lane row to the whole row; folded into the
// consuming multiply as a DPP operand (row_newbcast).
template <int J>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + J, 0xf, 0xf, false));
}

// Few-rows product split between waves: one wave issues at most one
// vector instruction every few clocks, so a lane that forms, widens and adds
// its own products runs its chain at a quarter of the SIMD's pace.  Here the
// consumer wave (wave 0) owns 64 chains, 16 outputs (lane % 16) x 4 rows
// (lane / 16), and only adds: per chunk of 16 * kProducers inputs it reads its
// widened products from LDS, two per read, in k order.  Producer waves
// 1..kProducers each form 16 of the chunk's products per chain (f32 product,
// widened to f64) for the next chunk, taking the activation for input j from
// lane j of the 16-lane row and the weights from registers loaded kDepth
// chunks ahead.  The consumer's adds are the reference's chain exactly.
// K % 16 == 0.
template <int kEpi, int kDepth, int kProducers = 4, int kConsumers = 1>
__global__ __launch_bounds__(64 * (kProducers + kConsumers)) void k_q35_mvpc(
    const uint16_t *__restrict__ w, int valid_rows, int K, const float *__restrict__ x, int ldx,
    int R, float *out, int ldo, unsigned long long *__restrict__ part, uint32_t *row_err,
    const uint32_t *__restrict__ err_row) {
  constexpr int kPcChunk = 16 * kProducers;
  __shared__ __align__(16) double2 pb[2][kPcChunk / 2][64];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int o16 = lane % 16, tile = blockIdx.x;
  const int r = blockIdx.y * 4 + lane / 16;
  const int o = tile * 16 + o16;
  const bool live = r < R;
  const int nc = (K + kPcChunk - 1) / kPcChunk, ng = K / 16;
  double acc = -0.0;
  // consumer wave c (< kConsumers) adds the chains of lanes
  // [c * 64/kConsumers, (c + 1) * 64/kConsumers); producer p = wave -
  // kConsumers forms group kProducers * chunk + p of 16 inputs for all 64
  const bool producer = wave >= kConsumers;
  const bool mine = !producer && lane / (64 / kConsumers) == wave;
  const int pg = wave - kConsumers;
  const uint4 *wt = reinterpret_cast<const uint4 *>(w) + (size_t)tile * (K / 8) * 16 + o16;
  const float *xr = x + (size_t)(live ? r : 0) * ldx + o16;
  // two register batches of kDepth chunks each: while one batch is turned
  // into products, the other is loading (no copies between them, so no load
  // is waited for before a whole batch of work has passed)
  float xa[kDepth], xb[kDepth];
  uint4 wa0[kDepth], wa1[kDepth], wb0[kDepth], wb1[kDepth];
  auto load = [&](float (&xv)[kDepth], uint4 (&w0)[kDepth], uint4 (&w1)[kDepth], int c0) {
#pragma unroll
    for (int j = 0; j < kDepth; j++) {
      const int g = min(kProducers * (c0 + j) + pg, ng - 1);
      xv[j] = xr[g * 16];
      w0[j] = wt[(size_t)(2 * g) * 16];
      w1[j] = wt[(size_t)(2 * g + 1) * 16];
    }
  };
  auto produce = [&](float xc, uint4 a, uint4 b, int c) {
    const int g = kProducers * c + pg;
    if (g >= ng) return;
    float wf[16] = {bf_lo(a.x), bf_hi(a.x), bf_lo(a.y), bf_hi(a.y), bf_lo(a.z), bf_hi(a.z),
                    bf_lo(a.w), bf_hi(a.w), bf_lo(b.x), bf_hi(b.x), bf_lo(b.y), bf_hi(b.y),
                    bf_lo(b.z), bf_hi(b.z), bf_lo(b.w), bf_hi(b.w)};
    pin_vgprs(wf);
    float pr[16] = {wf[0] * row_bcast<0>(xc),   wf[1] * row_bcast<1>(xc),
                    wf[2] * row_bcast<2>(xc),   wf[3] * row_bcast<3>(xc),
                    wf[4] * row_bcast<4>(xc),   wf[5] * row_bcast<5>(xc),
                    wf[6] * row_bcast<6>(xc),   wf[7] * row_bcast<7>(xc),
                    wf[8] * row_bcast<8>(xc),   wf[9] * row_bcast<9>(xc),
                    wf[10] * row_bcast<10>(xc), wf[11] * row_bcast<11>(xc),
                    wf[12] * row_bcast<12>(xc), wf[13] * row_bcast<13>(xc),
                    wf[14] * row_bcast<14>(xc), wf[15] * row_bcast<15>(xc)};
    double2 *dst = &pb[c & 1][pg * 8][lane];
#pragma unroll
    for (int e = 0; e < 8; e++) dst[e * 64] = make_double2((double)pr[2 * e], (double)pr[2 * e + 1]);
  };
  auto consume = [&](int c) {  // chunk c is full (not the last)
    const double2 *src = &pb[c & 1][0][lane];
#pragma unroll
    for (int e0 = 0; e0 < kPcChunk / 2; e0 += 16) {
      double2 d[16];
#pragma unroll
      for (int e = 0; e < 16; e++) d[e] = src[(e0 + e) * 64];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        acc += d[e].x;
        acc += d[e].y;
      }
    }
  };
  if (producer) load(xa, wa0, wa1, 0);
  // whole turns of 2*kDepth chunks; steps past the last chunk only keep the
  // barrier count uniform.  Step c: producers fill chunk c, the consumer adds
  // chunk c-1.
  const int ncp = (nc + 2 * kDepth - 1) / (2 * kDepth) * (2 * kDepth);
  for (int c0 = 0; c0 < ncp; c0 += 2 * kDepth) {
    if (producer) load(xb, wb0, wb1, c0 + kDepth);
#pragma unroll
    for (int j = 0; j < kDepth; j++) {
      const int c = c0 + j;
      if (producer) produce(xa[j], wa0[j], wa1[j], c);
      else if (mine && c > 0 && c < nc) consume(c - 1);
      __syncthreads();
    }
    if (producer) load(xa, wa0, wa1, c0 + 2 * kDepth);
#pragma unroll
    for (int j = 0; j < kDepth; j++) {
      const int c = c0 + kDepth + j;
      if (producer) produce(xb[j], wb0[j], wb1[j], c);
      else if (mine && c > 0 && c < nc) consume(c - 1);
      __syncthreads();
    }
  }
  if (!mine) return;
  {
    const int c = nc - 1;
    const int n2 = min(kPcChunk, K - c * kPcChunk) / 2;
    const double2 *src = &pb[c & 1][0][lane];
    for (int e = 0; e < n2; e++) {
      const double2 d = src[e * 64];
      acc += d.x;
      acc += d.y;
    }
  }
  const float v = (float)acc;
  const bool ok = live && o < valid_rows;
  if (kEpi == kQ35Argmax) {
    unsigned long long key = ok ? argmax_key(v, o) : 0ull;
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
      const unsigned long long other = __shfl_xor(key, m, 16);
      key = other > key ? other : key;
    }
    if (ok && out) out[(size_t)r * ldo + o] = v;
    if (live && o16 == 0) part[(size_t)r * gridDim.x + tile] = key;
  } else if (ok) {
    float *p = out + (size_t)r * ldo + o;
    *p = kEpi == kQ35Residual ? *p + v : v;
  }
  if (ok && !finitef(v)) atomicOr(&row_err[err_row ? err_row[r] : r], kErrNonFinite);
}

// cpu.rs:74-78 swiglu
__global__ __launch_bounds__(256) void k_q35_swiglu(const float *__restrict__ gu, int ldgu, int F,
                                                    int up_off, float *__restrict__ h, int ldh) {
  const int r = blockIdx.y;
  for (int f = blockIdx.x * 256 + threadIdx.x; f < F; f += gridDim.x * 256) {
    const float g = gu[(size_t)r * ldgu + f], u = gu[(size_t)r * ldgu + up_off + f];
    h[(size_t)r * ldh + f] = (g / (1.0f + exp_f32(-g))) * u;
  }
}

// ---------------------------------------------------------------------------
// Causal depthwise conv (kernels.rs:54-120), one thread per channel walking
// its lane's tokens in order.  The ring is kept in time order in registers
// (oldest first), which is exactly the reference's slot order
// (cursor + 1 + i) % kernel after the new input is written; the cursor of a
// sequence is position % kernel, since every layer steps once per token.
// ---------------------------------------------------------------------------
constexpr int kMaxConv = 8;
__global__ __launch_bounds__(256) void k_q35_conv(Q35Lanes L, const float *__restrict__ mix,
                                                  int ldm, const float *__restrict__ w, int C,
                                                  int K, float *hist, size_t hist_seq,
                                                  float *__restrict__ out, int ldo,
                                                  uint32_t *row_err) {
  const int ln = blockIdx.x, ch = blockIdx.y * 256 + threadIdx.x;
  if (ch >= C) return;
  const uint32_t first = L.first[ln], n = L.n[ln], start = L.start[ln];
  float *h = hist + (size_t)L.seq[ln] * hist_seq + (size_t)ch * K;
  const int c0 = (int)(start % (uint32_t)K);
  float tap[kMaxConv], wv[kMaxConv];
#pragma unroll
  for (int i = 0; i < kMaxConv; i++) {
    tap[i] = i < K ? h[(c0 + i) % K] : 0.0f;
    wv[i] = i < K ? w[(size_t)ch * K + i] : 0.0f;
  }
  // the inputs load a group of kAhead tokens at a time, the next group
  // requested before the current one is folded in, so a chunk's walk waits
  // on memory once per group rather than once per token
  constexpr int kAhead = 8;
  const float *mc = mix + ch;
  float cur[kAhead], nxt[kAhead];
#pragma unroll
  for (int j = 0; j < kAhead; j++) cur[j] = (uint32_t)j < n ? mc[(size_t)(first + j) * ldm] : 0.0f;
  for (uint32_t t0 = 0; t0 < n; t0 += kAhead) {
#pragma unroll
    for (int j = 0; j < kAhead; j++) {
      const uint32_t tn = t0 + kAhead + j;
      nxt[j] = tn < n ? mc[(size_t)(first + tn) * ldm] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kAhead; j++) {
      if (t0 + j >= n) break;
      const uint32_t row = first + t0 + j;
      const float in = cur[j];
#pragma unroll
      for (int i = 0; i < kMaxConv - 1; i++)
        if (i < K - 1) tap[i] = tap[i + 1];
#pragma unroll
      for (int i = 0; i < kMaxConv; i++)
        if (i == K - 1) tap[i] = in;
      double sum = -0.0;
#pragma unroll
      for (int i = 0; i < kMaxConv; i++)
        if (i < K) sum += (double)(tap[i] * wv[i]);
      const float y = silu_f32((float)sum);
      out[(size_t)row * ldo + ch] = y;
      if (!finitef(in) || !finitef(y)) atomicOr(&row_err[row], kErrRequest);
    }
#pragma unroll
    for (int j = 0; j < kAhead; j++) cur[j] = nxt[j];
  }
  const int c1 = (int)((start + n) % (uint32_t)K);
#pragma unroll
  for (int i = 0; i < kMaxConv; i++)
    if (i < K) h[(c1 + i) % K] = tap[i];
}

// ---------------------------------------------------------------------------
// Gated delta rule (kernels.rs:122-214) in three passes.
// Gates, per (row, value head): the q/k norms (ordered f64 sums of f32
// squares), q_scale = (1/sqrt(qn + 1e-6))/sqrt(key_dim), k_scale =
// 1/sqrt(kn + 1e-6), decay = exp(log_decay) with log_decay = -exp(A_log) *
// softplus(a + dt_bias), beta = sigmoid(b) (execution.rs:376-388).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q35_gates(const float *__restrict__ conv, int ldc,
                                                   int keys, const float *__restrict__ mix,
                                                   int ldm, int a_off, int b_off,
                                                   const float *__restrict__ a_log,
                                                   const float *__restrict__ dt, int KH, int VH,
                                                   int KD, float4 *__restrict__ gates,
                                                   uint32_t *row_err) {
  __shared__ double sq[2][128];
  __shared__ float norms[2];
  const int row = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int src = (h / (VH / KH)) * KD;
  const float *cr = conv + (size_t)row * ldc;
  for (int i = tid; i < KD; i += blockDim.x) {
    const float q = cr[src + i], k = cr[keys + src + i];
    sq[0][i] = (double)(q * q);
    sq[1][i] = (double)(k * k);
  }
  __syncthreads();
  if (tid % kWave == 0 && tid / kWave < 2) {  // one lane of each of two waves
    const int which = tid / kWave;
    norms[which] = (float)ordered_sum_f64(sq[which], KD, -0.0);
  }
  __syncthreads();
  if (tid == 0) {
    const float qn = norms[0], kn = norms[1];
    const float *mr = mix + (size_t)row * ldm;
    const float ld = -exp_f32(a_log[h]) * softplus_f32(mr[a_off + h] + dt[h]);
    const float beta = sigmoid_f32(mr[b_off + h]);
    gates[(size_t)row * VH + h] = make_float4((1.0f / sqrtf(qn + 1e-6f)) / sqrtf((float)KD),
                                              1.0f / sqrtf(kn + 1e-6f), exp_f32(ld), beta);
    if (!finitef(qn) || !finitef(kn) || !finitef(ld) || !finitef(beta) || ld > 0.0f ||
        !(beta >= 0.0f && beta <= 1.0f))
      atomicOr(&row_err[row], kErrRequest);
  }
}

// The recurrence: one workgroup per (lane, value head); thread j keeps state
// column j (kKD cells) in registers across the lane's tokens.  Per token the
// cells decay, the prediction chain sum_i f64(cell * k_i*k_scale) runs in key
// order from +0.0, corr = (v_j - f32(pred)) * beta, then the cells take
// k_i*k_scale*corr and the read chain sum_i f64(cell * q_i*q_scale) gives
// the head's raw output.
template <int kKD>
__global__ __launch_bounds__(256) void k_q35_delta(Q35Lanes L, const float *__restrict__ conv,
                                                   int ldc, int keys,
                                                   const float4 *__restrict__ gates, int KH,
                                                   int VH, int VD, float *state, size_t state_seq,
                                                   float *__restrict__ o_out, int ldo,
                                                   uint32_t *row_err) {
  __shared__ __align__(16) float s_qq[kKD], s_kk[kKD];
  const int ln = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const uint32_t first = L.first[ln], n = L.n[ln];
  const int src = (h / (VH / KH)) * kKD;
  float *S = state + (size_t)L.seq[ln] * state_seq + (size_t)h * kKD * VD;
  const bool active = j < VD;
  // the column moves through a buffer resource: lane offset j*4 in one VGPR,
  // key offset i*VD*4 as a scalar, so no per-key address stays live
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(S, (short)0, (int)(kKD * VD * 4), 0x00020000);
  const int voff = active ? j * 4 : 0;
  float col[kKD];
#pragma unroll
  for (int i = 0; i < kKD; i++)
    col[i] = active ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, i * VD * 4, 0))
                    : 0.0f;
  // token t + 1's gates, q/k channel j and v channel j are requested while
  // token t's chains run (the launcher gives at least kKD threads)
  float4 gt_n = make_float4(0.f, 0.f, 0.f, 0.f);
  float q_n = 0.0f, k_n = 0.0f, v_n = 0.0f;
  auto fetch = [&](uint32_t t) {
    const float *cr = conv + (size_t)(first + t) * ldc;
    gt_n = gates[(size_t)(first + t) * VH + h];
    if (j < kKD) {
      q_n = cr[src + j];
      k_n = cr[keys + src + j];
    }
    if (active) v_n = cr[2 * keys + h * VD + j];
  };
  if (n) fetch(0);
  for (uint32_t t = 0; t < n; t++) {
    const uint32_t row = first + t;
    const float4 gt = gt_n;
    const float qc = q_n, kc = k_n, v = v_n;
    __syncthreads();
    if (j < kKD) {
      s_qq[j] = qc * gt.x;
      s_kk[j] = kc * gt.y;
    }
    if (t + 1 < n) fetch(t + 1);
    __syncthreads();
    if (!active) continue;
    const float decay = gt.z, beta = gt.w;
    // the keys' LDS values are requested two groups of 4 ahead of their use,
    // so the chains do not wait on LDS at every group
    const float4 *kk4 = reinterpret_cast<const float4 *>(s_kk);
    const float4 *qq4 = reinterpret_cast<const float4 *>(s_qq);
    constexpr int kG4 = kKD / 4;
    double pred = 0.0;
    float4 ka = kk4[0], kb = kG4 > 1 ? kk4[1] : ka;
#pragma unroll
    for (int i0 = 0; i0 < kKD; i0 += 4) {
      asm volatile("" ::: "memory");
      const float4 kq = ka;
      ka = kb;
      if (i0 / 4 + 2 < kG4) kb = kk4[i0 / 4 + 2];
      const float kv[4] = {kq.x, kq.y, kq.z, kq.w};
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        col[i0 + e] *= decay;
        p[e] = col[i0 + e] * kv[e];
      }
      pin_vgprs(p);
      double wd[4];
#pragma unroll
      for (int e = 0; e < 4; e++) wd[e] = (double)p[e];
      pin_vgprs(wd);
#pragma unroll
      for (int e = 0; e < 4; e++) pred += wd[e];
    }
    const float corr = (v - (float)pred) * beta;
    double rd = 0.0;
    ka = kk4[0];
    kb = kG4 > 1 ? kk4[1] : ka;
    float4 qa = qq4[0], qb = kG4 > 1 ? qq4[1] : qa;
#pragma unroll
    for (int i0 = 0; i0 < kKD; i0 += 4) {
      asm volatile("" ::: "memory");
      const float4 kq = ka, qv4 = qa;
      ka = kb;
      qa = qb;
      if (i0 / 4 + 2 < kG4) {
        kb = kk4[i0 / 4 + 2];
        qb = qq4[i0 / 4 + 2];
      }
      const float kv[4] = {kq.x, kq.y, kq.z, kq.w}, qv[4] = {qv4.x, qv4.y, qv4.z, qv4.w};
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        col[i0 + e] += kv[e] * corr;
        p[e] = col[i0 + e] * qv[e];
      }
      pin_vgprs(p);
      double wd[4];
#pragma unroll
      for (int e = 0; e < 4; e++) wd[e] = (double)p[e];
      pin_vgprs(wd);
#pragma unroll
      for (int e = 0; e < 4; e++) rd += wd[e];
    }
    const float o = (float)rd;
    // a non-finite cell makes its read product non-finite (inf * 0 is NaN),
    // and no f64 sum brings an inf or NaN term back to a finite value, so o
    // is non-finite whenever any updated cell is: o covers the cells' check
    const bool bad = !finitef(o) || !finitef(v);
    o_out[(size_t)row * ldo + h * VD + j] = o;
    if (bad) atomicOr(&row_err[row], kErrRequest);
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < kKD; i++)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, col[i]), rs, voff,
                                            i * VD * 4, 0);
  }
}

// ---------------------------------------------------------------------------
// The whole linear-attention mixer of one (lane, value head) in one
// workgroup, token after token (execution.rs:357-411): the causal conv of the
// head's q, k (its key head's channels) and v channels, the q/k norms and
// gates, the delta-rule column updates, and the output norm times SiLU(z).
// Thread j owns q/k channel j of the key head (j < kKD), v channel and state
// column j of the value head (j < VD).  The arithmetic of each stage is the
// one the separate kernels above restate; only the launches are merged.
// Used when every value head has its own key head: a workgroup then owns all
// the conv channels it reads and writes back (with shared key heads the ring
// would be read by one workgroup after another had advanced it).  Conv
// kernels up to kFusedConv taps.
// ---------------------------------------------------------------------------
constexpr int kFusedConv = 4;
struct ConvTaps {
  float tap[kFusedConv], w[kFusedConv];
};
__device__ __forceinline__ void conv_load(ConvTaps &c, const float *h, const float *w, int K,
                                          int c0) {
#pragma unroll
  for (int i = 0; i < kFusedConv; i++) {
    c.tap[i] = i < K ? h[(c0 + i) % K] : 0.0f;
    c.w[i] = i < K ? w[i] : 0.0f;
  }
}
__device__ __forceinline__ float conv_step(ConvTaps &c, float in, int K) {
#pragma unroll
  for (int i = 0; i < kFusedConv - 1; i++)
    if (i < K - 1) c.tap[i] = c.tap[i + 1];
#pragma unroll
  for (int i = 0; i < kFusedConv; i++)
    if (i == K - 1) c.tap[i] = in;
  double sum = -0.0;
#pragma unroll
  for (int i = 0; i < kFusedConv; i++)
    if (i < K) sum += (double)(c.tap[i] * c.w[i]);
  return silu_f32((float)sum);
}
__device__ __forceinline__ void conv_store(const ConvTaps &c, float *h, int K, int c1) {
#pragma unroll
  for (int i = 0; i < kFusedConv; i++)
    if (i < K) h[(c1 + i) % K] = c.tap[i];
}

template <int kKD>
__global__ __launch_bounds__(256) void k_q35_linear(
    Q35Lanes L, const float *__restrict__ mix, int ldm, int keys, int z_off, int a_off, int b_off,
    const float *__restrict__ conv_w, int K, float *hist, size_t hist_seq,
    const float *__restrict__ a_log, const float *__restrict__ dt,
    const float *__restrict__ norm_w, int KH, int VH, int VD, float eps, float *state,
    size_t state_seq, float *__restrict__ tgt, int ldt, uint32_t *row_err) {
  __shared__ __align__(16) float qv[kKD], kv[kKD], s_qq[kKD], s_kk[kKD];
  __shared__ double qsq[kKD], ksq[kKD], osq[256];
  __shared__ float s_qn, s_kn, s_scale;
  __shared__ float4 s_gate;
  __shared__ int s_bad;
  const int ln = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const int rep = VH / KH, src = (h / rep) * kKD;
  const uint32_t first = L.first[ln], n = L.n[ln], start = L.start[ln];
  const uint32_t seq = L.seq[ln];
  const bool has_qk = j < kKD, has_v = j < VD;
  float *hs = hist + (size_t)seq * hist_seq;
  const int c0 = (int)(start % (uint32_t)K);
  const int qc = src + j, kc = keys + src + j, vc = 2 * keys + h * VD + j;
  ConvTaps cq, ck, cv;
  if (has_qk) {
    conv_load(cq, hs + (size_t)qc * K, conv_w + (size_t)qc * K, K, c0);
    conv_load(ck, hs + (size_t)kc * K, conv_w + (size_t)kc * K, K, c0);
  }
  if (has_v) conv_load(cv, hs + (size_t)vc * K, conv_w + (size_t)vc * K, K, c0);
  float *S = state + (size_t)seq * state_seq + (size_t)h * kKD * VD;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(S, (short)0, (int)(kKD * VD * 4), 0x00020000);
  const int voff = has_v ? j * 4 : 0;
  float col[kKD];
#pragma unroll
  for (int i = 0; i < kKD; i++)
    col[i] = has_v ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, voff, i * VD * 4, 0))
                   : 0.0f;
  const int T = blockDim.x;
  const float nw = has_v ? norm_w[j] : 0.0f;
  for (uint32_t t = 0; t < n; t++) {
    const uint32_t row = first + t;
    const float *mr = mix + (size_t)row * ldm;
    bool bad = false;
    // causal conv + SiLU (kernels.rs:54-120)
    if (has_qk) {
      const float iq = mr[qc], ik = mr[kc];
      const float q = conv_step(cq, iq, K), k = conv_step(ck, ik, K);
      qv[j] = q;
      kv[j] = k;
      qsq[j] = (double)(q * q);
      ksq[j] = (double)(k * k);
      bad |= !finitef(iq) || !finitef(ik) || !finitef(q) || !finitef(k);
    }
    float v = 0.0f;
    if (has_v) {
      const float iv = mr[vc];
      v = conv_step(cv, iv, K);
      bad |= !finitef(iv) || !finitef(v);
    }
    __syncthreads();
    // q/k norms: ordered f64 sums of the f32 squares, in two waves when there are two
    if (j == 0) s_qn = (float)ordered_sum_f64(qsq, kKD, -0.0);
    if (j == (T > kWave ? kWave : 0)) s_kn = (float)ordered_sum_f64(ksq, kKD, -0.0);
    __syncthreads();
    if (j == 0) {
      const float qn = s_qn, kn = s_kn;
      const float ld = -exp_f32(a_log[h]) * softplus_f32(mr[a_off + h] + dt[h]);
      const float beta = sigmoid_f32(mr[b_off + h]);
      s_gate = make_float4((1.0f / sqrtf(qn + 1e-6f)) / sqrtf((float)kKD), 1.0f / sqrtf(kn + 1e-6f),
                           exp_f32(ld), beta);
      s_bad = !finitef(qn) || !finitef(kn) || !finitef(ld) || !finitef(beta) || ld > 0.0f ||
              !(beta >= 0.0f && beta <= 1.0f);
    }
    __syncthreads();
    const float4 gt = s_gate;
    if (has_qk) {
      s_qq[j] = qv[j] * gt.x;
      s_kk[j] = kv[j] * gt.y;
    }
    __syncthreads();
    // the delta rule on state column j (kernels.rs:122-214)
    float o = 0.0f;
    if (has_v) {
      const float decay = gt.z, beta = gt.w;
      // LDS values two groups of 4 ahead of their use, as in k_q35_delta
      const float4 *kk4 = reinterpret_cast<const float4 *>(s_kk);
      const float4 *qq4 = reinterpret_cast<const float4 *>(s_qq);
      constexpr int kG4 = kKD / 4;
      double pred = 0.0;
      float4 ka = kk4[0], kb = kG4 > 1 ? kk4[1] : ka;
#pragma unroll
      for (int i0 = 0; i0 < kKD; i0 += 4) {
        asm volatile("" ::: "memory");
        const float4 kq = ka;
        ka = kb;
        if (i0 / 4 + 2 < kG4) kb = kk4[i0 / 4 + 2];
        const float k4[4] = {kq.x, kq.y, kq.z, kq.w};
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          col[i0 + e] *= decay;
          p[e] = col[i0 + e] * k4[e];
        }
        pin_vgprs(p);
        double wd[4];
#pragma unroll
        for (int e = 0; e < 4; e++) wd[e] = (double)p[e];
        pin_vgprs(wd);
#pragma unroll
        for (int e = 0; e < 4; e++) pred += wd[e];
      }
      const float corr = (v - (float)pred) * beta;
      double rd = 0.0;
      ka = kk4[0];
      kb = kG4 > 1 ? kk4[1] : ka;
      float4 qa = qq4[0], qb = kG4 > 1 ? qq4[1] : qa;
#pragma unroll
      for (int i0 = 0; i0 < kKD; i0 += 4) {
        asm volatile("" ::: "memory");
        const float4 kq = ka, qq = qa;
        ka = kb;
        qa = qb;
        if (i0 / 4 + 2 < kG4) {
          kb = kk4[i0 / 4 + 2];
          qb = qq4[i0 / 4 + 2];
        }
        const float k4[4] = {kq.x, kq.y, kq.z, kq.w}, q4[4] = {qq.x, qq.y, qq.z, qq.w};
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          col[i0 + e] += k4[e] * corr;
          p[e] = col[i0 + e] * q4[e];
        }
        pin_vgprs(p);
        double wd[4];
#pragma unroll
        for (int e = 0; e < 4; e++) wd[e] = (double)p[e];
        pin_vgprs(wd);
#pragma unroll
        for (int e = 0; e < 4; e++) rd += wd[e];
      }
      o = (float)rd;
      // a non-finite updated cell makes o non-finite (its read product is
      // inf or NaN, and no f64 sum returns from those), so o covers the cells
      bad |= !finitef(o);
      osq[j] = (double)(o * o);
    }
    __syncthreads();
    // output norm over the head (zero_centered false) times SiLU(z) (execution.rs:397-411)
    if (j == 0) {
      const double sum = ordered_sum_f64(osq, VD, -0.0);
      const double mean = sum / (double)VD;
      s_bad |= !(__builtin_isfinite(mean) && finitef((float)mean));
      s_scale = 1.0f / sqrtf((float)mean + eps);
    }
    __syncthreads();
    if (has_v) {
      const float z = mr[z_off + h * VD + j];
      const float y = ((o * s_scale) * (nw + 0.0f)) * silu_f32(z);
      tgt[(size_t)row * ldt + h * VD + j] = y;
      bad |= !finitef(y);
    }
    if (bad || (j == 0 && s_bad)) atomicOr(&row_err[row], kErrRequest);
    __syncthreads();  // the LDS stages are rewritten by the next token
  }
  const int c1 = (int)((start + n) % (uint32_t)K);
  if (has_qk) {
    conv_store(cq, hs + (size_t)qc * K, K, c1);
    conv_store(ck, hs + (size_t)kc * K, K, c1);
  }
  if (has_v) {
    conv_store(cv, hs + (size_t)vc * K, K, c1);
#pragma unroll
    for (int i = 0; i < kKD; i++)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, col[i]), rs, voff,
                                            i * VD * 4, 0);
  }
}

// Per value head: the output norm (zero_centered false) times SiLU(z)
// (execution.rs:397-411).
__global__ __launch_bounds__(256) void k_q35_headnorm(const float *__restrict__ o_in, int ldo,
                                                      const float *__restrict__ mix, int ldm,
                                                      int z_off, const float *__restrict__ w,
                                                      int VD, float eps, float *__restrict__ tgt,
                                                      int ldt, uint32_t *row_err) {
  __shared__ double sq[256];
  __shared__ float s_scale;
  __shared__ int s_bad;
  const int row = blockIdx.x, h = blockIdx.y, j = threadIdx.x;
  const float o = j < VD ? o_in[(size_t)row * ldo + h * VD + j] : 0.0f;
  if (j < VD) sq[j] = (double)(o * o);
  __syncthreads();
  if (j == 0) {
    const double sum = ordered_sum_f64(sq, VD, -0.0);
    const double mean = sum / (double)VD;
    s_bad = !(__builtin_isfinite(mean) && finitef((float)mean));
    s_scale = 1.0f / sqrtf((float)mean + eps);
  }
  __syncthreads();
  bool bad = false;
  if (j < VD) {
    const float z = mix[(size_t)row * ldm + z_off + h * VD + j];
    const float y = ((o * s_scale) * (w[j] + 0.0f)) * silu_f32(z);
    tgt[(size_t)row * ldt + h * VD + j] = y;
    bad = !finitef(y);
  }
  if (bad || (j == 0 && s_bad)) atomicOr(&row_err[row], kErrRequest);
}

// ---------------------------------------------------------------------------
// Full-attention q/k preparation (execution.rs:436-497): per head the
// zero-centred norm, then the partial rotary embedding (kernels.rs:226-268)
// from the host table (cos, sin) of angle pos * base^(-2i/rotary); q and its
// gate to the q/z buffers, k and v appended to the sequence's cache rows.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(576) void k_q35_qk(Q35Rows Rw, const float *__restrict__ mix,
                                                int ldm, int k_off, int v_off,
                                                const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm, int NH, int NKV,
                                                int D, int rotary, float eps,
                                                const float2 *__restrict__ rope, float *q,
                                                float *z, int ldq, float *kc, float *vc,
                                                size_t cache_seq, uint32_t *row_err) {
  __shared__ float y[512];
  __shared__ double sq[512];
  __shared__ float s_scale;
  __shared__ int s_bad;
  const int row = blockIdx.x, hh = blockIdx.y, d = threadIdx.x;
  const uint32_t pos = Rw.pos[row], seq = Rw.seq[row];
  const bool is_q = hh < NH;
  const int kh = hh - NH, kvw = NKV * D;
  const float *srcp = mix + (size_t)row * ldm + (is_q ? hh * 2 * D : k_off + kh * D);
  const float xv = d < D ? srcp[d] : 0.0f;
  if (d < D) sq[d] = (double)(xv * xv);
  __syncthreads();
  if (d == 0) {
    const double sum = ordered_sum_f64(sq, D, -0.0);
    const double mean = sum / (double)D;
    s_bad = !(__builtin_isfinite(mean) && finitef((float)mean));
    s_scale = 1.0f / sqrtf((float)mean + eps);
  }
  __syncthreads();
  bool bad = d < D && !finitef(xv);
  if (d < D) {
    y[d] = (xv * s_scale) * ((is_q ? q_norm : k_norm)[d] + 1.0f);
    bad |= !finitef(y[d]);
  }
  __syncthreads();
  float *dst = is_q ? q + (size_t)row * ldq + hh * D
                    : kc + (size_t)seq * cache_seq + (size_t)pos * kvw + kh * D;
  const int half = rotary / 2;
  if (d < half) {
    const float a = y[d], b = y[d + half];
    const float2 cs = rope[(size_t)pos * half + d];
    const float ra = a * cs.x - b * cs.y, rb = b * cs.x + a * cs.y;
    dst[d] = ra;
    dst[d + half] = rb;
    bad |= !finitef(ra) || !finitef(rb);
  } else if (d >= rotary && d < D) {
    dst[d] = y[d];
  }
  if (d < D) {
    if (is_q)
      z[(size_t)row * ldq + hh * D + d] = mix[(size_t)row * ldm + hh * 2 * D + D + d];
    else
      vc[(size_t)seq * cache_seq + (size_t)pos * kvw + kh * D + d] =
          mix[(size_t)row * ldm + v_off + kh * D + d];
  }
  if (bad || (d == 0 && s_bad)) atomicOr(&row_err[row], kErrRequest);
}

// ---------------------------------------------------------------------------
// Attention scores s_t = f32(sum_i f64(q_i * k_t,i)) / sqrt(D) (cpu.rs:80-124
// dot products), every (row, head, key) an independent ordered chain: a
// workgroup takes one row, one KV group and 256/G keys, the G heads of the
// group side by side so each K load serves them all.  Scores go to
// sc[row][head][key].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q35_scores(Q35Rows Rw, const float *__restrict__ q,
                                                    int ldq, const float *__restrict__ kc,
                                                    size_t cache_seq, int NH, int NKV, int D,
                                                    float *__restrict__ sc, int ldsc) {
  __shared__ __align__(16) float qs[kQ35MaxGroup * kQ35MaxHeadDim];
  const int row = blockIdx.x, kvh = blockIdx.y, G = NH / NKV, kb = 256 / G;
  const int kv = (int)Rw.pos[row] + 1, t0 = blockIdx.z * kb;
  if (t0 >= kv) return;
  const uint32_t seq = Rw.seq[row];
  const int kvw = NKV * D;
  const float *qg = q + (size_t)row * ldq + (size_t)kvh * G * D;
  for (int i = threadIdx.x; i < G * D; i += 256) qs[i] = qg[i];
  __syncthreads();
  const int hg = threadIdx.x % G, t = t0 + (int)threadIdx.x / G;
  if (t >= kv || (int)threadIdx.x >= kb * G) return;
  const float4 *kr =
      reinterpret_cast<const float4 *>(kc + (size_t)seq * cache_seq + (size_t)t * kvw + kvh * D);
  const float4 *qh = reinterpret_cast<const float4 *>(qs + hg * D);
  double a = -0.0;
  const int n4 = D / 4;
  for (int i0 = 0; i0 < n4; i0 += 8) {
    float4 kk[8];
#pragma unroll
    for (int j = 0; j < 8; j++) kk[j] = i0 + j < n4 ? kr[i0 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (i0 + j < n4) {
        const float4 qq = qh[i0 + j];
        a += (double)(qq.x * kk[j].x);
        a += (double)(qq.y * kk[j].y);
        a += (double)(qq.z * kk[j].z);
        a += (double)(qq.w * kk[j].w);
      }
    }
  }
  sc[((size_t)row * NH + kvh * G + hg) * ldsc + t] = (float)a / sqrtf((float)D);
}

// ---------------------------------------------------------------------------
// Online-softmax attention (cpu.rs:80-124) in the reference's exact order.
// The running maximum m_t is a prefix maximum (exact in any order), so the
// maxima and both exponentials old_t = exp(m_{t-1} - m_t), new_t =
// exp(s_t - m_t) are formed in parallel from the scores; the two f32
// recurrences den = den*old + new and o_d = o_d*old + new*v_d then run in key
// order, one thread per output element (and one for the denominator), V
// loads running eight keys ahead.  The output is o/den times sigmoid(gate)
// (execution.rs:506-508).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(576) void k_q35_attn(Q35Rows Rw, const float *__restrict__ scores,
                                                  int ldsc, const float *__restrict__ z, int ldq,
                                                  const float *__restrict__ vc, size_t cache_seq,
                                                  int NH, int NKV, int D, int maxc4,
                                                  float *__restrict__ out, int ldo) {
  extern __shared__ __align__(16) float sm[];
  float *sc = sm, *mx = sc + maxc4, *old = mx + maxc4, *seg = old + maxc4;
  __shared__ float s_den;
  const int row = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, nt = blockDim.x;
  const int dthreads = nt - kWave;  // the last wave runs the denominator
  const uint32_t pos = Rw.pos[row], seq = Rw.seq[row];
  const int kv = (int)pos + 1, kvh = h / (NH / NKV), kvw = NKV * D;
  const float *V = vc + (size_t)seq * cache_seq + kvh * D;
  const float *srow = scores + ((size_t)row * NH + h) * ldsc;
  __shared__ uint64_t s_tab[32];  // expf's table, read per lane in the exponent loops
  if (tid < 32) s_tab[tid] = kExp2Tab[tid];
  for (int t = tid; t < kv; t += nt) sc[t] = srow[t];
  __syncthreads();
  // prefix maxima: contiguous segments, then an exclusive scan of segment maxima
  const int per = (kv + nt - 1) / nt, lo = min(kv, tid * per), hi = min(kv, lo + per);
  float m = -__builtin_inff();
  for (int t = lo; t < hi; t++) {
    m = fmaxf(m, sc[t]);
    mx[t] = m;
  }
  // exclusive prefix maxima of the segment maxima (a maximum is exact in any
  // order): a shuffle scan within each wave, then the earlier waves' totals
  // (the block is whole waves)
  const int lane = tid % kWave, wave = tid / kWave;
  float inc = m;
#pragma unroll
  for (int d = 1; d < kWave; d *= 2) {
    const float u = __shfl_up(inc, d, kWave);
    if (lane >= d) inc = fmaxf(inc, u);
  }
  float base = __shfl_up(inc, 1, kWave);
  if (lane == 0) base = -__builtin_inff();
  if (lane == kWave - 1) seg[wave] = inc;
  __syncthreads();
  for (int i = 0; i < wave; i++) base = fmaxf(base, seg[i]);
  for (int t = lo; t < hi; t++) mx[t] = fmaxf(base, mx[t]);
  __syncthreads();
  for (int t = lo; t < hi; t++) {
    const float prev = t ? mx[t - 1] : -__builtin_inff();
    old[t] = exp_f32_tab(prev - mx[t], s_tab);
  }
  __syncthreads();
  for (int t = lo; t < hi; t++) sc[t] = exp_f32_tab(sc[t] - mx[t], s_tab);  // new_t
  __syncthreads();
  if (tid == dthreads) {
    float den = 0.0f;
    for (int t = 0; t < kv; t++) den = den * old[t] + sc[t];
    s_den = den;
  }
  float o = 0.0f;
  if (tid < D) {
    // whole groups of 8 keys without branches, the next group's V values
    // loading while the current group is folded in; then the tail
    const float *vp = V + tid;
    const int full = kv / 8;
    float cur[8], nxt[8];
#pragma unroll
    for (int j = 0; j < 8; j++) cur[j] = full ? vp[(size_t)j * kvw] : 0.0f;
    for (int g = 0; g < full; g++) {
      const int tn = min(g + 1, full - 1) * 8;
#pragma unroll
      for (int j = 0; j < 8; j++) nxt[j] = vp[(size_t)(tn + j) * kvw];
      const float4 o0 = *reinterpret_cast<const float4 *>(old + 8 * g);
      const float4 o1 = *reinterpret_cast<const float4 *>(old + 8 * g + 4);
      const float4 n0 = *reinterpret_cast<const float4 *>(sc + 8 * g);
      const float4 n1 = *reinterpret_cast<const float4 *>(sc + 8 * g + 4);
      o = o * o0.x + n0.x * cur[0];
      o = o * o0.y + n0.y * cur[1];
      o = o * o0.z + n0.z * cur[2];
      o = o * o0.w + n0.w * cur[3];
      o = o * o1.x + n1.x * cur[4];
      o = o * o1.y + n1.y * cur[5];
      o = o * o1.z + n1.z * cur[6];
      o = o * o1.w + n1.w * cur[7];
#pragma unroll
      for (int j = 0; j < 8; j++) cur[j] = nxt[j];
    }
    for (int t = full * 8; t < kv; t++) o = o * old[t] + sc[t] * vp[(size_t)t * kvw];
  }
  __syncthreads();
  if (tid < D) {
    const float gate = z[(size_t)row * ldq + h * D + tid];
    out[(size_t)row * ldo + h * D + tid] = (o / s_den) * sigmoid_f32(gate);
  }
}

// ---------------------------------------------------------------------------
// Packed-prefill regime (steps of 128+ rows): the linears run on the
// matrix-core GEMM (gemm.h) over the tiled BF16 matrices.  An f32 activation x enters
// as hi = bf16(x) and lo = bf16(x - hi) (round to nearest even), so hi + lo
// is x to a relative 2^-17 or better, every product of two bfloat16 values is
// exact in f32, and the f32 sums of hi . w + lo . w are what differ from the
// reference's f64 dot (cpu.rs:31-48).  Thread = 4 consecutive inputs.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_q35_split(const float *__restrict__ x, int ldx, int K,
                                                   uint16_t *__restrict__ hi, uint16_t *__restrict__ lo) {
  const int r = blockIdx.y, k = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (k >= K) return;
  const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)r * ldx + k);
  const float f[4] = {v.x, v.y, v.z, v.w};
  uint16_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const __bf16 bh = (__bf16)f[i];
    const __bf16 bl = (__bf16)(f[i] - (float)bh);
    h[i] = __builtin_bit_cast(uint16_t, bh);
    l[i] = __builtin_bit_cast(uint16_t, bl);
  }
  *reinterpret_cast<uint2 *>(hi + (size_t)r * K + k) =
      make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
  *reinterpret_cast<uint2 *>(lo + (size_t)r * K + k) =
      make_uint2(l[0] | (uint32_t)l[1] << 16, l[2] | (uint32_t)l[3] << 16);
}

}  // namespace

// ---- launchers ---------------------------------------------------------------

void q35_embed(hipStream_t s, int rows, const uint16_t *embed, const uint32_t *tokens, int H,
               float *x) {
  hipLaunchKernelGGL(k_q35_embed, dim3(rows), dim3(256), 0, s, embed, tokens, H, x);
}

void q35_norm(hipStream_t s, int rows, const float *x, int ldx, const uint32_t *src,
              const float *w, int n, float eps, int zc, float *out, int ldo, uint32_t *row_err,
              const uint32_t *err_row) {
  hipLaunchKernelGGL(k_q35_norm, dim3(rows), dim3(256), 0, s, x, ldx, src, w, n, eps, zc, out,
                     ldo, row_err, err_row);
}

int q35_matvec_blocks(int rows_w) { return (rows_w + 15) / 16; }

// Up to this many rows the one-chain-per-lane form runs (and always for the
// argmax head, whose partials are per 16-output tile).
constexpr int kMvdMaxRows = 64;

void q35_matvec(hipStream_t s, int epi, const uint16_t *w, int rows_w, int valid_rows, int K,
                const float *x, int ldx, int R, float *out, int ldo, unsigned long long *part,
                uint32_t *row_err, const uint32_t *err_row) {
  if (R <= kMvdMaxRows || epi == kQ35Argmax) {
    const int tiles = rows_w / 16;
    // Few (16-output tile, 4-row group) pairs: one chain per lane leaves most
    // SIMDs with a single wave, so the chains' adds go to consumer waves fed
    // by producer waves.  Otherwise the one-wave-per-chain-set form, four
    // waves per workgroup, three workgroups per CU.
    if (epi != kQ35Argmax && K % 16 == 0 && tiles * ((R + 3) / 4) <= 512) {
      const dim3 grid(tiles, (R + 3) / 4);
      // eight producers (128-input chunks, 128 KB of LDS, one workgroup per
      // CU) against four: C5 one-token steps 3.76 -> 3.65 ms
      if (epi == kQ35Store)
        hipLaunchKernelGGL((k_q35_mvpc<kQ35Store, 2, 8, 1>), grid, dim3(576), 0, s, w, valid_rows,
                           K, x, ldx, R, out, ldo, part, row_err, err_row);
      else
        hipLaunchKernelGGL((k_q35_mvpc<kQ35Residual, 2, 8, 1>), grid, dim3(576), 0, s, w,
                           valid_rows, K, x, ldx, R, out, ldo, part, row_err, err_row);
      return;
    }
    const dim3 grid(tiles, (R + 15) / 16);
    if (epi == kQ35Store)
      hipLaunchKernelGGL((k_q35_mvd<kQ35Store, 128, 4>), grid, dim3(256), 0, s, w, valid_rows, K, x,
                         ldx, R, out, ldo, part, row_err, err_row);
    else if (epi == kQ35Residual)
      hipLaunchKernelGGL((k_q35_mvd<kQ35Residual, 128, 4>), grid, dim3(256), 0, s, w, valid_rows,
                         K, x, ldx, R, out, ldo, part, row_err, err_row);
    else
      hipLaunchKernelGGL((k_q35_mvd<kQ35Argmax, 128, 4>), grid, dim3(256), 0, s, w, valid_rows, K,
                         x, ldx, R, out, ldo, part, row_err, err_row);
    return;
  }
  const dim3 grid((rows_w + 63) / 64, (R + kMvRows - 1) / kMvRows);
  if (epi == kQ35Store)
    hipLaunchKernelGGL(k_q35_mv<kQ35Store>, grid, dim3(256), 0, s, w, rows_w, valid_rows, K, x,
                       ldx, R, out, ldo, part, row_err, err_row);
  else if (epi == kQ35Residual)
    hipLaunchKernelGGL(k_q35_mv<kQ35Residual>, grid, dim3(256), 0, s, w, rows_w, valid_rows, K,
                       x, ldx, R, out, ldo, part, row_err, err_row);
  else
    hipLaunchKernelGGL(k_q35_mv<kQ35Argmax>, grid, dim3(256), 0, s, w, rows_w, valid_rows, K, x,
                       ldx, R, out, ldo, part, row_err, err_row);
}

void q35_split_bf16(hipStream_t s, int rows, int K, const float *x, int ldx, uint16_t *hi, uint16_t *lo) {
  hipLaunchKernelGGL(k_q35_split, dim3((K / 4 + 255) / 256, rows), dim3(256), 0, s, x, ldx, K, hi, lo);
}

// Tiles measured on the Qwen3.5 prompt-chunk shapes (4,096 rows, hi and lo
// products counted): 128 x 128 on eight waves of 64 features x 32 rows with
// two K steps in flight (mix 8,224 x 1024: 170 us; gate+up 7,168 x 1024:
// 130 us; out K 2048: 41 us; down K 3584: 63 us; on four waves of 64 x 64:
// 181, 128, 48, 72).
void q35_gemm_split(hipStream_t s, bool accumulate, const uint16_t *w, int N, int K, const uint16_t *hi,
                    const uint16_t *lo, int rows, float *out, int ldo, uint32_t *row_err) {
  using namespace gemm;
  Args g{};
  g.w = w;
  g.w_tiled = 1;
  g.x = hi;
  g.xlo = lo;
  g.N = N;
  g.K = K;
  g.M = rows;
  g.ldx = K;
  g.out = out;
  g.ldo = ldo;
  g.row_err = row_err;
  const dim3 grid(tile_order(g, N, 128, 128));
  constexpr int lds = lds_bytes<2, 4, 4, 2, true, kStore>();
  if (accumulate)
    hipLaunchKernelGGL((k_gemm<kBF16, true, 2, 4, 4, 2, 2, kAccumulate>), grid, dim3(512), lds, s, g);
  else
    hipLaunchKernelGGL((k_gemm<kBF16, true, 2, 4, 4, 2, 2, kStore>), grid, dim3(512), lds, s, g);
}

bool q35_matvec_swiglu(hipStream_t s, const uint16_t *w, int up_off, int F, int K, const float *x,
                       int ldx, int R, float *h, int ldh, uint32_t *row_err) {
  const int tiles = 2 * up_off / 16;  // gate and up tiles, as q35_matvec sees the matrix
  if (R > kMvdMaxRows || up_off % 16 || K % 8 || ldh != F ||
      (K % 16 == 0 && tiles * ((R + 3) / 4) <= 512))
    return false;
  hipLaunchKernelGGL((k_q35_mvd<kQ35Swiglu, 128, 8>), dim3(up_off / 16, (R + 15) / 16), dim3(512), 0,
                     s, w, up_off, K, x, ldx, R, h, F, nullptr, row_err, nullptr);
  return true;
}

void q35_swiglu(hipStream_t s, int rows, const float *gu, int ldgu, int F, int up_off, float *h,
                int ldh) {
  hipLaunchKernelGGL(k_q35_swiglu, dim3((F + 255) / 256, rows), dim3(256), 0, s, gu, ldgu, F,
                     up_off, h, ldh);
}

void q35_conv(hipStream_t s, int lanes, Q35Lanes L, const float *mix, int ldm, const float *w,
              int C, int K, float *hist, size_t hist_seq, float *out, int ldo, uint32_t *row_err) {
  hipLaunchKernelGGL(k_q35_conv, dim3(lanes, (C + 255) / 256), dim3(256), 0, s, L, mix, ldm, w, C,
                     K, hist, hist_seq, out, ldo, row_err);
}

bool q35_linear_fused(int conv_kernel, int key_heads, int value_heads) {
  return conv_kernel <= kFusedConv && key_heads == value_heads;
}

void q35_linear(hipStream_t s, int lanes, Q35Lanes L, const float *mix, int ldm, int keys,
                int z_off, int a_off, int b_off, const float *conv_w, int K, float *hist,
                size_t hist_seq, const float *a_log, const float *dt, const float *norm_w,
                int key_heads, int value_heads, int key_dim, int value_dim, float eps,
                float *state, size_t state_seq, float *tgt, int ldt, uint32_t *row_err) {
  const dim3 grid(lanes, value_heads);
  const dim3 block(((std::max(key_dim, value_dim) + kWave - 1) / kWave) * kWave);
#define LIN_(KD)                                                                               \
  case KD:                                                                                     \
    hipLaunchKernelGGL(k_q35_linear<KD>, grid, block, 0, s, L, mix, ldm, keys, z_off, a_off,  \
                       b_off, conv_w, K, hist, hist_seq, a_log, dt, norm_w, key_heads,           \
                       value_heads, value_dim, eps, state, state_seq, tgt, ldt, row_err);      \
    break;
  switch (key_dim) {
    LIN_(16) LIN_(32) LIN_(64) LIN_(128)
    default: break;
  }
#undef LIN_
}

bool q35_delta_supported(int key_dim, int value_dim) {
  return (key_dim == 16 || key_dim == 32 || key_dim == 64 || key_dim == 128) && value_dim >= 1 &&
         value_dim <= 256;
}

void q35_delta(hipStream_t s, int rows, int lanes, Q35Lanes L, const float *conv, int ldc, int keys,
               const float *mix, int ldm, int z_off, int a_off, int b_off, const float *a_log,
               const float *dt, const float *norm_w, int key_heads, int value_heads, int key_dim,
               int value_dim, float eps, float *state, size_t state_seq, float4 *gates,
               float *o_raw, float *tgt, int ldt, uint32_t *row_err) {
  hipLaunchKernelGGL(k_q35_gates, dim3(rows, value_heads), dim3(128), 0, s, conv, ldc, keys, mix,
                     ldm, a_off, b_off, a_log, dt, key_heads, value_heads, key_dim, gates, row_err);
  // at least key_dim threads: thread j stages q/k channel j of each token
  const dim3 grid(lanes, value_heads),
      block(((std::max(value_dim, key_dim) + kWave - 1) / kWave) * kWave);
#define L_(KD)                                                                                 \
  case KD:                                                                                     \
    hipLaunchKernelGGL(k_q35_delta<KD>, grid, block, 0, s, L, conv, ldc, keys, gates, key_heads, \
                       value_heads, value_dim, state, state_seq, o_raw, ldt, row_err);         \
    break;
  switch (key_dim) {
    L_(16) L_(32) L_(64) L_(128)
    default: break;
  }
#undef L_
  hipLaunchKernelGGL(k_q35_headnorm, dim3(rows, value_heads), block, 0, s, o_raw, ldt, mix, ldm,
                     z_off, norm_w, value_dim, eps, tgt, ldt, row_err);
}

void q35_qk(hipStream_t s, int rows, Q35Rows Rw, const float *mix, int ldm, int k_off, int v_off,
            const float *q_norm, const float *k_norm, int heads, int kv_heads, int D, int rotary,
            float eps, const float2 *rope, float *q, float *z, int ldq, float *kc, float *vc,
            size_t cache_seq, uint32_t *row_err) {
  const int threads = ((D + kWave - 1) / kWave) * kWave;
  hipLaunchKernelGGL(k_q35_qk, dim3(rows, heads + kv_heads), dim3(threads), 0, s, Rw, mix, ldm,
                     k_off, v_off, q_norm, k_norm, heads, kv_heads, D, rotary, eps, rope, q, z,
                     ldq, kc, vc, cache_seq, row_err);
}

void q35_attention(hipStream_t s, int rows, Q35Rows Rw, const float *q, const float *z, int ldq,
                   const float *kc, const float *vc, size_t cache_seq, int heads, int kv_heads,
                   int D, int max_context, float *scores, float *out, int ldo) {
  const int G = heads / kv_heads, kb = 256 / G;
  hipLaunchKernelGGL(k_q35_scores, dim3(rows, kv_heads, (max_context + kb - 1) / kb), dim3(256), 0,
                     s, Rw, q, ldq, kc, cache_seq, heads, kv_heads, D, scores, max_context);
  const int threads = ((D + kWave - 1) / kWave) * kWave + kWave;
  const int maxc4 = (max_context + 3) / 4 * 4;
  const size_t lds = (size_t)(3 * maxc4 + threads) * sizeof(float);
  hipLaunchKernelGGL(k_q35_attn, dim3(rows, heads), dim3(threads), lds, s, Rw, scores, max_context,
                     z, ldq, vc, cache_seq, heads, kv_heads, D, maxc4, out, ldo);
}

}  // namespace cohx
