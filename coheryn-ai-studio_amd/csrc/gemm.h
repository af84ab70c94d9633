// The packed-prefill regime's matrix-core GEMM (gfx950):
//
//   C[m][n] = sum_k X[m][k] * W[n][k]  (+ Xlo[m][k] * W[n][k])
//
// W is an [N][K] matrix of binary16 (Qwen2 F16 weights, row-major) or
// bfloat16 (Qwen3.5 weights, read in place from the exact matvecs' 16-row
// tiles), X the packed token rows [M][ldx] in the same type (the
// activations already rounded as the reference rounds them, cpu.rs:37-48, or
// the hi part of an f32 activation split hi + lo for bfloat16).  Every
// product of two such values is exact in f32; the sums are f32 in MFMA order,
// where the reference sums in f64 (cpu.rs:31-48): the regime's tolerance.
//
// Tiling.  A workgroup of kWM x kWN waves owns BM = 16 kWM kTM output
// features by BN = 16 kWN kTN token rows; each wave a kTM x kTN grid of
// v_mfma_f32_16x16x32 tiles (lane l holds features 4 (l/16) + i of token
// column l % 16).  K advances 32 at a time.  Each thread keeps kR K steps of
// its share of the operands in flight in registers (16-byte global loads);
// the LDS holds two steps: while the waves multiply step ks out of one half,
// step ks + 1 is written into the other from the registers loaded kR - 1
// steps earlier, and those registers are refilled with step ks + kR.  (A
// ring of direct-to-LDS loads, global_load_lds_dwordx4, measured slower: at
// about 10 TB/s of L2-to-LDS traffic its loads alone took longer than this
// whole kernel, and they slowed the LDS reads beside them.)  Within a step a
// row's 64 bytes are four 16-byte segments; segment s of row R sits at slot
// 4R + (s ^ ((R >> 1) & 3)).  The LDS serves a 16-byte access eight lanes at
// a time, free of bank conflicts when the eight addresses differ modulo 128
// bytes; a fragment read gives those eight lanes rows R..R+7 of one segment,
// and this swizzle puts them on eight distinct 16-byte positions.  (With
// (R >> 2) & 3 rows R and R + 2 met, and about a third of all LDS cycles
// were bank conflicts.)
//
// Epilogues: store or accumulate f32 rows (ldo), SwiGLU of a [gate | up]
// matrix into the down projection's binary16 operand (gate waves and their up
// partner waves hold the same positions; the up sums cross through LDS), the
// argmax head keys, and the qkv projection's bias, rotation and K/V append
// (kQkvRope).  Non-finite outputs set the row's error bit.
#pragma once
#include <type_traits>

#include "device.h"

namespace cohx {
namespace gemm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;  // K per ring stage: one MFMA step

// kSwigluQ8: SwiGLU rounded as the reference's Q8_0 operand of the down
// projection (q * f16(d) per 32-feature block, as binary16; quant.rs:193-213)
// kQkvRope: the qkv projection's bias, RoPE and K/V append (the operations
// of the separate post pass, cohx k_qkv_post) applied to the tile in place of
// a store
enum Epi { kStore = 0, kAccumulate = 1, kSwigluF16 = 2, kArgmax = 3, kSwigluQ8 = 4, kQkvRope = 5 };
enum Type { kF16 = 0, kBF16 = 1 };

struct Args {
  const uint16_t *w;    // [N][K] row-major, or in 16-row tiles (w_tiled)
  int w_tiled;          // W as [N/16][K/8][16][8] (the Qwen3.5 matvecs' layout): each
                        // row's 8 consecutive inputs stay 16 contiguous bytes
  const uint16_t *x;    // [M][ldx]
  const uint16_t *xlo;  // [M][ldx] second operand summed into the same tiles (bfloat16 lo parts), or null
  int N, K, M, ldx;
  float *out;           // kStore / kAccumulate: [M][ldo]
  int ldo;
  uint16_t *out16;      // kSwigluF16: [M][F] binary16, F = N / 2
  unsigned long long *keys;  // kArgmax: [M][ktiles] per 16-feature tile
  int ktiles;
  float *logits;        // kArgmax: optional [M][N]
  uint32_t *row_err;
  const uint32_t *err_rows;  // optional: the error slot of each token row
  // tile order (see tile_of): tiles along features (nf) and token rows (nr),
  // tiles per XCD, and whether feature blocks are the major index
  int nf, nr, per_xcd, feature_major;
  // k_gemm_q: W as the exact matvecs' 16-row tiles of Q8_0 (int8 values) or
  // Q4_0 (nibbles) blocks and their binary16 scales [tile][nbp][16]
  // (device.h q8_byte / q4_byte / q8_scale); SwiGLU matrices hold gate tile
  // i at tile 2i and up tile i at tile 2i + 1
  const void *qs;
  const uint16_t *ds;
  int nbp;
  // kStore: features [0, rope_rows) are query and key heads of rope_d
  // features uploaded in rope order (cohx.cpp rope_row); each is stored at
  // its source column
  int rope_d, rope_rows;
  // kQkvRope: features [0, H) query heads, [H, H + KVD) key heads, then value
  // heads, of D = 64 features each (rope_rows > 0: the query and key rows in
  // rope order as above, else in source order, where a wave's 64 features
  // are one head); bias in source order, rope [position][D/2] (cos, sin),
  // the rows' positions and KV slots (< 0: no append), the rotated queries
  // [M][H] and the layer's pools
  const float *qk_bias;
  const float2 *qk_rope;
  const uint32_t *qk_pos;
  const int32_t *qk_slot;
  float *qk_q, *qk_kpool, *qk_vpool;
  int qk_H, qk_KVD, qk_NKV;
};

// SwiGLU's gate activation g / (1 + e^-g) in the regime's epilogues, on the
// hardware exp2 and reciprocal (about 1 ulp each, ~1e-6 relative in all:
// far inside the regime's binary16 operand rounding; the exact kernels keep
// the reference's expf and IEEE division).  Large negative g gives -0, +inf
// gives +inf, -inf and NaN give NaN, as the exact formula does.
__device__ __forceinline__ float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.44269504f));
}

// Source column of feature f of a rope-ordered head block: even features are
// a head's first half in order, odd ones its second half.
__device__ __forceinline__ int rope_col(int f, int d) {
  const int i = f % d;
  return f - i + ((i & 1) ? (i >> 1) + d / 2 : (i >> 1));
}

// Workgroup -> output tile.  The dispatcher hands workgroup ids to the 8 XCDs
// round robin (id % 8), and each XCD has its own L2.  Tiles are numbered in
// one major order (feature blocks major, token blocks minor, or the reverse)
// and XCD x takes the contiguous range [x per_xcd, (x + 1) per_xcd): its
// tiles share one or a few major blocks and cover the minor blocks, so the
// operand slices one XCD needs stay few and its concurrent tiles read the
// same major block.
// Returns the tile as (feature block, token block), or (-1, -1) for the ids
// past the last tile.
__device__ __forceinline__ int2 tile_of(const Args &g) {
  const int L = blockIdx.x, t = (L % 8) * g.per_xcd + L / 8;
  if (t >= g.nf * g.nr || L / 8 >= g.per_xcd) return make_int2(-1, -1);
  const int minor = g.feature_major ? g.nr : g.nf;
  const int hi = t / minor, lo = t - hi * minor;
  return g.feature_major ? make_int2(hi, lo) : make_int2(lo, hi);
}

// Operand fragments are read from LDS as the MFMA's own vector type, and the
// staged operand bytes live in a plain vector type (HIP's uint4 struct made
// the compiler keep the staging registers in scratch memory).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int kType>
using frag_t = std::conditional_t<kType == kF16, f16x8, bf16x8>;

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Fills the tile-order fields of `g` for tiles of bm features by bn rows
// (bm: output features per tile, halved for SwiGLU by the caller) and
// returns the 1-D grid size.  The major index is the one whose blocks are the
// more expensive to re-read: an XCD's range then spans few major blocks and
// all minor ones, and the smaller of the two slice sums wins.
// w_bytes: bytes per weight value in HBM (2 for binary16 and bfloat16,
// 34/32 for Q8_0 blocks, 18/32 for Q4_0).
inline int tile_order(Args &g, int out_features, int bm, int bn, double w_bytes = 2.0) {
  g.nf = (out_features + bm - 1) / bm;
  g.nr = (g.M + bn - 1) / bn;
  const int tiles = g.nf * g.nr;
  g.per_xcd = (tiles + 7) / 8;
  const double wb = (double)bm * g.K * w_bytes, xb = 2.0 * bn * g.K * (g.xlo ? 2 : 1);
  const double f_major = (double)g.per_xcd / g.nr * wb + (double)g.nr * xb;  // few W blocks, all X
  const double r_major = (double)g.per_xcd / g.nf * xb + (double)g.nf * wb;  // few X blocks, all W
  g.feature_major = f_major <= r_major;
  return 8 * g.per_xcd;
}

// LDS bytes one workgroup of this configuration takes: two K steps of both
// operands, or the SwiGLU exchange of the up sums if that is larger.
template <int kWM, int kWN, int kTM, int kTN, bool kLo, int kEpi>
constexpr int lds_bytes() {
  constexpr int ring = 2 * (16 * kWM * kTM + (kLo ? 2 : 1) * 16 * kWN * kTN) * 64;
  constexpr int park = kEpi == kSwigluF16 ? (kWM / 2) * kWN * kTM * kTN * 4 * 64 * 4 : 0;
  return ring > park ? ring : park;
}

// Output tile of a workgroup: the accumulators of its waves at features
// f0 + ..., token rows r0 + ... (SwiGLU: f0 counts gate features).  The LDS
// is free (all waves are past the main loop's last barrier).
template <int kWM, int kWN, int kTM, int kTN, int kEpi>
__device__ __forceinline__ void epilogue(const Args &g, f32x4 (&acc)[kTM][kTN], int f0, int r0,
                                         uint4 *smem) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWN, wn = wave % kWN, lr = lane % 16;
  const int F = g.N / 2;
  if constexpr (kEpi == kQkvRope) {
    constexpr int kD = 64, kHalf = 32;
    static_assert(kTM == 4, "source order: a wave's four 16-feature tiles are one head");
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int r = r0 + (wn * kTN + b) * 16 + lr;
      if (r >= g.M) continue;
      const uint32_t pos = g.qk_pos[r];
      const int32_t slot = g.qk_slot[r];
      const float2 *rp = g.qk_rope + (size_t)pos * kHalf;
      const int page = slot / kPage, off = slot % kPage;
      bool bad = false;
      // n consecutive (i, i + D/2) pairs of one head, element i of the first
      // at source index src, rotated as k_qkv_post does it and stored as
      // vectors (n = 4: one K quad; n = 2: half of one)
      auto rotate = [&](auto N, int src, int i, const float *x, const float *y) __attribute__((always_inline)) {
        constexpr int n = decltype(N)::value;
        float lo[n], hi[n];
#pragma unroll
        for (int u = 0; u < n; u++) {
          const float qa = x[u] + g.qk_bias[src + u], qb = y[u] + g.qk_bias[src + u + kHalf];
          const float2 cs = rp[i + u];
          lo[u] = fmaf(qa, cs.x, -(qb * cs.y));
          hi[u] = fmaf(qa, cs.y, qb * cs.x);
        }
        float *dlo, *dhi;
        if (src < g.qk_H) {
          dlo = g.qk_q + (size_t)r * g.qk_H + src;
          dhi = dlo + kHalf;
        } else if (slot >= 0) {
          const int kg = (src - g.qk_H) / kD;
          dlo = g.qk_kpool + k_at(page, pos / kPage, kg, g.qk_NKV, off, i, kD);
          dhi = g.qk_kpool + k_at(page, pos / kPage, kg, g.qk_NKV, off, i + kHalf, kD);
        } else {
          return;
        }
        if constexpr (n == 4) {
          *reinterpret_cast<float4 *>(dlo) = make_float4(lo[0], lo[1], lo[2], lo[3]);
          *reinterpret_cast<float4 *>(dhi) = make_float4(hi[0], hi[1], hi[2], hi[3]);
        } else {
          *reinterpret_cast<float2 *>(dlo) = make_float2(lo[0], lo[1]);
          *reinterpret_cast<float2 *>(dhi) = make_float2(hi[0], hi[1]);
        }
      };
#pragma unroll
      for (int a = 0; a < kTM; a++) {
        const int fb = f0 + (wm * kTM + a) * 16 + 4 * (lane / 16);
        if (fb >= g.N) continue;
        const float *v = reinterpret_cast<const float *>(&acc[a][b]);
#pragma unroll
        for (int i = 0; i < 4; i++) bad |= !finitef(v[i]);
        if (fb >= g.qk_H + g.qk_KVD) {  // value features: bias and append
          if (slot >= 0) {
            const int e = fb - g.qk_H - g.qk_KVD;
            *reinterpret_cast<float4 *>(g.qk_vpool + v_at(page, e / kD, g.qk_NKV, off, e % kD, kD)) =
                make_float4(v[0] + g.qk_bias[fb], v[1] + g.qk_bias[fb + 1], v[2] + g.qk_bias[fb + 2],
                            v[3] + g.qk_bias[fb + 3]);
          }
        } else if (g.rope_rows > 0) {  // rope order: pairs (2i, 2i + 1) adjacent
          const int i = (fb % kD) / 2;
          const float x[2] = {v[0], v[2]}, y[2] = {v[1], v[3]};
          rotate(std::integral_constant<int, 2>{}, fb - fb % kD + i, i, x, y);
        } else if (a < 2) {  // source order: element i in tile a, i + D/2 in tile a + 2
          const float *y = reinterpret_cast<const float *>(&acc[a + 2][b]);
          rotate(std::integral_constant<int, 4>{}, fb, fb % kD, v, y);
        }
      }
      if (bad) atomicOr(&g.row_err[g.err_rows ? (int)g.err_rows[r] : r], kErrNonFinite);
    }
    return;
  } else if constexpr (kEpi == kArgmax) {
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int r = r0 + (wn * kTN + b) * 16 + lr;
      const bool rvalid = r < g.M;
      bool bad = false;
#pragma unroll
      for (int a = 0; a < kTM; a++) {
        const int ft = f0 + (wm * kTM + a) * 16, fb = ft + 4 * (lane / 16);
        unsigned long long key = 0ull;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float v = acc[a][b][i];
          if (rvalid && fb + i < g.N) {
            bad |= !finitef(v);
            if (g.logits) g.logits[(size_t)r * g.N + fb + i] = v;
            const unsigned long long k = argmax_key(v, fb + i);
            key = k > key ? k : key;
          }
        }
        unsigned long long o = __shfl_xor(key, 16, kWave);
        key = o > key ? o : key;
        o = __shfl_xor(key, 32, kWave);
        key = o > key ? o : key;
        if (lane < 16 && rvalid && ft < g.N) g.keys[(size_t)r * g.ktiles + ft / 16] = key;
      }
      if (bad) atomicOr(&g.row_err[g.err_rows ? (int)g.err_rows[r] : r], kErrNonFinite);
    }
    return;
  } else if constexpr (kEpi == kSwigluQ8) {
    // Every wave parks its sums in LDS as [token][feature] rows, gate
    // features [0, BM/2) and up features apart; then each thread takes whole
    // 32-feature blocks of one token: SwiGLU, the block's Q8_0 rounding and
    // one contiguous 64-byte store.  Rows hold BM/2 features as float4
    // quads, quad c of token t at slot 16 t' + (c ^ (t % 16)) within each
    // 16-quad group (conflict-free for 16 consecutive tokens on both sides).
    constexpr int kHalf = 16 * kWM * kTM / 2, kBN = 16 * kWN * kTN, kQuads = kHalf / 4;
    static_assert(kHalf % 64 == 0, "whole 16-quad groups per row");
    float4 *park = reinterpret_cast<float4 *>(smem);
    auto slot = [](int t, int c) { return (t * kQuads + (c & ~15)) + ((c & 15) ^ (t & 15)); };
#pragma unroll
    for (int a = 0; a < kTM; a++) {
      const int R = (wm * kTM + a) * 16 + 4 * (lane / 16);  // feature row within the tile
      const bool up = R >= kHalf;
      const int c = (R - (up ? kHalf : 0)) / 4;
#pragma unroll
      for (int b = 0; b < kTN; b++) {
        const int t = (wn * kTN + b) * 16 + lr;
        park[(up ? kBN * kQuads : 0) + slot(t, c)] =
            make_float4(acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]);
      }
    }
    __syncthreads();
    constexpr int kTasks = kBN * (kHalf / 32), kThreads = 64 * kWM * kWN;
    for (int task = tid; task < kTasks; task += kThreads) {
      const int t = task % kBN, blk = task / kBN;
      const int r = r0 + t, fb = f0 + 32 * blk;
      if (r >= g.M || fb >= F) continue;  // F % 32 == 0: whole blocks in or out
      float h[32];
      float m = 0.0f;
      bool bad = false;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float4 gv = park[slot(t, 8 * blk + q)];
        const float4 uv = park[kBN * kQuads + slot(t, 8 * blk + q)];
        const float gq[4] = {gv.x, gv.y, gv.z, gv.w}, uq[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float v = silu_fast(gq[i]) * uq[i];
          h[4 * q + i] = v;
          bad |= !finitef(v);
          m = fmaxf(m, fabsf(v));
        }
      }
      const Q8Scale sc = q8_scale_of(m);
      const float dh = h2f(sc.hd);
      bad |= !finitef(dh) || !finitef(sc.inv);
      uint32_t w[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint16_t lo = q8_value_h(q8_round(h[2 * i], sc.inv), dh);
        const uint16_t hi = q8_value_h(q8_round(h[2 * i + 1], sc.inv), dh);
        bad |= !finitef(h2f(lo)) || !finitef(h2f(hi));
        w[i] = lo | (uint32_t)hi << 16;
      }
      uint4 *dst = reinterpret_cast<uint4 *>(g.out16 + (size_t)r * F + fb);
#pragma unroll
      for (int i = 0; i < 4; i++) dst[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
      if (bad) atomicOr(&g.row_err[g.err_rows ? (int)g.err_rows[r] : r], kErrNonFinite);
    }
  } else if constexpr (kEpi == kSwigluF16) {
    // up waves (wm >= kWM/2) park their sums; the gate wave at wm - kWM/2
    // holds the matching gate sums in the same registers
    float *park = reinterpret_cast<float *>(smem);
    constexpr int kPair = kTM * kTN * 4;  // floats per lane per wave
    const int pair = (wm % (kWM / 2)) * kWN + wn;
    if (wm >= kWM / 2) {
#pragma unroll
      for (int a = 0; a < kTM; a++)
#pragma unroll
        for (int b = 0; b < kTN; b++)
#pragma unroll
          for (int i = 0; i < 4; i++) park[((pair * kPair) + (a * kTN + b) * 4 + i) * kWave + lane] = acc[a][b][i];
    }
    __syncthreads();
    if (wm >= kWM / 2) return;
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int r = r0 + (wn * kTN + b) * 16 + lr;
      if (r >= g.M) continue;
      bool bad = false;
#pragma unroll
      for (int a = 0; a < kTM; a++) {
        const int fb = f0 + (wm * kTM + a) * 16 + 4 * (lane / 16);
        uint16_t h[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float gv = acc[a][b][i];
          const float uv = park[((pair * kPair) + (a * kTN + b) * 4 + i) * kWave + lane];
          bad |= !finitef(gv) || !finitef(uv);
          h[i] = f2h(silu_fast(gv) * uv);
          bad |= !finitef(h2f(h[i]));
        }
        if (fb + 3 < F && F % 4 == 0) {
          *reinterpret_cast<uint2 *>(g.out16 + (size_t)r * F + fb) =
              make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (fb + i < F) g.out16[(size_t)r * F + fb + i] = h[i];
        }
      }
      if (bad) atomicOr(&g.row_err[g.err_rows ? (int)g.err_rows[r] : r], kErrNonFinite);
    }
  } else {
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int r = r0 + (wn * kTN + b) * 16 + lr;
      if (r >= g.M) continue;
      bool bad = false;
#pragma unroll
      for (int a = 0; a < kTM; a++) {
        const int fb = f0 + (wm * kTM + a) * 16 + 4 * (lane / 16);
        if (kEpi == kStore && fb < g.rope_rows) {  // query/key features back in source order
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float v = acc[a][b][i];
            bad |= !finitef(v);
            g.out[(size_t)r * g.ldo + rope_col(fb + i, g.rope_d)] = v;
          }
          continue;
        }
        float *p = g.out + (size_t)r * g.ldo + fb;
        if (fb + 3 < g.N && g.ldo % 4 == 0) {
          float4 v = make_float4(acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]);
          if (kEpi == kAccumulate) {
            const float4 q = *reinterpret_cast<const float4 *>(p);
            v = make_float4(q.x + v.x, q.y + v.y, q.z + v.z, q.w + v.w);
          }
          bad |= !finitef(v.x) || !finitef(v.y) || !finitef(v.z) || !finitef(v.w);
          *reinterpret_cast<float4 *>(p) = v;
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            if (fb + i >= g.N) continue;
            const float v = kEpi == kAccumulate ? p[i] + acc[a][b][i] : acc[a][b][i];
            bad |= !finitef(v);
            p[i] = v;
          }
        }
      }
      if (bad) atomicOr(&g.row_err[g.err_rows ? (int)g.err_rows[r] : r], kErrNonFinite);
    }
  }
}

template <int kType, bool kLo, int kWM, int kWN, int kTM, int kTN, int kR, int kEpi>
__global__ __launch_bounds__(64 * kWM * kWN) void k_gemm(Args g) {
  constexpr int kThreads = 64 * kWM * kWN;
  constexpr int kBM = 16 * kWM * kTM, kBN = 16 * kWN * kTN;
  constexpr int kWSlots = kBM * 4, kXSlots = kBN * 4;
  constexpr int kSlots = kWSlots + (kLo ? 2 : 1) * kXSlots;  // 16-byte slots per K step
  static_assert(kSlots % kThreads == 0, "whole loads per thread");
  constexpr int kPer = kSlots / kThreads;  // 16-byte loads per thread per K step
  static_assert(kR == 2 || kR == 4, "two or four K steps in flight (K / 32 a multiple of kR)");
  static_assert(kEpi != kSwigluF16 || kWM % 2 == 0, "gate and up waves in pairs");
  extern __shared__ __align__(16) uint4 smem[];
  u32x4 *lds = reinterpret_cast<u32x4 *>(smem);
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWN, wn = wave % kWN;
  const int nk = g.K / kBK;
  // feature rows of this workgroup: BM consecutive rows, or for SwiGLU BM/2
  // gate rows and the BM/2 matching up rows (F = N/2 apart)
  const int F = g.N / 2;
  const int2 tile = tile_of(g);
  if (tile.x < 0) return;
  const int fb = tile.x, rb = tile.y;
  const int f0 = fb * (kEpi == kSwigluF16 ? kBM / 2 : kBM);
  const int r0 = rb * kBN;
  // this thread's slots of a K step: source row and segment (rows past the
  // end clamp to the last; their results are never stored); successive K
  // steps are wstep (W) or kBK (X) elements apart
  const uint16_t *src[kPer];
  int step_of[kPer];
  const int wstep = g.w_tiled ? 4 * 16 * 8 : kBK;
#pragma unroll
  for (int i = 0; i < kPer; i++) {
    const int slot = (wave * kPer + i) * kWave + lane;
    if (slot < kWSlots) {
      const int row = slot >> 2, seg = (slot & 3) ^ ((row >> 1) & 3);
      int f = f0 + row;
      if (kEpi == kSwigluF16) f = row < kBM / 2 ? f0 + row : F + f0 + row - kBM / 2;
      f = min(f, g.N - 1);
      src[i] = g.w + (g.w_tiled ? ((size_t)(f / 16) * (g.K / 8) + seg) * 128 + (f % 16) * 8
                                : (size_t)f * g.K + seg * 8);
      step_of[i] = wstep;
    } else {
      const int xs = slot - kWSlots;
      const bool lo = kLo && xs >= kXSlots;
      const int row = (xs - (lo ? kXSlots : 0)) >> 2, seg = (slot & 3) ^ ((row >> 1) & 3);
      src[i] = (lo ? g.xlo : g.x) + (size_t)min(r0 + row, g.M - 1) * g.ldx + seg * 8;
      step_of[i] = kBK;
    }
  }
  // K steps ks .. ks + kR - 1 in flight: reg[ks % kR]; steps past the end
  // reload the last one (never used)
  u32x4 reg[kR][kPer];
#pragma unroll
  for (int j = 0; j < kR; j++)
#pragma unroll
    for (int i = 0; i < kPer; i++)
      reg[j][i] = *reinterpret_cast<const u32x4 *>(src[i] + (size_t)min(j, nk - 1) * step_of[i]);
#pragma unroll
  for (int i = 0; i < kPer; i++) lds[(wave * kPer + i) * kWave + lane] = reg[0][i];
  f32x4 acc[kTM][kTN];
#pragma unroll
  for (int a = 0; a < kTM; a++)
#pragma unroll
    for (int b = 0; b < kTN; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int seg = lane / 16, lr = lane % 16;
  // K step k0 + J (J a compile-time constant, so every register index is)
  auto step = [&](auto J, int k0) __attribute__((always_inline)) {
    constexpr int j = decltype(J)::value;
    const int ks = k0 + j;
    // step ks is in LDS half j % 2 (kR is even, so ks % 2 == j % 2); the
    // other half's readers (step ks - 1) are past this barrier
    __syncthreads();
    const uint4 *stage = smem + (j % 2) * kSlots;
    using frag = frag_t<kType>;
    frag af[kTM], bf[kTN], lf[kLo ? kTN : 1];
#pragma unroll
    for (int a = 0; a < kTM; a++) {
      const int R = (wm * kTM + a) * 16 + lr;
      af[a] = *reinterpret_cast<const frag *>(stage + R * 4 + (seg ^ ((R >> 1) & 3)));
    }
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int R = (wn * kTN + b) * 16 + lr;
      bf[b] = *reinterpret_cast<const frag *>(stage + kWSlots + R * 4 + (seg ^ ((R >> 1) & 3)));
      if constexpr (kLo)
        lf[b] = *reinterpret_cast<const frag *>(stage + kWSlots + kXSlots + R * 4 + (seg ^ ((R >> 1) & 3)));
    }
    // step ks + 1 into the other half, then step ks + kR into its registers
    constexpr int jn = (j + 1) % kR;
#pragma unroll
    for (int i = 0; i < kPer; i++) lds[((j + 1) % 2) * kSlots + (wave * kPer + i) * kWave + lane] = reg[jn][i];
    const int kc = min(ks + kR, nk - 1);
#pragma unroll
    for (int i = 0; i < kPer; i++) reg[j][i] = *reinterpret_cast<const u32x4 *>(src[i] + (size_t)kc * step_of[i]);
#pragma unroll
    for (int a = 0; a < kTM; a++)
#pragma unroll
      for (int b = 0; b < kTN; b++) {
        acc[a][b] = mfma(af[a], bf[b], acc[a][b]);
        if constexpr (kLo) acc[a][b] = mfma(af[a], lf[b], acc[a][b]);
      }
  };
  for (int k0 = 0; k0 < nk; k0 += kR) {
    step(std::integral_constant<int, 0>{}, k0);
    step(std::integral_constant<int, 1>{}, k0);
    if constexpr (kR == 4) {
      step(std::integral_constant<int, 2>{}, k0);
      step(std::integral_constant<int, 3>{}, k0);
    }
  }
  // the last step's readers are done before the LDS is reused by the epilogue
  __syncthreads();
  epilogue<kWM, kWN, kTM, kTN, kEpi>(g, acc, f0, r0, smem);
}

// ---------------------------------------------------------------------------
// Quantized weights (the packed-prefill regime over Q8_0 / Q5_0 / Q4_0
// models).  W stays in the exact matvecs' 16-row tiles: per (tile, block
// pair) lane l of a 64-lane slot row holds row l % 16, inputs 8 (l / 16) ..
// + 8 of both blocks (Q8: 16 bytes, Q4: 8), which is the MFMA's own operand
// order.  Each ring stage covers one block pair (K advances 64): every thread
// loads its (row, input group) slot and the row's two block scales, and on
// the way into LDS turns each value into binary16 times its block's scale,
// rounded once (int8 and nibble values are exact in binary16, and the
// product of an 8-bit value and an 11-bit scale is exact in f32 before the
// rounding).  The reference multiplies Q8_0 activations with the int8
// weights per block and applies both scales in an f32 chain
// (quant.rs:245-292).  The operand rows here hold the same Q8_0 activation
// values, q * f16(d) as binary16 (their producers round each row block as
// the reference does; the SwiGLU epilogue kSwigluQ8 too), so the regime keeps
// the reference's activation rounding; its tolerance covers the binary16
// rounding of q * d on both sides and the f32 sums in MFMA order.
//
// LDS per stage: BM weight rows and BN token rows of 64 binary16 inputs
// (eight 16-byte segments each); segment s of row R sits at slot
// 8R + (s ^ (R & 7)), so the eight rows that one pass of a 16-byte LDS
// access serves (R..R+7 of one segment, in the fragment reads and the weight
// stores alike) sit at eight distinct positions modulo 128 bytes, free of
// bank conflicts.  ((R >> 1) & 7 paired rows R and R + 1: a sixth of the
// LDS cycles were conflicts.)
// ---------------------------------------------------------------------------
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int kQ>
struct QSlot;
template <>
struct QSlot<8> {
  typedef u32x4 type;
  static constexpr int kBytes = 16, kPair = 1024;  // per lane / per tile, one block pair
};
template <>
struct QSlot<4> {
  typedef u32x2 type;
  static constexpr int kBytes = 8, kPair = 512;
};

// Eight signed values (bytes of lo then hi, in order) times their block
// scale as binary16.
__device__ __forceinline__ f16x8 scale8(uint32_t lo, uint32_t hi, _Float16 d) {
  f16x8 v;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[j] = (_Float16)(short)(signed char)(lo >> (8 * j));
    v[4 + j] = (_Float16)(short)(signed char)(hi >> (8 * j));
  }
  return v * d;
}

__device__ __forceinline__ int qswz(int R) { return R & 7; }

template <int kWM, int kWN, int kTM, int kTN, int kEpi>
constexpr int lds_bytes_q() {
  constexpr int ring = 2 * (16 * kWM * kTM + 16 * kWN * kTN) * 128;
  constexpr int park = kEpi == kSwigluQ8 ? 16 * kWM * kTM * 16 * kWN * kTN * 4 : 0;
  return ring > park ? ring : park;
}

template <int kQ, int kWM, int kWN, int kTM, int kTN, int kR, int kEpi>
__global__ __launch_bounds__(64 * kWM * kWN) void k_gemm_q(Args g) {
  constexpr int kThreads = 64 * kWM * kWN;
  constexpr int kBM = 16 * kWM * kTM, kBN = 16 * kWN * kTN;
  constexpr int kWLoads = kBM * 4, kXLoads = kBN * 8;  // per stage
  static_assert(kWLoads % kThreads == 0 && kXLoads % kThreads == 0, "whole loads per thread");
  constexpr int kPW = kWLoads / kThreads, kPX = kXLoads / kThreads;
  constexpr int kStage = (kBM + kBN) * 8;  // 16-byte LDS slots per stage
  static_assert(kR == 2 || kR == 4, "two or four block pairs in flight");
  constexpr bool kGlu = kEpi == kSwigluF16 || kEpi == kSwigluQ8;
  static_assert(!kGlu || kWM % 2 == 0, "gate and up waves in pairs");
  using QT = typename QSlot<kQ>::type;
  extern __shared__ __align__(16) uint4 smem[];
  f16x8 *lds = reinterpret_cast<f16x8 *>(smem);
  u32x4 *ldsx = reinterpret_cast<u32x4 *>(smem);
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int wm = wave / kWN, wn = wave % kWN;
  const int nk = g.K / 64;
  const int2 tile = tile_of(g);
  if (tile.x < 0) return;
  const int f0 = tile.x * (kGlu ? kBM / 2 : kBM);
  const int r0 = tile.y * kBN;
  // weight slots: a 64-slot row of the load index is one 16-row tile of the
  // workgroup (tl), lane = the tile's own lane order; tiles past the end
  // clamp to the last (their results are never stored)
  const char *qsrc[kPW];
  const uint16_t *dsrc[kPW];
  int wdst[kPW];  // LDS row of the slot
  const int last = kGlu ? (g.N / 2 - 1) / 16 : (g.N - 1) / 16;
#pragma unroll
  for (int i = 0; i < kPW; i++) {
    const int tl = wave * kPW + i;
    int dt;
    if (kGlu) {
      const bool up = tl >= kBM / 32;
      dt = 2 * min(f0 / 16 + tl - (up ? kBM / 32 : 0), last) + (up ? 1 : 0);
    } else {
      dt = min(f0 / 16 + tl, last);
    }
    qsrc[i] = static_cast<const char *>(g.qs) + (size_t)dt * (g.nbp / 2) * QSlot<kQ>::kPair +
              lane * QSlot<kQ>::kBytes;
    dsrc[i] = g.ds + (size_t)dt * g.nbp * 16 + lane % 16;
    wdst[i] = tl * 16 + lane % 16;
  }
  const uint16_t *xsrc[kPX];
  int xdst[kPX];
#pragma unroll
  for (int i = 0; i < kPX; i++) {
    const int slot = (wave * kPX + i) * kWave + lane, row = slot >> 3, sg = slot & 7;
    xsrc[i] = g.x + (size_t)min(r0 + row, g.M - 1) * g.ldx + sg * 8;
    xdst[i] = kBM * 8 + row * 8 + (sg ^ qswz(row));
  }
  QT qreg[kR][kPW];
  uint32_t dreg[kR][kPW];
  u32x4 xreg[kR][kPX];
  auto load = [&](int j, int kc) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPW; i++) {
      qreg[j][i] = *reinterpret_cast<const QT *>(qsrc[i] + (size_t)kc * QSlot<kQ>::kPair);
      dreg[j][i] = (uint32_t)dsrc[i][kc * 32] | (uint32_t)dsrc[i][kc * 32 + 16] << 16;
    }
#pragma unroll
    for (int i = 0; i < kPX; i++) xreg[j][i] = *reinterpret_cast<const u32x4 *>(xsrc[i] + (size_t)kc * 64);
  };
  // ring registers j -> LDS stage st (dequantizing the weights)
  auto store = [&](int j, int st) __attribute__((always_inline)) {
    const int base = st * kStage;
#pragma unroll
    for (int i = 0; i < kPW; i++) {
      const int R = wdst[i], sw = qswz(R), kg = lane / 16;
      uint32_t b0lo, b0hi, b1lo, b1hi;
      if constexpr (kQ == 8) {
        b0lo = qreg[j][i][0], b0hi = qreg[j][i][1], b1lo = qreg[j][i][2], b1hi = qreg[j][i][3];
      } else {
        const long a = q4_operand(qreg[j][i][0]), b = q4_operand(qreg[j][i][1]);
        b0lo = (uint32_t)a, b0hi = (uint32_t)((unsigned long)a >> 32);
        b1lo = (uint32_t)b, b1hi = (uint32_t)((unsigned long)b >> 32);
      }
      const _Float16 d0 = __builtin_bit_cast(_Float16, (uint16_t)(dreg[j][i] & 0xffffu));
      const _Float16 d1 = __builtin_bit_cast(_Float16, (uint16_t)(dreg[j][i] >> 16));
      lds[base + R * 8 + (kg ^ sw)] = scale8(b0lo, b0hi, d0);
      lds[base + R * 8 + ((4 + kg) ^ sw)] = scale8(b1lo, b1hi, d1);
    }
#pragma unroll
    for (int i = 0; i < kPX; i++) ldsx[base + xdst[i]] = xreg[j][i];
  };
#pragma unroll
  for (int j = 0; j < kR; j++) load(j, min(j, nk - 1));
  store(0, 0);
  f32x4 acc[kTM][kTN];
#pragma unroll
  for (int a = 0; a < kTM; a++)
#pragma unroll
    for (int b = 0; b < kTN; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int seg = lane / 16, lr = lane % 16;
  // the last round of kR steps may run past the end (K / 64 need not be a
  // multiple of kR): those steps do nothing (ks is the same in every thread)
  auto step = [&](auto J, int k0) __attribute__((always_inline)) {
    constexpr int j = decltype(J)::value;
    const int ks = k0 + j;
    if (ks >= nk) return;
    __syncthreads();
    const f16x8 *stage = lds + (j % 2) * kStage;
    f16x8 af[2][kTM], bf[2][kTN];
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
      for (int a = 0; a < kTM; a++) {
        const int R = (wm * kTM + a) * 16 + lr;
        af[h][a] = stage[R * 8 + ((4 * h + seg) ^ qswz(R))];
      }
#pragma unroll
      for (int b = 0; b < kTN; b++) {
        const int R = (wn * kTN + b) * 16 + lr;
        bf[h][b] = stage[kBM * 8 + R * 8 + ((4 * h + seg) ^ qswz(R))];
      }
    }
    store((j + 1) % kR, (j + 1) % 2);
    load(j, min(ks + kR, nk - 1));
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int a = 0; a < kTM; a++)
#pragma unroll
        for (int b = 0; b < kTN; b++) acc[a][b] = mfma(af[h][a], bf[h][b], acc[a][b]);
  };
  for (int k0 = 0; k0 < nk; k0 += kR) {
    step(std::integral_constant<int, 0>{}, k0);
    step(std::integral_constant<int, 1>{}, k0);
    if constexpr (kR == 4) {
      step(std::integral_constant<int, 2>{}, k0);
      step(std::integral_constant<int, 3>{}, k0);
    }
  }
  __syncthreads();
  epilogue<kWM, kWN, kTM, kTN, kEpi>(g, acc, f0, r0, smem);
}

}  // namespace gemm
}  // namespace cohx
