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
// 4R + (s ^ ((R >> 2) & 3)), so the 16 rows x 4 segments a wave reads for one
// operand spread over all banks.
//
// Epilogues: store or accumulate f32 rows (ldo), SwiGLU of a [gate | up]
// matrix into the down projection's binary16 operand (gate waves and their up
// partner waves hold the same positions; the up sums cross through LDS), and
// the argmax head keys.  Non-finite outputs set the row's error bit.
#pragma once
#include <type_traits>

#include "device.h"

namespace cohx {
namespace gemm {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;  // K per ring stage: one MFMA step

enum Epi { kStore = 0, kAccumulate = 1, kSwigluF16 = 2, kArgmax = 3 };
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
};

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
inline int tile_order(Args &g, int out_features, int bm, int bn) {
  g.nf = (out_features + bm - 1) / bm;
  g.nr = (g.M + bn - 1) / bn;
  const int tiles = g.nf * g.nr;
  g.per_xcd = (tiles + 7) / 8;
  const double wb = (double)bm * g.K, xb = (double)bn * g.K * (g.xlo ? 2 : 1);
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
      const int row = slot >> 2, seg = (slot & 3) ^ ((row >> 2) & 3);
      int f = f0 + row;
      if (kEpi == kSwigluF16) f = row < kBM / 2 ? f0 + row : F + f0 + row - kBM / 2;
      f = min(f, g.N - 1);
      src[i] = g.w + (g.w_tiled ? ((size_t)(f / 16) * (g.K / 8) + seg) * 128 + (f % 16) * 8
                                : (size_t)f * g.K + seg * 8);
      step_of[i] = wstep;
    } else {
      const int xs = slot - kWSlots;
      const bool lo = kLo && xs >= kXSlots;
      const int row = (xs - (lo ? kXSlots : 0)) >> 2, seg = (slot & 3) ^ ((row >> 2) & 3);
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
      af[a] = *reinterpret_cast<const frag *>(stage + R * 4 + (seg ^ ((R >> 2) & 3)));
    }
#pragma unroll
    for (int b = 0; b < kTN; b++) {
      const int R = (wn * kTN + b) * 16 + lr;
      bf[b] = *reinterpret_cast<const frag *>(stage + kWSlots + R * 4 + (seg ^ ((R >> 2) & 3)));
      if constexpr (kLo)
        lf[b] = *reinterpret_cast<const frag *>(stage + kWSlots + kXSlots + R * 4 + (seg ^ ((R >> 2) & 3)));
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

  if constexpr (kEpi == kArgmax) {
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
          h[i] = f2h((gv / (1.0f + exp_f32(-gv))) * uv);
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

}  // namespace gemm
}  // namespace cohx
