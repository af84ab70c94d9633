// Device helpers shared by the step kernels (gfx950, wave64).
//
// Everything here is compiled with -ffp-contract=off: the engine's float
// semantics (crates/coheryn-engine/src/cpu.rs, quant.rs) never fuse a*b+c
// except where the Rust source calls mul_add, which these kernels spell fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "expf.h"

namespace cohx {

constexpr int kWave = 64;
constexpr int kPage = 16;         // tokens per KV page
constexpr int kChunk = 128;       // tokens per attention work item
constexpr int kMaxGroup = 8;      // q heads per kv head handled by one work item

// Row error bits (per packed row); folded into per-lane statuses on the host.
constexpr uint32_t kErrNonFinite = 1u;  // Error::invalid (non-finite value)
constexpr uint32_t kErrScale = 2u;      // Error::invalid (activation scale overflow)
constexpr uint32_t kErrPage = 4u;       // Error::resource (slot outside the page table)

typedef int v4i __attribute__((ext_vector_type(4)));

// glibc-identical expf (expf.h); the table in constant memory for kernels
// that do not stage it in LDS.
__constant__ static const uint64_t kExp2Tab[32] = COHX_EXP2_TABLE;
__device__ __forceinline__ float exp_f32(float x) { return exp_f32_tab(x, kExp2Tab); }

// binary16 <-> binary32 (round to nearest even; the `half` crate contract).
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ bool finitef(float v) { return __builtin_isfinite(v); }

// Orderable key of (value, row): larger value wins, then the lower row
// (greedy sampling keeps the first maximum, sampling.rs:160-173); -0 ties +0.
__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
  if (v == 0.0f) v = 0.0f;
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)row);
}

// Empty asm that takes each value as a VGPR operand: every value is live and
// computed at this point, which fixes the issue order of a group (the
// scheduler would otherwise chain every f64 triple through one temporary).
template <typename T, int kN>
__device__ __forceinline__ void pin_vgprs(T (&v)[kN]) {
#pragma unroll
  for (int i = 0; i < kN; i++) asm volatile("" : "+v"(v[i]));
}

// Rust `f as i8` (saturating; NaN -> 0).
__device__ __forceinline__ int8_t sat_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v;
}

// Q8_0 activation rounding (QuantizedInput::prepare, quant.rs:193-213) of a
// block whose largest magnitude is m: d = m/127, inv = 1/d (0 when d == 0),
// stored scale f16(d), value q = round-half-away(x*inv) as i8.
struct Q8Scale {
  float inv;
  uint16_t hd;  // the stored binary16 scale
};
__device__ __forceinline__ Q8Scale q8_scale_of(float m) {
  const float d = m / 127.0f;
  return Q8Scale{d == 0.0f ? 0.0f : 1.0f / d, f2h(d)};
}
__device__ __forceinline__ int8_t q8_round(float v, float inv) { return sat_i8(roundf(v * inv)); }
// The value the reference's dot product multiplies for q, q * f16(d), as
// binary16 (q * d is exact in f32; one rounding).
__device__ __forceinline__ uint16_t q8_value_h(int8_t q, float dh) { return f2h((float)q * dh); }

// Wave-level reductions (butterfly: every lane ends with the result; the
// combination order is fixed, so results are deterministic).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
// Max over aligned groups of 32 lanes.
__device__ __forceinline__ float half_max_f32(float v) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Block reduction of one f64 per thread, fixed order; all threads get the sum.
template <int kThreads>
__device__ __forceinline__ double block_sum_f64(double v, double *scratch) {
  constexpr int kWaves = kThreads / kWave;
  v = wave_sum_f64(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) scratch[w] = v;
  __syncthreads();
  double total = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; i++) total += scratch[i];
  return total;
}
template <int kThreads>
__device__ __forceinline__ float block_max_f32(float v, float *scratch) {
  constexpr int kWaves = kThreads / kWave;
  v = wave_max_f32(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x % kWave) == 0) scratch[w] = v;
  __syncthreads();
  float m = scratch[0];
#pragma unroll
  for (int i = 1; i < kWaves; i++) m = fmaxf(m, scratch[i]);
  return m;
}

// ---------------------------------------------------------------------------
// Q8 tile layout shared by weights (A operand, 16 matrix rows per tile) and
// activations (B operand, 16 batch rows per tile).  For tile t, 32-element
// block b (nbp = blocks rounded up to even) and lane l of a wave:
//   bytes  ((t*(nbp/2) + b/2)*64 + l)*16 + (b%2)*8 + j,  j < 8
// hold row t*16 + l%16, elements b*32 + (l/16)*8 + j — the per-lane operand
// of v_mfma_i32_16x16x32_i8, two blocks per 16-byte lane load.
// Block scales (binary16) sit at (t*nbp + b)*16 + row%16.
// ---------------------------------------------------------------------------
// KV pages.  A page holds kPage consecutive tokens of one sequence; per layer
// the pool is [page][kv_head][...] with kPage * D floats per (page, head).
// V rows are token-major: token o of the page, element j at o * D + j, so a
// wave with lane = element reads one row per instruction.  K is stored
// element-quad-major: [D/4][kPage][4], so with one thread per token the
// float4 of elements 4q..4q+3 of a page's 16 tokens are 256 contiguous bytes,
// and each wave-wide K load covers whole cache lines exactly once.  The quads
// are rotated by the page's place in its sequence (lpage = position / kPage)
// and the head: quad q at slot (q + lpage * NKV + head) % (D/4), so waves
// that read quad q of different pages at the same time spread over all cache
// channels instead of one 256-byte offset.  The rotation depends on the
// logical page, not the physical one, so copying a page (copy-on-write) or
// sharing it between sequences at the same positions keeps its meaning.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint32_t k_rot(uint32_t lpage, int g, int NKV, int D) {
  return (lpage * (uint32_t)NKV + (uint32_t)g) % (uint32_t)(D / 4);
}
__host__ __device__ __forceinline__ size_t k_at(size_t page, uint32_t lpage, int g, int NKV, int off, int j,
                                                int D) {
  const size_t slot = ((size_t)(j / 4) + k_rot(lpage, g, NKV, D)) % (size_t)(D / 4);
  return (page * (size_t)NKV + (size_t)g) * (size_t)(kPage * D) + slot * (kPage * 4) + (size_t)off * 4 +
         (size_t)(j % 4);
}
__host__ __device__ __forceinline__ size_t v_at(size_t page, int g, int NKV, int off, int j, int D) {
  return ((page * (size_t)NKV + (size_t)g) * kPage + (size_t)off) * (size_t)D + (size_t)j;
}

// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ size_t q8_byte(size_t tile, int nbp, int b, int lane, int j) {
  return ((tile * (size_t)(nbp / 2) + (size_t)(b / 2)) * 64 + (size_t)lane) * 16 +
         (size_t)(b % 2) * 8 + (size_t)j;
}
__host__ __device__ __forceinline__ size_t q8_scale(size_t tile, int nbp, int b, int row16) {
  return (tile * (size_t)nbp + (size_t)b) * 16 + (size_t)row16;
}

// Q4_0 weights keep 4 bits per value in the same tile order: lane l holds the
// 8 values of k-group l/16 of row l%16 for blocks 2p and 2p+1 in 8 bytes
// (4 per block).  Byte k (0..3) of a block's word holds value k in its low
// nibble and value k+4 in its high nibble, so one AND and one shift yield the
// 8 operand bytes in order.  Scales use the Q8_0 scale layout.
__host__ __device__ __forceinline__ size_t q4_byte(size_t tile, int nbp, int b, int lane, int k) {
  return ((tile * (size_t)(nbp / 2) + (size_t)(b / 2)) * 64 + (size_t)lane) * 8 +
         (size_t)(b % 2) * 4 + (size_t)(k % 4);
}

// ---------------------------------------------------------------------------
// K-quant tiles (Q4_K / Q6_K weights as the A operand, Q8_K activations as
// the B operand).  The engine's K-format dot keeps eight integer sums per
// 256-element block, sum[i % 8] over element i (quant.rs:294-341).  So each
// block is stored as 8 lane-classes: class c holds elements c, c+8, ...,
// c+248, and its 32 values are exactly the K run of one
// v_mfma_i32_16x16x32_i8.  For tile t, block b (nb blocks per row), class c
// and lane l, the 8 bytes at ((t*nb + b)*8 + c)*512 + l*8 + j hold row
// t*16 + l%16, element c + 8*(8*(l/16) + j), as one int8 value (Q4_K 0..15,
// Q6_K -32..31; activations -128..127).
// Weight side data per (tile, block):
//  * scales: 64 dwords; lane l's dword at (t*nb + b)*64 + l holds in byte s
//    the integer scale of the 16-element sub-group 4*(l/16) + s of row l%16
//    (Q4_K: its 32-element group's 6-bit scale; Q6_K: the int8 scale), which
//    are exactly the sub-groups of the lane's 8 operand values (value j is in
//    sub-group 4*(l/16) + j/2);
//  * d and dmin (binary16) at (t*nb + b)*16 + row%16 (Q6_K: dmin = 0);
//  * mins: 8 bytes per row at ((t*nb + b)*16 + row%16)*8 (Q6_K: zeros).
// Activation side data per (batch tile, block): d (f32) at (t*nb + b)*16 +
// row%16 and the 16 sums of 16 consecutive values (int16) at
// ((t*nb + b)*16 + row%16)*16, as QuantizedInput stores them.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ size_t kq_byte(size_t tile, int nb, int b, int c, int lane, int j) {
  return (((tile * (size_t)nb + (size_t)b) * 8 + (size_t)c) * 64 + (size_t)lane) * 8 + (size_t)j;
}
__host__ __device__ __forceinline__ size_t kq_row(size_t tile, int nb, int b, int row16) {
  return (tile * (size_t)nb + (size_t)b) * 16 + (size_t)row16;
}

// One block's 4-byte word -> the 8 signed operand bytes (nibble - 8), as the
// low 64 bits of an MFMA A/B operand.  Bytewise (n | 0x80) - 8 never borrows
// across bytes; the final XOR removes the 0x80 bias.
__device__ __forceinline__ long q4_operand(uint32_t x) {
  const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
  const uint32_t a = ((lo | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  const uint32_t b = ((hi | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
  return (long)(((unsigned long)b << 32) | a);
}

}  // namespace cohx
