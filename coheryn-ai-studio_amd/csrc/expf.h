// expf for binary32 with the same results as glibc's expf on x86-64, which is
// what the engine's f32::exp calls on Linux (cpu.rs:74-78 SwiGLU, cpu.rs:133-210
// softmax).  Method: Szabolcs Nagy's exp2 table reduction (ARM
// optimized-routines, glibc >= 2.28 e_expf.c): x*32/ln2 = k + r, 2^(k/32)
// from a 32-entry table, a cubic in r, all in binary64, one final rounding.
// Table entries are asuint64(2^(i/32)) - (i<<47) with 2^(i/32) correctly
// rounded; the reduction uses fused multiply-adds, matching the FMA build
// that glibc selects on CPUs with FMA.  Plain C++ arithmetic, so the same
// text compiles for the GPU and for the host check against the C library
// (tests/host_expf.cpp).
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifndef COHX_HD
#ifdef __HIPCC__
#define COHX_HD __host__ __device__
#else
#define COHX_HD
#endif
#endif

#define COHX_EXP2_TABLE                                                                          \
  {0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,    \
   0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,    \
   0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,    \
   0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,    \
   0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,    \
   0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,    \
   0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,    \
   0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL}

namespace cohx {

COHX_HD inline uint32_t ef_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
COHX_HD inline uint64_t ed_bits(double x) {
  uint64_t u;
  memcpy(&u, &x, 8);
  return u;
}
COHX_HD inline double ed_from(uint64_t u) {
  double x;
  memcpy(&x, &u, 8);
  return x;
}

// expf with the 2^(i/32) table read from `tab` (on the GPU the constant
// table or a copy a kernel has staged in LDS: a per-lane indexed constant
// load is a memory round trip per call, an LDS read is not).
COHX_HD inline float exp_f32_tab(float x, const uint64_t *tab) {
  const uint32_t ux = ef_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 or nan
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = fma(inv_ln2_n, xd, shift);
  const uint64_t ki = ed_bits(kd);
  kd -= shift;
  const double r = fma(inv_ln2_n, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = ed_from(t);
  const double z = fma(c0, r, c1), r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace cohx
