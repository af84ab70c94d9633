// log1pf as glibc 2.35 computes it (sysdeps/ieee754/flt-32/s_log1pf.c, the
// fdlibm method: argument reduction to 1+f in [sqrt(2)/2, sqrt(2)) with a
// correction term c, s = f/(2+f), log(1+f) = f - (hfsq - s*(hfsq + R(s^2))),
// R a degree-7 odd-power polynomial, result k*ln2_hi + (... + k*ln2_lo)).
// The engine's softplus calls f32::ln_1p, which is that libm routine on Linux
// (qwen35/kernels.rs:22-24).  Plain C++ float arithmetic, so the same text
// compiles for the GPU and for a host check against the C library.  Defined
// for the non-negative arguments softplus produces (x = exp(-|y|) in [0, 1])
// and for every finite x > -1.
#pragma once
#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define COHX_HD __host__ __device__
#else
#define COHX_HD
#endif

namespace cohx {

COHX_HD inline uint32_t l1p_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
COHX_HD inline float l1p_float(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

COHX_HD inline float log1p_f32(float x) {
  const float ln2_hi = l1p_float(0x3f317180u), ln2_lo = l1p_float(0x3717f7d1u);
  const float Lp1 = l1p_float(0x3F2AAAABu), Lp2 = l1p_float(0x3ECCCCCDu),
              Lp3 = l1p_float(0x3E924925u), Lp4 = l1p_float(0x3E638E29u),
              Lp5 = l1p_float(0x3E3A3325u), Lp6 = l1p_float(0x3E1CD04Fu),
              Lp7 = l1p_float(0x3E178897u);
  const int32_t hx = (int32_t)l1p_bits(x), ax = hx & 0x7fffffff;
  int32_t k = 1, hu = 0;
  float f = 0.0f, c = 0.0f, u;
  if (hx < 0x3ed413d7) {                        // 1 + x < sqrt(2)+
    if (ax >= 0x3f800000) return l1p_float(0x7fc00000u);  // x <= -1 (unused here)
    if (ax < 0x31000000) {                      // |x| < 2^-29
      if (ax < 0x24800000) return x;            // |x| < 2^-54
      return x - x * x * 0.5f;
    }
    if (hx > 0 || hx <= (int32_t)0xbe95f61fu) { // -0.2929 < x < 0.41422
      k = 0;
      f = x;
      hu = 1;
    }
  } else if (hx >= 0x7f800000) {
    return x + x;
  }
  if (k != 0) {
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)l1p_bits(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // correction term
      c /= u;
    } else {
      u = x;
      hu = (int32_t)l1p_bits(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = l1p_float((uint32_t)hu | 0x3f800000u);  // normalize u
    } else {
      k += 1;
      u = l1p_float((uint32_t)hu | 0x3f000000u);  // normalize u/2
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  const float hfsq = 0.5f * f * f;
  if (hu == 0) {  // |f| < 2^-20
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += (float)k * ln2_lo;
      return (float)k * ln2_hi + c;
    }
    const float R = hfsq * (1.0f - 0.66666666666666666f * f);
    if (k == 0) return f - R;
    return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
  }
  const float s = f / (2.0f + f), z = s * s;
  const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

}  // namespace cohx
