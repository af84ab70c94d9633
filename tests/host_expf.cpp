// Host check of the expf restatement the GPU kernels use (csrc/expf.h):
// compares cohx::exp_f32_tab with the C library's expf bit for bit over the
// whole binary32 range at the given stride (both signs, subnormals,
// infinities and NaNs included), plus every float in the softmax range
// [-104, 0] at a finer stride.  Prints the number of mismatches and the
// first few.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "expf.h"

static const uint64_t kTab[32] = COHX_EXP2_TABLE;

static float from_bits(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

static unsigned long check(uint64_t lo, uint64_t hi, uint32_t stride, unsigned long *n) {
  unsigned long bad = 0;
  for (uint64_t u = lo; u <= hi; u += stride) {
    const float x = from_bits((uint32_t)u);
    const float a = cohx::exp_f32_tab(x, kTab), b = expf(x);
    ++*n;
    const bool both_nan = a != a && b != b;
    if (!both_nan && cohx::ef_bits(a) != cohx::ef_bits(b)) {
      if (bad < 4) printf("x=%a: got %a want %a\n", x, a, b);
      bad++;
    }
  }
  return bad;
}

int main(int argc, char **argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 0) : 1;
  unsigned long n = 0, bad = 0;
  bad += check(0x00000000u, 0xffffffffu, stride * 4 + 1, &n);  // everything, coarse
  bad += check(0x80000000u, 0xc2d00000u, stride, &n);          // [-104, -0]: softmax, SiLU
  bad += check(0x00000000u, 0x42b17218u, stride, &n);          // [0, ln(FLT_MAX)]
  printf("checked %lu mismatches %lu\n", n, bad);
  return bad != 0;
}
