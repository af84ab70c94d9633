// Host check of the log1pf restatement used by the GPU softplus: compares
// cohx::log1p_f32 with the C library's log1pf bit for bit over every float
// in [0, 1] at the given stride (the arguments softplus produces) and over
// every float in (-1, 0) and (1, 2^64) at a coarser stride.  Prints the
// number of mismatches and the first few.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "log1pf.h"

static unsigned long check(uint32_t lo, uint32_t hi, uint32_t stride, unsigned long *n) {
  unsigned long bad = 0;
  for (uint64_t u = lo; u <= hi; u += stride) {
    const float x = cohx::l1p_float((uint32_t)u);
    const float a = cohx::log1p_f32(x), b = log1pf(x);
    ++*n;
    if (cohx::l1p_bits(a) != cohx::l1p_bits(b)) {
      if (bad < 4) printf("x=%a: got %a want %a\n", x, a, b);
      bad++;
    }
  }
  return bad;
}

int main(int argc, char **argv) {
  const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], 0, 0) : 1;
  unsigned long n = 0, bad = 0;
  bad += check(0x00000000u, 0x3f800000u, stride, &n);           // [0, 1]
  bad += check(0x80000001u, 0xbf7fffffu, stride * 8, &n);       // (-1, 0)
  bad += check(0x3f800001u, 0x5f800000u, stride * 8, &n);       // (1, 2^64]
  printf("checked %lu mismatches %lu\n", n, bad);
  return bad != 0;
}
