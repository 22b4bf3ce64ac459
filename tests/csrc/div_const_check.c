/* Exhaustive check of the kernels' division by a float32 constant c:
 *   (float)((double)x * (1.0 / (double)c))  ==  x / c  (IEEE float32, round to nearest)
 * for all 2^32 float32 bit patterns x. The right side is formed as the float64 quotient
 * rounded to float32, which is the correctly rounded float32 quotient (float64 carries
 * more than 2 * 24 + 2 bits). Any NaN equals any NaN. Prints the mismatch count; exits 1
 * on any mismatch. Usage: div_const_check <c as a C float literal, e.g. 0x1.19999ap+0>. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

static uint32_t to_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

int main(int argc, char** argv) {
  if (argc != 2) return 2;
  const float c = strtof(argv[1], NULL);
  const double inv_c = 1.0 / (double)c;
  unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long i = 0; i < (1ll << 32); ++i) {
    const float x = from_bits((uint32_t)i);
    const float want = (float)((double)x / (double)c);
    const float got = (float)((double)x * inv_c);
    if (to_bits(got) != to_bits(want) && !(isnan(got) && isnan(want))) ++bad;
  }
  printf("c=%a mismatches=%llu\n", c, bad);
  return bad != 0;
}
