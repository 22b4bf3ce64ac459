/* Checks of the kernels' division through a shared float64 reciprocal (DivRecip):
 *   q = (float)((double)a * (1.0 / (double)d))
 * 1. all 2^32 float32 bit patterns: the key (bits << 1) - 2 (uint32) is <= 0xFFFFFC exactly
 *    for the nonzero subnormals;
 * 2. random operand pairs over the whole exponent range, special values included, plus
 *    quotients placed on and next to float32 rounding midpoints (subnormal and normal):
 *    whenever q is not a nonzero subnormal it equals IEEE a / d, bit for bit (any NaN
 *    equals any NaN);
 * 3. exact subnormal midpoints a / d = (2j + 1) 2^-150 exist where q differs from IEEE
 *    a / d, which is why a subnormal q is recomputed.
 * Prints counts; exits 1 when 1 or 2 fails or 3 finds no such case. Usage: div_recip_check <pairs>. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t to_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static uint64_t s_state = 0x9E3779B97F4A7C15ull;
static uint64_t next64(void) { /* splitmix64 */
  uint64_t z = (s_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static int is_subnormal_nonzero(float q) { uint32_t b = to_bits(q) & 0x7FFFFFFFu; return b != 0 && b <= 0x7FFFFFu; }
static float fast_div(float a, float d) { return (float)((double)a * (1.0 / (double)d)); }
static int same(float x, float y) { return to_bits(x) == to_bits(y) || (isnan(x) && isnan(y)); }

int main(int argc, char** argv) {
  const long long pairs = argc > 1 ? atoll(argv[1]) : 20000000;
  /* 1: the key, exhaustively */
  unsigned long long key_bad = 0;
#pragma omp parallel for reduction(+ : key_bad) schedule(static)
  for (long long i = 0; i < (1ll << 32); ++i) {
    const uint32_t b = (uint32_t)i;
    const uint32_t key = (b << 1) - 2u;
    if ((key <= 0x00FFFFFCu) != is_subnormal_nonzero(from_bits(b))) ++key_bad;
  }
  /* 2: random pairs */
  unsigned long long bad = 0, flagged = 0, checked = 0;
  const float specials[] = {0.0f, -0.0f, INFINITY, -INFINITY, NAN, 1e-45f, -1e-45f, 1.1754942e-38f, 1.17549435e-38f,
                            3.4028235e38f, -3.4028235e38f, 1.0f, -1.0f, 2.0f, 0.5f};
  const int ns = sizeof(specials) / sizeof(specials[0]);
  for (long long t = 0; t < pairs; ++t) {
    const uint64_t r = next64();
    float a = from_bits((uint32_t)r), d = from_bits((uint32_t)(r >> 32));
    const int mode = (int)(t % 8);
    if (mode == 1) a = specials[(r >> 5) % ns];
    if (mode == 2) d = specials[(r >> 9) % ns];
    if (mode >= 3 && mode <= 5) {            /* operands of moderate size: quotients near 1 */
      a = ldexpf(1.0f + (float)((r >> 8) & 0xFFFFFF) / 16777216.0f, (int)((r >> 40) % 40) - 20);
      d = ldexpf(1.0f + (float)((r >> 16) & 0xFFFFFF) / 16777216.0f, (int)((r >> 48) % 40) - 20);
      if (r & 1) a = -a;
    }
    if (mode >= 6) {                          /* a = m * d for a float32 midpoint m, rounded to float32 */
      const double m = ldexp((double)(2 * ((r >> 8) & 0x7FFFFF) + 1), (int)((r >> 40) % 300) - 175);
      const double dd = ldexp(1.0 + (double)((r >> 16) & 0xFFF) / 4096.0, (int)((r >> 52) % 60) - 30);
      d = (float)dd;
      a = (float)(m * (double)d);
    }
    const float q = fast_div(a, d), want = a / d;
    if (is_subnormal_nonzero(q)) { ++flagged; continue; }
    ++checked;
    if (!same(q, want)) { if (bad < 5) printf("mismatch a=%a d=%a q=%a want=%a\n", a, d, q, want); ++bad; }
  }
  /* 3: exact subnormal midpoints that the product rounds the wrong way */
  unsigned long long wrong_midpoints = 0;
  for (uint32_t dodd = 3; dodd < 4096; dodd += 2) {
    for (int j = 0; j < 64; ++j) {
      for (int e = 1; e < 8; ++e) {
        const float d = ldexpf((float)dodd, e);                 /* odd significand, not a power of 2 */
        const double m = ldexp((double)(2 * j + 1), -150);      /* a subnormal midpoint */
        const double ad = m * (double)d;
        const float a = (float)ad;
        if ((double)a != ad) continue;                         /* need a = m * d exactly */
        const float q = fast_div(a, d), want = a / d;
        if (!same(q, want)) {
          ++wrong_midpoints;
          if (!is_subnormal_nonzero(q)) { printf("unflagged midpoint error a=%a d=%a\n", a, d); ++bad; }
        }
      }
    }
  }
  printf("key_mismatches=%llu pairs_checked=%llu flagged_subnormal=%llu mismatches=%llu wrong_midpoints=%llu\n",
         key_bad, checked, flagged, bad, wrong_midpoints);
  return (key_bad == 0 && bad == 0 && wrong_midpoints > 0) ? 0 : 1;
}
