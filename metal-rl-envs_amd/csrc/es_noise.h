// Antithetic Gaussian perturbations from the counter RNG, for ES generations that never
// materialise the (P, D) noise (the reference draws and stores it: es.py:218-222).
//
// Member pair m (members m and m + P/2) has key k = pcg(seed ^ pcg(m + kMemberSalt)).
// Weight pair j (weights 2j, 2j + 1) takes h1 = pcg(k + 2j * golden) and
// h2 = pcg(k + (2j + 1) * golden), and Box-Muller on 24-bit fixed point:
//   u1 = ((h1 >> 8) + 1) * 2^-24 in (0, 1],  t = h2 >> 8,
//   r = sqrt(-2 ln u1),  eps[2j] = r cos(2 pi t / 2^24),  eps[2j + 1] = r sin(...).
// Member m + P/2 carries -eps. ln, sin and cos below are float32 elementary operations
// (bit manipulation, one IEEE division, Horner polynomials with the Taylor coefficients)
// under -ffp-contract=off, so a numpy restatement reproduces every bit. Accuracy against
// float64 over every input: ln within 1.7 ulp, sin and cos within 1e-7 absolute.
#pragma once

#include "hipenvs_device.h"

namespace hipenvs {
namespace esn {

constexpr uint32_t kMemberSalt = 0x6A09E667u;

__device__ __forceinline__ uint32_t member_key(uint32_t seed, uint32_t m) {
  return pcg_hash(seed ^ pcg_hash(m + kMemberSalt));
}

// ln(n * 2^-24) for n in [1, 2^24]. n = m * 2^e with m in (sqrt(1/2), sqrt(2)] (exact),
// ln m = 2 atanh(s), s = (m - 1) / (m + 1), then k ln 2 in two pieces (k * LN2_HI exact).
__device__ __forceinline__ float ln_fixed24(uint32_t n) {
  const uint32_t bits = __float_as_uint((float)n);
  const int e = (int)(bits >> 23) - 127;
  float m = __uint_as_float((bits & 0x007FFFFFu) | 0x3F800000u);
  const bool big = m > 0x1.6a09e6p+0f;
  m = big ? m * 0.5f : m;
  const float k = (float)(e + (big ? 1 : 0) - 24);
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  const float poly = 0x1.555556p-1f + z * (0x1.99999ap-2f + z * (0x1.24924ap-2f + z * (0x1.c71c72p-3f +
                                                                                        z * 0x1.745d18p-3f)));
  const float ln_m = (s + s) + s * (z * poly);
  return k * 0x1.62e4p-1f + (k * 0x1.7f7d1cp-20f + ln_m);
}

__device__ __forceinline__ float sin_poly(float x) {
  const float z = x * x;
  return x + x * (z * (-0x1.555556p-3f + z * (0x1.111112p-7f + z * (-0x1.a01a02p-13f + z * 0x1.71de3ap-19f))));
}

__device__ __forceinline__ float cos_poly(float x) {
  const float z = x * x;
  return 1.0f + z * (-0x1p-1f + z * (0x1.555556p-5f + z * (-0x1.6c16c2p-10f + z * (0x1.a01a02p-16f +
                                                                                   z * -0x1.27e4fcp-22f))));
}

// sin and cos of 2 pi t / 2^24 for t in [0, 2^24): the octant from the top three bits,
// the angle within it as (f or 2^21 - f) * pi / 2^23 in [0, pi/4], then the quadrant's
// swaps and signs.
__device__ __forceinline__ void sincos_turn24(uint32_t t, float& s, float& c) {
  constexpr uint32_t kOctant = 1u << 21;
  const uint32_t octant = t >> 21, f = t & (kOctant - 1u);
  const bool odd = (octant & 1u) != 0u;
  const float phi = (float)(odd ? kOctant - f : f) * 0x1.921fb6p-22f;
  const float sp = sin_poly(phi), cp = cos_poly(phi);
  const float s_psi = odd ? cp : sp, c_psi = odd ? sp : cp;
  switch (octant >> 1) {
    case 0: s = s_psi; c = c_psi; break;
    case 1: s = c_psi; c = -s_psi; break;
    case 2: s = -s_psi; c = -c_psi; break;
    default: s = -c_psi; c = s_psi; break;
  }
}

// The standard-normal pair (eps[2j], eps[2j + 1]) of a member key.
__device__ __forceinline__ void gauss_pair(uint32_t key, uint32_t j, float& z0, float& z1) {
  const uint32_t h1 = pcg_hash(key + (2u * j) * kGolden);
  const uint32_t h2 = pcg_hash(key + (2u * j + 1u) * kGolden);
  const float r = __builtin_sqrtf(-2.0f * ln_fixed24((h1 >> 8) + 1u));
  float s, c;
  sincos_turn24(h2 >> 8, s, c);
  z0 = r * c;
  z1 = r * s;
}

// Member pairs per partial sum of the update: a multiple of 64 giving at most 256 partials.
__host__ __device__ constexpr int64_t chunk_members(int64_t half) {
  const int64_t blocks = (half + 64 * 256 - 1) / (64 * 256);
  return 64 * (blocks > 0 ? blocks : 1);
}

}  // namespace esn

// Population layouts written by launch_perturb.
enum PerturbLayout : int { kPerturbRows = 0, kPerturbColumns = 1 };

// theta + sigma * [eps; -eps] for p (even) members into out: rows (p, d) or columns (d, p).
// Arguments are checked by the caller.
int launch_perturb(const float* theta, int64_t d, int64_t p, uint32_t seed, float sigma, int layout, float* out,
                   hipStream_t s);

}  // namespace hipenvs
