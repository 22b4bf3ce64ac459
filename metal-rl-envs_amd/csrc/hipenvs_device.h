// Device-side building blocks shared by every hipenvs kernel: the counter RNG,
// deterministic float32 transcendentals, launch geometry and the C-ABI error
// plumbing. Compiled for gfx950 with -ffp-contract=off: every a*b+c below is a
// rounded multiply followed by a rounded add, exactly as numpy evaluates it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/hipenvs.h"

namespace hipenvs {

// ---------------------------------------------------------------------------
// Counter RNG: the PCG hash of Jarzynski & Olano (JCGT 2020), the generator of
// the reference's Metal kernels (cartpole_metal.py:39-51). Per-env stream
// base seed ^ (env * 0x9E3779B9) (cartpole_metal.py:89).
// ---------------------------------------------------------------------------
constexpr uint32_t kGolden = 0x9E3779B9u;
constexpr uint32_t kRowStride = 0x85EBCA6Bu;        // generic row offset (pendulum_aba_metal.py:111)
constexpr uint32_t kRowOff1 = 0x85EBCA6Bu;          // 4-row bodies (cartpole_metal.py:91-93)
constexpr uint32_t kRowOff2 = 0xC2B2AE35u;
constexpr uint32_t kRowOff3 = 0x27D4EB2Fu;
constexpr uint32_t kActionOffset = 0x165667B1u;     // in-kernel actions (no reference counterpart)
constexpr uint32_t kTorqueOffset = 0xD3A2646Cu;     // continuous torques (no reference counterpart)

__device__ __forceinline__ uint32_t pcg_hash(uint32_t v) {
  uint32_t s = v * 747796405u + 2891336453u;
  uint32_t w = ((s >> ((s >> 28u) + 4u)) ^ s) * 277803737u;
  return (w >> 22u) ^ w;
}

// float in [-bound, bound) from the top 24 bits of a hash (cartpole_metal.py:47-50):
// ((h >> 8) * 2^-24 * 2 - 1) * bound. Every step before the last multiply is exact,
// so the value is (m * 2^-23) * bound with m = (h >> 8) - 2^23 (|m| <= 2^23, exact in
// float32), and m * (bound * 2^-23) rounds the same real number: one convert, one multiply.
__device__ __forceinline__ float uniform_pm(uint32_t h, float bound) {
  return (float)((int32_t)(h >> 8) - 0x800000) * (bound * 0x1p-23f);
}

__device__ __forceinline__ uint32_t env_hash(uint32_t seed, uint32_t env) { return seed ^ (env * kGolden); }

__device__ __forceinline__ int32_t action_bit(uint32_t h) { return (int32_t)(pcg_hash(h + kActionOffset) >> 31); }

__device__ __forceinline__ int32_t action_uniform(uint32_t h, uint32_t m) {
  return (int32_t)(((pcg_hash(h + kActionOffset) >> 8) * m) >> 24);
}

// ---------------------------------------------------------------------------
// Deterministic float32 sin/cos/tanh. Built from IEEE operations only (no FMA,
// no hardware transcendental), so numpy reproduces every bit; the numpy twin
// and the derivation of every constant live with the CPU oracle. Accuracy vs
// float64: <= 1.5 ULP (sin, cos), <= 2.5 ULP (tanh).
// ---------------------------------------------------------------------------
namespace dm {
// pi/2 in four pieces of 12, 12, 12 and 24 significant bits: k*P1..k*P3 exact for |k| < 2^12.
constexpr float PIO2_1 = 0x1.92p+0f;
constexpr float PIO2_2 = 0x1.fb4p-12f;
constexpr float PIO2_3 = 0x1.444p-24f;
constexpr float PIO2_4 = 0x1.68c234p-39f;
constexpr float TWO_OVER_PI = 0x1.45f306p-1f;
// float64 fallback for |x| > 256: 33-bit head (exact products for |k| < 2^20) and tail.
constexpr double PIO2_1D = 0x1.921fb544p+0;
constexpr double PIO2_2D = 0x1.0b4611a626331p-34;
constexpr double TWO_OVER_PI_D = 0x1.45f306dc9c883p-1;
constexpr float SMALL_ARG = 256.0f;
// Taylor coefficients 1/n! rounded to float32.
constexpr float S3 = -0x1.555556p-3f, S5 = 0x1.111112p-7f, S7 = -0x1.a01a02p-13f, S9 = 0x1.71de3ap-19f;
constexpr float C2 = -0x1p-1f, C4 = 0x1.555556p-5f, C6 = -0x1.6c16c2p-10f, C8 = 0x1.a01a02p-16f,
                C10 = -0x1.27e4fcp-22f;
// ln 2 in a 16-bit head and a float32 tail; log2(e).
constexpr float LN2_HI = 0x1.62e4p-1f;
constexpr float LN2_LO = 0x1.7f7d1cp-20f;
constexpr float LOG2E = 0x1.715476p+0f;
constexpr float E2 = 0x1p-1f, E3 = 0x1.555556p-3f, E4 = 0x1.555556p-5f, E5 = 0x1.111112p-7f,
                E6 = 0x1.6c16c2p-10f, E7 = 0x1.a01a02p-13f, E8 = 0x1.a01a02p-16f;
constexpr float TANH_CLAMP = 10.0f;
}  // namespace dm

// sin and cos of a reduced argument r, |r| <= pi/4, by the Taylor polynomials.
__device__ __forceinline__ void sincos_poly(float r, float* sin_out, float* cos_out) {
  const float z = r * r;
  float sp = dm::S7 + z * dm::S9;
  sp = dm::S5 + z * sp;
  sp = dm::S3 + z * sp;
  *sin_out = r + (r * z) * sp;
  float cp = dm::C8 + z * dm::C10;
  cp = dm::C6 + z * cp;
  cp = dm::C4 + z * cp;
  cp = dm::C2 + z * cp;
  *cos_out = 1.0f + z * cp;
}

__device__ __forceinline__ void det_sincos(float x, float* sin_out, float* cos_out) {
  // float32 reduction, computed for every lane on an argument clamped into its range (so
  // no branch precedes it and independent work can overlap the loads that feed x) ...
  const bool small = fabsf(x) <= dm::SMALL_ARG;
  const float xs = small ? x : 0.0f;
  const float k = rintf(xs * dm::TWO_OVER_PI);
  float r = (((xs - k * dm::PIO2_1) - k * dm::PIO2_2) - k * dm::PIO2_3) - k * dm::PIO2_4;
  int q = (int)k & 3;
  if (!small) {  // ... and the float64 reduction for |x| > 256, inf and NaN
    const double xd = (double)x;
    const double kd = rint(xd * dm::TWO_OVER_PI_D);
    r = (float)((xd - kd * dm::PIO2_1D) - kd * dm::PIO2_2D);
    const double qd = kd - 4.0 * floor(kd * 0.25);
    q = (qd >= 0.0 && qd < 4.0) ? ((int)qd & 3) : 0;  // inf/NaN: quadrant 0, result NaN
  }
  float s, c;
  sincos_poly(r, &s, &c);
  const float a = (q & 1) ? c : s;
  const float b = (q & 1) ? s : c;
  *sin_out = (q & 2) ? -a : a;
  *cos_out = ((q + 1) & 2) ? -b : b;
}

// Deterministic float64 sin/cos, for the reference-precision legged step (the reference's
// numpy evaluates np.sin/np.cos on float64 arrays once its state has been promoted).
// Cody-Waite reduction by pi/2 in three float64 pieces (33 + 33 + 53 significant bits, so
// k * PIO2_D1 and k * PIO2_D2 are exact for |k| < 2^20), then the Taylor series of sin to
// r^19 and of cos to r^20 (coefficients 1/n! rounded to float64). Every argument takes the
// same operations; NaN and infinities give NaN. Within 1.7 ulp of the exact values for
// |x| < 2^20 pi/2.
namespace dm {
constexpr double PIO2_D1 = 0x1.921fb54400000p+0;
constexpr double PIO2_D2 = 0x1.0b4611a600000p-34;
constexpr double PIO2_D3 = 0x1.3198a2e037073p-69;
constexpr double TWO_OVER_PI_64 = 0x1.45f306dc9c883p-1;
constexpr double SIN64_C[9] = {-0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13,
                               0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33,
                               -0x1.ae7f3e733b81fp-41, 0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57};
constexpr double COS64_C[10] = {-0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
                                0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29,
                                -0x1.93974a8c07c9dp-37, 0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53,
                                0x1.e542ba4020225p-62};
}  // namespace dm

__device__ __forceinline__ void det_sincos64(double x, double* sin_out, double* cos_out) {
  const double k = __builtin_rint(x * dm::TWO_OVER_PI_64);
  const double r = ((x - k * dm::PIO2_D1) - k * dm::PIO2_D2) - k * dm::PIO2_D3;
  const double z = r * r;
  double sp = dm::SIN64_C[8];
#pragma unroll
  for (int i = 7; i >= 0; --i) sp = dm::SIN64_C[i] + z * sp;
  const double s = r + (r * z) * sp;
  double cp = dm::COS64_C[9];
#pragma unroll
  for (int i = 8; i >= 0; --i) cp = dm::COS64_C[i] + z * cp;
  const double c = 1.0 + z * cp;
  const double q = k - 4.0 * __builtin_floor(k * 0.25);  // 0..3 exactly for finite k; NaN otherwise
  *sin_out = (q == 0.0) ? s : (q == 1.0) ? c : (q == 2.0) ? -s : -c;
  *cos_out = (q == 0.0) ? c : (q == 1.0) ? -s : (q == 2.0) ? -c : s;
}

// det_sincos for arguments that are usually near zero (CartPole's pole angle). When every
// active lane of the wave has |x| <= 0.78, rint(x * 2/pi) is 0 on every lane, the reduction
// returns x itself (a zero of either sign gives the same sin and cos), and the quadrant is
// 0, so the polynomial alone returns det_sincos's bits. Otherwise the wave takes det_sincos.
// Lanes with `counts` false take no part in the vote, and their results are not det_sincos's
// when the wave takes the polynomial: for callers that discard those lanes' results.
__device__ __forceinline__ void det_sincos_near_zero(float x, float* sin_out, float* cos_out, bool counts = true) {
  if (__all(!counts || fabsf(x) <= 0.78f)) {
    sincos_poly(x, sin_out, cos_out);
  } else {
    det_sincos(x, sin_out, cos_out);
  }
}

// Whether every active lane of the wave has |x[i]| <= 0.78 for each of its K values (NaN
// counts as far): then det_sincos(x[i]) equals sincos_poly(x[i]) for all of them, for the
// reason given at det_sincos_near_zero. One vote for K arguments; a chain near rest (the
// pendulums' hanging equilibrium) passes it.
template <int K>
__device__ __forceinline__ bool wave_near_zero(const float* x) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < K; ++i) ok &= fabsf(x[i]) <= 0.78f;
  return __all(ok);
}

// det_sincos of K arguments; the polynomial alone when the wave's vote allows it.
template <int K>
__device__ __forceinline__ void det_sincos_all(const float* x, float* sin_out, float* cos_out) {
  if (wave_near_zero<K>(x)) {
#pragma unroll
    for (int i = 0; i < K; ++i) sincos_poly(x[i], &sin_out[i], &cos_out[i]);
  } else {
#pragma unroll
    for (int i = 0; i < K; ++i) det_sincos(x[i], &sin_out[i], &cos_out[i]);
  }
}

// Lane L's value of each 16-lane row of the wave, on every lane of that row (DPP
// row_newbcast:L): how a 16-lane group shares a value one of its lanes computed. Every lane
// of every row is written, so the destination needs no prior value (mov_dpp, not update_dpp
// with an initialised old value, which costs a v_mov per broadcast).
template <int L>
__device__ __forceinline__ float group_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + L, 0xF, 0xF, false));
}

// Lane L (< 8) of each 8-lane half of every 16-lane row, on every lane of that half: how an
// 8-lane group shares a value. Two DPP row broadcasts of v: lane L into the first half
// (banks 0 and 1), then lane 8 + L into the second (banks 2 and 3; the first half keeps
// what the first move wrote). Neither reads the other's result, so no wait states sit
// between them.
template <int L>
__device__ __forceinline__ float half_bcast(float v) {
  static_assert(L >= 0 && L < 8, "a lane of the 8-lane half");
  const int x = __float_as_int(v);
  const int lo = __builtin_amdgcn_mov_dpp(x, 0x150 + L, 0xF, 0x3, false);
  return __int_as_float(__builtin_amdgcn_update_dpp(lo, x, 0x150 + 8 + L, 0xF, 0xC, false));
}

// Lane L of each G-lane group (G = 4, 8 or 16) on every lane of that group; a 4-lane group
// is a DPP quad, broadcast by one quad_perm move.
template <int G, int L>
__device__ __forceinline__ float lane_bcast(float v) {
  static_assert(G == 4 || G == 8 || G == 16, "groups of 4, 8 or 16 lanes");
  if constexpr (G == 16) {
    return group_bcast<L>(v);
  } else if constexpr (G == 8) {
    return half_bcast<L>(v);
  } else {
    static_assert(L >= 0 && L < 4, "a lane of the quad");
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), L * 0x55, 0xF, 0xF, false));
  }
}

__device__ __forceinline__ float det_sin(float x) {
  float s, c;
  det_sincos(x, &s, &c);
  return s;
}

__device__ __forceinline__ float det_cos(float x) {
  float s, c;
  det_sincos(x, &s, &c);
  return c;
}

__device__ __forceinline__ float det_tanh(float x) {
  float a = fabsf(x);
  a = (a > dm::TANH_CLAMP) ? dm::TANH_CLAMP : a;  // NaN compares false and stays NaN
  const float y = a + a;
  const float k = rintf(y * dm::LOG2E);
  const float r = (y - k * dm::LN2_HI) - k * dm::LN2_LO;
  float p = dm::E7 + r * dm::E8;
  p = dm::E6 + r * p;
  p = dm::E5 + r * p;
  p = dm::E4 + r * p;
  p = dm::E3 + r * p;
  p = dm::E2 + r * p;
  p = r + (r * r) * p;
  const int ki = (k >= 0.0f && k <= 64.0f) ? (int)k : 0;
  const float two_k = __int_as_float((ki + 127) << 23);
  const float e = two_k * p + (two_k - 1.0f);
  const float t = e / (e + 2.0f);
  return copysignf(t, x);
}

// x / c for a float32 constant c, as one float64 product with inv_c = 1 / (double)c
// rounded once to float32. The float64 product is within 2^-52 (relative) of x / c, and
// a quotient of two float32 values never lies that close to a float32 rounding boundary
// without being on it, which it cannot be; so this equals the IEEE float32 quotient for
// every x, zeros, subnormals, infinities and NaN included. Each divisor used is also
// checked against IEEE division over all 2^32 float32 inputs by the test suite.
__device__ __forceinline__ float div_const(float x, double inv_c) { return (float)((double)x * inv_c); }

// Division by a divisor used many times, through its correctly rounded float64 reciprocal
// r = recip(d): q = RN32(RN64(a * r)). The float64 product is within 2^-52 (relative) of the
// exact a / d. A quotient of two float32 values that is not itself a midpoint of the float32
// grid lies at least 2^-49 (relative) from every midpoint (write a, d and the midpoint with
// 24-, 24- and 25-bit significands, the midpoint's odd, and compare integer numerators),
// and in the normal range it is never exactly on one. So q is the IEEE quotient whenever
// that quotient is normal, zero, infinite or NaN (special operands pass through 1 / d and
// the product as through IEEE division). Only a subnormal quotient can sit exactly on a
// midpoint, where the product may round either way. DivRecip marks a lane whose quotient
// came out nonzero subnormal (a compare and a select, no branch); its caller then redoes
// the computation with IEEE division (DivIEEE), a path these bodies never take in practice.
//
// recip(d) is IEEE 1.0 / (double)d, formed from the hardware float64 reciprocal estimate
// and two Newton steps, e = 1 - d r, r += r e (each one fused multiply-add): six
// instructions where the IEEE float64 division takes eleven. For d = +-0, +-inf or NaN the
// residual is NaN and the estimate (+-inf, +-0, NaN) is the answer. Equal to
// 1.0 / (double)d bit for bit for all 2^32 float32 d (hipenvs_sqrt_recip_check, run by the
// GPU tests), so the argument above holds unchanged.
__device__ __forceinline__ double recip(float d) {
  const double x = (double)d;
  const double r0 = __builtin_amdgcn_rcp(x);
  double e = __builtin_fma(-x, r0, 1.0);
  double r = __builtin_fma(r0, e, r0);
  e = __builtin_fma(-x, r, 1.0);
  r = __builtin_fma(r, e, r);
  return (e == e) ? r : r0;
}

// IEEE sqrtf(x), formed in float64 from the hardware reciprocal square root estimate r:
// g = x r, then one Newton step g += (r / 2)(x - g^2), rounded to float32; +-0 and +inf pass
// through, negative inputs and NaN give NaN. Nine instructions where the correctly rounded
// float32 expansion takes about sixteen. Equal to IEEE sqrtf bit for bit (NaN for NaN) for
// all 2^32 float32 x (hipenvs_sqrt_recip_check, run by the GPU tests).
__device__ __forceinline__ float sqrt_rn(float x) {
  const double d = (double)x;
  const double r = __builtin_amdgcn_rsq(d);
  const double g = d * r;
  const double e = __builtin_fma(-g, g, d);
  const float y = (float)__builtin_fma(0.5 * r, e, g);
  return __builtin_amdgcn_classf(x, 0x260) ? x : y;  // class bits 5, 6, 9: -0, +0, +inf
}

struct DivRecip {
  // Per lane, the least (bits << 1) - 2 over the quotients, in uint32 arithmetic: the shift
  // drops the sign, and the subtraction sends zero to the top, so a nonzero subnormal
  // (0 < |bits| <= 0x7FFFFF) maps to at most 0xFFFFFC and every other value above it. One
  // shift-add and one min per quotient, kept in a vector register.
  uint32_t least = 0xFFFFFFFFu;
  __device__ __forceinline__ float operator()(float a, float /*d*/, double r) {
    const float q = (float)((double)a * r);
    const uint32_t key = (__float_as_uint(q) << 1) - 2u;
    least = key < least ? key : least;
    return q;
  }
  __device__ __forceinline__ bool saw_subnormal() const { return least <= 0x00FFFFFCu; }
};

struct DivIEEE {
  __device__ __forceinline__ float operator()(float a, float d, double /*r*/) const { return a / d; }
};

// Per-step streams (an action or torque row read once, reward and done rows written once)
// move with non-temporal hints, so they do not displace the state rows that the next step
// reads back from the caches: 2.90 vs 3.31 us for the CartPole step at N = 2^18, 8.28 vs
// 9.08 us at 2^20. The state itself uses ordinary accesses.
template <class T>
__device__ __forceinline__ T stream_load(const T* p) {
  return __builtin_nontemporal_load(p);
}

template <class T>
__device__ __forceinline__ void stream_store(T v, T* p) {
  __builtin_nontemporal_store(v, p);
}

// NaN-propagating clamp, numpy's np.clip semantics.
__device__ __forceinline__ float clip(float v, float lo, float hi) {
  v = (v < lo) ? lo : v;
  return (v > hi) ? hi : v;
}

// ---------------------------------------------------------------------------
// Launch geometry and C-ABI plumbing.
// ---------------------------------------------------------------------------
constexpr int kBlock = 256;

void set_last_hip_error(int err);

constexpr int kMaxDevices = 64;

// The current device's index into per-device caches; HIPENVS_E_HIP (error recorded) when
// hipGetDevice fails, HIPENVS_E_ARG past kMaxDevices devices.
int current_device(int* dev);

// Compute units of the current device, queried once per device (the answer cannot change
// while the process runs); a negative status when the query fails.
int device_cus(int* cus);

// Populations up to this size run the fused ES rollouts with a lane group per member: 16
// members per CU, i.e. one four-member wave per SIMD.
inline int group_rollout_limit(int64_t* limit) {
  int cus = 0;
  const int status = device_cus(&cus);
  *limit = 16 * (int64_t)cus;
  return status;
}

// Resident 64-thread workgroups per CU of `kernel` on the current device, queried once per
// device for each kernel (Tag distinguishes the callers' caches); a negative status on failure.
template <class Tag, class Kernel>
int resident_blocks_per_cu(Kernel kernel, int* per_cu) {
  static int cache[kMaxDevices];  // 0: not yet queried; written once per device under the lock below
  static std::atomic<int> ready[kMaxDevices];
  static std::mutex lock;
  int dev = 0;
  const int status = current_device(&dev);
  if (status != HIPENVS_OK) return status;
  if (!ready[dev].load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> guard(lock);
    if (!ready[dev].load(std::memory_order_relaxed)) {
      int blocks = 0;
      const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 64, 0);
      if (e != hipSuccess) {
        set_last_hip_error((int)e);
        return HIPENVS_E_HIP;
      }
      cache[dev] = blocks > 0 ? blocks : 1;
      ready[dev].store(1, std::memory_order_release);
    }
  }
  *per_cu = cache[dev];
  return HIPENVS_OK;
}

inline unsigned grid_for(int64_t items, int block = kBlock) {
  return (unsigned)((items + block - 1) / block);
}

// Checks the launch just enqueued; returns HIPENVS_OK or HIPENVS_E_HIP.
inline int launch_status() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_hip_error((int)e);
    return HIPENVS_E_HIP;
  }
  return HIPENVS_OK;
}

inline hipStream_t as_stream(hipenvs_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace hipenvs
