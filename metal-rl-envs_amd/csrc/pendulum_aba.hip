// The K-link planar pendulum by Featherstone's articulated-body algorithm on
// MI355X: accelerations, the RK4 step of the reference (dt 0.02, discrete root
// torque) and the semi-implicit Euler step with a continuous root torque
// (dt 0.01), each one thread per environment with the chain in registers.
//
// The three passes follow pendulum_aba_np.py:30-99 operation by operation:
// outward link velocities; inward articulated inertia Ia = IA - U U^T / D and
// bias pa = p + Ia c + U u / D folded into the parent through X^T (.) X; outward
// accelerations with the base accelerating at -g; the running sum turns joint
// accelerations into absolute ones. Per link the kernel keeps cos/sin of the
// joint angle, the link velocity and U, u (9 floats); K is a template constant,
// and for K <= 16 every per-link array is indexed statically and lives in
// VGPRs/AGPRs.
//
// Algorithmic bytes per env-step: 2K floats in, 2K floats out, 4 B action or
// torque, 4 B reward, 1 B done = 16K + 9 B.

#include "hipenvs_device.h"

namespace hipenvs {
namespace aba {

constexpr float GRAVITY = 0x1.39999ap+3f;     // float32(9.8)
constexpr float DT = 0x1.47ae14p-6f;          // float32(0.02)
constexpr float DT_2 = 0x1.47ae14p-7f;        // float32(0.02 / 2)
constexpr float DT_6 = 0x1.b4e81cp-9f;        // float32(0.02 / 6)
constexpr float DT_EULER = 0x1.47ae14p-7f;    // float32(0.01)
constexpr float MAX_VEL = 0x1.f6a7a2p+4f;     // float32(10 * pi)
constexpr float RESET_BOUND = 0x1.99999ap-4f; // float32(0.1)
constexpr float TWO_PI = 0x1.921fb6p+2f;      // float32(2 * pi)
constexpr float PI = 0x1.921fb6p+1f;          // float32(pi)

constexpr double INV_TWO_PI = 1.0 / (double)TWO_PI;  // for div_const(x, .) == x / TWO_PI

__device__ __forceinline__ float wrap(float x) { return x - TWO_PI * floorf(div_const(x + PI, INV_TWO_PI)); }

// Per-link loops are unrolled (U = K), so every per-link array is a set of
// registers, except in the RK4 step past K = 16: its four chained evaluations no
// longer fit the register file, so there the loops stay rolled (U = 1) and the
// per-link arrays live in private (scratch) memory.

// Velocity-product bias p = v x* (I v) of a unit mass at (1, 0) (pendulum_aba_np.py:46-47).
__device__ __forceinline__ void own_bias(float w, float x, float y, float& p0, float& p1, float& p2) {
  const float f = w + y;
  p0 = x * f - y * x;
  p1 = (-w) * f;
  p2 = w * x;
}

// Absolute angular accelerations acc[K] from absolute angles th[K] and velocities om[K],
// dividing with Div: a link's eight quotients share its pivot D, whose float64 reciprocal
// is formed once in each pass.
template <int K, int U, class Div>
__device__ __forceinline__ void accelerations_with(const float* th, const float* om, float torque, float* acc,
                                                   Div& div) {
  float cs[K], sn[K], vw[K], vx[K], vy[K], U0[K], U1[K], U2[K], uu[K];
  // the joints' sin and cos, by one wave vote for all K joint angles
  {
    float q[K];
#pragma unroll U
    for (int i = 0; i < K; ++i) q[i] = (i == 0) ? th[0] : th[i] - th[i > 0 ? i - 1 : 0];
    det_sincos_all<K>(q, sn, cs);
  }
  // outward: link velocities in link frames (pendulum_aba_np.py:36-50)
  {
    float w = 0.0f, x = 0.0f, y = 0.0f;
#pragma unroll U
    for (int i = 0; i < K; ++i) {
      const int im = i > 0 ? i - 1 : 0;
      const float qd = (i == 0) ? om[0] : om[i] - om[im];
      const float xy = (i == 0) ? (y + w * 0.0f) : (y + w);
      const float nw = w + qd;
      const float nx = cs[i] * x + sn[i] * xy;
      const float ny = (-sn[i]) * x + cs[i] * xy;
      vw[i] = nw;
      vx[i] = nx;
      vy[i] = ny;
      w = nw;
      x = nx;
      y = ny;
    }
  }
  // inward: articulated inertia A and bias P of the current link, folded into the parent
  // (pendulum_aba_np.py:51-82)
  {
    float A0 = 1.0f, A1 = 0.0f, A2 = 1.0f, A3 = 1.0f, A4 = 0.0f, A5 = 1.0f;
    float P0, P1, P2;
    own_bias(vw[K - 1], vx[K - 1], vy[K - 1], P0, P1, P2);
#pragma unroll U
    for (int i = K - 1; i >= 0; --i) {
      U0[i] = A0;
      U1[i] = A1;
      U2[i] = A2;
      uu[i] = (i == 0 ? torque : 0.0f) - P0;
      if (i == 0) break;
      const float D = A0;
      const double rD = recip(D);
      const float I0 = A0 - div(A0 * A0, D, rD), I1 = A1 - div(A0 * A1, D, rD), I2 = A2 - div(A0 * A2, D, rD);
      const float I3 = A3 - div(A1 * A1, D, rD), I4 = A4 - div(A1 * A2, D, rD), I5 = A5 - div(A2 * A2, D, rD);
      const float qd = om[i] - om[i - 1];
      const float c1 = qd * vy[i], c2 = (-qd) * vx[i];
      // Ia c with c = (0, c1, c2); the reference adds the exact zero term Ia_j0 * 0 first.
      const float Iac0 = I1 * c1 + I2 * c2;
      const float Iac1 = I3 * c1 + I4 * c2;
      const float Iac2 = I4 * c1 + I5 * c2;
      const float g = div(uu[i], D, rD);
      const float pa0 = (P0 + Iac0) + A0 * g;
      const float pa1 = (P1 + Iac1) + A1 * g;
      const float pa2 = (P2 + Iac2) + A2 * g;
      const float c = cs[i], s = sn[i];
      // B = Ia X, X = [[1, 0, 0], [s, c, s], [c, -s, c]] (joint at (1, 0) in the parent)
      const float B00 = (I0 + I1 * s) + I2 * c, B01 = I1 * c - I2 * s, B02 = I1 * s + I2 * c;
      const float B10 = (I1 + I3 * s) + I4 * c, B11 = I3 * c - I4 * s, B12 = I3 * s + I4 * c;
      const float B20 = (I2 + I4 * s) + I5 * c, B21 = I4 * c - I5 * s, B22 = I4 * s + I5 * c;
      // parent's own inertia (1, 0, 1, 1, 0, 1) + X^T B
      A0 = 1.0f + ((B00 + s * B10) + c * B20);
      A1 = (B01 + s * B11) + c * B21;
      A2 = 1.0f + ((B02 + s * B12) + c * B22);
      A3 = 1.0f + (c * B11 - s * B21);
      A4 = c * B12 - s * B22;
      A5 = 1.0f + (s * B12 + c * B22);
      // parent's own bias + X^T pa
      float pp0, pp1, pp2;
      own_bias(vw[i - 1], vx[i - 1], vy[i - 1], pp0, pp1, pp2);
      P0 = ((pp0 + pa0) + s * pa1) + c * pa2;
      P1 = (pp1 + c * pa1) - s * pa2;
      P2 = (pp2 + s * pa1) + c * pa2;
    }
  }
  // outward: accelerations from a base accelerating at -g (pendulum_aba_np.py:83-99)
  {
    float aw = 0.0f, ax = -GRAVITY, ay = 0.0f, run = 0.0f;
#pragma unroll U
    for (int i = 0; i < K; ++i) {
      const int im = i > 0 ? i - 1 : 0;
      const float c = cs[i], s = sn[i];
      const float xy = (i == 0) ? (ay + aw * 0.0f) : (ay + aw);
      const float qd = (i == 0) ? om[0] : om[i] - om[im];
      const float c1 = qd * vy[i], c2 = (-qd) * vx[i];
      const float ap0 = aw;
      const float ap1 = (c * ax + s * xy) + c1;
      const float ap2 = ((-s) * ax + c * xy) + c2;
      const float qdd = div(uu[i] - ((U0[i] * ap0 + U1[i] * ap1) + U2[i] * ap2), U0[i], recip(U0[i]));
      aw = ap0 + qdd;
      ax = ap1;
      ay = ap2;
      run = run + qdd;
      acc[i] = run;
    }
  }
}

// accelerations_with through the pivots' shared float64 reciprocals (DivRecip: the IEEE
// quotient unless it is subnormal); a lane on which a quotient came out subnormal
// evaluates again with IEEE division, so the results are IEEE's bit for bit. At N = 65,536:
// the Euler step at K = 16 11.98 -> 11.35 us, at K = 4 3.23 -> 3.14 us; the RK4 step at
// K = 4 6.77 -> 6.46 us. Past K = 16 the second copy of the evaluation costs scratch (the
// K = 32 Euler step spilled 184 B/lane). So K = 2..16 divide this way, the others with IEEE
// division (one link has one quotient to share its reciprocal with).
#ifndef ABA_RECIP_MIN_K
#define ABA_RECIP_MIN_K 2
#endif
template <int K, int U = K>
__device__ __forceinline__ void accelerations(const float* th, const float* om, float torque, float* acc) {
  if constexpr (K >= ABA_RECIP_MIN_K && K <= 16) {
    DivRecip fast;
    accelerations_with<K, U>(th, om, torque, acc, fast);
    if (fast.saw_subnormal()) {
      DivIEEE ieee;
      accelerations_with<K, U>(th, om, torque, acc, ieee);
    }
  } else {
    DivIEEE ieee;
    accelerations_with<K, U>(th, om, torque, acc, ieee);
  }
}

// Absolute angular accelerations from the Lagrangian mass-matrix form (pendulum_np.py:68-79,
// the reference's pendulum_metal.py): M_ij = mu_ij cos(th_i - th_j) and
// rhs_i = -sum_j mu_ij sin(th_i - th_j) om_j^2 - g mu_ii sin th_i (+ torque at the root),
// with mu_ij = K - max(i, j) and the differences' cos/sin from K cosines and K sines by the
// addition formulas, then the Cholesky solve of pendulum_np.py:85-107 (the IEEE square root
// and quotients, bit for bit). Sums run in numpy's order: over j for each row, the factor's
// rows left to right.
template <int K, class Div>
__device__ __forceinline__ void mass_matrix_accelerations_with(const float* th, const float* om, float torque,
                                                               float* acc, Div& div) {
  float c[K], s[K], w2[K];
  det_sincos_all<K>(th, s, c);
#pragma unroll
  for (int i = 0; i < K; ++i) w2[i] = om[i] * om[i];
  float L[K][K], y[K];
#pragma unroll
  for (int i = 0; i < K; ++i) {
    float r = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const float mu = (float)(K - (i > j ? i : j));
      const float t = (mu * (s[i] * c[j] - c[i] * s[j])) * w2[j];
      r = (j == 0) ? t : r + t;
      if (j <= i) L[i][j] = mu * (c[i] * c[j] + s[i] * s[j]);
    }
    y[i] = (-r) - (GRAVITY * (float)(K - i)) * s[i];
  }
  y[0] = y[0] + torque;
  // L L^T = M in place, then L y' = y and L^T x = y'; every quotient divides by a pivot,
  // whose float64 reciprocal is formed once
  double rL[K];
#pragma unroll
  for (int i = 0; i < K; ++i) {
#pragma unroll
    for (int j = 0; j <= i; ++j) {
      float t = L[i][j];
#pragma unroll
      for (int p = 0; p < j; ++p) t = t - L[i][p] * L[j][p];
      if (i == j) {
        L[i][i] = sqrt_rn(t);
        rL[i] = recip(L[i][i]);
      } else {
        L[i][j] = div(t, L[j][j], rL[j]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < K; ++i) {
    float t = y[i];
#pragma unroll
    for (int p = 0; p < i; ++p) t = t - L[i][p] * y[p];
    y[i] = div(t, L[i][i], rL[i]);
  }
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    float t = y[i];
#pragma unroll
    for (int p = i + 1; p < K; ++p) t = t - L[p][i] * acc[p];
    acc[i] = div(t, L[i][i], rL[i]);
  }
}

// The mass-matrix model's accelerations (pendulum_np.py:69-95). Divisions go through the
// pivots' shared float64 reciprocals (DivRecip: the IEEE quotient unless it is subnormal);
// a lane on which a quotient came out subnormal evaluates again with IEEE division. RK4 at
// N = 65,536: K = 16 55.5 -> 48.4 us per step, K = 8 16.1 -> 15.2, K = 4 6.85 -> 6.63; at
// K = 2 (3.97 -> 4.17 us) it divides with IEEE division alone.
template <int K>
__device__ __forceinline__ void mass_matrix_accelerations(const float* th, const float* om, float torque,
                                                          float* acc) {
  if constexpr (K > 2) {
    DivRecip fast;
    mass_matrix_accelerations_with<K>(th, om, torque, acc, fast);
    if (fast.saw_subnormal()) {
      DivIEEE ieee;
      mass_matrix_accelerations_with<K>(th, om, torque, acc, ieee);
    }
  } else {
    DivIEEE ieee;
    mass_matrix_accelerations_with<K>(th, om, torque, acc, ieee);
  }
}

// Tip above half the chain's length: -(sum_i cos th_i) > K / 2 (pendulum_np.py:81-82).
template <int K, int U = K>
__device__ __forceinline__ bool terminal(const float* th) {
  float s = 0.0f;
  if (wave_near_zero<K>(th)) {
#pragma unroll U
    for (int i = 0; i < K; ++i) {
      float sn, cs;
      sincos_poly(th[i], &sn, &cs);
      s = (i == 0) ? cs : s + cs;
    }
  } else {
#pragma unroll U
    for (int i = 0; i < K; ++i) s = (i == 0) ? det_cos(th[0]) : s + det_cos(th[i]);
  }
  return -s > (float)K * 0.5f;
}

// The accelerations of either model: the articulated-body algorithm or the mass matrix.
template <int K, int U, bool kMassMatrix>
__device__ __forceinline__ void model_accelerations(const float* th, const float* om, float torque, float* acc) {
  if constexpr (kMassMatrix)
    mass_matrix_accelerations<K>(th, om, torque, acc);
  else
    accelerations<K, U>(th, om, torque, acc);
}

// RK4 at dt 0.02 in place (pendulum_aba_np.py:117-123, pendulum_np.py:59-66), stage sums
// accumulated in numpy's order.
template <int K, int U = (K <= 16 ? K : 1), bool kMassMatrix = false>
__device__ __forceinline__ void rk4(float* th, float* om, float torque) {
  float acc[K], t[K], o[K], sth[K], som[K];
  model_accelerations<K, U, kMassMatrix>(th, om, torque, acc);
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    sth[p] = om[p];
    som[p] = acc[p];
    t[p] = th[p] + DT_2 * om[p];
    o[p] = om[p] + DT_2 * acc[p];
  }
  model_accelerations<K, U, kMassMatrix>(t, o, torque, acc);
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    sth[p] = sth[p] + 2.0f * o[p];
    som[p] = som[p] + 2.0f * acc[p];
    t[p] = th[p] + DT_2 * o[p];
    o[p] = om[p] + DT_2 * acc[p];
  }
  model_accelerations<K, U, kMassMatrix>(t, o, torque, acc);
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    sth[p] = sth[p] + 2.0f * o[p];
    som[p] = som[p] + 2.0f * acc[p];
    t[p] = th[p] + DT * o[p];
    o[p] = om[p] + DT * acc[p];
  }
  model_accelerations<K, U, kMassMatrix>(t, o, torque, acc);
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    th[p] = wrap(th[p] + DT_6 * (sth[p] + o[p]));
    om[p] = clip(om[p] + DT_6 * (som[p] + acc[p]), -MAX_VEL, MAX_VEL);
  }
}

// Semi-implicit Euler at dt 0.01 in place: omega first, then theta with the new omega.
template <int K, int U = K>
__device__ __forceinline__ void euler(float* th, float* om, float torque) {
  float acc[K];
  accelerations<K>(th, om, torque, acc);
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    const float om_new = om[p] + DT_EULER * acc[p];
    const float th_new = th[p] + DT_EULER * om_new;
    th[p] = wrap(th_new);
    om[p] = clip(om_new, -MAX_VEL, MAX_VEL);
  }
}

template <int K, int U = K>
__device__ __forceinline__ void load(const float* __restrict__ state, int64_t n, int64_t e, float* th, float* om) {
#pragma unroll U
  for (int p = 0; p < K; ++p) {
    th[p] = state[p * n + e];
    om[p] = state[(K + p) * n + e];
  }
}

// Masked reset: all 2K rows U[+-0.1] (RK4 task) or angles U[+-0.1] and zero velocities (Euler task),
// row p of env e hashed at (seed ^ e*golden) + p * 0x85EBCA6B (pendulum_aba_metal.py:109-113).
// The reference draws for every env and selects; the draws here sit on the terminated lanes'
// branch, so a wave with no termination (the common case: K up to 2K hashes saved) skips them.
template <int K, bool kZeroVelocity, int U = K>
__device__ __forceinline__ void store_with_reset(float* __restrict__ next, int64_t n, int64_t e, float* th,
                                                 float* om, bool d, uint32_t seed) {
  if (d) {
    const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll U
    for (int p = 0; p < K; ++p) th[p] = uniform_pm(pcg_hash(h + (uint32_t)p * kRowStride), RESET_BOUND);
#pragma unroll U
    for (int p = 0; p < K; ++p)
      om[p] = kZeroVelocity ? 0.0f : uniform_pm(pcg_hash(h + (uint32_t)(K + p) * kRowStride), RESET_BOUND);
  }
#pragma unroll U
  for (int p = 0; p < K; ++p) next[p * n + e] = th[p];
#pragma unroll U
  for (int p = 0; p < K; ++p) next[(K + p) * n + e] = om[p];
}

// kMassMatrix: the reference's pendulum_metal step (the same task with the mass-matrix
// accelerations, pendulum_metal.py:59-101); otherwise pendulum_aba_metal's.
template <int K, bool kMassMatrix = false>
__global__ __launch_bounds__(kBlock) void step_rk4_kernel(const float* __restrict__ state,
                                                          const int32_t* __restrict__ action, uint32_t seed,
                                                          float* __restrict__ next, float* __restrict__ reward,
                                                          uint8_t* __restrict__ done, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  constexpr int U = K <= 16 ? K : 1;
  float th[K], om[K];
  load<K, U>(state, n, e, th, om);
  rk4<K, U, kMassMatrix>(th, om, (float)(stream_load(action + e) - 1) * 1.0f);
  const bool d = terminal<K, U>(th);
  store_with_reset<K, false, U>(next, n, e, th, om, d, seed);
  stream_store(d ? 0.0f : -1.0f, reward + e);
  stream_store((uint8_t)(d ? 1 : 0), done + e);
}

template <int K, bool kArrayTorque>
__global__ __launch_bounds__(kBlock) void step_euler_kernel(const float* __restrict__ state,
                                                            const float* __restrict__ torque, uint32_t seed,
                                                            float* __restrict__ next, float* __restrict__ reward,
                                                            uint8_t* __restrict__ done, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float th[K], om[K];
  load<K>(state, n, e, th, om);
  const float tq = kArrayTorque ? stream_load(torque + e)
                                : uniform_pm(pcg_hash(env_hash(seed, (uint32_t)e) + kTorqueOffset), 1.0f);
  euler<K>(th, om, tq);
  const bool d = terminal<K>(th);
  store_with_reset<K, true>(next, n, e, th, om, d, seed);
  stream_store(d ? 0.0f : -1.0f, reward + e);
  stream_store((uint8_t)(d ? 1 : 0), done + e);
}

#ifndef ABA_STAGE_LINKS
#define ABA_STAGE_LINKS 4
#endif
// The staged K = 64 kernel's passes read their LDS rows (and the last pass its inputs)
// kStageLinks links ahead of their use, and hold later reads back with a memory barrier
// every kStageLinks links; its first pass reads its inputs kOutwardAhead links ahead. 2, 8
// or 16 instead of 4 change the K = 64 step by 1.2 us or less (54.2 us at N = 65,536).
constexpr int kStageLinks = ABA_STAGE_LINKS;
#ifndef ABA_OUTWARD_AHEAD
#define ABA_OUTWARD_AHEAD 4
#endif
constexpr int kOutwardAhead = ABA_OUTWARD_AHEAD;

// A (rows, n) float32 array seen by one env through a buffer resource: row r of env e is
// at byte (r * n + e) * 4, addressed as a per-lane offset e * 4 plus a uniform row offset in
// a scalar register, so a thread's 2K loads or stores need one address register instead
// of one per row. Requires rows * n * 4 < 2^31 (checked by the caller); accesses past the
// array's bytes read 0 and write nothing. 0x00020000 is the gfx9 resource word 3 for a raw
// 32-bit buffer.
struct RowBuffer {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t row_bytes, lane_bytes;
  __device__ RowBuffer(const float* base, int rows, int64_t n, int64_t e)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)(rows * n * 4), 0x00020000)),
        row_bytes((uint32_t)(n * 4)),
        lane_bytes((uint32_t)(e * 4)) {}
  __device__ float load(int r) const {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)lane_bytes, (int)(r * row_bytes), 0));
  }
  __device__ void store(int r, float v) const {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rsrc, (int)lane_bytes, (int)(r * row_bytes), 0);
  }
};

// The staged kernel's first pass (pendulum_aba_np.py:36-50): link velocities in link frames
// and joint rates from the inputs (read kOutwardAhead links ahead of their use), the joints'
// sin and cos into the LDS rows.
template <int K>
__device__ __forceinline__ void staged_outward(const RowBuffer& in, float* sn_l, float* cs_l, float (&vw)[K],
                                               float (&vx)[K], float (&vy)[K], float (&qdv)[K]) {
  float w = 0.0f, x = 0.0f, y = 0.0f, th_prev = 0.0f, om_prev = 0.0f;
  float th0[K], om0[K];  // the inputs, read kOutwardAhead links ahead of their use
#pragma unroll
  for (int j = 0; j < K && j < kOutwardAhead; ++j) {
    th0[j] = in.load(j);
    om0[j] = in.load(K + j);
  }
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (i + kOutwardAhead < K) {
      th0[i + kOutwardAhead] = in.load(i + kOutwardAhead);
      om0[i + kOutwardAhead] = in.load(K + i + kOutwardAhead);
    }
    const float th_i = th0[i], om_i = om0[i];
    const float q = (i == 0) ? th_i : th_i - th_prev;
    const float qd = (i == 0) ? om_i : om_i - om_prev;
    float sn, cs;
    det_sincos(q, &sn, &cs);
    sn_l[i * kBlock] = sn;
    cs_l[i * kBlock] = cs;
    const float xy = (i == 0) ? (y + w * 0.0f) : (y + w);
    const float nw = w + qd;
    const float nx = cs * x + sn * xy;
    const float ny = (-sn) * x + cs * xy;
    vw[i] = nw;
    vx[i] = nx;
    vy[i] = ny;
    qdv[i] = qd;
    w = nw;
    x = nx;
    y = ny;
    th_prev = th_i;
    om_prev = om_i;
  }
}

// The staged kernel's inward pass (pendulum_aba_np.py:51-82): articulated inertia and bias
// folded into the parent, writing U and u per link; a link's seven quotients divide by its
// pivot D through Div. cv, sv are rotating registers for the LDS rows of cos and sin.
template <int K, class Div>
__device__ __forceinline__ void staged_inward(const float (&vw)[K], const float (&vx)[K], const float (&vy)[K],
                                              const float (&qdv)[K], const float* cs_l, const float* sn_l,
                                              float tq, float (&U0)[K], float (&U1)[K], float (&U2)[K],
                                              float (&uu)[K], float (&cv)[K], float (&sv)[K], Div& div) {
  float A0 = 1.0f, A1 = 0.0f, A2 = 1.0f, A3 = 1.0f, A4 = 0.0f, A5 = 1.0f;
  float P0, P1, P2;
  own_bias(vw[K - 1], vx[K - 1], vy[K - 1], P0, P1, P2);
#pragma unroll
  for (int j = K - 1; j >= 1 && j > K - 1 - kStageLinks; --j) {
    cv[j] = cs_l[j * kBlock];
    sv[j] = sn_l[j * kBlock];
  }
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    U0[i] = A0;
    U1[i] = A1;
    U2[i] = A2;
    uu[i] = (i == 0 ? tq : 0.0f) - P0;
    if (i == 0) break;
    if (i - kStageLinks >= 1) {
      cv[i - kStageLinks] = cs_l[(i - kStageLinks) * kBlock];
      sv[i - kStageLinks] = sn_l[(i - kStageLinks) * kBlock];
    }
    const float D = A0;
    const double rD = recip(D);
    const float I0 = A0 - div(A0 * A0, D, rD), I1 = A1 - div(A0 * A1, D, rD), I2 = A2 - div(A0 * A2, D, rD);
    const float I3 = A3 - div(A1 * A1, D, rD), I4 = A4 - div(A1 * A2, D, rD), I5 = A5 - div(A2 * A2, D, rD);
    const float c1 = qdv[i] * vy[i], c2 = (-qdv[i]) * vx[i];
    const float Iac0 = I1 * c1 + I2 * c2;
    const float Iac1 = I3 * c1 + I4 * c2;
    const float Iac2 = I4 * c1 + I5 * c2;
    const float g = div(uu[i], D, rD);
    const float pa0 = (P0 + Iac0) + A0 * g;
    const float pa1 = (P1 + Iac1) + A1 * g;
    const float pa2 = (P2 + Iac2) + A2 * g;
    const float c = cv[i], s = sv[i];
    const float B00 = (I0 + I1 * s) + I2 * c, B01 = I1 * c - I2 * s, B02 = I1 * s + I2 * c;
    const float B10 = (I1 + I3 * s) + I4 * c, B11 = I3 * c - I4 * s, B12 = I3 * s + I4 * c;
    const float B20 = (I2 + I4 * s) + I5 * c, B21 = I4 * c - I5 * s, B22 = I4 * s + I5 * c;
    A0 = 1.0f + ((B00 + s * B10) + c * B20);
    A1 = (B01 + s * B11) + c * B21;
    A2 = 1.0f + ((B02 + s * B12) + c * B22);
    A3 = 1.0f + (c * B11 - s * B21);
    A4 = c * B12 - s * B22;
    A5 = 1.0f + (s * B12 + c * B22);
    float pp0, pp1, pp2;
    own_bias(vw[i - 1], vx[i - 1], vy[i - 1], pp0, pp1, pp2);
    P0 = ((pp0 + pa0) + s * pa1) + c * pa2;
    P1 = (pp1 + c * pa1) - s * pa2;
    P2 = (pp2 + s * pa1) + c * pa2;
    if ((i & (kStageLinks - 1)) == 0) asm volatile("" ::: "memory");  // LDS reads kStageLinks links ahead at most
  }
}

// The Euler step for long chains with the per-link state staged by lifetime. At K = 64 the
// step of the generic form holds the input angles and velocities and every per-link array
// for the whole step, about 790 floats per lane, and spills past the 512 registers. Here:
// - cos/sin of the joint angles sit in LDS (one 4-byte slot per link and thread,
//   2 * K * 4 * kBlock bytes per workgroup), read by all three passes;
// - the outward pass keeps, per link, the link velocity and the joint rate qd (4 floats);
// - the inward pass forms c1, c2 from them as it needs them, and each link it passes
//   trades those 4 floats for U and u (4 floats), so about 256 floats per lane are live;
// - the last pass runs the outward velocity recursion again next to the accelerations
//   (the same operations on the same values, so c1, c2 come out the same bits), rereads
//   each link's inputs, and finishes the link's Euler update, wrap, clip and cosine there.
// Every value is the generic form's, from the same operations in the same order
// (accelerations, euler, terminal, store_with_reset).
template <int K, bool kArrayTorque>
__global__ __launch_bounds__(kBlock) void step_euler_staged_kernel(const float* __restrict__ state,
                                                                   const float* __restrict__ torque, uint32_t seed,
                                                                   float* __restrict__ next,
                                                                   float* __restrict__ reward,
                                                                   uint8_t* __restrict__ done, int64_t n) {
  __shared__ float trig_lds[2 * K * kBlock];
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float* sn_l = trig_lds + threadIdx.x;          // sin of joint i at sn_l[i * kBlock]
  float* cs_l = trig_lds + K * kBlock + threadIdx.x;
  const float tq = kArrayTorque ? stream_load(torque + e)
                                : uniform_pm(pcg_hash(env_hash(seed, (uint32_t)e) + kTorqueOffset), 1.0f);
  float vw[K], vx[K], vy[K], qdv[K], U0[K], U1[K], U2[K], uu[K];
  const RowBuffer in(state, 2 * K, n, e);
  staged_outward<K>(in, sn_l, cs_l, vw, vx, vy, qdv);
  asm volatile("" ::: "memory");  // each pass reads its LDS rows in its own order, not hoisted into the last
  // inward: articulated inertia and bias folded into the parent (pendulum_aba_np.py:51-82)
  // Each pass below issues its reads kStageLinks links ahead of their use (rotating
  // registers), so their latency overlaps the links in between.
  float cv[K], sv[K];
  {
    // through the pivots' shared float64 reciprocals; a lane on which a quotient came out
    // subnormal runs the first two passes again, with IEEE division (nothing is stored
    // before the last pass and the inputs are only read, so the redo starts from them and
    // no first-pass value has to outlive the first attempt)
    DivRecip fast;
    staged_inward<K>(vw, vx, vy, qdv, cs_l, sn_l, tq, U0, U1, U2, uu, cv, sv, fast);
    if (fast.saw_subnormal()) {
      staged_outward<K>(in, sn_l, cs_l, vw, vx, vy, qdv);
      asm volatile("" ::: "memory");
      DivIEEE ieee;
      staged_inward<K>(vw, vx, vy, qdv, cs_l, sn_l, tq, U0, U1, U2, uu, cv, sv, ieee);
    }
  }
  asm volatile("" ::: "memory");
  // The last pass reads the inputs again, through a copy of the pointer that the compiler
  // cannot see through, so the reads are not hoisted above the passes (the input is
  // read-only, and a plain memory barrier does not hold its loads back).
  const float* again = state;
  asm volatile("" : "+s"(again)::"memory");
  const RowBuffer in2(again, 2 * K, n, e), out(next, 2 * K, n, e);
  // outward: accelerations from a base accelerating at -g (pendulum_aba_np.py:83-99), with
  // the velocity recursion of the first pass repeated for c1, c2, and each link's
  // semi-implicit Euler update, wrap, clip and cosine for the termination test
  float cos_sum = 0.0f;
  {
    float aw = 0.0f, ax = -GRAVITY, ay = 0.0f, run = 0.0f;
    float w = 0.0f, x = 0.0f, y = 0.0f, om_prev = 0.0f;
    float thv[K], omv[K];
#pragma unroll
    for (int j = 0; j < K && j < kStageLinks; ++j) {
      thv[j] = in2.load(j);
      omv[j] = in2.load(K + j);
      cv[j] = cs_l[j * kBlock];
      sv[j] = sn_l[j * kBlock];
    }
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (i + kStageLinks < K) {
        thv[i + kStageLinks] = in2.load(i + kStageLinks);
        omv[i + kStageLinks] = in2.load(K + i + kStageLinks);
        cv[i + kStageLinks] = cs_l[(i + kStageLinks) * kBlock];
        sv[i + kStageLinks] = sn_l[(i + kStageLinks) * kBlock];
      }
      const float th_i = thv[i], om_i = omv[i];
      const float qd = (i == 0) ? om_i : om_i - om_prev;
      const float c = cv[i], s = sv[i];
      const float vxy = (i == 0) ? (y + w * 0.0f) : (y + w);
      const float nw = w + qd;
      const float nx = c * x + s * vxy;
      const float ny = (-s) * x + c * vxy;
      w = nw;
      x = nx;
      y = ny;
      const float c1 = qd * ny, c2 = (-qd) * nx;
      const float xy = (i == 0) ? (ay + aw * 0.0f) : (ay + aw);
      const float ap0 = aw;
      const float ap1 = (c * ax + s * xy) + c1;
      const float ap2 = ((-s) * ax + c * xy) + c2;
      const float qdd = (uu[i] - ((U0[i] * ap0 + U1[i] * ap1) + U2[i] * ap2)) / U0[i];
      aw = ap0 + qdd;
      ax = ap1;
      ay = ap2;
      run = run + qdd;
      const float om_new = om_i + DT_EULER * run;
      const float th_new = wrap(th_i + DT_EULER * om_new);
      out.store(i, th_new);
      out.store(K + i, clip(om_new, -MAX_VEL, MAX_VEL));
      cos_sum = (i == 0) ? det_cos(th_new) : cos_sum + det_cos(th_new);
      om_prev = om_i;
      if ((i & (kStageLinks - 1)) == kStageLinks - 1) asm volatile("" ::: "memory");
    }
  }
  const bool d = -cos_sum > (float)K * 0.5f;
  if (d) {  // angles U[+-0.1], zero velocities, overwriting the stepped state
    const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
    for (int p = 0; p < K; ++p) {
      out.store(p, uniform_pm(pcg_hash(h + (uint32_t)p * kRowStride), RESET_BOUND));
      out.store(K + p, 0.0f);
    }
  }
  stream_store(d ? 0.0f : -1.0f, reward + e);
  stream_store((uint8_t)(d ? 1 : 0), done + e);
}

// ---------------------------------------------------------------------------
// Staged RK4 step for long chains (K = 32, 64): the reference's drop-in step
// (pendulum_aba_np.py:117-123, pendulum_aba_metal.py:85-116) with the per-link state kept
// by lifetime, as in the staged Euler kernel. The generic RK4 kernel holds nine per-link
// arrays per evaluation next to the stage sums, and past K = 16 keeps them in scratch
// memory. Here, per evaluation:
// - pass 1 (outward) forms the joint angles and rates from the stage input (t, o), writes
//   the joints' sin and cos into the LDS rows and keeps each link's velocity (3 floats);
// - pass 2 (inward) trades each link's velocity for U and u (4 floats), reading the
//   joint rate back from o;
// - pass 3 (outward) repeats the velocity recursion next to the accelerations (the same
//   operations on the same values, so the same bits), and finishes each link's stage at
//   once: the stage sums and the next stage's input (t, o), or in the last stage the
//   link's update, wrap and clip, stored.
// Across the stages each lane keeps t, o and (kSumsInNext false) the stage sums of the
// angles and velocities in registers; with kSumsInNext the sums live in the output rows of
// `next` between stages (the lane's own column, overwritten by the result in the last
// stage), which is what fits 64 links in the register file. Every value is the generic
// kernel's, from the same operations in the same order (rk4, terminal, store_with_reset).
// ---------------------------------------------------------------------------

// Pass 1 of one evaluation: joint angles and rates from (t, o), the joints' sin and cos
// into the LDS rows (the polynomial alone when the caller's wave vote found every joint
// angle within 0.78 of zero), link velocities in link frames (pendulum_aba_np.py:36-50).
template <int K, bool kNear>
__device__ __forceinline__ void rk4_outward(const float (&t)[K], const float (&o)[K], float* sn_l, float* cs_l,
                                            float (&vw)[K], float (&vx)[K], float (&vy)[K]) {
  float w = 0.0f, x = 0.0f, y = 0.0f;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const float q = (i == 0) ? t[0] : t[i] - t[i > 0 ? i - 1 : 0];
    const float qd = (i == 0) ? o[0] : o[i] - o[i > 0 ? i - 1 : 0];
    float sn, cs;
    if constexpr (kNear)
      sincos_poly(q, &sn, &cs);
    else
      det_sincos(q, &sn, &cs);
    sn_l[i * kBlock] = sn;
    cs_l[i * kBlock] = cs;
    const float xy = (i == 0) ? (y + w * 0.0f) : (y + w);
    const float nw = w + qd;
    const float nx = cs * x + sn * xy;
    const float ny = (-sn) * x + cs * xy;
    vw[i] = nw;
    vx[i] = nx;
    vy[i] = ny;
    w = nw;
    x = nx;
    y = ny;
  }
}

// Pass 2 of one evaluation (pendulum_aba_np.py:51-82): staged_inward with the joint rates
// read back from o instead of kept per link.
template <int K, class Div>
__device__ __forceinline__ void rk4_inward(const float (&vw)[K], const float (&vx)[K], const float (&vy)[K],
                                           const float (&o)[K], const float* cs_l, const float* sn_l, float tq,
                                           float (&U0)[K], float (&U1)[K], float (&U2)[K], float (&uu)[K],
                                           float (&cv)[K], float (&sv)[K], Div& div) {
  float A0 = 1.0f, A1 = 0.0f, A2 = 1.0f, A3 = 1.0f, A4 = 0.0f, A5 = 1.0f;
  float P0, P1, P2;
  own_bias(vw[K - 1], vx[K - 1], vy[K - 1], P0, P1, P2);
#pragma unroll
  for (int j = K - 1; j >= 1 && j > K - 1 - kStageLinks; --j) {
    cv[j] = cs_l[j * kBlock];
    sv[j] = sn_l[j * kBlock];
  }
#pragma unroll
  for (int i = K - 1; i >= 0; --i) {
    U0[i] = A0;
    U1[i] = A1;
    U2[i] = A2;
    uu[i] = (i == 0 ? tq : 0.0f) - P0;
    if (i == 0) break;
    if (i - kStageLinks >= 1) {
      cv[i - kStageLinks] = cs_l[(i - kStageLinks) * kBlock];
      sv[i - kStageLinks] = sn_l[(i - kStageLinks) * kBlock];
    }
    const float D = A0;
    const double rD = recip(D);
    const float I0 = A0 - div(A0 * A0, D, rD), I1 = A1 - div(A0 * A1, D, rD), I2 = A2 - div(A0 * A2, D, rD);
    const float I3 = A3 - div(A1 * A1, D, rD), I4 = A4 - div(A1 * A2, D, rD), I5 = A5 - div(A2 * A2, D, rD);
    const float qd = o[i] - o[i - 1];
    const float c1 = qd * vy[i], c2 = (-qd) * vx[i];
    const float Iac0 = I1 * c1 + I2 * c2;
    const float Iac1 = I3 * c1 + I4 * c2;
    const float Iac2 = I4 * c1 + I5 * c2;
    const float g = div(uu[i], D, rD);
    const float pa0 = (P0 + Iac0) + A0 * g;
    const float pa1 = (P1 + Iac1) + A1 * g;
    const float pa2 = (P2 + Iac2) + A2 * g;
    const float c = cv[i], s = sv[i];
    const float B00 = (I0 + I1 * s) + I2 * c, B01 = I1 * c - I2 * s, B02 = I1 * s + I2 * c;
    const float B10 = (I1 + I3 * s) + I4 * c, B11 = I3 * c - I4 * s, B12 = I3 * s + I4 * c;
    const float B20 = (I2 + I4 * s) + I5 * c, B21 = I4 * c - I5 * s, B22 = I4 * s + I5 * c;
    A0 = 1.0f + ((B00 + s * B10) + c * B20);
    A1 = (B01 + s * B11) + c * B21;
    A2 = 1.0f + ((B02 + s * B12) + c * B22);
    A3 = 1.0f + (c * B11 - s * B21);
    A4 = c * B12 - s * B22;
    A5 = 1.0f + (s * B12 + c * B22);
    float pp0, pp1, pp2;
    own_bias(vw[i - 1], vx[i - 1], vy[i - 1], pp0, pp1, pp2);
    P0 = ((pp0 + pa0) + s * pa1) + c * pa2;
    P1 = (pp1 + c * pa1) - s * pa2;
    P2 = (pp2 + s * pa1) + c * pa2;
    if ((i & (kStageLinks - 1)) == 0) asm volatile("" ::: "memory");  // LDS reads kStageLinks links ahead at most
  }
}

// Passes 1 and 2 of one evaluation; the quotients of pass 2 through the pivots' shared
// float64 reciprocals when kRecip (a lane on which one came out subnormal runs both passes
// again with IEEE division, from t and o, which no pass writes), else IEEE division.
// o's values passed through an empty asm statement: the same bits, but values the compiler
// cannot match with the earlier ones, so a pass that recomputes a joint rate o[i] - o[i-1]
// does not keep the previous pass's copy alive across the passes in between (K more
// registers live).
template <int K>
__device__ __forceinline__ void opaque_rows(float (&o)[K]) {
#pragma unroll
  for (int i = 0; i < K; ++i) asm volatile("" : "+v"(o[i]));
}

template <int K, bool kRecip>
__device__ __forceinline__ void rk4_passes12(const float (&t)[K], float (&o)[K], float* sn_l, float* cs_l,
                                             float tq, float (&U0)[K], float (&U1)[K], float (&U2)[K],
                                             float (&uu)[K], float (&cv)[K], float (&sv)[K]) {
  // one wave vote for the K joint angles of this stage
  bool ok = true;
#pragma unroll
  for (int i = 0; i < K; ++i) ok &= fabsf((i == 0) ? t[0] : t[i] - t[i > 0 ? i - 1 : 0]) <= 0.78f;
  const bool near = __all(ok);
  float vw[K], vx[K], vy[K];
  if (near)
    rk4_outward<K, true>(t, o, sn_l, cs_l, vw, vx, vy);
  else
    rk4_outward<K, false>(t, o, sn_l, cs_l, vw, vx, vy);
  asm volatile("" ::: "memory");  // each pass reads its LDS rows in its own order
  opaque_rows<K>(o);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kRecip) {
    DivRecip fast;
    rk4_inward<K>(vw, vx, vy, o, cs_l, sn_l, tq, U0, U1, U2, uu, cv, sv, fast);
    if (fast.saw_subnormal()) {
      asm volatile("" ::: "memory");
      if (near)
        rk4_outward<K, true>(t, o, sn_l, cs_l, vw, vx, vy);
      else
        rk4_outward<K, false>(t, o, sn_l, cs_l, vw, vx, vy);
      asm volatile("" ::: "memory");
      DivIEEE ieee;
      rk4_inward<K>(vw, vx, vy, o, cs_l, sn_l, tq, U0, U1, U2, uu, cv, sv, ieee);
    }
  } else {
    DivIEEE ieee;
    rk4_inward<K>(vw, vx, vy, o, cs_l, sn_l, tq, U0, U1, U2, uu, cv, sv, ieee);
  }
  asm volatile("" ::: "memory");
}

// Pass 3 of evaluation kStage (0..3): accelerations from a base accelerating at -g
// (pendulum_aba_np.py:83-99) with the velocity recursion repeated, and each link's stage
// finished (rk4's stage loops, in the same order). The input rows th, om are re-read
// kStageLinks links ahead (stage 0 has them in t, o); with kSumsInNext the stage sums are
// read from and written to the lane's column of `next`.
template <int K, int kStage, bool kSumsInNext>
__device__ __forceinline__ void rk4_pass3(const RowBuffer& in, const RowBuffer& out, const float* cs_l,
                                          const float* sn_l, const float (&U0)[K], const float (&U1)[K],
                                          const float (&U2)[K], const float (&uu)[K], float (&cv)[K], float (&sv)[K],
                                          float (&t)[K], float (&o)[K], float (&sth)[K], float (&som)[K]) {
  constexpr bool kReread = kStage > 0;               // stage 0's t, o are the inputs themselves
  constexpr bool kReadSums = kSumsInNext && kStage > 0;
  float thv[K], omv[K], stv[K], sov[K];              // rotating read-ahead registers
#pragma unroll
  for (int j = 0; j < K && j < kStageLinks; ++j) {
    cv[j] = cs_l[j * kBlock];
    sv[j] = sn_l[j * kBlock];
    if constexpr (kReread) {
      thv[j] = in.load(j);
      omv[j] = in.load(K + j);
    }
    if constexpr (kReadSums) {
      stv[j] = out.load(j);
      sov[j] = out.load(K + j);
    }
  }
  float aw = 0.0f, ax = -GRAVITY, ay = 0.0f, run = 0.0f;
  float w = 0.0f, x = 0.0f, y = 0.0f, o_prev = 0.0f;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    if (i + kStageLinks < K) {
      cv[i + kStageLinks] = cs_l[(i + kStageLinks) * kBlock];
      sv[i + kStageLinks] = sn_l[(i + kStageLinks) * kBlock];
      if constexpr (kReread) {
        thv[i + kStageLinks] = in.load(i + kStageLinks);
        omv[i + kStageLinks] = in.load(K + i + kStageLinks);
      }
      if constexpr (kReadSums) {
        stv[i + kStageLinks] = out.load(i + kStageLinks);
        sov[i + kStageLinks] = out.load(K + i + kStageLinks);
      }
    }
    const float o_i = o[i];
    const float qd = (i == 0) ? o_i : o_i - o_prev;
    const float c = cv[i], s = sv[i];
    const float vxy = (i == 0) ? (y + w * 0.0f) : (y + w);
    const float nw = w + qd;
    const float nx = c * x + s * vxy;
    const float ny = (-s) * x + c * vxy;
    w = nw;
    x = nx;
    y = ny;
    const float c1 = qd * ny, c2 = (-qd) * nx;
    const float xy = (i == 0) ? (ay + aw * 0.0f) : (ay + aw);
    const float ap0 = aw;
    const float ap1 = (c * ax + s * xy) + c1;
    const float ap2 = ((-s) * ax + c * xy) + c2;
    const float qdd = (uu[i] - ((U0[i] * ap0 + U1[i] * ap1) + U2[i] * ap2)) / U0[i];
    aw = ap0 + qdd;
    ax = ap1;
    ay = ap2;
    run = run + qdd;
    const float acc = run;
    const float th_i = kReread ? thv[i] : t[i];
    const float om_i = kReread ? omv[i] : o_i;
    float st, so;  // the stage sums before this stage
    if constexpr (kStage > 0) {
      st = kSumsInNext ? stv[i] : sth[i];
      so = kSumsInNext ? sov[i] : som[i];
    }
    if constexpr (kStage < 3) {
      if constexpr (kStage == 0) {
        st = o_i;
        so = acc;
      } else {
        st = st + 2.0f * o_i;
        so = so + 2.0f * acc;
      }
      if constexpr (kSumsInNext) {
        out.store(i, st);
        out.store(K + i, so);
      } else {
        sth[i] = st;
        som[i] = so;
      }
      constexpr float h = kStage == 2 ? DT : DT_2;
      t[i] = th_i + h * o_i;
      o[i] = om_i + h * acc;
    } else {
      const float th_new = wrap(th_i + DT_6 * (st + o_i));
      out.store(i, th_new);
      out.store(K + i, clip(om_i + DT_6 * (so + acc), -MAX_VEL, MAX_VEL));
      t[i] = th_new;  // kept for the termination test
    }
    o_prev = o_i;
    if ((i & (kStageLinks - 1)) == kStageLinks - 1) asm volatile("" ::: "memory");
  }
}

template <int K, int kStage, bool kSumsInNext, bool kRecip>
__device__ __forceinline__ void rk4_stage(const RowBuffer& in, const RowBuffer& out, float* sn_l, float* cs_l, float tq,
                                          float (&t)[K], float (&o)[K], float (&sth)[K], float (&som)[K]) {
  float U0[K], U1[K], U2[K], uu[K], cv[K], sv[K];
  rk4_passes12<K, kRecip>(t, o, sn_l, cs_l, tq, U0, U1, U2, uu, cv, sv);
  opaque_rows<K>(o);
  __builtin_amdgcn_sched_barrier(0);
  rk4_pass3<K, kStage, kSumsInNext>(in, out, cs_l, sn_l, U0, U1, U2, uu, cv, sv, t, o, sth, som);
  asm volatile("" ::: "memory");
}

template <int K, bool kSumsInNext, bool kRecip>
__global__ __launch_bounds__(kBlock) void step_rk4_staged_kernel(const float* __restrict__ state,
                                                                 const int32_t* __restrict__ action, uint32_t seed,
                                                                 float* __restrict__ next, float* __restrict__ reward,
                                                                 uint8_t* __restrict__ done, int64_t n) {
  __shared__ float trig_lds[2 * K * kBlock];
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float* sn_l = trig_lds + threadIdx.x;  // sin of joint i at sn_l[i * kBlock]
  float* cs_l = trig_lds + K * kBlock + threadIdx.x;
  const float tq = (float)(stream_load(action + e) - 1) * 1.0f;
  const RowBuffer in(state, 2 * K, n, e), out(next, 2 * K, n, e);
  float t[K], o[K], sth[K], som[K];  // sth, som unused (no registers) with kSumsInNext
#pragma unroll
  for (int p = 0; p < K; ++p) {
    t[p] = in.load(p);
    o[p] = in.load(K + p);
  }
  rk4_stage<K, 0, kSumsInNext, kRecip>(in, out, sn_l, cs_l, tq, t, o, sth, som);
  rk4_stage<K, 1, kSumsInNext, kRecip>(in, out, sn_l, cs_l, tq, t, o, sth, som);
  rk4_stage<K, 2, kSumsInNext, kRecip>(in, out, sn_l, cs_l, tq, t, o, sth, som);
  rk4_stage<K, 3, kSumsInNext, kRecip>(in, out, sn_l, cs_l, tq, t, o, sth, som);
  const bool d = terminal<K, K>(t);
  if (d) {  // every row U[+-0.1], overwriting the stepped state
    const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
    for (int p = 0; p < 2 * K; ++p) out.store(p, uniform_pm(pcg_hash(h + (uint32_t)p * kRowStride), RESET_BOUND));
  }
  stream_store(d ? 0.0f : -1.0f, reward + e);
  stream_store((uint8_t)(d ? 1 : 0), done + e);
}

template <int K>
__global__ __launch_bounds__(kBlock) void accelerations_kernel(const float* __restrict__ state,
                                                               const float* __restrict__ torque,
                                                               float* __restrict__ acc_out, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float th[K], om[K], acc[K];
  load<K>(state, n, e, th, om);
  accelerations<K>(th, om, torque[e], acc);
#pragma unroll
  for (int p = 0; p < K; ++p) acc_out[p * n + e] = acc[p];
}

template <int K>
__global__ __launch_bounds__(kBlock) void mass_matrix_accelerations_kernel(const float* __restrict__ state,
                                                                           const float* __restrict__ torque,
                                                                           float* __restrict__ acc_out, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float th[K], om[K], acc[K];
  load<K>(state, n, e, th, om);
  mass_matrix_accelerations<K>(th, om, torque[e], acc);
#pragma unroll
  for (int p = 0; p < K; ++p) acc_out[p * n + e] = acc[p];
}

template <int K, bool kZeroVelocity>
__global__ __launch_bounds__(kBlock) void reset_kernel(float* __restrict__ state, uint32_t seed, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float th[K], om[K];
  store_with_reset<K, kZeroVelocity>(state, n, e, th, om, true, seed);
}

// Chains at least this long take the staged Euler kernel.
#ifndef ABA_STAGED_EULER_MIN_K
#define ABA_STAGED_EULER_MIN_K 64
#endif
constexpr int kStagedEulerMinK = ABA_STAGED_EULER_MIN_K;

// Chains at least this long take the staged RK4 kernel; up to ABA_RK4_SUMS_IN_REGS_MAX_K links
// it keeps the stage sums in registers (past it, in the output rows), and up to
// ABA_RK4_RECIP_MAX_K links it divides through the pivots' shared reciprocals.
#ifndef ABA_STAGED_RK4_MIN_K
#define ABA_STAGED_RK4_MIN_K 32
#endif
#ifndef ABA_RK4_SUMS_IN_REGS_MAX_K
#define ABA_RK4_SUMS_IN_REGS_MAX_K 32
#endif
#ifndef ABA_RK4_RECIP_MAX_K
#define ABA_RK4_RECIP_MAX_K 32
#endif
constexpr int kStagedRk4MinK = ABA_STAGED_RK4_MIN_K;

enum Op { kRk4, kEulerArray, kEulerRng, kAcc, kReset, kResetZeroVel, kMassRk4, kMassAcc };

template <int K>
int launch(Op op, const float* state, const void* in, uint32_t seed, float* out, float* reward, uint8_t* done,
           int64_t n, hipStream_t s) {
  const dim3 grid(grid_for(n)), block(kBlock);
  switch (op) {
    case kRk4: {
      // the staged kernel addresses the (2K, n) arrays with 32-bit byte offsets
      const bool staged = K >= kStagedRk4MinK && (int64_t)2 * K * n * 4 < ((int64_t)1 << 31);
      if constexpr (K >= kStagedRk4MinK) {
        constexpr bool kSumsInNext = K > ABA_RK4_SUMS_IN_REGS_MAX_K;
        constexpr bool kRecip = K <= ABA_RK4_RECIP_MAX_K;
        if (staged)
          hipLaunchKernelGGL((step_rk4_staged_kernel<K, kSumsInNext, kRecip>), grid, block, 0, s, state,
                             (const int32_t*)in, seed, out, reward, done, n);
      }
      if (!staged)
        hipLaunchKernelGGL(step_rk4_kernel<K>, grid, block, 0, s, state, (const int32_t*)in, seed, out, reward, done,
                           n);
      break;
    }
    case kEulerArray:
    case kEulerRng: {
      // the staged kernel addresses the (2K, n) arrays with 32-bit byte offsets
      const bool staged = K >= kStagedEulerMinK && (int64_t)2 * K * n * 4 < ((int64_t)1 << 31);
      const bool array = op == kEulerArray;
      if constexpr (K >= kStagedEulerMinK) {
        if (staged && array)
          hipLaunchKernelGGL((step_euler_staged_kernel<K, true>), grid, block, 0, s, state, (const float*)in, seed,
                             out, reward, done, n);
        if (staged && !array)
          hipLaunchKernelGGL((step_euler_staged_kernel<K, false>), grid, block, 0, s, state, (const float*)in, seed,
                             out, reward, done, n);
      }
      if (!staged && array)
        hipLaunchKernelGGL((step_euler_kernel<K, true>), grid, block, 0, s, state, (const float*)in, seed, out, reward,
                           done, n);
      if (!staged && !array)
        hipLaunchKernelGGL((step_euler_kernel<K, false>), grid, block, 0, s, state, (const float*)in, seed, out,
                           reward, done, n);
      break;
    }
    case kAcc:
      hipLaunchKernelGGL(accelerations_kernel<K>, grid, block, 0, s, state, (const float*)in, out, n);
      break;
    case kReset:
      hipLaunchKernelGGL((reset_kernel<K, false>), grid, block, 0, s, out, seed, n);
      break;
    case kResetZeroVel:
      hipLaunchKernelGGL((reset_kernel<K, true>), grid, block, 0, s, out, seed, n);
      break;
    case kMassRk4:
      if constexpr (K <= 16) {
        hipLaunchKernelGGL((step_rk4_kernel<K, true>), grid, block, 0, s, state, (const int32_t*)in, seed, out, reward,
                           done, n);
      } else {
        return HIPENVS_E_UNSUPPORTED;
      }
      break;
    case kMassAcc:
      if constexpr (K <= 16) {
        hipLaunchKernelGGL(mass_matrix_accelerations_kernel<K>, grid, block, 0, s, state, (const float*)in, out, n);
      } else {
        return HIPENVS_E_UNSUPPORTED;
      }
      break;
  }
  return launch_status();
}

int dispatch(int32_t k, Op op, const float* state, const void* in, uint32_t seed, float* out, float* reward,
             uint8_t* done, int64_t n, hipStream_t s) {
  switch (k) {
    case 1: return launch<1>(op, state, in, seed, out, reward, done, n, s);
    case 2: return launch<2>(op, state, in, seed, out, reward, done, n, s);
    case 3: return launch<3>(op, state, in, seed, out, reward, done, n, s);
    case 4: return launch<4>(op, state, in, seed, out, reward, done, n, s);
    case 8: return launch<8>(op, state, in, seed, out, reward, done, n, s);
    case 16: return launch<16>(op, state, in, seed, out, reward, done, n, s);
    case 32: return launch<32>(op, state, in, seed, out, reward, done, n, s);
    case 64: return launch<64>(op, state, in, seed, out, reward, done, n, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

}  // namespace aba
}  // namespace hipenvs

using namespace hipenvs;

extern "C" int hipenvs_pendulum_aba_reset(int32_t k, int32_t zero_velocity, float* state, int64_t n, uint32_t seed,
                                          hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && !state)) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, zero_velocity ? aba::kResetZeroVel : aba::kReset, nullptr, nullptr, seed, state, nullptr,
                       nullptr, n, as_stream(stream));
}

extern "C" int hipenvs_pendulum_aba_step(int32_t k, const float* state, const int32_t* action, uint32_t seed,
                                         float* next_state, float* reward, uint8_t* done, int64_t n,
                                         hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !action || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, aba::kRk4, state, action, seed, next_state, reward, done, n, as_stream(stream));
}

extern "C" int hipenvs_pendulum_aba_step_euler(int32_t k, const float* state, const float* torque, uint32_t seed,
                                               float* next_state, float* reward, uint8_t* done, int64_t n,
                                               hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, torque ? aba::kEulerArray : aba::kEulerRng, state, torque, seed, next_state, reward, done,
                       n, as_stream(stream));
}

extern "C" int hipenvs_pendulum_aba_accelerations(int32_t k, const float* state, const float* torque, float* acc,
                                                  int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !torque || !acc))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, aba::kAcc, state, torque, 0, acc, nullptr, nullptr, n, as_stream(stream));
}

extern "C" int hipenvs_pendulum_step(int32_t k, const float* state, const int32_t* action, uint32_t seed,
                                     float* next_state, float* reward, uint8_t* done, int64_t n,
                                     hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !action || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, aba::kMassRk4, state, action, seed, next_state, reward, done, n, as_stream(stream));
}

extern "C" int hipenvs_pendulum_accelerations(int32_t k, const float* state, const float* torque, float* acc,
                                              int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !torque || !acc))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  return aba::dispatch(k, aba::kMassAcc, state, torque, 0, acc, nullptr, nullptr, n, as_stream(stream));
}
