// Acrobot on MI355X: the single-step kernel (RK4 at dt 0.2, wrap, clip, masked
// reset) and the fused ES rollout kernel (6-H-3 tanh policy + the same physics
// for the whole horizon in registers), with their C-ABI entry points.
//
// The derivative follows acrobot_np.py:64-84 operation by operation, with the
// Python-scalar products already folded to the float32 constants numpy uses
// (each constant's defining expression is beside it); RK4/wrap/clip follow
// acrobot_np.py:47-61,87-89, termination acrobot_np.py:92-93, reset the
// counter RNG of acrobot_metal.py:78-83. Per env-step the step kernel moves 41
// algorithmic bytes; it is VALU-bound (14 sin/cos, 18 IEEE divisions).

#include "es_noise.h"

namespace hipenvs {
namespace ac {

constexpr float D1_C0 = 0x1p-2f;              // float32(1.0 * 0.5**2)
constexpr float D1_C1 = 0x1.4p+0f;            // float32(1.0**2 + 0.5**2)
constexpr float D2_C0 = 0x1p-2f;              // float32(0.5**2)
constexpr float D2_C1 = 0x1p-1f;              // float32(1.0 * 0.5)
constexpr float PHI2_C = 0x1.39999ap+2f;      // float32(1.0 * 0.5 * 9.8)
constexpr float HALF_PI = 0x1.921fb6p+0f;     // float32(pi / 2)
constexpr float PHI1_A = -0x1p-1f;            // float32(-1.0 * 1.0 * 0.5)
constexpr float PHI1_C = 0x1.d66666p+3f;      // float32((1.0 * 0.5 + 1.0 * 1.0) * 9.8)
constexpr float DD2_C = 0x1p-1f;              // float32(1.0 * 1.0 * 0.5)
constexpr float DEN_C = 0x1.4p+0f;            // float32(1.0 * 0.5**2 + 1.0)
constexpr float DT = 0x1.99999ap-3f;          // float32(0.2)
constexpr float DT_2 = 0x1.99999ap-4f;        // float32(0.2 / 2)
constexpr float DT_6 = 0x1.111112p-5f;        // float32(0.2 / 6)
constexpr float TWO_PI = 0x1.921fb6p+2f;      // float32(2 * pi)
constexpr float PI = 0x1.921fb6p+1f;          // float32(pi)
constexpr float MAX_VEL_1 = 0x1.921fb6p+3f;   // float32(4 * pi)
constexpr float MAX_VEL_2 = 0x1.c463acp+4f;   // float32(9 * pi)
constexpr float RESET_BOUND = 0x1.99999ap-4f; // float32(0.1)

struct S4 {
  float a, b, c, d;  // theta1, theta2, dtheta1, dtheta2 (or their derivatives)
};

// acrobot_np.py:64-84. The numpy expression's multiplications by the Python
// float 1.0 (m2 *, 2 * l1 * lc2 *) are exact and omitted.
__device__ __forceinline__ S4 dsdt(const S4& s, float torque) {
  float s2, c2;
  det_sincos(s.b, &s2, &c2);
  const float d1 = ((D1_C0 + (D1_C1 + c2)) + 1.0f) + 1.0f;
  const float d2 = (D2_C0 + D2_C1 * c2) + 1.0f;
  const float phi2 = PHI2_C * det_cos((s.a + s.b) - HALF_PI);
  const float t1 = (PHI1_A * (s.d * s.d)) * s2;
  const float t2 = (s.d * s.c) * s2;
  const float t3 = PHI1_C * det_cos(s.a - HALF_PI);
  const float phi1 = ((t1 - t2) + t3) + phi2;
  const float num = ((torque + (d2 / d1) * phi1) - (DD2_C * (s.c * s.c)) * s2) - phi2;
  const float den = DEN_C - (d2 * d2) / d1;
  const float dd2 = num / den;
  const float dd1 = (-((d2 * dd2) + phi1)) / d1;
  return S4{s.c, s.d, dd1, dd2};
}

constexpr double INV_TWO_PI = 1.0 / (double)TWO_PI;  // for div_const(x, .) == x / TWO_PI

__device__ __forceinline__ float wrap(float x) { return x - TWO_PI * floorf(div_const(x + PI, INV_TWO_PI)); }

// RK4 + wrap + clip in place (acrobot_np.py:47-61).
__device__ __forceinline__ void rk4(S4& s, float torque) {
  const S4 k1 = dsdt(s, torque);
  const S4 k2 = dsdt(S4{s.a + DT_2 * k1.a, s.b + DT_2 * k1.b, s.c + DT_2 * k1.c, s.d + DT_2 * k1.d}, torque);
  const S4 k3 = dsdt(S4{s.a + DT_2 * k2.a, s.b + DT_2 * k2.b, s.c + DT_2 * k2.c, s.d + DT_2 * k2.d}, torque);
  const S4 k4 = dsdt(S4{s.a + DT * k3.a, s.b + DT * k3.b, s.c + DT * k3.c, s.d + DT * k3.d}, torque);
  const float na = s.a + DT_6 * (((k1.a + 2.0f * k2.a) + 2.0f * k3.a) + k4.a);
  const float nb = s.b + DT_6 * (((k1.b + 2.0f * k2.b) + 2.0f * k3.b) + k4.b);
  const float nc = s.c + DT_6 * (((k1.c + 2.0f * k2.c) + 2.0f * k3.c) + k4.c);
  const float nd = s.d + DT_6 * (((k1.d + 2.0f * k2.d) + 2.0f * k3.d) + k4.d);
  s.a = wrap(na);
  s.b = wrap(nb);
  s.c = clip(nc, -MAX_VEL_1, MAX_VEL_1);
  s.d = clip(nd, -MAX_VEL_2, MAX_VEL_2);
}

// acrobot_np.py:92-93: -cos(th1) - cos(th2 + th1) > 1.
__device__ __forceinline__ bool terminal(const S4& s) { return (-det_cos(s.a)) - det_cos(s.b + s.a) > 1.0f; }

__global__ __launch_bounds__(kBlock) void reset_kernel(float* __restrict__ state, uint32_t seed, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint32_t h = env_hash(seed, (uint32_t)i);
  state[i] = uniform_pm(pcg_hash(h), RESET_BOUND);
  state[n + i] = uniform_pm(pcg_hash(h + kRowOff1), RESET_BOUND);
  state[2 * n + i] = uniform_pm(pcg_hash(h + kRowOff2), RESET_BOUND);
  state[3 * n + i] = uniform_pm(pcg_hash(h + kRowOff3), RESET_BOUND);
}

__global__ __launch_bounds__(kBlock) void step_kernel(const float* __restrict__ state, const int32_t* __restrict__ action,
                                                      uint32_t seed, float* __restrict__ next, float* __restrict__ reward,
                                                      uint8_t* __restrict__ done, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  S4 s{state[i], state[n + i], state[2 * n + i], state[3 * n + i]};
  const float torque = (float)(stream_load(action + i) - 1);
  rk4(s, torque);
  const bool d = terminal(s);
  if (d) {  // fresh draws only on terminated lanes; the reference selects (acrobot_metal.py:76-80)
    const uint32_t h = env_hash(seed, (uint32_t)i);
    s.a = uniform_pm(pcg_hash(h), RESET_BOUND);
    s.b = uniform_pm(pcg_hash(h + kRowOff1), RESET_BOUND);
    s.c = uniform_pm(pcg_hash(h + kRowOff2), RESET_BOUND);
    s.d = uniform_pm(pcg_hash(h + kRowOff3), RESET_BOUND);
  }
  next[i] = s.a;
  next[n + i] = s.b;
  next[2 * n + i] = s.c;
  next[3 * n + i] = s.d;
  stream_store(d ? 0.0f : -1.0f, reward + i);
  stream_store((uint8_t)(d ? 1 : 0), done + i);
}

// Fused ES rollout: one thread per member, the member's 10H+3 weights in
// registers (es.unflatten layout: w1 (6, H), b1 (H), w2 (H, 3), b2 (3)),
// Gym's observation, first-index argmax over three torques, RK4 physics, stop
// at the first termination. acrobot_rollout_metal.py:21-58.
template <int H>
__global__ __launch_bounds__(64) void rollout_kernel(const float* __restrict__ state, const float* __restrict__ theta,
                                                     int64_t member_stride, int64_t p, int32_t horizon,
                                                     float out_sign, float* __restrict__ steps_out) {
  constexpr int D = 10 * H + 3;
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i >= p) return;
  const float* row = theta + i * member_stride;
  float w[D];
#pragma unroll
  for (int d = 0; d < D; ++d) w[d] = row[d];
  S4 s{state[i], state[p + i], state[2 * p + i], state[3 * p + i]};
  float steps = 0.0f;
  for (int32_t t = 0; t < horizon; ++t) {
    float o[6];
    det_sincos(s.a, &o[1], &o[0]);
    det_sincos(s.b, &o[3], &o[2]);
    o[4] = s.c;
    o[5] = s.d;
    float l0 = w[10 * H], l1 = w[10 * H + 1], l2 = w[10 * H + 2];
#pragma unroll
    for (int j = 0; j < H; ++j) {
      float pre = o[0] * w[j];
#pragma unroll
      for (int k = 1; k < 6; ++k) pre = pre + o[k] * w[k * H + j];
      const float h = det_tanh(pre + w[6 * H + j]);
      l0 = l0 + h * w[7 * H + 3 * j];
      l1 = l1 + h * w[7 * H + 3 * j + 1];
      l2 = l2 + h * w[7 * H + 3 * j + 2];
    }
    float torque = -1.0f, best = l0;
    if (l1 > best) { torque = 0.0f; best = l1; }
    if (l2 > best) { torque = 1.0f; }
    rk4(s, torque);
    if (terminal(s)) break;
    steps += 1.0f;
  }
  steps_out[i] = out_sign * steps + 0.0f;  // + 0: a score of -0 reads +0
}

// The same rollout with a group of kRolloutLanes lanes per member (four members to a
// single-wave workgroup), for populations that would fill only a fraction of the SIMDs with
// one member per lane: lane g computes hidden units g, g + 16, ... from the weights it holds;
// lanes 0..2 sum the three heads over all hidden values, read in order from the group's LDS
// row; observation and RK4 physics run identically on all 16 lanes. Same bits as the one-lane
// form.
constexpr int kRolloutLanes = 16;
constexpr int kRolloutMembers = 64 / kRolloutLanes;

// The group's physics, with the transcendentals and the two quotients by d1 spread over the
// group's lanes: lanes 0, 1, 2 evaluate one det_sincos each (one instruction stream for the
// three) and every lane of the 16-lane group (one DPP row) receives the results by row
// broadcast. Each value is the single-lane function's on the same argument, so the bits
// are those of dsdt/rk4/terminal.
struct GroupTrig {
  float sin_a, cos_a, sin_b, cos_b, cos_ab;  // theta1, theta2, theta2 + theta1
};

__device__ __forceinline__ GroupTrig group_trig(const S4& s, int g) {
  const float x = (g == 1) ? s.b : (g == 2) ? (s.b + s.a) : s.a;
  float sn, cs;
  det_sincos(x, &sn, &cs);
  return GroupTrig{group_bcast<0>(sn), group_bcast<0>(cs), group_bcast<1>(sn), group_bcast<1>(cs),
                   group_bcast<2>(cs)};
}

__device__ __forceinline__ S4 dsdt_group(const S4& s, float torque, int g) {
  const float x = (g == 1) ? ((s.a + s.b) - HALF_PI) : (g == 2) ? (s.a - HALF_PI) : s.b;
  float sn, cs;
  det_sincos(x, &sn, &cs);
  const float s2 = group_bcast<0>(sn), c2 = group_bcast<0>(cs);
  const float d1 = ((D1_C0 + (D1_C1 + c2)) + 1.0f) + 1.0f;
  const float d2 = (D2_C0 + D2_C1 * c2) + 1.0f;
  const float phi2 = PHI2_C * group_bcast<1>(cs);
  const float t1 = (PHI1_A * (s.d * s.d)) * s2;
  const float t2 = (s.d * s.c) * s2;
  const float t3 = PHI1_C * group_bcast<2>(cs);
  const float phi1 = ((t1 - t2) + t3) + phi2;
  const float q = ((g == 1) ? d2 * d2 : d2) / d1;  // lane 0: d2 / d1, lane 1: (d2 * d2) / d1
  const float num = ((torque + group_bcast<0>(q) * phi1) - (DD2_C * (s.c * s.c)) * s2) - phi2;
  const float den = DEN_C - group_bcast<1>(q);
  const float dd2 = num / den;
  const float dd1 = (-((d2 * dd2) + phi1)) / d1;
  return S4{s.c, s.d, dd1, dd2};
}

__device__ __forceinline__ void rk4_group(S4& s, float torque, int g) {
  const S4 k1 = dsdt_group(s, torque, g);
  const S4 k2 = dsdt_group(S4{s.a + DT_2 * k1.a, s.b + DT_2 * k1.b, s.c + DT_2 * k1.c, s.d + DT_2 * k1.d}, torque, g);
  const S4 k3 = dsdt_group(S4{s.a + DT_2 * k2.a, s.b + DT_2 * k2.b, s.c + DT_2 * k2.c, s.d + DT_2 * k2.d}, torque, g);
  const S4 k4 = dsdt_group(S4{s.a + DT * k3.a, s.b + DT * k3.b, s.c + DT * k3.c, s.d + DT * k3.d}, torque, g);
  const float na = s.a + DT_6 * (((k1.a + 2.0f * k2.a) + 2.0f * k3.a) + k4.a);
  const float nb = s.b + DT_6 * (((k1.b + 2.0f * k2.b) + 2.0f * k3.b) + k4.b);
  const float nc = s.c + DT_6 * (((k1.c + 2.0f * k2.c) + 2.0f * k3.c) + k4.c);
  const float nd = s.d + DT_6 * (((k1.d + 2.0f * k2.d) + 2.0f * k3.d) + k4.d);
  s.a = wrap(na);
  s.b = wrap(nb);
  s.c = clip(nc, -MAX_VEL_1, MAX_VEL_1);
  s.d = clip(nd, -MAX_VEL_2, MAX_VEL_2);
}

template <int H>
__global__ __launch_bounds__(64) void rollout_group_kernel(const float* __restrict__ state,
                                                           const float* __restrict__ theta, int64_t member_stride,
                                                           int64_t p, int32_t horizon, float out_sign,
                                                           float* __restrict__ steps_out) {
  constexpr int G = kRolloutLanes, U = (H + G - 1) / G;
  __shared__ float xp_all[kRolloutMembers * 3 * H];
  __shared__ float xl_all[kRolloutMembers * 4];
  const int g = (int)threadIdx.x % G, mloc = (int)threadIdx.x / G;
  float* xp = xp_all + mloc * 3 * H;  // head o's terms h_j * w2[j][o] at o * H + j
  float* xl = xl_all + mloc * 4;
  const int64_t i = (int64_t)blockIdx.x * kRolloutMembers + mloc;
  bool alive = i < p;
  const int64_t m = alive ? i : p - 1;  // a group past p steps member p - 1, unused
  const float* row = theta + m * member_stride;
  float w1[U][6], b1[U], w2[U][3];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = g + G * u < H ? g + G * u : 0;  // lanes past H recompute unit 0, unused
#pragma unroll
    for (int k = 0; k < 6; ++k) w1[u][k] = row[k * H + j];
    b1[u] = row[6 * H + j];
#pragma unroll
    for (int oo = 0; oo < 3; ++oo) w2[u][oo] = row[7 * H + 3 * j + oo];
  }
  const int o = g < 3 ? g : 0;
  const float b2 = row[10 * H + o];
  const float* xo = xp + o * H;
  S4 s{state[m], state[p + m], state[2 * p + m], state[3 * p + m]};
  float steps = 0.0f;
  int32_t t = 0;
  alive = alive && horizon > 0;
  GroupTrig tr = group_trig(s, g);  // the observation's trig; after each step also the termination's
  while (__any(alive)) {  // every lane steps, so the barriers and row broadcasts stay uniform
    float ob[6];
    ob[0] = tr.cos_a;
    ob[1] = tr.sin_a;
    ob[2] = tr.cos_b;
    ob[3] = tr.sin_b;
    ob[4] = s.c;
    ob[5] = s.d;
    // each lane forms its units' head terms h_j * w2[j][o], and lanes 0-2 add them in
    // order: the same products and sums as one lane summing l + h_j * w2[j][o], with the
    // multiplications spread over the group instead of repeated on the head lanes
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float pre = ob[0] * w1[u][0];
#pragma unroll
      for (int k = 1; k < 6; ++k) pre = pre + ob[k] * w1[u][k];
      const float h = det_tanh(pre + b1[u]);
      if (g + G * u < H) {
#pragma unroll
        for (int oo = 0; oo < 3; ++oo) xp[oo * H + g + G * u] = h * w2[u][oo];
      }
    }
    __syncthreads();
    if (g < 3) {
      float l = b2;
#pragma unroll
      for (int j = 0; j < H; ++j) l = l + xo[j];
      xl[g] = l;
    }
    __syncthreads();
    const float l0 = xl[0], l1 = xl[1], l2 = xl[2];
    __syncthreads();  // the group's rows are read before the next step writes them
    float torque = -1.0f, best = l0;
    if (l1 > best) { torque = 0.0f; best = l1; }
    if (l2 > best) { torque = 1.0f; }
    rk4_group(s, torque, g);
    tr = group_trig(s, g);
    const bool done = (-tr.cos_a) - tr.cos_ab > 1.0f;  // terminal(s)
    if (alive) {
      if (done) {
        alive = false;
      } else {
        steps += 1.0f;
        alive = ++t < horizon;
      }
    }
  }
  if (g == 0 && i < p) steps_out[i] = out_sign * steps + 0.0f;  // + 0: a score of -0 reads +0
}

// member_stride D and out_sign 1 for a population's rollout; stride 0 (one shared policy)
// and sign -1 for the greedy evaluation, whose per-env score is minus the steps.
template <int H>
int launch_rollout(const float* state, const float* theta, int64_t member_stride, int64_t p, int32_t horizon,
                   float out_sign, float* out, hipStream_t s) {
  int64_t limit = 0;
  const int status = group_rollout_limit(&limit);
  if (status != HIPENVS_OK) return status;
  if (p <= limit) {
    hipLaunchKernelGGL(rollout_group_kernel<H>, dim3((unsigned)((p + kRolloutMembers - 1) / kRolloutMembers)),
                       dim3(64), 0, s, state, theta, member_stride, p, horizon, out_sign, out);
  } else {
    hipLaunchKernelGGL(rollout_kernel<H>, dim3(grid_for(p, 64)), dim3(64), 0, s, state, theta, member_stride, p,
                       horizon, out_sign, out);
  }
  return launch_status();
}

template <int H>
int launch_rollout(const float* state, const float* theta, int64_t p, int32_t horizon, float* out, hipStream_t s) {
  return launch_rollout<H>(state, theta, (int64_t)(10 * H + 3), p, horizon, 1.0f, out, s);
}

}  // namespace ac
}  // namespace hipenvs

using namespace hipenvs;

extern "C" int hipenvs_acrobot_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && !state)) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(ac::reset_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, seed, n);
  return launch_status();
}

extern "C" int hipenvs_acrobot_step(const float* state, const int32_t* action, uint32_t seed, float* next_state,
                                    float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !action || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(ac::step_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, action, seed,
                     next_state, reward, done, n);
  return launch_status();
}

extern "C" int hipenvs_acrobot_es_rollout(const float* state, const float* theta, int64_t p, int32_t hidden,
                                          int32_t horizon, float* steps, hipenvs_stream_t stream) {
  if (p < 0 || horizon < 0 || (p > 0 && (!state || !theta || !steps))) return HIPENVS_E_ARG;
  if (p == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (hidden) {
    case 4: return ac::launch_rollout<4>(state, theta, p, horizon, steps, s);
    case 8: return ac::launch_rollout<8>(state, theta, p, horizon, steps, s);
    case 16: return ac::launch_rollout<16>(state, theta, p, horizon, steps, s);
    case 32: return ac::launch_rollout<32>(state, theta, p, horizon, steps, s);
    case 64: return ac::launch_rollout<64>(state, theta, p, horizon, steps, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int hipenvs_acrobot_es_rollout_seeded(const float* state, const float* theta, int64_t p, uint32_t seed,
                                                 double sigma, int32_t hidden, int32_t horizon, float* steps,
                                                 void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream) {
  if (p < 2 || (p & 1) || p > 0x7fffffffLL || horizon < 0 || !state || !theta || !steps || !workspace)
    return HIPENVS_E_ARG;
  if (hidden != 4 && hidden != 8 && hidden != 16 && hidden != 32 && hidden != 64) return HIPENVS_E_UNSUPPORTED;
  const int64_t d = 10 * (int64_t)hidden + 3;
  if (workspace_bytes < (int64_t)sizeof(float) * p * d) return HIPENVS_E_ARG;
  float* population = static_cast<float*>(workspace);  // (p, d) rows, written here, read by the rollout
  const int status = launch_perturb(theta, d, p, seed, (float)sigma, kPerturbRows, population, as_stream(stream));
  if (status != HIPENVS_OK) return status;
  return hipenvs_acrobot_es_rollout(state, population, p, hidden, horizon, steps, stream);
}

extern "C" int hipenvs_acrobot_evaluate(const float* state, const float* theta, int64_t n, int32_t hidden,
                                        int32_t steps, float* fitness, hipenvs_stream_t stream) {
  if (n < 0 || steps < 0 || (n > 0 && (!state || !theta || !fitness))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (hidden) {  // every env reads the one policy: member stride 0; score = -steps
    case 4: return ac::launch_rollout<4>(state, theta, 0, n, steps, -1.0f, fitness, s);
    case 8: return ac::launch_rollout<8>(state, theta, 0, n, steps, -1.0f, fitness, s);
    case 16: return ac::launch_rollout<16>(state, theta, 0, n, steps, -1.0f, fitness, s);
    case 32: return ac::launch_rollout<32>(state, theta, 0, n, steps, -1.0f, fitness, s);
    case 64: return ac::launch_rollout<64>(state, theta, 0, n, steps, -1.0f, fitness, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}
