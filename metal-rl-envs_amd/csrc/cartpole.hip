// CartPole on MI355X: the single-step kernel, the K-step fused kernel, the
// reset kernel and the device action sampler, plus their C-ABI entry points.
//
// One thread per environment, state in VGPRs, SoA fp32 rows (x, x_dot, theta,
// theta_dot; row r of env i at r * n + i) so every access is coalesced. The physics is
// Gym's CartPole-v1 Euler step in the operation order of cartpole_np.py:58-76,
// termination cartpole_np.py:79-83, masked reset from the counter RNG exactly
// as cartpole_metal.py:84-95 writes it. Per env-step the single-step kernel
// moves 41 algorithmic bytes: 16 B state in, 4 B action, 16 B state out,
// 4 B reward, 1 B done.

#include "es_noise.h"

namespace hipenvs {
namespace cp {

constexpr float GRAVITY = 0x1.39999ap+3f;           // float32(9.8)
constexpr float POLE_MASS = 0x1.99999ap-4f;         // float32(0.1)
constexpr float TOTAL_MASS = 0x1.19999ap+0f;        // float32(1.0 + 0.1)
constexpr float HALF_POLE_LENGTH = 0x1p-1f;         // float32(0.5)
constexpr float POLE_MASS_LENGTH = 0x1.99999ap-5f;  // float32(0.1 * 0.5)
constexpr float FORCE_MAG = 0x1.4p+3f;              // float32(10.0)
constexpr float TAU = 0x1.47ae14p-6f;               // float32(0.02)
constexpr float FOUR_THIRDS = 0x1.555556p+0f;       // float32(4.0 / 3.0)
constexpr float X_LIMIT = 0x1.333334p+1f;           // float32(2.4)
constexpr float THETA_LIMIT = 0x1.aceeap-3f;        // float32(12 * 2 * pi / 360)
constexpr float RESET_BOUND = 0x1.99999ap-5f;       // float32(0.05)
constexpr double INV_TOTAL_MASS = 1.0 / (double)TOTAL_MASS;  // for div_const(x, .) == x / TOTAL_MASS

// One explicit-Euler step in place; returns the termination flag.
// cartpole_np.py:58-83, each line evaluated in numpy's order.
// `exact` false marks a lane whose results are discarded (see det_sincos_near_zero).
__device__ __forceinline__ bool advance(float& x, float& xd, float& th, float& thd, int32_t action,
                                        bool exact = true) {
  const float force = (action == 1) ? FORCE_MAG : -FORCE_MAG;
  float s, c;
  det_sincos_near_zero(th, &s, &c, exact);  // the pole angle stays within +-0.78 but for a terminating step
  const float temp = div_const(force + (POLE_MASS_LENGTH * (thd * thd)) * s, INV_TOTAL_MASS);
  const float theta_acc = (GRAVITY * s - c * temp) /
                          (HALF_POLE_LENGTH * (FOUR_THIRDS - div_const(POLE_MASS * (c * c), INV_TOTAL_MASS)));
  const float x_acc = temp - div_const((POLE_MASS_LENGTH * theta_acc) * c, INV_TOTAL_MASS);
  x = x + TAU * xd;
  xd = xd + TAU * x_acc;
  th = th + TAU * thd;
  thd = thd + TAU * theta_acc;
  return (fabsf(x) > X_LIMIT) || (fabsf(th) > THETA_LIMIT);
}

// Masked reset (cartpole_metal.py:86-93): a terminated env takes four fresh draws. The
// reference computes the draws for every env and selects; here they sit on the branch of
// the terminated lanes, so a wave in which no env terminates skips the four hashes.
__device__ __forceinline__ void reset_select(bool d, uint32_t h, float& x, float& xd, float& th, float& thd) {
  if (d) {
    x = uniform_pm(pcg_hash(h), RESET_BOUND);
    xd = uniform_pm(pcg_hash(h + kRowOff1), RESET_BOUND);
    th = uniform_pm(pcg_hash(h + kRowOff2), RESET_BOUND);
    thd = uniform_pm(pcg_hash(h + kRowOff3), RESET_BOUND);
  }
}

// ---- kernels ---------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void reset_kernel(float* __restrict__ state, uint32_t seed, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  float x = 0.f, xd = 0.f, th = 0.f, thd = 0.f;
  reset_select(true, env_hash(seed, (uint32_t)i), x, xd, th, thd);
  state[i] = x;
  state[n + i] = xd;
  state[2 * n + i] = th;
  state[3 * n + i] = thd;
}

// One env per thread, any n and alignment. At every batch size this beats packing four
// envs per thread into 16-byte accesses (2.96 vs 3.81 us at N = 2^18, 7.9 vs 9.3 us at
// 2^20): a step is short, and the extra waves hide more of the load latency.
// The four reset draws depend only on the seed and the env index, so they are computed
// for every env (as the reference's select does) while its state loads are in flight;
// the empty asm marks the draws as needed there, which keeps the compiler from sinking
// them past the physics, where they would add to the step's latency instead.
__global__ __launch_bounds__(kBlock) void step_kernel(const float* __restrict__ state, const int32_t* __restrict__ action,
                                                      uint32_t seed, float* __restrict__ next, float* __restrict__ reward,
                                                      uint8_t* __restrict__ done, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  float x = state[i], xd = state[n + i], th = state[2 * n + i], thd = state[3 * n + i];
  const int32_t a = stream_load(action + i);
  const uint32_t h = env_hash(seed, (uint32_t)i);
  float f0 = uniform_pm(pcg_hash(h), RESET_BOUND);
  float f1 = uniform_pm(pcg_hash(h + kRowOff1), RESET_BOUND);
  float f2 = uniform_pm(pcg_hash(h + kRowOff2), RESET_BOUND);
  float f3 = uniform_pm(pcg_hash(h + kRowOff3), RESET_BOUND);
  asm volatile("" : "+v"(f0), "+v"(f1), "+v"(f2), "+v"(f3));
  const bool d = advance(x, xd, th, thd, a);
  next[i] = d ? f0 : x;
  next[n + i] = d ? f1 : xd;
  next[2 * n + i] = d ? f2 : th;
  next[3 * n + i] = d ? f3 : thd;
  stream_store(1.0f, reward + i);
  stream_store((uint8_t)(d ? 1 : 0), done + i);
}

// k chained steps, one env per thread (any n): rewards and dones written per step as
// (k, n) rows, the state once at the end. One env per thread also wins here over four
// per thread (31.9 vs 44.3 us for k = 32 at N = 2^18): the loop is VALU-bound and more
// waves per SIMD keep the issue slots full.
template <bool kArrayActions>
__global__ __launch_bounds__(kBlock) void step_k_kernel(const float* __restrict__ state, const int32_t* __restrict__ actions,
                                                        uint32_t seed, int32_t k, float* __restrict__ next,
                                                        float* __restrict__ rewards, uint8_t* __restrict__ dones, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  float x = state[i], xd = state[n + i], th = state[2 * n + i], thd = state[3 * n + i];
  for (int32_t t = 0; t < k; ++t) {
    const uint32_t h = env_hash(seed + (uint32_t)t, (uint32_t)i);
    const int32_t a = kArrayActions ? stream_load(actions + (int64_t)t * n + i) : action_bit(h);
    const bool d = advance(x, xd, th, thd, a);
    reset_select(d, h, x, xd, th, thd);
    stream_store(1.0f, rewards + (int64_t)t * n + i);
    stream_store((uint8_t)(d ? 1 : 0), dones + (int64_t)t * n + i);
  }
  next[i] = x;
  next[n + i] = xd;
  next[2 * n + i] = th;
  next[3 * n + i] = thd;
}

__global__ __launch_bounds__(kBlock) void sample_actions_kernel(int32_t* __restrict__ action, int64_t n, uint32_t m,
                                                                uint32_t seed) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const uint32_t h = env_hash(seed, (uint32_t)i);
  action[i] = (m == 2u) ? action_bit(h) : action_uniform(h, m);
}

// Fused ES rollout: one thread per member, the member's 7H+2 weights in
// registers (es.unflatten layout: w1 (4, H), b1 (H), w2 (H, 2), b2 (2)), the
// 4-H-2 tanh policy with first-index argmax, the step physics, and an early
// exit at the first termination; writes the steps survived (the terminating
// step not counted). cartpole_rollout_metal.py:46-77. Member i's weights start
// at theta + i * member_stride: D for a population, 0 for one policy shared by
// every env (the greedy evaluation).
template <int H>
__global__ __launch_bounds__(64) void rollout_kernel(const float* __restrict__ state, const float* __restrict__ theta,
                                                     int64_t member_stride, int64_t p, int32_t horizon,
                                                     float* __restrict__ fitness) {
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (i >= p) return;
  constexpr int D = 7 * H + 2;
  const float* row = theta + i * member_stride;
  float w[D];
#pragma unroll
  for (int d = 0; d < D; ++d) w[d] = row[d];
  float x = state[i], xd = state[p + i], th = state[2 * p + i], thd = state[3 * p + i];
  float survived = 0.0f;
  for (int32_t t = 0; t < horizon; ++t) {
    float l0 = w[7 * H], l1 = w[7 * H + 1];
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const float pre = (((x * w[j] + xd * w[H + j]) + th * w[2 * H + j]) + thd * w[3 * H + j]) + w[4 * H + j];
      const float h = det_tanh(pre);
      l0 = l0 + h * w[5 * H + 2 * j];
      l1 = l1 + h * w[5 * H + 2 * j + 1];
    }
    if (advance(x, xd, th, thd, (l1 > l0) ? 1 : 0)) break;
    survived += 1.0f;
  }
  fitness[i] = survived;
}

// The same rollout with a group of kRolloutLanes lanes per member (four members to a
// single-wave workgroup), for populations that would fill only a fraction of the SIMDs with
// one member per lane: lane g computes hidden units g, g + 16, ... from the weights it holds;
// lanes 0 and 1 sum the two heads over all hidden values, read in order from the group's LDS
// row; the physics runs identically on all 16 lanes. A member's step then costs about a
// quarter of the one-lane form's instruction latency, and the results are the same bits.
constexpr int kRolloutLanes = 16;
constexpr int kRolloutMembers = 64 / kRolloutLanes;

template <int H>
__global__ __launch_bounds__(64) void rollout_group_kernel(const float* __restrict__ state,
                                                           const float* __restrict__ theta, int64_t member_stride,
                                                           int64_t p, int32_t horizon, float* __restrict__ fitness) {
  constexpr int G = kRolloutLanes, U = (H + G - 1) / G;
  __shared__ float xp_all[kRolloutMembers * 2 * H];
  __shared__ float xl_all[kRolloutMembers * 2];
  const int g = (int)threadIdx.x % G, mloc = (int)threadIdx.x / G;
  float* xp = xp_all + mloc * 2 * H;  // head o's terms h_j * w2[j][o] at o * H + j
  float* xl = xl_all + mloc * 2;
  const int64_t i = (int64_t)blockIdx.x * kRolloutMembers + mloc;
  bool alive = i < p;
  const int64_t m = alive ? i : p - 1;  // a group past p steps member p - 1, unused
  const float* row = theta + m * member_stride;
  float w1[U][4], b1[U], w2[U][2];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = g + G * u < H ? g + G * u : 0;  // lanes past H recompute unit 0, unused
#pragma unroll
    for (int k = 0; k < 4; ++k) w1[u][k] = row[k * H + j];
    b1[u] = row[4 * H + j];
    w2[u][0] = row[5 * H + 2 * j];
    w2[u][1] = row[5 * H + 2 * j + 1];
  }
  const int o = g < 2 ? g : 0;
  const float b2 = row[7 * H + o];
  const float* xo = xp + o * H;
  float x = state[m], xd = state[p + m], th = state[2 * p + m], thd = state[3 * p + m];
  float survived = 0.0f;
  int32_t t = 0;
  alive = alive && horizon > 0;
  while (__any(alive)) {  // every lane steps, so the barriers stay uniform
    // each lane forms its units' head terms h_j * w2[j][o], and lanes 0 and 1 add them in
    // order: the same products and sums as one lane summing l + h_j * w2[j][o], with the
    // multiplications spread over the group instead of repeated on the head lanes
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float pre = (((x * w1[u][0] + xd * w1[u][1]) + th * w1[u][2]) + thd * w1[u][3]) + b1[u];
      const float h = det_tanh(pre);
      if (g + G * u < H) {
        xp[g + G * u] = h * w2[u][0];
        xp[H + g + G * u] = h * w2[u][1];
      }
    }
    __syncthreads();
    if (g < 2) {
      float l = b2;
#pragma unroll
      for (int j = 0; j < H; ++j) l = l + xo[j];
      xl[g] = l;
    }
    __syncthreads();
    const float l0 = xl[0], l1 = xl[1];
    __syncthreads();  // the group's rows are read before the next step writes them
    // every member steps (no branch around the physics); the near-zero sin/cos vote counts
    // the live members alone, since a terminated member's results are discarded
    const bool done = advance(x, xd, th, thd, (l1 > l0) ? 1 : 0, alive);
    if (alive) {
      if (done) {
        alive = false;
      } else {
        survived += 1.0f;
        alive = ++t < horizon;
      }
    }
  }
  if (g == 0 && i < p) fitness[i] = survived;
}

template <int H>
int launch_rollout(const float* state, const float* theta, int64_t member_stride, int64_t p, int32_t horizon,
                   float* out, hipStream_t s) {
  int64_t limit = 0;
  const int status = group_rollout_limit(&limit);
  if (status != HIPENVS_OK) return status;
  if (p <= limit) {
    hipLaunchKernelGGL(rollout_group_kernel<H>, dim3((unsigned)((p + kRolloutMembers - 1) / kRolloutMembers)),
                       dim3(64), 0, s, state, theta, member_stride, p, horizon, out);
  } else {
    hipLaunchKernelGGL(rollout_kernel<H>, dim3(grid_for(p, 64)), dim3(64), 0, s, state, theta, member_stride, p,
                       horizon, out);
  }
  return launch_status();
}

template <int H>
int launch_rollout(const float* state, const float* theta, int64_t p, int32_t horizon, float* out, hipStream_t s) {
  return launch_rollout<H>(state, theta, (int64_t)(7 * H + 2), p, horizon, out, s);
}

}  // namespace cp
}  // namespace hipenvs

using namespace hipenvs;

extern "C" int hipenvs_cartpole_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && !state)) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(cp::reset_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, seed, n);
  return launch_status();
}

extern "C" int hipenvs_cartpole_step(const float* state, const int32_t* action, uint32_t seed, float* next_state,
                                     float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !action || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(cp::step_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, action, seed,
                     next_state, reward, done, n);
  return launch_status();
}

extern "C" int hipenvs_cartpole_step_k(const float* state, const int32_t* actions, uint32_t seed, int32_t k,
                                       float* next_state, float* rewards, uint8_t* dones, int64_t n,
                                       hipenvs_stream_t stream) {
  if (n < 0 || k < 0 || (n > 0 && (!state || !next_state || (k > 0 && (!rewards || !dones)))))
    return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  if (actions)
    hipLaunchKernelGGL(cp::step_k_kernel<true>, dim3(grid_for(n)), dim3(kBlock), 0, s, state, actions, seed, k,
                       next_state, rewards, dones, n);
  else
    hipLaunchKernelGGL(cp::step_k_kernel<false>, dim3(grid_for(n)), dim3(kBlock), 0, s, state, actions, seed, k,
                       next_state, rewards, dones, n);
  return launch_status();
}

extern "C" int hipenvs_sample_actions(int32_t* action, int64_t n, int32_t m, uint32_t seed, hipenvs_stream_t stream) {
  if (n < 0 || m < 1 || m > 256 || (n > 0 && !action)) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(cp::sample_actions_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), action, n,
                     (uint32_t)m, seed);
  return launch_status();
}

extern "C" int hipenvs_cartpole_es_rollout(const float* state, const float* theta, int64_t p, int32_t hidden,
                                           int32_t horizon, float* fitness, hipenvs_stream_t stream) {
  if (p < 0 || horizon < 0 || (p > 0 && (!state || !theta || !fitness))) return HIPENVS_E_ARG;
  if (p == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (hidden) {
    case 4: return cp::launch_rollout<4>(state, theta, p, horizon, fitness, s);
    case 8: return cp::launch_rollout<8>(state, theta, p, horizon, fitness, s);
    case 16: return cp::launch_rollout<16>(state, theta, p, horizon, fitness, s);
    case 32: return cp::launch_rollout<32>(state, theta, p, horizon, fitness, s);
    case 64: return cp::launch_rollout<64>(state, theta, p, horizon, fitness, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int hipenvs_cartpole_es_rollout_seeded(const float* state, const float* theta, int64_t p, uint32_t seed,
                                                 double sigma, int32_t hidden, int32_t horizon, float* fitness,
                                                 void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream) {
  if (p < 2 || (p & 1) || p > 0x7fffffffLL || horizon < 0 || !state || !theta || !fitness || !workspace)
    return HIPENVS_E_ARG;
  if (hidden != 4 && hidden != 8 && hidden != 16 && hidden != 32 && hidden != 64) return HIPENVS_E_UNSUPPORTED;
  const int64_t d = 7 * (int64_t)hidden + 2;
  if (workspace_bytes < (int64_t)sizeof(float) * p * d) return HIPENVS_E_ARG;
  float* population = static_cast<float*>(workspace);  // (p, d) rows, written here, read by the rollout
  const int status = launch_perturb(theta, d, p, seed, (float)sigma, kPerturbRows, population, as_stream(stream));
  if (status != HIPENVS_OK) return status;
  return hipenvs_cartpole_es_rollout(state, population, p, hidden, horizon, fitness, stream);
}

extern "C" int hipenvs_cartpole_evaluate(const float* state, const float* theta, int64_t n, int32_t hidden,
                                         int32_t steps, float* fitness, hipenvs_stream_t stream) {
  if (n < 0 || steps < 0 || (n > 0 && (!state || !theta || !fitness))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (hidden) {  // every env reads the one policy: member stride 0
    case 4: return cp::launch_rollout<4>(state, theta, 0, n, steps, fitness, s);
    case 8: return cp::launch_rollout<8>(state, theta, 0, n, steps, fitness, s);
    case 16: return cp::launch_rollout<16>(state, theta, 0, n, steps, fitness, s);
    case 32: return cp::launch_rollout<32>(state, theta, 0, n, steps, fitness, s);
    case 64: return cp::launch_rollout<64>(state, theta, 0, n, steps, fitness, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}
