// The C-legged body in the reference's own precision: legged_np.py:57-132 evaluated as
// numpy evaluates it, dtype promotions included.
//
// In hopper_np.py:100 the sliding sign `np.where(slip_p <= 0.0, 1.0, -1.0)` is a float64
// array (two Python floats), so every tangential impulse is float64. From there numpy
// promotes the Gauss-Seidel sums of the other contacts, the velocity update and the
// position update (legged_np.py:93-97), and the step returns a float64 state; every later
// substep and step is then float64 throughout (np.cos/np.sin of float64 angles included).
// From a float32 state the first substep is float32 up to its first contact solve.
//
// This file restates that flow. Each value has the dtype numpy gives it: T is the
// dtype of the substep's q and v (float for the first substep of a float32 state, double
// otherwise), a Python float constant takes the dtype of the array it meets (T(c)), and a
// float32 array meeting a float64 one is converted exactly before the float64 operation,
// which is C++'s own float/double promotion. Sums run in numpy's order, starting from
// Python's int 0 (sum() over a generator), and no term the reference multiplies by an
// exact zero or one is dropped. Transcendentals are the deterministic det_sincos
// (float32) and det_sincos64 (float64); division and sqrt are IEEE.
//
// It is the parity path, not the throughput path: legged.hip runs the Metal kernel's
// float32 arithmetic (legged_metal.py:13-155) for the env step and the rollouts.

#include "hipenvs_device.h"

namespace hipenvs {
namespace lgr {

constexpr int kSubsteps = 4;
// hopper_np.py:26-33 as Python floats
constexpr double kMF = 0.2, kIT = 0.1, kMT = 1.0, kL = 1.0, kG = 9.8, kH = 0.01, kMu = 0.7;
constexpr double kBaumgarteOverH = 0.2 / 0.01;  // BAUMGARTE / H, evaluated first in Python
constexpr double kFallHeight = 0.6, kFallAngle = 1.0;
constexpr float kTorque = 0x1p+1f;          // float32(2.0)
constexpr float kResetBound = 0x1.99999ap-5f;  // float32(0.05)

template <class T>
constexpr bool kF32 = sizeof(T) == sizeof(float);

__device__ __forceinline__ void sincos_t(float x, float* s, float* c) { det_sincos(x, s, c); }
__device__ __forceinline__ void sincos_t(double x, double* s, double* c) { det_sincos64(x, s, c); }

// np.maximum(x, 0.0): NaN propagates.
template <class T>
__device__ __forceinline__ T max0(T x) {
  return (x < T(0)) ? T(0) : x;
}

// a * x, where a is an array of dtype T and x an impulse held as a double: x32 marks an
// impulse that is a float32 array in numpy, whose product with a float32 array is rounded
// to float32.
template <class T>
__device__ __forceinline__ double times(T a, double x, bool x32) {
  if constexpr (kF32<T>) {
    if (x32) return (double)(a * (float)x);
  }
  return (double)a * x;
}

// contact_impulse (hopper_np.py:80-109) when wt and wn are float32 arrays: float32
// throughout except the float64 sign, so lt is float64 and ln float32.
__device__ __forceinline__ void impulse_f32(float Att, float Atn, float Ann, float wt, float wn, float depth,
                                            double& lt_out, double& ln_out) {
  const float mu = (float)kMu;
  const bool touching = depth >= 0.0f;
  const float target = (float)kBaumgarteOverH * max0(depth);
  const float det = Att * Ann - Atn * Atn;
  const float ln_stick = (Att * (target - wn) + Atn * wt) / det;
  const float lt_stick = ((-Ann) * wt - Atn * (target - wn)) / det;
  const bool sticks = fabsf(lt_stick) <= mu * ln_stick;
  const float den_p = Ann + mu * Atn, den_m = Ann - mu * Atn;
  const float ln_p = (den_p > 0.0f) ? max0((target - wn) / den_p) : 0.0f;
  const float ln_m = (den_m > 0.0f) ? max0((target - wn) / den_m) : 0.0f;
  const float slip_p = wt + (Att * mu + Atn) * ln_p;
  const double s = (slip_p <= 0.0f) ? 1.0 : -1.0;
  const float ln_slide = (slip_p <= 0.0f) ? ln_p : ln_m;
  const double lt_slide = (kMu * s) * (double)ln_slide;
  const float ln = sticks ? ln_stick : ln_slide;
  const double lt = sticks ? (double)lt_stick : lt_slide;
  const bool active = touching && (ln > 0.0f) && (wn < target);
  lt_out = active ? lt : 0.0;
  ln_out = active ? (double)ln : 0.0;
}

// contact_impulse when wt and wn are float64 arrays; the Delassus block and the depth
// have dtype T (float32 in the first substep of a float32 state).
template <class T>
__device__ __forceinline__ void impulse_f64(T Att, T Atn, T Ann, double wt, double wn, T depth, double& lt_out,
                                            double& ln_out) {
  const bool touching = depth >= T(0);
  const T target = T(kBaumgarteOverH) * max0(depth);
  const T det = Att * Ann - Atn * Atn;
  const double ln_stick = ((double)Att * ((double)target - wn) + (double)Atn * wt) / (double)det;
  const double lt_stick = ((double)(-Ann) * wt - (double)Atn * ((double)target - wn)) / (double)det;
  const bool sticks = fabs(lt_stick) <= kMu * ln_stick;
  const T den_p = Ann + T(kMu) * Atn, den_m = Ann - T(kMu) * Atn;
  const double ln_p = (den_p > T(0)) ? max0(((double)target - wn) / (double)den_p) : 0.0;
  const double ln_m = (den_m > T(0)) ? max0(((double)target - wn) / (double)den_m) : 0.0;
  const double slip_p = wt + (double)(Att * T(kMu) + Atn) * ln_p;
  const double s = (slip_p <= 0.0) ? 1.0 : -1.0;
  const double ln_slide = (slip_p <= 0.0) ? ln_p : ln_m;
  const double lt_slide = (kMu * s) * ln_slide;
  const double ln = sticks ? ln_stick : ln_slide;
  const double lt = sticks ? lt_stick : lt_slide;
  const bool active = touching && (ln > 0.0) && (wn < (double)target);
  lt_out = active ? lt : 0.0;
  ln_out = active ? ln : 0.0;
}

// pendulum_np.cholesky_solve (pendulum_np.py:85-107) against the factor Lo: b in, x out.
template <int N, class T>
__device__ __forceinline__ void chol_solve(const T (&Lo)[N][N], T (&b)[N]) {
  T y[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    T s = b[i];
#pragma unroll
    for (int p = 0; p < i; ++p) s = s - Lo[i][p] * y[p];
    y[i] = s / Lo[i][i];
  }
#pragma unroll
  for (int i = N - 1; i >= 0; --i) {
    T s = y[i];
#pragma unroll
    for (int p = i + 1; p < N; ++p) s = s - Lo[p][i] * b[p];
    b[i] = s / Lo[i][i];
  }
}

template <class T>
__device__ __forceinline__ T sqrt_t(T x) {
  if constexpr (kF32<T>)
    return __builtin_sqrtf(x);
  else
    return __builtin_sqrt(x);
}

// sum(r[i] * s[i] for i in range(n)), legged_np.py:85
template <int N, class T>
__device__ __forceinline__ T dot(const T (&r)[N], const T (&s)[N]) {
  T acc = T(0) + r[0] * s[0];
#pragma unroll
  for (int i = 1; i < N; ++i) acc = acc + r[i] * s[i];
  return acc;
}

// One substep (legged_np.py:57-97) from q, v of dtype T; the new q, v are float64 (iters >= 1).
template <int C, class T>
__device__ __forceinline__ void substep(const T (&q)[3 + C], const T (&v)[3 + C], const float (&tq)[C], int iters,
                                        double assist, double (&qo)[3 + C], double (&vo)[3 + C]) {
  constexpr int N = 3 + C;
  const T zero = T(0);
  const T one = zero + T(1.0);
  T Jt[C][N], Jn[C][N], dx[C], dy[C], depth[C];
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const T a = q[2] + q[3 + k];
    T sa, ca;
    sincos_t(a, &sa, &ca);
    const T ad = v[2] + v[3 + k];
    Jt[k][0] = one;
    Jt[k][1] = zero;
    Jt[k][2] = T(kL) * ca;
    Jn[k][0] = zero;
    Jn[k][1] = one;
    Jn[k][2] = T(kL) * sa;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      Jt[k][3 + j] = (j == k) ? T(kL) * ca : zero;
      Jn[k][3 + j] = (j == k) ? T(kL) * sa : zero;
    }
    dx[k] = ((T(-kL) * sa) * ad) * ad;
    dy[k] = ((T(kL) * ca) * ad) * ad;
    depth[k] = -(q[1] - T(kL) * ca);
  }
  // mass matrix (lower triangle; the expression is symmetric bit for bit) and forces
  T Lo[N][N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
#pragma unroll
    for (int j = 0; j <= i; ++j) {
      T s = T(0) + (Jt[0][i] * Jt[0][j] + Jn[0][i] * Jn[0][j]);
#pragma unroll
      for (int k = 1; k < C; ++k) s = s + (Jt[k][i] * Jt[k][j] + Jn[k][i] * Jn[k][j]);
      const double base = (i != j) ? 0.0 : (i < 2) ? kMT : (i == 2) ? kIT : 0.0;
      Lo[i][j] = T(base) + T(kMF) * s;
    }
  }
  T f[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    T s1 = T(0) + (Jt[0][i] * dx[0] + Jn[0][i] * dy[0]);
    T s2 = T(0) + Jn[0][i];
#pragma unroll
    for (int k = 1; k < C; ++k) {
      s1 = s1 + (Jt[k][i] * dx[k] + Jn[k][i] * dy[k]);
      s2 = s2 + Jn[k][i];
    }
    f[i] = T(-kMF) * s1 - T(kG) * (T(kMF) * s2 + T(i == 1 ? kMT : 0.0));
  }
#pragma unroll
  for (int k = 0; k < C; ++k) f[3 + k] = f[3 + k] + tq[k];
  f[2] = (f[2] - T(assist) * q[2]) - T(0.1 * assist) * v[2];
  // Cholesky (pendulum_np.py:88-94), then M^-1 f and the columns M^-1 J^T
#pragma unroll
  for (int i = 0; i < N; ++i) {
#pragma unroll
    for (int j = 0; j <= i; ++j) {
      T s = Lo[i][j];
#pragma unroll
      for (int p = 0; p < j; ++p) s = s - Lo[i][p] * Lo[j][p];
      Lo[i][j] = (i == j) ? sqrt_t(s) : s / Lo[j][j];
    }
  }
  chol_solve<N>(Lo, f);
  T vf[N];
#pragma unroll
  for (int i = 0; i < N; ++i) vf[i] = v[i] + T(kH) * f[i];
  T MiJt[C][N], MiJn[C][N];
#pragma unroll
  for (int k = 0; k < C; ++k) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      MiJt[k][i] = Jt[k][i];
      MiJn[k][i] = Jn[k][i];
    }
    chol_solve<N>(Lo, MiJt[k]);
    chol_solve<N>(Lo, MiJn[k]);
  }
  // Delassus blocks (tt, tn, nt, nn) and free contact velocities (legged_np.py:87-88)
  T Att[C][C], Atn[C][C], Ant[C][C], Ann[C][C], w0t[C], w0n[C];
#pragma unroll
  for (int k = 0; k < C; ++k) {
#pragma unroll
    for (int l = 0; l < C; ++l) {
      Att[k][l] = dot<N>(Jt[k], MiJt[l]);
      Atn[k][l] = dot<N>(Jt[k], MiJn[l]);
      Ant[k][l] = dot<N>(Jn[k], MiJt[l]);
      Ann[k][l] = dot<N>(Jn[k], MiJn[l]);
    }
    w0t[k] = dot<N>(Jt[k], vf);
    w0n[k] = dot<N>(Jn[k], vf);
  }
  // block Gauss-Seidel (legged_np.py:89-95). Impulses are held as doubles; ln32[l] marks an
  // ln that numpy holds as a float32 array (a solve whose velocities were float32: the first
  // contact of the first sweep from a float32 substep, and every sweep of a one-leg body).
  // Unsolved impulses are float32 zeros, whose products and sums are the same in either dtype.
  double lt[C], ln[C];
  bool ln32[C];
#pragma unroll
  for (int l = 0; l < C; ++l) {
    lt[l] = 0.0;
    ln[l] = 0.0;
    ln32[l] = false;
  }
#pragma unroll 1
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < C; ++k) {
      double st = 0.0, sn = 0.0;  // sum() starts from the int 0
#pragma unroll
      for (int l = 0; l < C; ++l) {
        if (l == k) continue;
        st = st + ((double)Att[k][l] * lt[l] + times(Atn[k][l], ln[l], ln32[l]));
        sn = sn + ((double)Ant[k][l] * lt[l] + times(Ann[k][l], ln[l], ln32[l]));
      }
      bool in32 = false;
      if constexpr (kF32<T>) in32 = (C == 1) || (it == 0 && k == 0);
      if (in32) {
        impulse_f32((float)Att[k][k], (float)Atn[k][k], (float)Ann[k][k], (float)w0t[k] + (float)st,
                    (float)w0n[k] + (float)sn, (float)depth[k], lt[k], ln[k]);
        ln32[k] = true;
      } else {
        impulse_f64<T>(Att[k][k], Atn[k][k], Ann[k][k], (double)w0t[k] + st, (double)w0n[k] + sn, depth[k], lt[k],
                       ln[k]);
        ln32[k] = false;
      }
    }
  }
  // v_new = v_free + sum_k (M^-1 J_t^T lt + M^-1 J_n^T ln); q + H v_new (legged_np.py:96-97)
#pragma unroll
  for (int i = 0; i < N; ++i) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < C; ++k) s = s + ((double)MiJt[k][i] * lt[k] + times(MiJn[k][i], ln[k], ln32[k]));
    vo[i] = (double)vf[i] + s;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) qo[i] = (double)q[i] + kH * vo[i];
}

// legged_np.Legged.step (legged_np.py:114-121) from a state of dtype TIn; the next state
// is float64, as numpy's. Reward (v_x + 1) rounded to float32, 0 on a fall; fallen envs get
// the counter-RNG reset of the float32 step (float32 values, stored exactly).
template <int C, class TIn>
__global__ __launch_bounds__(kBlock) void step_kernel(const TIn* __restrict__ state,
                                                      const int32_t* __restrict__ action, uint32_t seed,
                                                      const float* __restrict__ stand, int iters, double assist,
                                                      double* __restrict__ next, float* __restrict__ reward,
                                                      uint8_t* __restrict__ done, int64_t n) {
  constexpr int N = 3 + C;
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  TIn q0[N], v0[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q0[i] = state[i * n + e];
    v0[i] = state[(N + i) * n + e];
  }
  // leg k gets ((a / 3^k) % 3 - 1) * TORQUE in float32 (legged_np.py:51-54)
  float tq[C];
  int32_t a = action[e];
#pragma unroll
  for (int k = 0; k < C; ++k) {
    tq[k] = (float)(a % 3 - 1) * kTorque;
    a /= 3;
  }
  double q[N], v[N];
  substep<C, TIn>(q0, v0, tq, iters, assist, q, v);
#pragma unroll 1
  for (int s = 1; s < kSubsteps; ++s) {
    double qi[N], vi[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      qi[i] = q[i];
      vi[i] = v[i];
    }
    substep<C, double>(qi, vi, tq, iters, assist, q, v);
  }
  const bool d = (q[1] < kFallHeight) || (fabs(q[2]) > kFallAngle);
  reward[e] = d ? 0.0f : (float)(v[0] + 1.0);
  done[e] = d ? 1 : 0;
  if (d) {
    const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
    for (int i = 0; i < 2 * N; ++i) {
      const double fresh = (double)(stand[i] + uniform_pm(pcg_hash(h + (uint32_t)i * kRowStride), kResetBound));
      if (i < N)
        q[i] = fresh;
      else
        v[i - N] = fresh;
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) next[i * n + e] = q[i];
#pragma unroll
  for (int i = 0; i < N; ++i) next[(N + i) * n + e] = v[i];
}

template <int C>
int launch_step(bool f64_in, const void* state, const int32_t* action, uint32_t seed, const float* stand, int iters,
                double assist, double* next, float* reward, uint8_t* done, int64_t n, hipStream_t s) {
  if (f64_in)
    hipLaunchKernelGGL((step_kernel<C, double>), dim3(grid_for(n)), dim3(kBlock), 0, s,
                       static_cast<const double*>(state), action, seed, stand, iters, assist, next, reward, done, n);
  else
    hipLaunchKernelGGL((step_kernel<C, float>), dim3(grid_for(n)), dim3(kBlock), 0, s,
                       static_cast<const float*>(state), action, seed, stand, iters, assist, next, reward, done, n);
  return launch_status();
}

}  // namespace lgr
}  // namespace hipenvs

using namespace hipenvs;

extern "C" int hipenvs_legged_step_reference(int32_t c, int32_t iters, double assist, const void* state,
                                             int32_t state_is_f64, const int32_t* action, uint32_t seed,
                                             const float* stand, double* next_state, float* reward, uint8_t* done,
                                             int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || iters < 1 || iters > 4096 || (state_is_f64 != 0 && state_is_f64 != 1) ||
      (n > 0 && (!state || !action || !stand || !next_state || !reward || !done)))
    return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  const bool f64 = state_is_f64 != 0;
  switch (c) {
    case 1: return lgr::launch_step<1>(f64, state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 2: return lgr::launch_step<2>(f64, state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 3: return lgr::launch_step<3>(f64, state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 4: return lgr::launch_step<4>(f64, state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}
