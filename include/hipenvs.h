/*
 * hipenvs: the C ABI of the MI355X (gfx950) batched-environment library.
 *
 * Every entry point enqueues its kernel(s) on `stream` and returns without
 * synchronising; the caller owns the device boundary. The caller allocates
 * every buffer (device memory, fp32 structure-of-arrays state of shape
 * (rows, n), row-major, contiguous); the library allocates nothing, frees
 * nothing and keeps no per-call state, so any host thread may call it on any
 * stream (the one exception, hipenvs_es_update_static, keeps its partial sums
 * in a static device array). Inputs are never written.
 *
 * Return value: HIPENVS_OK (0), or a negative HIPENVS_E_* code. On
 * HIPENVS_E_HIP the launch failed and hipenvs_last_hip_error() gives the
 * hipError_t of the calling thread's most recent failure.
 *
 * RNG: `seed` is the per-call counter of the reference's step modules
 * (cartpole_metal.py:106-117 pre-increments it before each launch). Reset
 * noise for env i at counter s is pcg_hash((s ^ (i * 0x9E3779B9)) + row
 * offset), uniform from the top 24 bits (cartpole_metal.py:39-51,89-93).
 *
 * Each declaration names the reference interface it replaces (file:line in
 * metal-rl-envs).
 */
#ifndef HIPENVS_H
#define HIPENVS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipenvs_stream_t; /* a hipStream_t; NULL = the null stream */

enum {
  HIPENVS_OK = 0,
  HIPENVS_E_ARG = -1,         /* null pointer with n > 0, negative size, bad parameter */
  HIPENVS_E_UNSUPPORTED = -2, /* a compile-time shape (hidden, K links, C legs) with no instantiation */
  HIPENVS_E_HIP = -3,         /* the HIP launch failed; see hipenvs_last_hip_error() */
  HIPENVS_E_SCRATCH = -4      /* the shape needs more than a static-scratch entry point holds */
};

/* Library version and build description, e.g. "hipenvs 0.1 gfx950 fp-contract=off". */
const char* hipenvs_version(void);

/* hipError_t (as int) of this thread's last failed launch; 0 if none. */
int hipenvs_last_hip_error(void);

/* ---- CartPole ---------------------------------------------------------- */

/* Fresh states (4, n): what a reset column gets at counter `seed`.
 * Replaces cartpole_mlx.reset (cartpole_mlx.py:30-31), re-exported by
 * cartpole_metal.py:20; uses the kernel's counter RNG instead of MLX's. */
int hipenvs_cartpole_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream);

/* One Gym CartPole step for n envs with masked auto-reset.
 * state (4, n) f32, action (n) i32 (1 pushes right, anything else left)
 * -> next_state (4, n) f32, reward (n) f32 (= 1), done (n) u8 (0/1).
 * Replaces the `cartpole_step` Metal kernel and cartpole_metal.step
 * (cartpole_metal.py:69-125). */
int hipenvs_cartpole_step(const float* state, const int32_t* action, uint32_t seed,
                          float* next_state, float* reward, uint8_t* done,
                          int64_t n, hipenvs_stream_t stream);

/* k chained CartPole steps in one launch, state kept in registers. Step t
 * (0-based) uses counter seed + t and action actions[t * n + i], or, when
 * `actions` is NULL, the in-kernel Bernoulli(0.5) action
 * pcg_hash((seed + t) ^ (i * 0x9E3779B9) + 0x165667B1) >> 31.
 * rewards and dones are (k, n). Identical to k calls of hipenvs_cartpole_step.
 * No reference kernel: the semantic reference is a chain of k cartpole_metal.step
 * calls evaluated once (bench.py:48-61, bench_kernel.py:14-22). */
int hipenvs_cartpole_step_k(const float* state, const int32_t* actions, uint32_t seed, int32_t k,
                            float* next_state, float* rewards, uint8_t* dones,
                            int64_t n, hipenvs_stream_t stream);

/* Bernoulli(0.5) (m == 2) or uniform [0, m) actions (m <= 256) for counter `seed`:
 * bit 31, or ((h >> 8) * m) >> 24, of pcg_hash((seed ^ (i * 0x9E3779B9)) + 0x165667B1).
 * The device-side action sampler of the benchmark loop (bench.py:55 samples
 * mx.random.randint inside the loop). */
int hipenvs_sample_actions(int32_t* action, int64_t n, int32_t m, uint32_t seed, hipenvs_stream_t stream);

/* Fused ES rollout on CartPole: one thread per member runs its own 4-H-2 tanh
 * policy (row i of theta (p, 7*hidden+2) in es.unflatten's layout: w1 (4, H)
 * row-major, b1 (H), w2 (H, 2) row-major, b2 (2)) from state (4, p) for up to
 * `horizon` steps and writes the steps survived before its first termination
 * (the terminating step not counted) to fitness (p) f32. No auto-reset, no RNG.
 * hidden in {4, 8, 16, 32, 64}.
 * Replaces the `cartpole_es_rollout` Metal kernel and
 * cartpole_rollout_metal.rollout_steps (cartpole_rollout_metal.py:46-100). */
int hipenvs_cartpole_es_rollout(const float* state, const float* theta, int64_t p, int32_t hidden,
                                int32_t horizon, float* fitness, hipenvs_stream_t stream);

/* ---- Acrobot ----------------------------------------------------------- */

/* Fresh states (4, n) uniform in +-0.1 at counter `seed`.
 * Replaces acrobot_mlx.reset, re-exported by acrobot_metal.py:8. */
int hipenvs_acrobot_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream);

/* One Gym Acrobot step (book dynamics, RK4 dt 0.2, wrap, clip) with masked
 * auto-reset. state (4, n) f32 rows theta1, theta2, dtheta1, dtheta2; action (n)
 * i32 in {0, 1, 2} (torque action - 1) -> next_state (4, n), reward (n) f32
 * (-1, or 0 on done), done (n) u8.
 * Replaces the `acrobot_step` Metal kernel and acrobot_metal.step
 * (acrobot_metal.py:57-111). */
int hipenvs_acrobot_step(const float* state, const int32_t* action, uint32_t seed,
                         float* next_state, float* reward, uint8_t* done,
                         int64_t n, hipenvs_stream_t stream);

/* Fused ES rollout on Acrobot: 6-H-3 tanh policy on (cos th1, sin th1, cos th2,
 * sin th2, dth1, dth2), first-index argmax over torques (-1, 0, +1); theta is
 * (p, 10*hidden+3) in es.unflatten's layout. Writes the steps taken before the
 * tip first clears height 1 (horizon if never) to steps (p) f32.
 * hidden in {4, 8, 16, 32, 64}.
 * Replaces the `acrobot_es_rollout` Metal kernel and
 * acrobot_rollout_metal.rollout_steps (acrobot_rollout_metal.py:21-81). */
int hipenvs_acrobot_es_rollout(const float* state, const float* theta, int64_t p, int32_t hidden,
                               int32_t horizon, float* steps, hipenvs_stream_t stream);

/* ---- K-link pendulum, articulated-body algorithm ----------------------- */
/* k (links) in {1, 2, 3, 4, 8, 16, 32, 64}; state (2k, n) f32: absolute angles
 * then angular velocities. */

/* Fresh states: every row U[+-0.1] (zero_velocity == 0, the RK4 task's reset),
 * or angles U[+-0.1] and zero velocities (the Euler task's), at counter `seed`;
 * row p hashed at (seed ^ (i * 0x9E3779B9)) + p * 0x85EBCA6B.
 * Replaces pendulum_aba_mlx.Pendulum.reset (MLX RNG) used beside
 * pendulum_aba_metal.py:119-144. */
int hipenvs_pendulum_aba_reset(int32_t k, int32_t zero_velocity, float* state, int64_t n, uint32_t seed,
                               hipenvs_stream_t stream);

/* One RK4 step (dt 0.02) of the ABA dynamics, root torque action - 1 for action
 * (n) i32 in {0, 1, 2}, wrap, clip at 10 pi, terminate when -sum cos th > k/2,
 * reward -1 (0 on done), masked reset. Replaces the `pendulum{k}_aba_step` Metal
 * kernel and pendulum_aba_metal.Pendulum.step (pendulum_aba_metal.py:85-144). */
int hipenvs_pendulum_aba_step(int32_t k, const float* state, const int32_t* action, uint32_t seed,
                              float* next_state, float* reward, uint8_t* done, int64_t n,
                              hipenvs_stream_t stream);

/* One semi-implicit Euler step (dt 0.01): omega += dt * acc, theta += dt * omega,
 * with a continuous root torque torque (n) f32, or, when `torque` is NULL,
 * U[-1, 1) from pcg_hash((seed ^ (i * 0x9E3779B9)) + 0xD3A2646C). Same wrap,
 * clip, termination and reward as the RK4 step; resets to angles U[+-0.1] and
 * zero velocities. No reference kernel: the reference integrates with RK4 only
 * (pendulum_aba_np.py:117-123); this is the integrator of the K-link benchmark
 * configuration. */
int hipenvs_pendulum_aba_step_euler(int32_t k, const float* state, const float* torque, uint32_t seed,
                                    float* next_state, float* reward, uint8_t* done, int64_t n,
                                    hipenvs_stream_t stream);

/* Absolute angular accelerations acc (k, n) of state (2k, n) under root torque
 * (n): the ABA alone. Replaces pendulum_aba_np.aba_accelerations
 * (pendulum_aba_np.py:30-99) / the `aba<K>` Metal function
 * (pendulum_aba_metal.py:24-82). */
int hipenvs_pendulum_aba_accelerations(int32_t k, const float* state, const float* torque, float* acc,
                                       int64_t n, hipenvs_stream_t stream);

/* ---- K-link pendulum, mass-matrix form --------------------------------- */

/* One RK4 step of the K-link pendulum with the Lagrangian mass matrix
 * M_ij = mu_ij cos(th_i - th_j), mu_ij = k - max(i, j), solved by Cholesky at each
 * stage; otherwise the task of hipenvs_pendulum_aba_step (action, wrap, clip,
 * termination, reward, all-row reset). k in {1, 2, 3, 4, 8, 16}.
 * Replaces the `pendulum{K}_step` Metal kernel and pendulum_metal.Pendulum.step
 * (pendulum_metal.py:59-131, pendulum_np.py:50-82). */
int hipenvs_pendulum_step(int32_t k, const float* state, const int32_t* action, uint32_t seed,
                          float* next_state, float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream);

/* Absolute angular accelerations acc (k, n) from the mass-matrix solve.
 * Replaces pendulum_np.Pendulum._dsdt's solve (pendulum_np.py:68-79) / the `dsdt<K>`
 * Metal function (pendulum_metal.py:21-54). */
int hipenvs_pendulum_accelerations(int32_t k, const float* state, const float* torque, float* acc, int64_t n,
                                   hipenvs_stream_t stream);

/* ---- Hopper ------------------------------------------------------------- */

/* Fresh states (8, n): the standing pose (0, 1, 0, 0, 0, 0, 0, 0) plus U[+-0.05] on
 * every row at counter `seed`. Replaces hopper_mlx.Hopper.reset (hopper_mlx.py:19-20). */
int hipenvs_hopper_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream);

/* One hopper step: torque (action - 1) * 2 at the hip, four substeps of mass matrix,
 * 4x4 Cholesky, three solves and the exact single-contact impulse, reward v_x + 1
 * (0 on a fall), masked reset. state (8, n) q = (x, y, phi, psi) then velocities.
 * Replaces the `hopper_step` Metal kernel and hopper_metal.Hopper.step
 * (hopper_metal.py:84-138, hopper_np.py:117-138). */
int hipenvs_hopper_step(const float* state, const int32_t* action, uint32_t seed, float* next_state,
                        float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream);

/* ---- C-legged body with hard contacts ---------------------------------- */
/* state (2(3+c), n) f32: q = (x, y, phi, psi_1..psi_c), then the velocities.
 * `stand` is the standing pose (2(3+c)) f32 (legged_np.stand_pose). */

/* Fresh states stand + U[+-0.05] at counter `seed`, row j hashed at
 * (seed ^ (i * 0x9E3779B9)) + j * 0x85EBCA6B; c in {1, 2, 3, 4}.
 * Replaces legged_mlx.Legged.reset (legged_mlx.py:21-22). */
int hipenvs_legged_reset(int32_t c, const float* stand, float* state, int64_t n, uint32_t seed,
                         hipenvs_stream_t stream);

/* One control step: four semi-implicit Euler substeps of 0.01 s, each with a
 * dense Cholesky of the (3+c)^2 mass matrix and `iters` (0..4096) sweeps of
 * block projected Gauss-Seidel over the c contacts; action (n) i32 in
 * [0, 3^c); `assist` is the torso spring-damper stiffness (the stiffness and
 * 0.1 * assist are rounded to f32 from the double, as numpy does). Reward
 * forward velocity + 1, 0 on a fall (y < 0.6 or |phi| > 1); masked reset.
 * Replaces the `legged{c}_step` Metal kernel and legged_metal.Legged.step
 * (legged_metal.py:13-185). */
int hipenvs_legged_step(int32_t c, int32_t iters, double assist, const float* state, const int32_t* action,
                        uint32_t seed, const float* stand, float* next_state, float* reward, uint8_t* done,
                        int64_t n, hipenvs_stream_t stream);

/* The same control step in the reference's own arithmetic: legged_np.Legged.step
 * (legged_np.py:57-132) as numpy evaluates it. numpy makes the contact solve's
 * tangential impulse float64 (hopper_np.py:100) and promotes the velocities and the
 * state with it, so the next state is float64 (d, n) and a float64 state runs every
 * substep in float64; from a float32 state the first substep is float32 up to its
 * first contact solve. state is float32 (state_is_f64 == 0) or float64 (1);
 * next_state (2(3+c), n) f64; reward (v_x + 1 rounded to f32, 0 on a fall) and done
 * as hipenvs_legged_step, same reset. c in {1, 2, 3, 4}, iters 1..4096. The parity
 * path for the reference's numpy; hipenvs_legged_step is the Metal kernel's float32. */
int hipenvs_legged_step_reference(int32_t c, int32_t iters, double assist, const void* state, int32_t state_is_f64,
                                  const int32_t* action, uint32_t seed, const float* stand, double* next_state,
                                  float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream);

/* Fused ES rollout on the legged body: one thread per member runs its
 * (5+2c)-H-3c tanh policy (one three-way head per leg) and the physics for up
 * to `horizon` steps; fitness (p) = sum of ((v_x if y >= height_gate else 0) +
 * alive_bonus) until the first fall, minus fall_penalty at it; steps (p) = steps
 * taken including the falling one. layout 0: theta (p, D) rows in es.unflatten's
 * layout; layout 1: theta (D, p) columns. c in {1, 2, 3, 4}, hidden in
 * {4, 8, 16, 32, 64}, iters 0..4096.
 * Replaces the `legged_es_rollout` Metal kernel and legged_rollout_metal.rollout
 * (legged_rollout_metal.py:19-83), whose ITERS the reference fixes at 8. */
int hipenvs_legged_es_rollout(int32_t c, int32_t hidden, int32_t iters, int32_t layout, const float* state,
                              const float* theta, int64_t p, int32_t horizon, float alive_bonus,
                              float fall_penalty, float height_gate, double assist, float* fitness, float* steps,
                              hipenvs_stream_t stream);

/* Bytes of device workspace hipenvs_legged_es_rollout_chunked needs for p
 * members: two packed member sets of p rounded up to 64 slots (state, weights in
 * 64-member tiles, accumulators, ids) and two counters; -1 for an unsupported c
 * or hidden. */
int64_t hipenvs_legged_es_rollout_workspace_bytes(int32_t c, int32_t hidden, int64_t p);

/* The same rollout, scheduled in chunks of `chunk_steps` steps (for c <= 2 the
 * first chunk is 16 steps when chunk_steps is longer): after each
 * chunk the surviving members (state, accumulators and weights) are packed
 * into a dense column buffer in `workspace`, so later chunks run full waves
 * despite heavy-tailed episode lengths; the counts stay on the device and the
 * whole rollout is enqueued without a host round trip. theta_cols is (D, p)
 * columns; p < 2^31; workspace_bytes >= hipenvs_legged_es_rollout_workspace_bytes.
 * Results identical to hipenvs_legged_es_rollout. Calls that share a workspace
 * must not overlap. */
int hipenvs_legged_es_rollout_chunked(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                      const float* state, const float* theta_cols, int64_t p, int32_t horizon,
                                      float alive_bonus, float fall_penalty, float height_gate, double assist,
                                      float* fitness, float* steps, void* workspace, int64_t workspace_bytes,
                                      hipenvs_stream_t stream);

/* hipenvs_legged_es_rollout_chunked on the caller's theta_rows (p, D) in
 * es.unflatten's layout, the reference's own theta_pop (legged_rollout_metal.py:70-83,
 * es.py:152-164), with no transpose: the first chunk reads each member's row front to
 * back (16-byte loads at any 4-byte alignment; HIPENVS_E_ARG for a theta_rows that is not
 * 4-byte aligned) and fetches only live members' weights. The rows are addressed with
 * 32-bit byte offsets: HIPENVS_E_UNSUPPORTED when p * D * 4 >= 2^31 (use the columns
 * form). Results identical to hipenvs_legged_es_rollout_chunked on the transpose. */
int hipenvs_legged_es_rollout_chunked_rows(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                           const float* state, const float* theta_rows, int64_t p, int32_t horizon,
                                           float alive_bonus, float fall_penalty, float height_gate, double assist,
                                           float* fitness, float* steps, void* workspace, int64_t workspace_bytes,
                                           hipenvs_stream_t stream);

/* ---- Greedy evaluation of one policy ----------------------------------- */
/* The reference's evaluate (es.py:308-322) steps n fresh envs with the mean
 * policy for `steps` steps through the env step and sums, per env,
 * (reward - 1 + eval_bonus) while no termination has happened. These run the
 * whole loop in one launch with theta (D) shared by every env (es.unflatten's
 * layout), stopping each env at its first termination, which adds nothing,
 * and write the per-env sum to fitness (n) f32; its mean is the score.
 * hidden in {4, 8, 16, 32, 64}; the policy sums as the fused rollouts do. */

/* CartPole: reward 1, eval_bonus 1 -> steps survived.
 * Replaces evaluate with mean_policy for the CartPole task (es.py:302-322). */
int hipenvs_cartpole_evaluate(const float* state, const float* theta, int64_t n, int32_t hidden, int32_t steps,
                              float* fitness, hipenvs_stream_t stream);

/* Acrobot: reward -1, eval_bonus 1 -> minus the steps before the tip clears height 1.
 * Replaces evaluate for the Acrobot task (es.py:302-322). */
int hipenvs_acrobot_evaluate(const float* state, const float* theta, int64_t n, int32_t hidden, int32_t steps,
                             float* fitness, hipenvs_stream_t stream);

/* Legged body with c in {1, 2, 3, 4}, no assist: sum of ((v_x + 1) - 1) + eval_bonus
 * while standing (the reference's legged tasks use eval_bonus 0: forward distance).
 * Replaces evaluate for the legged tasks (es.py:302-322, legged_np.py:114-121). */
int hipenvs_legged_evaluate(int32_t c, int32_t hidden, int32_t iters, const float* state, const float* theta,
                            int64_t n, int32_t steps, float eval_bonus, float* fitness, hipenvs_stream_t stream);

/* ---- Seeded ES generation ---------------------------------------------- */
/* The reference's generation (es.py:218-227) draws half = (P/2, D) normals,
 * materialises eps = [half; -half] and theta + sigma * eps, and reduces
 * sum(ranks[:, None] * eps, 0) / (P * sigma). These entry points replace those
 * lines with noise regenerated from a counter RNG: member pair m has key
 * pcg(seed ^ pcg(m + 0x6A09E667)); weight pair j is Box-Muller on
 * h1 = pcg(key + 2j * 0x9E3779B9), h2 = pcg(key + (2j+1) * 0x9E3779B9) at
 * 24-bit fixed point (ln, sin, cos in float32 elementary operations), giving
 * eps[2j] = r cos, eps[2j+1] = r sin; member m + P/2 carries -eps[m].
 * p is even, 2 <= p < 2^31; sigma and lr are rounded to float32 as numpy
 * rounds Python scalars against float32 arrays. */

/* The population theta (d) + sigma * [eps; -eps] for p members into out:
 * layout 0 rows (p, d), layout 1 columns (d, p).
 * Replaces `theta[None, :] + cfg.sigma * eps` with its noise draw (es.py:219-222). */
int hipenvs_es_perturb(const float* theta, int64_t d, int64_t p, uint32_t seed, double sigma, int32_t layout,
                       float* out, hipenvs_stream_t stream);

/* Bytes of device workspace hipenvs_es_update needs (-1 for an unsupported shape). */
int64_t hipenvs_es_update_workspace_bytes(int64_t d, int64_t p);

/* theta_out (d) = theta + f32(lr) * (S / f32(p * sigma)), S[k] = sum over member pairs of
 * (ranks[m] - ranks[m + p/2]) * eps[m][k]: float32 partial sums over chunks of
 * 64 * ceil(p/2 / 16384) pairs in member order, then the partials in chunk order.
 * ranks (p) f32 are the centered ranks of the fitness. theta_out may alias theta.
 * Replaces the gradient and update lines of es.py:224-226. */
int hipenvs_es_update(const float* theta, const float* ranks, int64_t d, int64_t p, uint32_t seed, double sigma,
                      double lr, float* theta_out, void* workspace, int64_t workspace_bytes,
                      hipenvs_stream_t stream);

/* Bytes of the static device array behind hipenvs_es_update_static (2 MiB: the partial
 * sums of any population at d <= 2048, which covers every task's policy up to hidden 64). */
#define HIPENVS_ES_UPDATE_STATIC_BYTES (2 * 1024 * 1024)

/* hipenvs_es_update without a workspace argument and without any allocation: the
 * partial sums go to a file-scope device array of HIPENVS_ES_UPDATE_STATIC_BYTES that
 * each GPU holds until the process ends (its address is looked up once per device, on
 * the first call with that device current). Same results as hipenvs_es_update.
 * Returns HIPENVS_E_SCRATCH when hipenvs_es_update_workspace_bytes(d, p) exceeds the
 * array. Calls on one GPU share the array: calls that overlap on one GPU (different
 * streams, or host threads) race and must be ordered by the caller.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
int hipenvs_es_update_static(const float* theta, const float* ranks, int64_t d, int64_t p, uint32_t seed,
                             double sigma, double lr, float* theta_out, hipenvs_stream_t stream);

/* hipenvs_cartpole_es_rollout on the population of hipenvs_es_perturb (rows),
 * which is written to workspace (workspace_bytes >= 4 * p * (7*hidden+2)) and
 * never returned. Identical results to perturbing and rolling out separately.
 * Replaces MetalBackend.rollout of a materialised population
 * (es.py:222, es.py:263-267, cartpole_rollout_metal.py:88-100). */
int hipenvs_cartpole_es_rollout_seeded(const float* state, const float* theta, int64_t p, uint32_t seed,
                                       double sigma, int32_t hidden, int32_t horizon, float* fitness,
                                       void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream);

/* The same for Acrobot (workspace_bytes >= 4 * p * (10*hidden+3));
 * acrobot_rollout_metal.py:69-81. */
int hipenvs_acrobot_es_rollout_seeded(const float* state, const float* theta, int64_t p, uint32_t seed,
                                      double sigma, int32_t hidden, int32_t horizon, float* steps,
                                      void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream);

/* hipenvs_legged_es_rollout_chunked on the population of hipenvs_es_perturb, whose
 * weights are generated straight into the packed member tiles of the workspace
 * (same size: hipenvs_legged_es_rollout_workspace_bytes), so no (p, D) array
 * exists. Identical results to the chunked rollout of the perturbed columns.
 * legged_rollout_metal.py:70-83 with es.py:218-222. */
int hipenvs_legged_es_rollout_seeded(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                     const float* state, const float* theta, int64_t p, uint32_t seed,
                                     double sigma, int32_t horizon, float alive_bonus, float fall_penalty,
                                     float height_gate, double assist, float* fitness, float* steps,
                                     void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream);

/* ---- Diagnostics (no reference counterpart) ---------------------------- */

/* Elementwise deterministic sin, cos, tanh of x (n) as the kernels compute them;
 * used by the parity tests to check the device transcendentals bit for bit. */
int hipenvs_detmath(const float* x, float* sin_out, float* cos_out, float* tanh_out,
                    int64_t n, hipenvs_stream_t stream);

/* Elementwise q = a / d (n) computed as the legged kernels divide by a shared divisor:
 * through the float64 reciprocal of d, with an IEEE redo where that quotient came out
 * subnormal (marked (n) u8 = 1 there). q must equal IEEE float32 a / d everywhere; used
 * by the parity tests. */
int hipenvs_div_recip(const float* a, const float* d, float* q, uint8_t* marked, int64_t n,
                      hipenvs_stream_t stream);

/* For every float32 bit pattern first .. first + count - 1 (within 0 .. 2^32 - 1): the
 * kernels' square root (float64 reciprocal square root estimate and one Newton step,
 * rounded to float32) against IEEE sqrtf, and their float64 reciprocal (hardware estimate
 * and two Newton steps) against IEEE 1.0 / (double)x, bit for bit. Adds the mismatch
 * counts to counts[0] (square root) and counts[1] (reciprocal), device memory the caller
 * zeroes. */
int hipenvs_sqrt_recip_check(uint64_t first, uint64_t count, unsigned long long* counts,
                             hipenvs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HIPENVS_H */
