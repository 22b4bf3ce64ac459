// The C-legged body with hard ground contacts on MI355X: the env step and the
// fused legged ES rollout, one thread per environment, everything in VGPRs.
//
// Physics: legged_np.py:57-97 in float32, operation by operation. Per substep:
// foot Jacobians (C sincos), the (3+C)^2 mass matrix, a dense Cholesky reused
// for the free velocity and the 2C columns M^-1 J^T, the C^2 Delassus blocks,
// `iters` sweeps of block projected Gauss-Seidel with the exact single-contact
// solve (hopper_np.py:80-109), semi-implicit Euler. Terms the reference
// multiplies by an exact zero or one are elided where that leaves every value
// unchanged (x * 1 = x, x + (+-0) = x); the order of every remaining operation
// is numpy's.
//
// The rollout runs each member's (5+2C)-H-3C tanh policy (one three-way head
// per leg) and the physics for the whole horizon (legged_rollout_metal.py:19-59).
// The member's weights are streamed from memory every step (D = 1,676 floats at
// C = 4, H = 64 do not fit in registers), either from es.unflatten's rows
// (P, D) or from a column layout (D, P) in which a wave's 64 members read 256
// contiguous bytes per weight.

#include <type_traits>

#include "es_noise.h"

namespace hipenvs {
namespace lg {

constexpr float M_F = 0x1.99999ap-3f;              // float32(0.2)
constexpr float I_T = 0x1.99999ap-4f;              // float32(0.1)
constexpr float GRAVITY = 0x1.39999ap+3f;          // float32(9.8)
constexpr float NEG_M_F = -0x1.99999ap-3f;         // float32(-0.2)
constexpr float H = 0x1.47ae14p-7f;                // float32(0.01)
constexpr float MU = 0x1.666666p-1f;               // float32(0.7)
constexpr float BAUMGARTE_OVER_H = 0x1.4p+4f;      // float32(0.2 / 0.01)
constexpr float FALL_HEIGHT = 0x1.333334p-1f;      // float32(0.6)
constexpr float FALL_ANGLE = 0x1p+0f;              // float32(1.0)
constexpr float RESET_BOUND = 0x1.99999ap-5f;      // float32(0.05)
constexpr float TORQUE = 0x1p+1f;                  // float32(2.0)
constexpr int SUBSTEPS = 4;

// np.maximum(x, 0.0): NaN propagates.
__device__ __forceinline__ float max0(float x) { return (x < 0.0f) ? 0.0f : x; }

// Exact impulse of one contact given its Delassus block and relative velocity
// (hopper_np.py:80-109), float32 throughout.
// The per-substep constants of one contact's diagonal Delassus block: the 2x2 determinant
// and the two cone-edge denominators with their float64 reciprocals, formed once per
// substep instead of once per sweep (the values are the same float32 numbers either way).
struct ContactBlock {
  float Att, Atn, Ann, det, den_p, den_m;
  double rdet, rden_p, rden_m;
};

__device__ __forceinline__ ContactBlock contact_block(float Att, float Atn, float Ann) {
  ContactBlock b;
  b.Att = Att;
  b.Atn = Atn;
  b.Ann = Ann;
  b.det = Att * Ann - Atn * Atn;
  b.den_p = Ann + MU * Atn;
  b.den_m = Ann - MU * Atn;
  b.rdet = recip(b.det);
  b.rden_p = recip(b.den_p);
  b.rden_m = recip(b.den_m);
  return b;
}

template <class Div>
__device__ __forceinline__ void contact_impulse(const ContactBlock& b, float wt, float wn, float depth,
                                                float& lt_out, float& ln_out, Div& div) {
  const float Att = b.Att, Atn = b.Atn, Ann = b.Ann;
  const bool touching = depth >= 0.0f;
  const float target = BAUMGARTE_OVER_H * max0(depth);
  const float tw = target - wn;
  const float ln_stick = div(Att * tw + Atn * wt, b.det, b.rdet);
  const float lt_stick = div((-Ann) * wt - Atn * tw, b.det, b.rdet);
  const bool sticks = fabsf(lt_stick) <= MU * ln_stick;
  // both cone quotients are formed whatever the signs of their denominators and selected
  // after (no branch); a subnormal mark from an unused one only costs an exact redo
  const float q_p = div(tw, b.den_p, b.rden_p);
  const float q_m = div(tw, b.den_m, b.rden_m);
  const float ln_p = (b.den_p > 0.0f) ? max0(q_p) : 0.0f;
  const float ln_m = (b.den_m > 0.0f) ? max0(q_m) : 0.0f;
  const float slip_p = wt + (Att * MU + Atn) * ln_p;
  const float s = (slip_p <= 0.0f) ? 1.0f : -1.0f;
  const float ln_slide = (slip_p <= 0.0f) ? ln_p : ln_m;
  const float lt_slide = (MU * s) * ln_slide;
  const float ln = sticks ? ln_stick : ln_slide;
  const float lt = sticks ? lt_stick : lt_slide;
  const bool active = touching && (ln > 0.0f) && (wn < target);
  lt_out = active ? lt : 0.0f;
  ln_out = active ? ln : 0.0f;
}

// Solve L L^T x = b in place (pendulum_np.py:95-107): forward then backward substitution.
// rL[i] = recip(L[i][i]): the 2N divisions of a solve share the N diagonal reciprocals.
template <int N, class Div>
__device__ __forceinline__ void chol_solve(const float (&L)[N][N], const double (&rL)[N], float (&b)[N], Div& div) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float s = b[i];
#pragma unroll
    for (int p = 0; p < i; ++p) s = s - L[i][p] * b[p];
    b[i] = div(s, L[i][i], rL[i]);
  }
#pragma unroll
  for (int i = N - 1; i >= 0; --i) {
    float s = b[i];
#pragma unroll
    for (int p = i + 1; p < N; ++p) s = s - L[p][i] * b[p];
    b[i] = div(s, L[i][i], rL[i]);
  }
}

// sa[k], ca[k] = lane k's sn, cs, for k < K, on every lane of the G-lane group.
template <int G, int K>
__device__ __forceinline__ void row_trig(float sn, float cs, float* sa, float* ca) {
  if constexpr (K > 0) {
    row_trig<G, K - 1>(sn, cs, sa, ca);
    sa[K - 1] = lane_bcast<G, K - 1>(sn);
    ca[K - 1] = lane_bcast<G, K - 1>(cs);
  }
}

// out[i] = lane i's x, for i < K, on every lane of the G-lane group.
template <int G, int K>
__device__ __forceinline__ void row_gather(float x, float* out) {
  if constexpr (K > 0) {
    row_gather<G, K - 1>(x, out);
    out[K - 1] = lane_bcast<G, K - 1>(x);
  }
}

// One semi-implicit Euler substep with block PGS contacts, in place (legged_np.py:57-97).
// kGroup = 0: one lane computes the whole substep. kGroup = G (8 or 16): the G lanes
// g = 0..G-1 of a member's group (a 16-lane DPP row or half of one) all hold the member's
// state and compute everything identically, except that lane g < C evaluates foot g's sin
// and cos, shared by DPP broadcast, the Gauss-Seidel sweeps and the velocity update split
// their independent work over the lanes (below), and lane g solves right-hand sides g,
// g + G, ... of the 2C + 1 triangular solves
// (the forces, then the tangent, then the normal Jacobian rows), exchanged through the
// group's LDS rows xs ((2C + 1) x 8 floats). Every value is computed by the same expression
// as in the one-lane form, so the results are the same bits. Callers keep the group's
// lanes in one single-wave workgroup, so the barriers order its LDS traffic.
// kHopperSum (C = 1 only) adds the impulse terms as the reference's hopper does,
// (v_free + M^-1 J_t^T lt) + M^-1 J_n^T ln (hopper_np.py:76), instead of the legged body's
// v_free + (M^-1 J_t^T lt + M^-1 J_n^T ln) (legged_np.py:95); otherwise the hopper is this
// body at C = 1 with one sweep.
// kStage (one-lane form only) parks the M^-1 J^T columns in LDS during the Gauss-Seidel
// sweeps, at xs[e * 64] for element e (xs points at the lane's own column of a 64-lane
// block), which frees 2C(3 + C) registers there; they are read back for the velocity update.
template <int C, class Div, int kGroup = 0, bool kHopperSum = false, bool kStage = false>
__device__ __forceinline__ void substep(float (&q)[3 + C], float (&v)[3 + C], const float (&tq)[C], int iters,
                                        float assist, float assist_damping, Div& div, float* xs = nullptr,
                                        int g = 0, float* xd = nullptr) {
  constexpr int N = 3 + C;
  float ca[C], sa[C], dx[C], dy[C], depth[C], r2[C];
  if constexpr (kGroup >= 4 && kGroup >= C) {
    // lane g < C evaluates foot g's sin and cos, shared by DPP broadcast within the group
    static_assert(C <= kGroup, "one lane per foot");
    float a = q[2] + q[3];
#pragma unroll
    for (int k = 1; k < C; ++k) a = (g == k) ? q[2] + q[3 + k] : a;
    float sn, cs;
    det_sincos(a, &sn, &cs);
    row_trig<kGroup, C>(sn, cs, sa, ca);
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k) det_sincos(q[2] + q[3 + k], &sa[k], &ca[k]);
  }
#pragma unroll
  for (int k = 0; k < C; ++k) {
    const float ad = v[2] + v[3 + k];
    dx[k] = ((-sa[k]) * ad) * ad;
    dy[k] = (ca[k] * ad) * ad;
    depth[k] = -(q[1] - ca[k]);
    r2[k] = ca[k] * ca[k] + sa[k] * sa[k];
  }
  // sums over the feet in the reference's order
  float s_ca = ca[0], s_sa = sa[0], s_r2 = r2[0], s_dx = dx[0], s_dy = dy[0], s_f2 = ca[0] * dx[0] + sa[0] * dy[0];
#pragma unroll
  for (int k = 1; k < C; ++k) {
    s_ca = s_ca + ca[k];
    s_sa = s_sa + sa[k];
    s_r2 = s_r2 + r2[k];
    s_dx = s_dx + dx[k];
    s_dy = s_dy + dy[k];
    s_f2 = s_f2 + (ca[k] * dx[k] + sa[k] * dy[k]);
  }
  // mass matrix, lower triangle (M_T = 1: base 1 + M_F * C on x and y)
  float L[N][N];
  const float mxy = 1.0f + M_F * (float)C;
  L[0][0] = mxy;
  L[1][0] = M_F * 0.0f;
  L[1][1] = mxy;
  L[2][0] = M_F * s_ca;
  L[2][1] = M_F * s_sa;
  L[2][2] = I_T + M_F * s_r2;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    L[3 + j][0] = M_F * ca[j];
    L[3 + j][1] = M_F * sa[j];
    L[3 + j][2] = M_F * r2[j];
#pragma unroll
    for (int i = 0; i < j; ++i) L[3 + j][3 + i] = M_F * 0.0f;
    L[3 + j][3 + j] = M_F * r2[j];
  }
  // generalised forces: bias, gravity, leg torques, torso assist
  float f[N];
  f[0] = NEG_M_F * s_dx;
  f[1] = NEG_M_F * s_dy - GRAVITY * (M_F * (float)C + 1.0f);
  f[2] = NEG_M_F * s_f2 - GRAVITY * (M_F * s_sa);
#pragma unroll
  for (int j = 0; j < C; ++j) {
    f[3 + j] = NEG_M_F * (ca[j] * dx[j] + sa[j] * dy[j]) - GRAVITY * (M_F * sa[j]);
    f[3 + j] = f[3 + j] + tq[j];
  }
  f[2] = (f[2] - assist * q[2]) - assist_damping * v[2];
  // Cholesky in place (pendulum_np.py:88-94), keeping each pivot's float64 reciprocal
  double rL[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
#pragma unroll
    for (int j = 0; j <= i; ++j) {
      float s = L[i][j];
#pragma unroll
      for (int p = 0; p < j; ++p) s = s - L[i][p] * L[j][p];
      if (i == j) {
        L[i][i] = sqrt_rn(s);
        rL[i] = recip(L[i][i]);
      } else {
        L[i][j] = div(s, L[j][j], rL[j]);
      }
    }
  }
  // M^-1 f and the M^-1 J^T columns
  float MiJt[C][N], MiJn[C][N];
  if constexpr (kGroup == 0) {
    chol_solve<N>(L, rL, f, div);
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        MiJt[k][i] = (i == 0) ? 1.0f : (i == 2 || i == 3 + k) ? ca[k] : 0.0f;
        MiJn[k][i] = (i == 1) ? 1.0f : (i == 2 || i == 3 + k) ? sa[k] : 0.0f;
      }
      chol_solve<N>(L, rL, MiJt[k], div);
      chol_solve<N>(L, rL, MiJn[k], div);
    }
  } else {
    constexpr int kRow = 8;  // LDS floats per right-hand side
    constexpr int kRhs = 2 * C + 1, kRounds = (kRhs + kGroup - 1) / kGroup;
    float b[kRounds][N];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      // lane g solves right-hand sides g, g + kGroup, ...; past 2C it solves the forces again, unused
      const int rhs = g + r * kGroup < kRhs ? g + r * kGroup : 0;
      const bool normal = rhs > C;
      const int k = normal ? rhs - 1 - C : rhs - 1;
      float ck = ca[0], sk = sa[0];
#pragma unroll
      for (int kk = 1; kk < C; ++kk) {
        ck = (k == kk) ? ca[kk] : ck;
        sk = (k == kk) ? sa[kk] : sk;
      }
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const bool on = (i == 2 || i == 3 + k);
        const float jt = (i == 0) ? 1.0f : on ? ck : 0.0f;
        const float jn = (i == 1) ? 1.0f : on ? sk : 0.0f;
        b[r][i] = (rhs == 0) ? f[i] : normal ? jn : jt;
      }
      chol_solve<N>(L, rL, b[r], div);
    }
    __syncthreads();  // the rows' previous readers are done
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      if (g + r * kGroup < kRhs) {
#pragma unroll
        for (int i = 0; i < N; ++i) xs[(g + r * kGroup) * kRow + i] = b[r][i];
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) f[i] = xs[i];
    // the M^-1 J^T columns stay in xs until the velocity update reads them
  }
  float vf[N];
#pragma unroll
  for (int i = 0; i < N; ++i) vf[i] = v[i] + H * f[i];
  // Delassus blocks A[k][l] = (Jt_k.MiJt_l, Jt_k.MiJn_l, Jn_k.MiJt_l, Jn_k.MiJn_l) and free velocities
  float Att[C][C], Atn[C][C], Ant[C][C], Ann[C][C], w0t[C], w0n[C];
  if constexpr (kGroup > 0) {
    // lane g < C^2 forms block (g / C, g % C) from the solved rows in xs, and a lane of a
    // diagonal block also forms its contact's ContactBlock; the group reads the C^2 blocks
    // (4 floats each) and the C contact blocks (12 floats each) back from xd
    constexpr int kRow = 8;
    constexpr int kBlocks = C * C, kRounds = (kBlocks + kGroup - 1) / kGroup;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int gr = g + r * kGroup;
      const int gb = gr < kBlocks ? gr : 0;  // lanes past C^2 form block 0 again, unused
      const int kb = gb / C, lb = gb % C;
      float ck = ca[0], sk = sa[0];
#pragma unroll
      for (int kk = 1; kk < C; ++kk) {
        ck = (kb == kk) ? ca[kk] : ck;
        sk = (kb == kk) ? sa[kk] : sk;
      }
      const float* rt = xs + (1 + lb) * kRow;
      const float* rn = xs + (1 + C + lb) * kRow;
      const float t2 = rt[2], t3 = rt[3 + kb], n2 = rn[2], n3 = rn[3 + kb];
      const float4 blk4 = make_float4((rt[0] + ck * t2) + ck * t3, (rn[0] + ck * n2) + ck * n3,
                                      (rt[1] + sk * t2) + sk * t3, (rn[1] + sk * n2) + sk * n3);
      if (gr < kBlocks) *reinterpret_cast<float4*>(xd + 4 * gr) = blk4;
      const ContactBlock own = contact_block(blk4.x, blk4.y, blk4.w);
      if (gr < kBlocks && kb == lb) {
        float* xc = xd + 4 * C * C + 12 * kb;
        *reinterpret_cast<float4*>(xc) = make_float4(own.det, own.den_p, own.den_m, 0.0f);
        *reinterpret_cast<double2*>(xc + 4) = make_double2(own.rdet, own.rden_p);
        *reinterpret_cast<double*>(xc + 8) = own.rden_m;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int l = 0; l < C; ++l) {
        const float4 e = *reinterpret_cast<const float4*>(xd + 4 * (k * C + l));
        Att[k][l] = e.x;
        Atn[k][l] = e.y;
        Ant[k][l] = e.z;
        Ann[k][l] = e.w;
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int l = 0; l < C; ++l) {
        Att[k][l] = (MiJt[l][0] + ca[k] * MiJt[l][2]) + ca[k] * MiJt[l][3 + k];
        Atn[k][l] = (MiJn[l][0] + ca[k] * MiJn[l][2]) + ca[k] * MiJn[l][3 + k];
        Ant[k][l] = (MiJt[l][1] + sa[k] * MiJt[l][2]) + sa[k] * MiJt[l][3 + k];
        Ann[k][l] = (MiJn[l][1] + sa[k] * MiJn[l][2]) + sa[k] * MiJn[l][3 + k];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < C; ++k) {
    w0t[k] = (vf[0] + ca[k] * vf[2]) + ca[k] * vf[3 + k];
    w0n[k] = (vf[1] + sa[k] * vf[2]) + sa[k] * vf[3 + k];
  }
  if constexpr (kStage) {
    static_assert(kGroup == 0, "staging is for the one-lane form");
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        xs[(k * N + i) * 64] = MiJt[k][i];
        xs[((C + k) * N + i) * 64] = MiJn[k][i];
      }
    }
    asm volatile("" ::: "memory");  // the columns live in LDS until the velocity update
  }
  // block projected Gauss-Seidel, fixed contact order (legged_np.py:88-93)
  float lt[C], ln[C];
  ContactBlock blk[C];
#pragma unroll
  for (int k = 0; k < C; ++k) {
    lt[k] = 0.0f;
    ln[k] = 0.0f;
    if constexpr (kGroup > 0) {
      const float* xc = xd + 4 * C * C + 12 * k;
      const float4 f4 = *reinterpret_cast<const float4*>(xc);
      const double2 d2 = *reinterpret_cast<const double2*>(xc + 4);
      blk[k] = ContactBlock{Att[k][k], Atn[k][k], Ann[k][k], f4.x, f4.y, f4.z,
                            d2.x, d2.y, *reinterpret_cast<const double*>(xc + 8)};
    } else {
      blk[k] = contact_block(Att[k][k], Atn[k][k], Ann[k][k]);
    }
  }
  if constexpr (kGroup >= 4) {
    // The member's lanes split each contact's independent work and share the results by
    // DPP broadcast: lane 1 forms the normal coupling sum and every other lane the tangential
    // one (each with its own coefficient rows), and lanes 0-3 form the four quotients of the
    // contact solve, ln_stick, lt_stick, (target - wn) / den_p and (target - wn) / den_m
    // (lanes 4 and up repeat lane 0's). Every broadcast value is the expression the one-lane
    // sweep evaluates, so the impulses are the same bits.
    // Each lane reads its own coefficients from the group's LDS blocks at a lane-dependent
    // offset (block (k, l) holds Att, Atn, Ant, Ann; contact k's block holds det, den_p,
    // den_m and then their float64 reciprocals), and negates by flipping the sign bit: no
    // per-lane selects, which the compiler had turned into exec-mask branches.
    const bool nrow = (g == 1);
    const int sel = (g == 2) ? 1 : (g == 3) ? 2 : 0;       // det, den_p, den_m
    const uint32_t neg = nrow ? 0x80000000u : 0u;
    const int oA = nrow ? 2 : 0, oB = nrow ? 3 : 1, oQ = nrow ? 1 : 0;  // Ant|Att, Ann|Atn, Atn|Att
    // Lanes 2 and 3 clamp their cone-edge quotients before the broadcast, as the contact solve
    // does after it: (den > 0) ? max0(q) : 0, that is 0 where den > 0 fails or q < 0, else q
    // (-0 and NaN pass, as in max0). Lanes 0 and 1 compare against -inf, which nothing is
    // below, and pass their stick quotients on unchanged. One clamp on two lanes replaces two
    // on every lane. No mask on the chain from the quotients to the impulses is combined on
    // the scalar unit, which would wait for the vector compare to complete: the gate's mask
    // is formed before the quotients, and the clamp and the gate are each one compare.
    const bool edge = (g == 2 || g == 3);
    const float qlo = edge ? 0.0f : -__builtin_inff();
    float cA[C][C], cB[C][C], w0x[C], qP[C], qQ[C], qd[C], slipc[C];
    bool qzero[C];
    double qr[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int l = 0; l < C; ++l) {
        cA[k][l] = xd[4 * (k * C + l) + oA];
        cB[k][l] = xd[4 * (k * C + l) + oB];
      }
      w0x[k] = nrow ? w0n[k] : w0t[k];
      // numerators qP * wt + qQ * tw: lane 0 Atn wt + Att tw, which is the reference's
      // Att tw + Atn wt (a rounded sum commutes); lane 1 (-Ann) wt + (-Atn) tw, which is
      // the reference's (-Ann) wt - Atn tw exactly (a - b = a + (-b))
      const float* xb = xd + 4 * (k * C + k);
      qP[k] = __uint_as_float(__float_as_uint(xb[oB]) ^ neg);
      qQ[k] = __uint_as_float(__float_as_uint(xb[oQ]) ^ neg);
      const float* xc = xd + 4 * C * C + 12 * k;
      qd[k] = xc[sel];
      qr[k] = *reinterpret_cast<const double*>(xc + 4 + 2 * sel);
      qzero[k] = edge && !(qd[k] > 0.0f);  // lane 2 holds den_p, lane 3 den_m
      // such a lane divides -1 by 1 instead, whose quotient the clamp sets to 0: the clamp
      // then needs no mask of its own (a mask combined on the scalar unit between the
      // quotient and its broadcast waits for the vector compare)
      qd[k] = qzero[k] ? 1.0f : qd[k];
      qr[k] = qzero[k] ? 1.0 : qr[k];
      slipc[k] = blk[k].Att * MU + blk[k].Atn;
    }
    // -1 in a register the compiler cannot see through: an impulse whose contact is not
    // pushing (open below) is gated as max(-1, ...) would be, by one compare of a select
    // rather than two compares combined on the scalar unit
    float neg_one = -1.0f;
    asm volatile("" : "+v"(neg_one));
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < C; ++k) {
        float wt, wn;
        if constexpr (C == 1) {
          wt = w0t[k];
          wn = w0n[k];
        } else {
          float sx = 0.0f;
          bool first = true;
#pragma unroll
          for (int l = 0; l < C; ++l) {
            if (l == k) continue;
            const float tx = cA[k][l] * lt[l] + cB[k][l] * ln[l];
            sx = first ? tx : sx + tx;
            first = false;
          }
          const float wx = w0x[k] + sx;
          wt = lane_bcast<kGroup, 0>(wx);
          wn = lane_bcast<kGroup, 1>(wx);
        }
        const bool touching = depth[k] >= 0.0f;
        const float target = BAUMGARTE_OVER_H * max0(depth[k]);
        const float tw = target - wn;
        const bool open = touching && (wn < target);  // known before the quotients
        const float num = qzero[k] ? -1.0f : edge ? tw : qP[k] * wt + qQ[k] * tw;
        const float quo = div(num, qd[k], qr[k]);
        const float qc = (quo < qlo) ? 0.0f : quo;
        const float ln_stick = lane_bcast<kGroup, 0>(qc);
        const float lt_stick = lane_bcast<kGroup, 1>(qc);
        const float ln_p = lane_bcast<kGroup, 2>(qc);
        const float ln_m = lane_bcast<kGroup, 3>(qc);
        const bool sticks = fabsf(lt_stick) <= MU * ln_stick;
        const float slip_p = wt + slipc[k] * ln_p;
        const float sgn = (slip_p <= 0.0f) ? 1.0f : -1.0f;
        const float ln_slide = (slip_p <= 0.0f) ? ln_p : ln_m;
        const float lt_slide = (MU * sgn) * ln_slide;
        const float lnv = sticks ? ln_stick : ln_slide;
        const float ltv = sticks ? lt_stick : lt_slide;
        const bool active = (open ? lnv : neg_one) > 0.0f;  // open && lnv > 0
        lt[k] = active ? ltv : 0.0f;
        ln[k] = active ? lnv : 0.0f;
      }
    }
  } else {
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < C; ++k) {
        float st = 0.0f, sn = 0.0f;
        bool first = true;
#pragma unroll
        for (int l = 0; l < C; ++l) {
          if (l == k) continue;
          const float tt = Att[k][l] * lt[l] + Atn[k][l] * ln[l];
          const float nn = Ant[k][l] * lt[l] + Ann[k][l] * ln[l];
          st = first ? tt : st + tt;
          sn = first ? nn : sn + nn;
          first = false;
        }
        const float wt = (C == 1) ? w0t[k] : w0t[k] + st;
        const float wn = (C == 1) ? w0n[k] : w0n[k] + sn;
        contact_impulse(blk[k], wt, wn, depth[k], lt[k], ln[k], div);
      }
    }
  }
  // v = v_free + sum_k M^-1 J_k^T lambda_k; q += h v
  if constexpr (kStage) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        MiJt[k][i] = xs[(k * N + i) * 64];
        MiJn[k][i] = xs[((C + k) * N + i) * 64];
      }
    }
  } else if constexpr (kGroup >= 3 + C && !kHopperSum) {
    // lane i < N forms velocity i (its sum over the contacts in the same order as below,
    // from its own column of the solved rows) and the DPP broadcast gives it to the group
    static_assert(3 + C <= kGroup, "one lane per velocity");
    constexpr int kRow = 8;
    asm volatile("" ::: "memory");  // read here, not held in registers through the sweeps
    const int i = g < N ? g : 0;  // lanes past N form velocity 0 again, unused
    float vfi = vf[0];
#pragma unroll
    for (int r = 1; r < N; ++r) vfi = (i == r) ? vf[r] : vfi;
    float si = xs[(1 + 0) * kRow + i] * lt[0] + xs[(1 + C + 0) * kRow + i] * ln[0];
#pragma unroll
    for (int k = 1; k < C; ++k) si = si + (xs[(1 + k) * kRow + i] * lt[k] + xs[(1 + C + k) * kRow + i] * ln[k]);
    float vn[N];
    row_gather<kGroup, N>(vfi + si, vn);
#pragma unroll
    for (int r = 0; r < N; ++r) {
      v[r] = vn[r];
      q[r] = q[r] + H * vn[r];
    }
    return;
  } else if constexpr (kGroup > 0) {
    constexpr int kRow = 8;
    asm volatile("" ::: "memory");  // read here, not held in registers through the sweeps
#pragma unroll
    for (int k = 0; k < C; ++k) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        MiJt[k][i] = xs[(1 + k) * kRow + i];
        MiJn[k][i] = xs[(1 + C + k) * kRow + i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float vn;
    if constexpr (kHopperSum) {
      static_assert(C == 1, "the hopper has one contact");
      vn = (vf[i] + MiJt[0][i] * lt[0]) + MiJn[0][i] * ln[0];
    } else {
      float s = MiJt[0][i] * lt[0] + MiJn[0][i] * ln[0];
#pragma unroll
      for (int k = 1; k < C; ++k) s = s + (MiJt[k][i] * lt[k] + MiJn[k][i] * ln[k]);
      vn = vf[i] + s;
    }
    v[i] = vn;
    q[i] = q[i] + H * vn;
  }
}

// One substep dividing through the shared float64 reciprocals; a lane on which a quotient
// came out subnormal (never met in practice) redoes the substep from its saved state with
// IEEE division, so the result is always the IEEE one.
template <int C, bool kHopperSum = false, bool kStage = false>
__device__ __forceinline__ void substep_exact(float (&q)[3 + C], float (&v)[3 + C], const float (&tq)[C], int iters,
                                              float assist, float assist_damping, float* stage = nullptr) {
  constexpr int N = 3 + C;
  float q0[N], v0[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q0[i] = q[i];
    v0[i] = v[i];
  }
  DivRecip fast;
  substep<C, DivRecip, 0, kHopperSum, kStage>(q, v, tq, iters, assist, assist_damping, fast, stage);
  if (fast.saw_subnormal()) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      q[i] = q0[i];
      v[i] = v0[i];
    }
    DivIEEE ieee;
    substep<C, DivIEEE, 0, kHopperSum, kStage>(q, v, tq, iters, assist, assist_damping, ieee, stage);
  }
}

// The group form of substep_exact: the fast divisions, and when any live lane of the wave saw
// a subnormal quotient the whole wave redoes the substep with IEEE division (identical bits
// wherever nothing was marked), which keeps the group's barriers in uniform control flow.
template <int C, int G>
__device__ __forceinline__ void substep_exact_group(float (&q)[3 + C], float (&v)[3 + C], const float (&tq)[C],
                                                    int iters, float assist, float assist_damping, float* xs, int g,
                                                    bool live, float* xd) {
  constexpr int N = 3 + C;
  float q0[N], v0[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q0[i] = q[i];
    v0[i] = v[i];
  }
  DivRecip fast;
  substep<C, DivRecip, G>(q, v, tq, iters, assist, assist_damping, fast, xs, g, xd);
  if (__any(live && fast.saw_subnormal())) {  // lanes of finished members step on, unused
#pragma unroll
    for (int i = 0; i < N; ++i) {
      q[i] = q0[i];
      v[i] = v0[i];
    }
    DivIEEE ieee;
    substep<C, DivIEEE, G>(q, v, tq, iters, assist, assist_damping, ieee, xs, g, xd);
  }
}

template <int C>
__device__ __forceinline__ bool fallen(const float (&q)[3 + C]) {
  return (q[1] < FALL_HEIGHT) || (fabsf(q[2]) > FALL_ANGLE);
}

// Minimum resident waves per SIMD the rollout kernels are compiled for (bounds their VGPRs).
#ifndef LEGGED_ROLLOUT_MIN_WAVES
#define LEGGED_ROLLOUT_MIN_WAVES 1
#endif
// The same for the first chunk of the compacting schedule, which streams every member's
// weights from HBM.
#ifndef LEGGED_FIRST_CHUNK_MIN_WAVES
#define LEGGED_FIRST_CHUNK_MIN_WAVES 1
#endif
// Whether the first chunk's column base is made opaque to the compiler every step (see
// rollout_chunk_kernel).
#ifndef LEGGED_FIRST_CHUNK_OPAQUE_COLUMNS
#define LEGGED_FIRST_CHUNK_OPAQUE_COLUMNS 1
#endif
// Whether the chunk kernels park the substep's M^-1 J^T columns in LDS during the
// Gauss-Seidel sweeps (substep's kStage, 14 KB per single-wave workgroup at C = 4). The
// sweeps hold the most registers; with the columns in LDS the C = 4 chunk kernels need about
// 210 instead of 263-271, so two waves share a SIMD and one streams weights while the other
// runs the physics (ES rollout at N = 262,144: 64.2 -> 61.3 ms at 8 sweeps, 89.2 -> 83.7 ms
// at 16). Forcing two waves without it spilled to scratch and ran slower (94 ms at 8).
#ifndef LEGGED_CHUNK_STAGE
#define LEGGED_CHUNK_STAGE 1
#endif
// Steps of the first chunk of the compacting schedule at C <= 2, when shorter than the chunk
// length (0: the chunk length). Most bipeds fall early (at N = 262,144, 8 sweeps, 17 % stand
// after 32 steps): compacting after 16 steps drops their rows from the weight stream sooner
// (ES rollout 27.8 -> 26.0 ms; 8, 12, 20 steps: 27.2, 26.1, 26.4 ms). The quadruped keeps the
// chunk length (16, 24, 40, 48 steps: 46.7, 47.0, 47.3, 48.8 against 46.5 ms).
#ifndef LEGGED_BIPED_FIRST_CHUNK_STEPS
#define LEGGED_BIPED_FIRST_CHUNK_STEPS 16
#endif
template <int C>
constexpr int32_t kFirstChunkSteps = C <= 2 ? LEGGED_BIPED_FIRST_CHUNK_STEPS : 0;
template <int C>
inline int32_t first_chunk_steps(int32_t chunk_steps) {
  return kFirstChunkSteps<C> > 0 && kFirstChunkSteps<C> < chunk_steps ? kFirstChunkSteps<C> : chunk_steps;
}

// Rows of the policy weights. FlatRows is es.unflatten's layout (es.py:152-164): w1 (OBS, HID)
// row-major, b1 (HID), w2 (HID, OUT) row-major, b2 (OUT), the layout callers pass in.
// UnitRows is the compacted sets' layout: hidden unit j's bias, its OBS input weights and
// its OUT head weights on 1 + OBS + OUT consecutive rows, then b2; a unit's rows then lie
// within one immediate-offset range of a single address (26 rows of 256 B at C = 4).
template <int OBS, int HID, int OUT>
struct FlatRows {
  static constexpr int w1(int i, int j) { return i * HID + j; }
  static constexpr int b1(int j) { return OBS * HID + j; }
  static constexpr int w2(int j, int o) { return OBS * HID + HID + j * OUT + o; }
  static constexpr int b2(int o) { return OBS * HID + HID + HID * OUT + o; }
};

template <int OBS, int HID, int OUT>
struct UnitRows {
  static constexpr int kUnit = 1 + OBS + OUT;
  static constexpr int b1(int j) { return j * kUnit; }
  static constexpr int w1(int i, int j) { return j * kUnit + 1 + i; }
  static constexpr int w2(int j, int o) { return j * kUnit + 1 + OBS + o; }
  static constexpr int b2(int o) { return HID * kUnit + o; }
};

// The member's (5+2C)-HID-3C tanh policy and per-leg torques (legged_rollout_metal.py:217-236).
// Every accumulator sums in the reference kernel's order (hidden unit j: bias, then the
// observations in order; head o: bias, then the hidden units in order).
// Weight row r of the member is w[r * stride]; Rows maps each weight to its row. kStride > 0
// fixes the stride at compile time (the compacted sets' 64-member tiles), so neighbouring
// rows are immediate offsets from one address instead of one 64-bit address add per load.
template <int C, int HID, template <int, int, int> class Rows = FlatRows, int kStride = 0>
__device__ __forceinline__ void policy_torques(const float* __restrict__ w, int64_t runtime_stride,
                                               const float (&q)[3 + C], const float (&v)[3 + C], float (&tq)[C]) {
  const int64_t stride = kStride > 0 ? (int64_t)kStride : runtime_stride;
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  using R = Rows<OBS, HID, OUT>;
  float obs[OBS];
#pragma unroll
  for (int k = 1; k < N; ++k) obs[k - 1] = q[k];
#pragma unroll
  for (int k = 0; k < N; ++k) obs[N - 1 + k] = v[k];
  float logit[OUT];
#pragma unroll
  for (int o = 0; o < OUT; ++o) logit[o] = w[R::b2(o) * stride];
  // kBatch hidden units at a time: their weights are loaded before the first use and a
  // scheduling barrier keeps them there, so the loads of a batch share one memory round
  // trip whatever the scheduler would otherwise interleave (left to itself it has waited on
  // the biped's weights one at a time). Two units at C = 4 keep two waves per SIMD (236
  // registers; four-unit batches took 318); four at C <= 2 (169 registers) match the
  // biped's rollout before this form (ES rollout 25.0 ms at 8 sweeps; two units: 25.5;
  // eight units, 227 registers, were no faster).
  constexpr int kWant = C <= 2 ? 4 : 2;
  constexpr int kBatch = kWant <= HID ? kWant : HID;
  static_assert(HID % kBatch == 0, "whole batches of hidden units");
#pragma unroll 2
  for (int j0 = 0; j0 < HID; j0 += kBatch) {
    float wb[kBatch][1 + OBS + OUT];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u;
      wb[u][0] = w[R::b1(j) * stride];
#pragma unroll
      for (int k = 0; k < OBS; ++k) wb[u][1 + k] = w[R::w1(k, j) * stride];
#pragma unroll
      for (int o = 0; o < OUT; ++o) wb[u][1 + OBS + o] = w[R::w2(j, o) * stride];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      float s = wb[u][0];
#pragma unroll
      for (int k = 0; k < OBS; ++k) s = s + obs[k] * wb[u][1 + k];
      const float hj = det_tanh(s);
#pragma unroll
      for (int o = 0; o < OUT; ++o) logit[o] = logit[o] + hj * wb[u][1 + OBS + o];
    }
  }
#pragma unroll
  for (int leg = 0; leg < C; ++leg) {
    float torque = -1.0f, best = logit[3 * leg];
    if (logit[3 * leg + 1] > best) { torque = 0.0f; best = logit[3 * leg + 1]; }
    if (logit[3 * leg + 2] > best) { torque = 1.0f; }
    tq[leg] = torque * TORQUE;
  }
}

// One member's row of the caller's (P, D) weights, read through a buffer resource over the
// whole array: row i starts at byte i * D * 4 (a per-lane offset in one VGPR), and a
// position within the row is a wave-uniform byte offset (an immediate, or a scalar past
// 4 KB). With flat pointers the compiler had kept one 64-bit address per load batch alive
// across the policy and spilled them (496 B/lane at two waves per SIMD). The row offset
// passes through an empty asm statement where the reader is made (once per step), so the
// loads, which read the same addresses every step, are not hoisted out of the step loop
// into registers. Requires P * D * 4 < 2^31 (checked by the caller); a read past the
// array returns 0.
struct MemberRow {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t lane_bytes;
  __device__ MemberRow(const float* base, int64_t total_floats, int64_t i, int d)
      : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, (int)(total_floats * 4), 0x00020000)),
        lane_bytes((uint32_t)(i * d * 4)) {
    asm volatile("" : "+v"(lane_bytes));
  }
  // floats [first, first + M) of the row into out: 16-byte loads, then one 8- or 4-byte load
  // for a remainder. A row starts at any 4-byte boundary (D may be odd); the hardware serves
  // dword-aligned 16-byte loads, which hipcc itself emits for 4-byte aligned float4 data.
  template <int M>
  __device__ __forceinline__ void load(int first, float* out) const {
#pragma unroll
    for (int m = 0; m + 4 <= M; m += 4) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)lane_bytes, (first + m) * 4, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[m + e] = __uint_as_float(x[e]);
    }
    constexpr int m = M / 4 * 4;
    if constexpr (M - m >= 2) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b64(rsrc, (int)lane_bytes, (first + m) * 4, 0);
      out[m] = __uint_as_float(x[0]);
      out[m + 1] = __uint_as_float(x[1]);
    }
    if constexpr ((M - m) % 2 == 1)
      out[M - 1] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)lane_bytes, (first + M - 1) * 4, 0));
  }
};

// policy_torques on the member's own row of the caller's (P, D) array, es.unflatten's
// layout (es.py:152-164): w1 (OBS, HID) input-major, b1 (HID), w2 (HID, OUT), b2 (OUT).
// The hidden sums run input-major: each unit's accumulator starts at its bias and adds
// obs_k * w1[k][j] for k in order, then the heads add h_j * w2[j][o] for j in order, the
// same operations in the same order per accumulator as policy_torques. A lane therefore
// reads its row front to back in vectors, and a wave fetches only its live members' rows:
// in the columns layout a 128-byte line holds one weight of 32 members and is fetched
// while any of them lives. Each batch's loads (one input's HID weights, or eight hidden
// units' heads) issue before their first use.
template <int C, int HID>
__device__ __forceinline__ void policy_torques_rows(const MemberRow& row, const float (&q)[3 + C],
                                                    const float (&v)[3 + C], float (&tq)[C]) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  using F = FlatRows<OBS, HID, OUT>;
  float obs[OBS];
#pragma unroll
  for (int k = 1; k < N; ++k) obs[k - 1] = q[k];
#pragma unroll
  for (int k = 0; k < N; ++k) obs[N - 1 + k] = v[k];
  float s[HID];
  row.load<HID>(F::b1(0), s);
#pragma unroll
  for (int k = 0; k < OBS; ++k) {
    float wk[HID];
    row.load<HID>(F::w1(k, 0), wk);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < HID; ++j) s[j] = s[j] + obs[k] * wk[j];
    __builtin_amdgcn_sched_barrier(0);
  }
  float logit[OUT];
  row.load<OUT>(F::b2(0), logit);
  constexpr int kHeads = HID >= 8 ? 8 : HID;  // hidden units per batch of head weights
#pragma unroll
  for (int j0 = 0; j0 < HID; j0 += kHeads) {
    float w2b[kHeads * OUT];
    row.load<kHeads * OUT>(F::w2(j0, 0), w2b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kHeads; ++u) {
      const float hj = det_tanh(s[j0 + u]);
#pragma unroll
      for (int o = 0; o < OUT; ++o) logit[o] = logit[o] + hj * w2b[u * OUT + o];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int leg = 0; leg < C; ++leg) {
    float torque = -1.0f, best = logit[3 * leg];
    if (logit[3 * leg + 1] > best) { torque = 0.0f; best = logit[3 * leg + 1]; }
    if (logit[3 * leg + 2] > best) { torque = 1.0f; }
    tq[leg] = torque * TORQUE;
  }
}

// The group form of policy_torques for a compacted member (UnitRows tile, stride 64): lane g
// of the G-lane group computes hidden units g, g + G, ...; lane o < 3C sums head o over all
// hidden units in order; the group exchanges the hidden values and the logits through its
// LDS rows xh (HID floats) and xl (3C floats). Sums in the same order as policy_torques.
template <int C, int HID, int G>
__device__ __forceinline__ void policy_group(const float* __restrict__ w, const float (&q)[3 + C],
                                             const float (&v)[3 + C], float (&tq)[C], float* xh, float* xl, int g) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  using R = UnitRows<OBS, HID, OUT>;
  constexpr int64_t kStride = 64;
  float obs[OBS];
#pragma unroll
  for (int k = 1; k < N; ++k) obs[k - 1] = q[k];
#pragma unroll
  for (int k = 0; k < N; ++k) obs[N - 1 + k] = v[k];
  constexpr int kUnits = (HID + G - 1) / G;
  // the weights of the lane's hidden units are loaded in two batches (one for fewer than
  // eight units), each before its first use: two memory round trips. Left to itself the
  // scheduler may wait out one round trip per weight; one batch of all sixteen units at
  // H = 64 holds 160-224 weights at once and made the biped's kernel spill.
  constexpr int kBatch = kUnits >= 8 ? kUnits / 2 : kUnits;
  static_assert(kUnits % kBatch == 0, "whole batches");
  float hs[kUnits];
#pragma unroll
  for (int u0 = 0; u0 < kUnits; u0 += kBatch) {
    float wu[kBatch][1 + OBS];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int j = g + G * (u0 + b) < HID ? g + G * (u0 + b) : 0;  // lanes past HID recompute unit 0, unused
      wu[b][0] = w[R::b1(j) * kStride];
#pragma unroll
      for (int k = 0; k < OBS; ++k) wu[b][1 + k] = w[R::w1(k, j) * kStride];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      float sj = wu[b][0];
#pragma unroll
      for (int k = 0; k < OBS; ++k) sj = sj + obs[k] * wu[b][1 + k];
      hs[u0 + b] = det_tanh(sj);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // the rows' previous readers are done
#pragma unroll
  for (int u = 0; u < kUnits; ++u)
    if (g + G * u < HID) xh[g + G * u] = hs[u];
  __syncthreads();
  // lane g sums heads g, g + G, ... over the hidden values in order; a head's HID weights are
  // loaded together (one memory round trip per head), at an offset the compiler cannot see
  // (zero) so that the loads stay here, not hoisted out of the caller's step loop; offsetting
  // w keeps the loads global (an opaque pointer would make them flat loads, which also wait
  // with the LDS traffic)
  int opaque_zero = 0;
  asm volatile("" : "+s"(opaque_zero));
  const float* wh = w + opaque_zero;
#pragma unroll
  for (int o = g; o < OUT; o += G) {
    float w2r[HID];
#pragma unroll
    for (int j = 0; j < HID; ++j) w2r[j] = wh[R::w2(j, o) * kStride];
    // all HID loads issue before the first use: left to itself the scheduler may pair each
    // load with its product and wait out one memory round trip per weight
    __builtin_amdgcn_sched_barrier(0);
    float lo = w[R::b2(o) * kStride];
#pragma unroll
    for (int j = 0; j < HID; ++j) lo = lo + xh[j] * w2r[j];
    xl[o] = lo;
  }
  __syncthreads();
#pragma unroll
  for (int leg = 0; leg < C; ++leg) {
    float torque = -1.0f, best = xl[3 * leg];
    if (xl[3 * leg + 1] > best) { torque = 0.0f; best = xl[3 * leg + 1]; }
    if (xl[3 * leg + 2] > best) { torque = 1.0f; }
    tq[leg] = torque * TORQUE;
  }
}

// kHopper (C = 1): the reference's hopper step (hopper_metal.py:84-125): torque
// (a - 1) * TORQUE for any action value, its impulse sum order, and the standing pose
// (0, L, 0, 0) with zero velocities built in (stand is not read).
template <int C, bool kHopper = false>
__global__ __launch_bounds__(kBlock) void step_kernel(const float* __restrict__ state,
                                                      const int32_t* __restrict__ action, uint32_t seed,
                                                      const float* __restrict__ stand, int iters, float assist,
                                                      float assist_damping, float* __restrict__ next,
                                                      float* __restrict__ reward, uint8_t* __restrict__ done,
                                                      int64_t n) {
  constexpr int N = 3 + C;
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  float q[N], v[N], tq[C];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = state[i * n + e];
    v[i] = state[(N + i) * n + e];
  }
  // leg k gets ((a / 3^k) % 3 - 1) * TORQUE (legged_np.py:51-54)
  int32_t a = stream_load(action + e);
  if constexpr (kHopper) {
    tq[0] = (float)(a - 1) * TORQUE;
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k) {
      tq[k] = (float)(a % 3 - 1) * TORQUE;
      a /= 3;
    }
  }
#pragma unroll 1
  for (int s = 0; s < SUBSTEPS; ++s) substep_exact<C, kHopper>(q, v, tq, iters, assist, assist_damping);
  const bool d = fallen<C>(q);
  stream_store(d ? 0.0f : v[0] + 1.0f, reward + e);
  stream_store((uint8_t)(d ? 1 : 0), done + e);
  if (d) {  // fresh draws only on fallen lanes; the reference selects (legged_metal.py:148-152)
    const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float pose = kHopper ? (i == 1 ? 1.0f : 0.0f) : stand[i];  // hopper: y = L = 1
      q[i] = pose + uniform_pm(pcg_hash(h + (uint32_t)i * kRowStride), RESET_BOUND);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float pose = kHopper ? 0.0f : stand[N + i];
      v[i] = pose + uniform_pm(pcg_hash(h + (uint32_t)(N + i) * kRowStride), RESET_BOUND);
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) next[i * n + e] = q[i];
#pragma unroll
  for (int i = 0; i < N; ++i) next[(N + i) * n + e] = v[i];
}

template <int C>
__global__ __launch_bounds__(kBlock) void reset_kernel(const float* __restrict__ stand, float* __restrict__ state,
                                                       uint32_t seed, int64_t n) {
  constexpr int N = 3 + C;
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
  for (int i = 0; i < 2 * N; ++i)
    state[i * n + e] = stand[i] + uniform_pm(pcg_hash(h + (uint32_t)i * kRowStride), RESET_BOUND);
}

// The hopper's reset (hopper_mlx.py:19-20 with the counter RNG of hopper_metal.py:118-120):
// the standing pose (0, L, 0, 0, 0, 0, 0, 0) plus U[+-0.05] on every row.
__global__ __launch_bounds__(kBlock) void hopper_reset_kernel(float* __restrict__ state, uint32_t seed, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  const uint32_t h = env_hash(seed, (uint32_t)e);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    state[i * n + e] = (i == 1 ? 1.0f : 0.0f) + uniform_pm(pcg_hash(h + (uint32_t)i * kRowStride), RESET_BOUND);
}

// Fused ES rollout (legged_rollout_metal.py:19-59). Weight d of member i is
// theta[i * D + d] (rows) or theta[d * p + i] (columns).
template <int C, int HID, bool kColumns>
__global__ __launch_bounds__(64, LEGGED_ROLLOUT_MIN_WAVES) void rollout_kernel(const float* __restrict__ state, const float* __restrict__ theta,
                                                     int64_t p, int32_t horizon, int iters, float alive, float fall,
                                                     float gate, float assist, float assist_damping,
                                                     float* __restrict__ fitness, float* __restrict__ steps_out) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  const int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (e >= p) return;
  const float* w = kColumns ? theta + e : theta + e * D;
  const int64_t stride = kColumns ? p : 1;
  float q[N], v[N], tq[C];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = state[i * p + e];
    v[i] = state[(N + i) * p + e];
  }
  float total = 0.0f, taken = 0.0f;
  for (int32_t t = 0; t < horizon; ++t) {
    policy_torques<C, HID>(w, stride, q, v, tq);
#pragma unroll 1
    for (int s = 0; s < SUBSTEPS; ++s) substep_exact<C>(q, v, tq, iters, assist, assist_damping);
    if (fallen<C>(q)) {
      taken += 1.0f;
      total = total - fall;
      break;
    }
    total = total + (((q[1] >= gate) ? v[0] : 0.0f) + alive);
    taken += 1.0f;
  }
  fitness[e] = total;
  steps_out[e] = taken;
}

// A compacted member's policy weights held in the registers of its G-lane group for the
// rest of its episode (the group tail runs one or two waves per SIMD, so the registers are
// there):
// lane g keeps the bias and input weights of hidden units g, g + G, ... and, for g < 3C, the
// weights of head g over every hidden unit. policy() then computes policy_group's sums, in
// the same order, without reading memory; loading the weights from the packed tile once
// replaces a dependent chain of memory round trips per step (the head sums' loads).
template <int C, int HID, int G>
struct ResidentPolicy {
  static constexpr int OBS = 5 + 2 * C, OUT = 3 * C, U = (HID + G - 1) / G;
  static_assert(OUT <= G, "one head per lane");
  float w1[U][OBS], b1[U], w2[HID], b2;

  // from a member's weights in a 64-member tile (UnitRows, stride 64), or with R = FlatRows
  // and kStride 1 from one policy in es.unflatten's layout
  template <class R = UnitRows<OBS, HID, OUT>, int64_t kStride = 64>
  __device__ __forceinline__ void load(const float* __restrict__ w, int g) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = g + G * u < HID ? g + G * u : 0;  // lanes past HID hold unit 0, unused
      b1[u] = w[R::b1(j) * kStride];
#pragma unroll
      for (int k = 0; k < OBS; ++k) w1[u][k] = w[R::w1(k, j) * kStride];
    }
    const int o = g < OUT ? g : 0;  // lanes past the heads hold head 0, unused
    b2 = w[R::b2(o) * kStride];
#pragma unroll
    for (int j = 0; j < HID; ++j) w2[j] = w[R::w2(j, o) * kStride];
  }

  __device__ __forceinline__ void policy(const float (&q)[3 + C], const float (&v)[3 + C], float (&tq)[C],
                                         float* xh, float* xl, int g) const {
    constexpr int N = 3 + C;
    float obs[OBS];
#pragma unroll
    for (int k = 1; k < N; ++k) obs[k - 1] = q[k];
#pragma unroll
    for (int k = 0; k < N; ++k) obs[N - 1 + k] = v[k];
    float hs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float sj = b1[u];
#pragma unroll
      for (int k = 0; k < OBS; ++k) sj = sj + obs[k] * w1[u][k];
      hs[u] = det_tanh(sj);
    }
    __syncthreads();  // the rows' previous readers are done
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (g + G * u < HID) xh[g + G * u] = hs[u];
    __syncthreads();
    if (g < OUT) {
      float lo = b2;
#pragma unroll
      for (int j = 0; j < HID; ++j) lo = lo + xh[j] * w2[j];
      xl[g] = lo;
    }
    __syncthreads();
#pragma unroll
    for (int leg = 0; leg < C; ++leg) {
      float torque = -1.0f, best = xl[3 * leg];
      if (xl[3 * leg + 1] > best) { torque = 0.0f; best = xl[3 * leg + 1]; }
      if (xl[3 * leg + 2] > best) { torque = 1.0f; }
      tq[leg] = torque * TORQUE;
    }
  }
};

// The greedy evaluation of one policy (es.py:308-322): every env runs the shared weights
// theta (D) without assist from its own start state for up to `steps` steps. While the body
// stands, the score adds the evaluation's term (reward - 1) + eval_bonus with the
// environment's reward v_x + 1 (legged_np.py:118-121); the step that falls adds nothing
// and ends the episode. All lanes read the same weight at once.
template <int C, int HID>
__global__ __launch_bounds__(64, LEGGED_ROLLOUT_MIN_WAVES) void evaluate_kernel(const float* __restrict__ state,
                                                                             const float* __restrict__ theta,
                                                                             int64_t n, int32_t steps, int iters,
                                                                             float eval_bonus,
                                                                             float* __restrict__ fitness) {
  constexpr int N = 3 + C;
  const int64_t e = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (e >= n) return;
  float q[N], v[N], tq[C];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = state[i * n + e];
    v[i] = state[(N + i) * n + e];
  }
  float total = 0.0f;
  for (int32_t t = 0; t < steps; ++t) {
    policy_torques<C, HID>(theta, 1, q, v, tq);
#pragma unroll 1
    for (int s = 0; s < SUBSTEPS; ++s) substep_exact<C>(q, v, tq, iters, 0.0f, 0.0f);
    if (fallen<C>(q)) break;
    total = total + (((v[0] + 1.0f) - 1.0f) + eval_bonus);
  }
  fitness[e] = total;
}

// Survivor weight copies. A one-row-at-a-time copy waits out a memory round trip per row
// (the compiler may not move a row's load above the previous row's store, which it cannot
// prove disjoint). These load kCopyBatch rows into registers before storing them, through
// pointers declared disjoint, so a member's D rows take D / kCopyBatch round trips.
constexpr int kCopyBatch = 32;

// n rows, row r at src[r * src_stride] -> dst[r * dst_stride]
__device__ __forceinline__ void copy_rows(float* __restrict__ dst, int64_t dst_stride,
                                          const float* __restrict__ src, int64_t src_stride, int n) {
  int r = 0;
  for (; r + kCopyBatch <= n; r += kCopyBatch) {
    float b[kCopyBatch];
#pragma unroll
    for (int i = 0; i < kCopyBatch; ++i) b[i] = src[(r + i) * src_stride];
#pragma unroll
    for (int i = 0; i < kCopyBatch; ++i) dst[(r + i) * dst_stride] = b[i];
  }
  for (; r < n; ++r) dst[r * dst_stride] = src[r * src_stride];
}

// A member's weights from the caller's FlatRows columns (row stride src_stride) to a
// UnitRows tile (row stride dst_stride): hidden unit j's 1 + OBS + OUT rows at a time.
template <int OBS, int HID, int OUT>
__device__ __forceinline__ void copy_flat_to_units(float* __restrict__ dst, int64_t dst_stride,
                                                   const float* __restrict__ src, int64_t src_stride) {
  using F = FlatRows<OBS, HID, OUT>;
  using T = UnitRows<OBS, HID, OUT>;
  constexpr int kUnit = T::kUnit;
#pragma unroll 2
  for (int j = 0; j < HID; ++j) {
    float b[kUnit];
    b[0] = src[F::b1(j) * src_stride];
#pragma unroll
    for (int k = 0; k < OBS; ++k) b[1 + k] = src[F::w1(k, j) * src_stride];
#pragma unroll
    for (int o = 0; o < OUT; ++o) b[1 + OBS + o] = src[F::w2(j, o) * src_stride];
#pragma unroll
    for (int r = 0; r < kUnit; ++r) dst[(T::b1(j) + r) * dst_stride] = b[r];
  }
  float b2[OUT];
#pragma unroll
  for (int o = 0; o < OUT; ++o) b2[o] = src[F::b2(o) * src_stride];
#pragma unroll
  for (int o = 0; o < OUT; ++o) dst[T::b2(o) * dst_stride] = b2[o];
}

// Compacting schedule for the fused rollout. Episode lengths are heavy-tailed
// (at the ES benchmark's shape the mean is ~43 steps while a few members last
// the whole horizon), and a one-member-per-lane launch keeps each wave busy
// until its longest member ends. Here the rollout runs in chunks of
// `chunk_steps` steps. Each chunk reads a packed set of members in the column
// layout (D, cap), so a wave's loads of one weight stay 256 contiguous bytes.
// The survivors of a chunk are appended to the other packed buffer, with their
// state, accumulators and weights, at slots taken from a wave-aggregated atomic
// counter. The first chunk reads the caller's state and columns directly.
// Counts stay on the device: later chunks run a grid-stride loop over whatever
// count the previous chunk left, so the whole rollout is enqueued without a
// host round trip. Every loop is bounded (a member runs at most `horizon`
// steps, a chunk at most `chunk_steps`), and each member's arithmetic is the
// same as in the one-member-per-lane kernel, whatever slot it lands in.
// A compacted member set. cap is a multiple of 64; the weights are stored in tiles of 64
// members, tile t holding (D, 64) columns: weight d of slot s at
// (s / 64) * D * 64 + d * 64 + s % 64, so a wave (one tile) reads weight d of its 64
// members as one coalesced 256-byte row at a compile-time stride.
struct Packed {
  float* state;      // (2N, cap): q then v
  float* theta;      // (cap / 64) tiles of (D, 64)
  float* acc;        // (2, cap): total, taken
  int32_t* meta;     // (2, cap): member id, steps done
  uint32_t* count;
};

constexpr int kTile = 64;

__host__ __device__ constexpr int64_t round_to_tile(int64_t n) { return (n + kTile - 1) / kTile * kTile; }

// The tail of a rollout: once at most wide_max members survive (about one wave per SIMD in
// this form), each compacted member gets a group of kTailLanes<C> lanes and runs to the end
// of its episode (policy_group, substep_exact_group), kTailMembers<C> members per wave. The
// group shortens one member's step, which is what bounds the tail. Results are those of the
// one-lane schedule, bit for bit.
// At C <= 2 every lane role fits in 8 lanes (2C + 1 solves, C^2 Delassus blocks, 3C heads),
// so eight members share a wave and the tail runs one wave per SIMD from 32 survivors per CU.
// With 16 lanes it ran two 4-member waves per SIMD from the same count, which share the
// SIMD's issue to the end of the horizon: biped ES rollout at N = 262,144 19.6 -> 17.9,
// 23.8 -> 21.7 and 32.4 -> 30.2 ms at 4, 8 and 16 sweeps. Eight lanes at two waves per SIMD
// from 64 per CU (LEGGED_SMALL_TAIL_WAVES 2, no group chunks) took 20.6, 25.5 and 35.2 ms.
#ifndef LEGGED_SMALL_TAIL_LANES
#define LEGGED_SMALL_TAIL_LANES 8
#endif
template <int C>
constexpr int kTailLanes = C <= 2 ? LEGGED_SMALL_TAIL_LANES : 16;
template <int C>
constexpr int kTailMembers = 64 / kTailLanes<C>;
// Above the tail's bound and up to this many survivors per CU, a chunk runs in the group form
// (rollout_group_chunk_kernel) instead of one member per lane, with LEGGED_GROUP_CHUNK_LANES
// lanes per member. With the split Gauss-Seidel sweeps (a 4-lane group broadcasts with one
// DPP quad move), 4 lanes and up to 64 per CU at one 16-member wave per SIMD (256 + 107
// registers; at two waves it spilled 444 B/lane) beat 8 lanes up to 48 per CU at one or two
// waves (ES rollout at N = 262,144, 8 sweeps: 44.5 -> 43.7 ms). Before those sweeps, 8 lanes
// had beaten 16 (57.2 -> 56.3 ms) and a spilling 4-lane form (56.0 against 50.0 ms).
#ifndef LEGGED_GROUP_CHUNK_MEMBERS_PER_CU
#define LEGGED_GROUP_CHUNK_MEMBERS_PER_CU 64
#endif
#ifndef LEGGED_GROUP_CHUNK_LANES
#define LEGGED_GROUP_CHUNK_LANES 4
#endif
constexpr int kChunkGroupLanes = LEGGED_GROUP_CHUNK_LANES;
// Waves per SIMD the group tail runs at; it takes over at 4 x kTailWaves x kTailMembers
// survivors per CU. With its members' weights in registers the 16-lane form needed 218 VGPRs
// at C = 2 (H = 64), so two waves shared a SIMD; at C = 4 it needs 256 VGPRs + 14 AGPRs, one
// wave per SIMD. (Reloading the weights every step instead fits two waves at C = 4, 206 VGPRs,
// but the ES rollout at N = 262,144 and 8 sweeps took 60.6 instead of 50.0 ms: a SIMD holding
// two long-lived members' waves steps each at part speed to the end of the horizon.)
#ifndef LEGGED_SMALL_TAIL_WAVES
#define LEGGED_SMALL_TAIL_WAVES 1
#endif
template <int C>
constexpr int kTailWaves = C > 2 ? 1 : kTailLanes<C> == 16 ? 2 : LEGGED_SMALL_TAIL_WAVES;
// Whether chunks between the tail's bound and LEGGED_GROUP_CHUNK_MEMBERS_PER_CU run in the
// group form. At C <= 2 the tail already takes over at 32 per CU; with 4-lane groups at one
// wave per SIMD the biped's group chunks between 32 and 64 per CU also pay (biped ES rollout
// at N = 262,144: 20.2 -> 19.7, 24.9 -> 24.1 and 35.2 -> 33.0 ms at 4, 8, 16 sweeps; the
// earlier 8-lane groups spilled at C = 2 and were slower than one member per lane).
template <int C>
constexpr bool kGroupChunks = true;
// LDS floats per member for the group substep's Delassus and contact blocks (xd)
template <int C>
constexpr int kBlockFloats = 4 * C * C + 12 * C;

// kChunk false: every member runs to the end of its episode. kChunk true: at most chunk_steps
// steps, then the survivors are appended to dst like rollout_chunk_kernel's (the member's
// group copies its weight rows).
template <int C, int HID, int G, bool kChunk>
__device__ __forceinline__ void rollout_group(const Packed& src, const Packed& dst, int64_t count, int64_t cap,
                                              int32_t chunk_steps, int32_t horizon, int iters, float alive_bonus,
                                              float fall, float gate, float assist, float assist_damping,
                                              float* __restrict__ fitness, float* __restrict__ steps_out,
                                              float* xs_all, float* xh_all, float* xl_all, float* xd_all) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  constexpr int M = 64 / G;  // members per single-wave workgroup
  static_assert(G == 4 || G == 8 || G == 16, "groups of 4, 8 or 16 lanes");
  const int g = (int)threadIdx.x % G, mloc = (int)threadIdx.x / G;
  float* xs = xs_all + mloc * (2 * C + 1) * 8;
  float* xd = xd_all + mloc * kBlockFloats<C>;
  float* xh = xh_all + mloc * HID;
  float* xl = xl_all + mloc * 16;
  for (int64_t mbase = (int64_t)blockIdx.x * M; mbase < count; mbase += (int64_t)gridDim.x * M) {
    const int64_t i = mbase + mloc;
    bool live = i < count;
    const int64_t slot = live ? i : mbase;  // a lane group past the count steps slot mbase, unused
    float q[N], v[N], tq[C];
#pragma unroll
    for (int r = 0; r < N; ++r) {
      q[r] = src.state[r * cap + slot];
      v[r] = src.state[(N + r) * cap + slot];
    }
    float total = src.acc[slot], taken = src.acc[cap + slot];
    const int32_t id = src.meta[slot];
    int32_t t = src.meta[cap + slot];
    const float* w = src.theta + (slot / kTile) * (int64_t)D * kTile + (slot % kTile);
    // the tail (which runs each member to the end at one wave per SIMD) keeps the member's
    // weights in registers; a group chunk reads them from its tile every step
    struct NoResident {};
    std::conditional_t<kChunk, NoResident, ResidentPolicy<C, HID, G>> resident;
    if constexpr (!kChunk) resident.load(w, g);
    // every lane steps while any member of the wave is live, so the barriers stay uniform
    for (int32_t k = 0; (!kChunk || k < chunk_steps) && __any(live); ++k) {
      if constexpr (kChunk)
        policy_group<C, HID, G>(w, q, v, tq, xh, xl, g);
      else
        resident.policy(q, v, tq, xh, xl, g);
#pragma unroll 1
      for (int sub = 0; sub < SUBSTEPS; ++sub)
        substep_exact_group<C, G>(q, v, tq, iters, assist, assist_damping, xs, g, live, xd);
      if (live) {
        ++t;
        bool finished;
        if (fallen<C>(q)) {
          taken += 1.0f;
          total = total - fall;
          finished = true;
        } else {
          total = total + (((q[1] >= gate) ? v[0] : 0.0f) + alive_bonus);
          taken += 1.0f;
          finished = t >= horizon;
        }
        if (finished) {
          if (g == 0) {
            fitness[id] = total;
            steps_out[id] = taken;
          }
          live = false;
        }
      }
    }
    if constexpr (kChunk) {
      // one slot per surviving member (its lane 0 counts), in lane order
      const unsigned long long m = __ballot(live && g == 0);
      if (m) {
        const int leader = __ffsll((long long)m) - 1;
        unsigned int slot0 = 0;
        if ((int)threadIdx.x == leader) slot0 = atomicAdd(dst.count, (unsigned int)__popcll(m));
        slot0 = __shfl(slot0, leader);
        if (live) {
          const int64_t to = (int64_t)slot0 + __popcll(m & ((1ull << (mloc * G)) - 1ull));
          if (g == 0) {
#pragma unroll
            for (int r = 0; r < N; ++r) {
              dst.state[r * cap + to] = q[r];
              dst.state[(N + r) * cap + to] = v[r];
            }
            dst.acc[to] = total;
            dst.acc[cap + to] = taken;
            dst.meta[to] = id;
            dst.meta[cap + to] = t;
          }
          float* wd = dst.theta + (to / kTile) * (int64_t)D * kTile + (to % kTile);
          copy_rows(wd + g * kTile, (int64_t)G * kTile, w + g * kTile, (int64_t)G * kTile, (D - g + G - 1) / G);
        }
      }
    }
  }
}

// LDS of the group kernels: per member, the solve rows, the Delassus and contact blocks, the
// hidden values and the head values.
#define LEGGED_GROUP_LDS(C, HID, M)                                                \
  __shared__ float xs_all[(M) * (2 * (C) + 1) * 8];                                \
  __shared__ __align__(16) float xd_all[(M) * kBlockFloats<(C)>];                  \
  __shared__ float xh_all[(M) * (HID)];                                            \
  __shared__ float xl_all[(M) * 16]

// The group tail as a kernel of its own, launched after every later chunk: it runs when the
// set holds at most wide_max members and exits at once otherwise (the chunk kernels do the
// opposite). Kept apart so that the one-lane kernel's code is compiled on its own.
template <int C, int HID>
__global__ __launch_bounds__(64, kTailWaves<C>) void rollout_tail_kernel(Packed src, int64_t cap, int32_t horizon, int iters,
                                                          float alive_bonus, float fall, float gate, float assist,
                                                          float assist_damping, float* __restrict__ fitness,
                                                          float* __restrict__ steps_out, int64_t wide_max) {
  const int64_t count = (int64_t)*src.count;
  if (count > wide_max) return;
  LEGGED_GROUP_LDS(C, HID, kTailMembers<C>);
  rollout_group<C, HID, kTailLanes<C>, false>(src, src, count, cap, horizon, horizon, iters, alive_bonus, fall, gate,
                                            assist, assist_damping, fitness, steps_out, xs_all, xh_all, xl_all,
                                            xd_all);
}

// The greedy evaluation (evaluate_kernel) with a group of kTailLanes<C> lanes per env, for
// batches of at most one wave per SIMD: one env per lane leaves most SIMDs idle there, and a
// policy that stands steps every env to the end at one lane's latency. The shared policy's
// weights are loaded into the group's registers once; the step is the group tail's (same
// bits as the one-lane kernel).
template <int C, int HID>
__global__ __launch_bounds__(64, kTailWaves<C>) void evaluate_group_kernel(const float* __restrict__ state,
                                                                          const float* __restrict__ theta,
                                                                          int64_t n, int32_t steps, int iters,
                                                                          float eval_bonus,
                                                                          float* __restrict__ fitness) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C, G = kTailLanes<C>, M = kTailMembers<C>;
  LEGGED_GROUP_LDS(C, HID, M);
  const int g = (int)threadIdx.x % G, mloc = (int)threadIdx.x / G;
  float* xs = xs_all + mloc * (2 * C + 1) * 8;
  float* xd = xd_all + mloc * kBlockFloats<C>;
  float* xh = xh_all + mloc * HID;
  float* xl = xl_all + mloc * 16;
  const int64_t e = (int64_t)blockIdx.x * M + mloc;
  bool live = e < n && steps > 0;
  const int64_t slot = e < n ? e : n - 1;  // a group past n steps env n - 1, unused
  float q[N], v[N], tq[C];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = state[i * n + slot];
    v[i] = state[(N + i) * n + slot];
  }
  ResidentPolicy<C, HID, G> policy;
  policy.template load<FlatRows<OBS, HID, OUT>, 1>(theta, g);
  float total = 0.0f;
  // every lane steps while any env of the wave is live, so the barriers stay uniform
  for (int32_t t = 0; t < steps && __any(live); ++t) {
    policy.policy(q, v, tq, xh, xl, g);
#pragma unroll 1
    for (int sub = 0; sub < SUBSTEPS; ++sub)
      substep_exact_group<C, G>(q, v, tq, iters, 0.0f, 0.0f, xs, g, live, xd);
    if (live) {
      if (fallen<C>(q))
        live = false;
      else
        total = total + (((v[0] + 1.0f) - 1.0f) + eval_bonus);
    }
  }
  if (g == 0 && e < n) fitness[e] = total;
}

// The group form for one chunk, G lanes per member, when the set holds more than lo and at
// most hi members (a wave or two per SIMD): the survivors go to dst as after a one-lane chunk.
template <int C, int HID, int G>
__global__ __launch_bounds__(64, G >= 8 ? 2 : 1) void rollout_group_chunk_kernel(Packed src, Packed dst, int64_t cap,
                                                                    int32_t chunk_steps, int32_t horizon, int iters,
                                                                    float alive_bonus, float fall, float gate,
                                                                    float assist, float assist_damping,
                                                                    float* __restrict__ fitness,
                                                                    float* __restrict__ steps_out, int64_t lo,
                                                                    int64_t hi) {
  const int64_t count = (int64_t)*src.count;
  if (count <= lo || count > hi) return;
  LEGGED_GROUP_LDS(C, HID, 64 / G);
  rollout_group<C, HID, G, true>(src, dst, count, cap, chunk_steps, horizon, iters, alive_bonus, fall, gate, assist,
                                 assist_damping, fitness, steps_out, xs_all, xh_all, xl_all, xd_all);
}

// kRows (first chunk only): theta0 is the caller's (P, D) rows instead of its (D, P) columns.
template <int C, int HID, bool kFirst, bool kRows = false>
__global__ __launch_bounds__(64, kFirst ? LEGGED_FIRST_CHUNK_MIN_WAVES : LEGGED_ROLLOUT_MIN_WAVES) void rollout_chunk_kernel(const float* __restrict__ state0,
                                                           const float* __restrict__ theta0, int64_t p,
                                                           Packed src, Packed dst, int64_t cap,
                                                           int32_t chunk_steps, int32_t horizon, int iters,
                                                           float alive_bonus, float fall, float gate, float assist,
                                                           float assist_damping, float* __restrict__ fitness,
                                                           float* __restrict__ steps_out, int64_t group_max) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  constexpr bool kStage = LEGGED_CHUNK_STAGE != 0;
  __shared__ float stage_lds[kStage ? 2 * C * N * 64 : 1];
  const unsigned lane = threadIdx.x;
  const int64_t count = kFirst ? p : (int64_t)*src.count;
  if (!kFirst && count <= group_max) return;  // a group kernel takes the set (the same count everywhere)
  const int64_t src_stride = kFirst ? p : cap;  // state rows; the weights use tiles after the first chunk
  const float* sstate = kFirst ? state0 : src.state;
  const float* stheta = kFirst ? theta0 : src.theta;
  for (int64_t base = (int64_t)blockIdx.x * 64; base < count; base += (int64_t)gridDim.x * 64) {
    const int64_t i = base + lane;
    bool live = i < count;
    float q[N], v[N], tq[C];
    float total = 0.0f, taken = 0.0f;
    int32_t id = 0, t = 0;
    if (live) {
#pragma unroll
      for (int r = 0; r < N; ++r) {
        q[r] = sstate[r * src_stride + i];
        v[r] = sstate[(N + r) * src_stride + i];
      }
      if (kFirst) {
        id = (int32_t)i;
      } else {
        total = src.acc[i];
        taken = src.acc[cap + i];
        id = src.meta[i];
        t = src.meta[cap + i];
      }
    }
    // the caller's (D, p) columns or (p, D) rows in the first chunk; the set's tile of this
    // wave after
    static_assert(kFirst || !kRows, "rows are the caller's layout, read by the first chunk only");
    const float* w = kRows    ? stheta + i * (int64_t)D
                     : kFirst ? stheta + i
                              : stheta + (base / kTile) * (int64_t)D * kTile + lane;
    for (int32_t k = 0; k < chunk_steps; ++k) {
      if (!__any(live)) break;
      if (!live) continue;
      if constexpr (kRows) {
        policy_torques_rows<C, HID>(MemberRow(stheta, p * (int64_t)D, i, D), q, v, tq);
      } else if constexpr (kFirst) {
        // an offset of zero passes through an empty asm statement every step, so the loads
        // (the same addresses each step) stay in the loop: at H = 4 the compiler had
        // hoisted all 120 weights into registers and spilled 60 B/lane. The column pointer
        // keeps its base, so they stay global loads (an opaque pointer made them flat loads).
        uint32_t off = 0;
        if constexpr (LEGGED_FIRST_CHUNK_OPAQUE_COLUMNS != 0) asm volatile("" : "+v"(off));
        policy_torques<C, HID>(w + off, src_stride, q, v, tq);
      } else {
        policy_torques<C, HID, UnitRows, kTile>(w, kTile, q, v, tq);
      }
#pragma unroll 1
      for (int sub = 0; sub < SUBSTEPS; ++sub)
        substep_exact<C, false, kStage>(q, v, tq, iters, assist, assist_damping, stage_lds + lane);
      ++t;
      bool finished;
      if (fallen<C>(q)) {
        taken += 1.0f;
        total = total - fall;
        finished = true;
      } else {
        total = total + (((q[1] >= gate) ? v[0] : 0.0f) + alive_bonus);
        taken += 1.0f;
        finished = t >= horizon;
      }
      if (finished) {
        fitness[id] = total;
        steps_out[id] = taken;
        live = false;
      }
    }
    // append the survivors to the destination set
    const unsigned long long m = __ballot(live);
    if (m) {
      const int leader = __ffsll((long long)m) - 1;
      unsigned int slot0 = 0;
      if ((int)lane == leader) slot0 = atomicAdd(dst.count, (unsigned int)__popcll(m));
      slot0 = __shfl(slot0, leader);
      if (live) {
        const int64_t slot = (int64_t)slot0 + __popcll(m & ((1ull << lane) - 1ull));
#pragma unroll
        for (int r = 0; r < N; ++r) {
          dst.state[r * cap + slot] = q[r];
          dst.state[(N + r) * cap + slot] = v[r];
        }
        dst.acc[slot] = total;
        dst.acc[cap + slot] = taken;
        dst.meta[slot] = id;
        dst.meta[cap + slot] = t;
        float* wd = dst.theta + (slot / kTile) * (int64_t)D * kTile + (slot % kTile);
        if constexpr (kRows)  // caller's FlatRows row -> UnitRows tile
          copy_flat_to_units<OBS, HID, OUT>(wd, kTile, w, 1);
        else if constexpr (kFirst)  // caller's FlatRows columns -> UnitRows tile
          copy_flat_to_units<OBS, HID, OUT>(wd, kTile, w, src_stride);
        else  // tile -> tile, same rows
          copy_rows(wd, kTile, w, kTile, D);
      }
    }
  }
}

__global__ void set_count_kernel(uint32_t* count, uint32_t value) { *count = value; }

__global__ __launch_bounds__(kBlock) void zero_pair_kernel(float* __restrict__ a, float* __restrict__ b, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  a[i] = 0.0f;
  b[i] = 0.0f;
}

// Row of flat weight k (es.unflatten order: w1 (OBS, HID), b1, w2 (HID, OUT), b2) in the
// unit-major tile layout.
template <int OBS, int HID, int OUT>
__device__ __forceinline__ int unit_row_of_flat(int k) {
  using T = UnitRows<OBS, HID, OUT>;
  if (k < OBS * HID) return T::w1(k / HID, k % HID);
  k -= OBS * HID;
  if (k < HID) return T::b1(k);
  k -= HID;
  if (k < HID * OUT) return T::w2(k / OUT, k % OUT);
  return T::b2(k - HID * OUT);
}

// The first packed set of a seeded rollout: member m at slot m with its state from the
// caller's (2N, p) rows, zero accumulators, and weights theta + sigma * (+-eps) written
// straight into the 64-member tiles (es_noise.h generates eps). One thread per member pair
// writes both members; the lanes of a wave are consecutive slots of one tile.
template <int C, int HID>
__global__ __launch_bounds__(64) void seed_set_kernel(const float* __restrict__ state,
                                                      const float* __restrict__ theta, int64_t p, uint32_t seed,
                                                      float sigma, Packed dst, int64_t cap) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  const int64_t half = p / 2;
  const int64_t m = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (m >= half) return;
  const int64_t mb = m + half;
#pragma unroll
  for (int r = 0; r < 2 * N; ++r) {
    dst.state[r * cap + m] = state[r * p + m];
    dst.state[r * cap + mb] = state[r * p + mb];
  }
  dst.acc[m] = 0.0f;
  dst.acc[cap + m] = 0.0f;
  dst.acc[mb] = 0.0f;
  dst.acc[cap + mb] = 0.0f;
  dst.meta[m] = (int32_t)m;
  dst.meta[cap + m] = 0;
  dst.meta[mb] = (int32_t)mb;
  dst.meta[cap + mb] = 0;
  float* wa = dst.theta + (m / kTile) * (int64_t)D * kTile + (m % kTile);
  float* wb = dst.theta + (mb / kTile) * (int64_t)D * kTile + (mb % kTile);
  const uint32_t key = esn::member_key(seed, (uint32_t)m);
  for (int j = 0; j < (D + 1) / 2; ++j) {
    float z0, z1;
    esn::gauss_pair(key, (uint32_t)j, z0, z1);
    const int k = 2 * j;
    const float e0 = sigma * z0, t0 = theta[k];
    const int u0 = unit_row_of_flat<OBS, HID, OUT>(k);
    wa[u0 * kTile] = t0 + e0;
    wb[u0 * kTile] = t0 + -e0;
    if (k + 1 < D) {
      const float e1 = sigma * z1, t1 = theta[k + 1];
      const int u1 = unit_row_of_flat<OBS, HID, OUT>(k + 1);
      wa[u1 * kTile] = t1 + e1;
      wb[u1 * kTile] = t1 + -e1;
    }
  }
}

// ---- the seeded rollout's first chunk over antithetic pairs ----
// Members m and m + p/2 of a seeded population share one noise row e = sigma * eps_m (their
// weights are theta + e and theta + (-e)). The first chunk reads that row once for both. The
// rows lie in tiles of kPairTile pairs (UnitRows order, row r of pair q at
// ((q / kPairTile) * D + r) * kPairTile + q % kPairTile), a wave runs one tile, and lanes l
// and l + 32 hold members q and q + p/2, so their loads of a row are the same 128 bytes:
// half of the weight bytes a wave of 64 members reads from a full population. A lane forms
// each weight as fmaf(s, e, theta_k) with s = +1 or -1. The product is exact, so this is
// theta_k + e or theta_k + (-e) rounded once, the bits seed_set_kernel stores. theta is read
// with scalar loads, one copy for the wave.
constexpr int kPairTile = 32;

// policy_torques of one pair member: weight k is fmaf(sgn, e[row(k) * kPairTile], t0[k]) with
// e the lane's column of its pair tile and t0 the flat theta. The same batches, order of
// operations and torques as policy_torques.
template <int C, int HID>
__device__ __forceinline__ void policy_torques_pairs(const float* __restrict__ e, const float* __restrict__ t0,
                                                     float sgn, const float (&q)[3 + C], const float (&v)[3 + C],
                                                     float (&tq)[C]) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  using F = FlatRows<OBS, HID, OUT>;
  using R = UnitRows<OBS, HID, OUT>;
  constexpr int64_t kS = kPairTile;
  float obs[OBS];
#pragma unroll
  for (int k = 1; k < N; ++k) obs[k - 1] = q[k];
#pragma unroll
  for (int k = 0; k < N; ++k) obs[N - 1 + k] = v[k];
  float logit[OUT];
#pragma unroll
  for (int o = 0; o < OUT; ++o) logit[o] = __builtin_fmaf(sgn, e[R::b2(o) * kS], t0[F::b2(o)]);
  constexpr int kWant = C <= 2 ? 4 : 2;
  constexpr int kBatch = kWant <= HID ? kWant : HID;
  static_assert(HID % kBatch == 0, "whole batches of hidden units");
#pragma unroll 2
  for (int j0 = 0; j0 < HID; j0 += kBatch) {
    float eb[kBatch][1 + OBS + OUT], tb[kBatch][1 + OBS + OUT];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int j = j0 + u;
      eb[u][0] = e[R::b1(j) * kS];
      tb[u][0] = t0[F::b1(j)];
#pragma unroll
      for (int k = 0; k < OBS; ++k) {
        eb[u][1 + k] = e[R::w1(k, j) * kS];
        tb[u][1 + k] = t0[F::w1(k, j)];
      }
#pragma unroll
      for (int o = 0; o < OUT; ++o) {
        eb[u][1 + OBS + o] = e[R::w2(j, o) * kS];
        tb[u][1 + OBS + o] = t0[F::w2(j, o)];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      float s = __builtin_fmaf(sgn, eb[u][0], tb[u][0]);
#pragma unroll
      for (int k = 0; k < OBS; ++k) s = s + obs[k] * __builtin_fmaf(sgn, eb[u][1 + k], tb[u][1 + k]);
      const float hj = det_tanh(s);
#pragma unroll
      for (int o = 0; o < OUT; ++o)
        logit[o] = logit[o] + hj * __builtin_fmaf(sgn, eb[u][1 + OBS + o], tb[u][1 + OBS + o]);
    }
  }
#pragma unroll
  for (int leg = 0; leg < C; ++leg) {
    float torque = -1.0f, best = logit[3 * leg];
    if (logit[3 * leg + 1] > best) { torque = 0.0f; best = logit[3 * leg + 1]; }
    if (logit[3 * leg + 2] > best) { torque = 1.0f; }
    tq[leg] = torque * TORQUE;
  }
}

// A pair member's weights into a UnitRows tile (row stride dst_stride), formed as in
// policy_torques_pairs, hidden unit j's 1 + OBS + OUT rows at a time.
template <int OBS, int HID, int OUT>
__device__ __forceinline__ void copy_pair_to_units(float* __restrict__ dst, int64_t dst_stride,
                                                   const float* __restrict__ e, const float* __restrict__ t0,
                                                   float sgn) {
  using F = FlatRows<OBS, HID, OUT>;
  using T = UnitRows<OBS, HID, OUT>;
  constexpr int kUnit = T::kUnit;
  constexpr int64_t kS = kPairTile;
#pragma unroll 2
  for (int j = 0; j < HID; ++j) {
    float b[kUnit];
    b[0] = __builtin_fmaf(sgn, e[T::b1(j) * kS], t0[F::b1(j)]);
#pragma unroll
    for (int k = 0; k < OBS; ++k) b[1 + k] = __builtin_fmaf(sgn, e[T::w1(k, j) * kS], t0[F::w1(k, j)]);
#pragma unroll
    for (int o = 0; o < OUT; ++o) b[1 + OBS + o] = __builtin_fmaf(sgn, e[T::w2(j, o) * kS], t0[F::w2(j, o)]);
#pragma unroll
    for (int r = 0; r < kUnit; ++r) dst[(T::b1(j) + r) * dst_stride] = b[r];
  }
  float b2[OUT];
#pragma unroll
  for (int o = 0; o < OUT; ++o) b2[o] = __builtin_fmaf(sgn, e[T::b2(o) * kS], t0[F::b2(o)]);
#pragma unroll
  for (int o = 0; o < OUT; ++o) dst[T::b2(o) * dst_stride] = b2[o];
}

// The pair tiles: e = sigma * eps_q for pair q < p/2 (es_noise.h generates eps), one thread
// per pair.
template <int C, int HID>
__global__ __launch_bounds__(64) void seed_pairs_kernel(int64_t p, uint32_t seed, float sigma,
                                                        float* __restrict__ tiles) {
  constexpr int OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  const int64_t half = p / 2;
  const int64_t m = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (m >= half) return;
  float* e = tiles + (m / kPairTile) * (int64_t)D * kPairTile + (m % kPairTile);
  const uint32_t key = esn::member_key(seed, (uint32_t)m);
  for (int j = 0; j < (D + 1) / 2; ++j) {
    float z0, z1;
    esn::gauss_pair(key, (uint32_t)j, z0, z1);
    const int k = 2 * j;
    e[unit_row_of_flat<OBS, HID, OUT>(k) * kPairTile] = sigma * z0;
    if (k + 1 < D) e[unit_row_of_flat<OBS, HID, OUT>(k + 1) * kPairTile] = sigma * z1;
  }
}

// The seeded rollout's first chunk: wave t runs the pairs of tile t (members q and q + p/2 of
// each) for chunk_steps steps from the caller's (2N, p) state rows and appends the survivors,
// their weights formed, to dst. Otherwise as rollout_chunk_kernel's first chunk.
template <int C, int HID>
__global__ __launch_bounds__(64, LEGGED_FIRST_CHUNK_MIN_WAVES) void rollout_pairs_first_kernel(
    const float* __restrict__ state0, const float* __restrict__ theta, const float* __restrict__ tiles, int64_t p,
    Packed dst, int64_t cap, int32_t chunk_steps, int32_t horizon, int iters, float alive_bonus, float fall,
    float gate, float assist, float assist_damping, float* __restrict__ fitness, float* __restrict__ steps_out) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  constexpr bool kStage = LEGGED_CHUNK_STAGE != 0;
  __shared__ float stage_lds[kStage ? 2 * C * N * 64 : 1];
  static_assert(2 * kPairTile == 64, "a wave holds both members of its tile's pairs");
  const unsigned lane = threadIdx.x;
  const int64_t half = p / 2;
  const int64_t pair = (int64_t)blockIdx.x * kPairTile + (lane % kPairTile);
  bool live = pair < half;
  const bool minus = lane >= (unsigned)kPairTile;
  const float sgn = minus ? -1.0f : 1.0f;
  const int64_t i = minus ? half + pair : pair;
  float q[N], v[N], tq[C];
  float total = 0.0f, taken = 0.0f;
  int32_t t = 0;
  if (live) {
#pragma unroll
    for (int r = 0; r < N; ++r) {
      q[r] = state0[r * p + i];
      v[r] = state0[(N + r) * p + i];
    }
  }
  const float* e = tiles + (int64_t)blockIdx.x * D * kPairTile + (lane % kPairTile);
  for (int32_t k = 0; k < chunk_steps; ++k) {
    if (!__any(live)) break;
    if (!live) continue;
    // offsets of zero pass through empty asm statements every step, so the loads (the same
    // addresses each step) stay in the loop instead of being hoisted into registers; the
    // pointers keep their bases, so the noise loads stay global loads and theta's scalar
    uint32_t eoff = 0, toff = 0;
    asm volatile("" : "+v"(eoff));
    asm volatile("" : "+s"(toff));
    policy_torques_pairs<C, HID>(e + eoff, theta + toff, sgn, q, v, tq);
#pragma unroll 1
    for (int sub = 0; sub < SUBSTEPS; ++sub)
      substep_exact<C, false, kStage>(q, v, tq, iters, assist, assist_damping, stage_lds + lane);
    ++t;
    bool finished;
    if (fallen<C>(q)) {
      taken += 1.0f;
      total = total - fall;
      finished = true;
    } else {
      total = total + (((q[1] >= gate) ? v[0] : 0.0f) + alive_bonus);
      taken += 1.0f;
      finished = t >= horizon;
    }
    if (finished) {
      fitness[i] = total;
      steps_out[i] = taken;
      live = false;
    }
  }
  const unsigned long long m = __ballot(live);
  if (m) {
    const int leader = __ffsll((long long)m) - 1;
    unsigned int slot0 = 0;
    if ((int)lane == leader) slot0 = atomicAdd(dst.count, (unsigned int)__popcll(m));
    slot0 = __shfl(slot0, leader);
    if (live) {
      const int64_t slot = (int64_t)slot0 + __popcll(m & ((1ull << lane) - 1ull));
#pragma unroll
      for (int r = 0; r < N; ++r) {
        dst.state[r * cap + slot] = q[r];
        dst.state[(N + r) * cap + slot] = v[r];
      }
      dst.acc[slot] = total;
      dst.acc[cap + slot] = taken;
      dst.meta[slot] = (int32_t)i;
      dst.meta[cap + slot] = t;
      float* wd = dst.theta + (slot / kTile) * (int64_t)D * kTile + (slot % kTile);
      copy_pair_to_units<OBS, HID, OUT>(wd, kTile, e, theta, sgn);
    }
  }
}

// Member counts at which the schedule changes form: one member per lane above group_max,
// the group chunk kernel above wide_max, the group tail at or below wide_max.
struct GroupBounds {
  int64_t wide_max, group_max, group_grid, tail_grid;
};

template <int C>
inline GroupBounds group_bounds(int64_t p, int cus) {
  GroupBounds b;
  b.wide_max = (int64_t)4 * kTailWaves<C> * kTailMembers<C> * cus;
  const int64_t gm = kGroupChunks<C> ? (int64_t)LEGGED_GROUP_CHUNK_MEMBERS_PER_CU * cus : 0;
  b.group_max = gm > b.wide_max ? gm : b.wide_max;
  // one member group per workgroup: a kernel never holds more than min(p, its bound) members
  const int64_t group_members = p < b.group_max ? p : b.group_max;
  const int64_t tail_members = p < b.wide_max ? p : b.wide_max;
  constexpr int chunk_members = 64 / kChunkGroupLanes;  // per single-wave workgroup
  b.group_grid = (group_members + chunk_members - 1) / chunk_members;
  b.tail_grid = (tail_members + kTailMembers<C> - 1) / kTailMembers<C>;
  return b;
}

// One later chunk from set src into set dst: of the three kernels, the one whose member
// bound holds src's count runs, the others exit at once.
template <int C, int HID>
int launch_later_chunk(const float* state0, const float* theta0, int64_t p, const Packed& src, const Packed& dst,
                       int64_t cap, int64_t grid, const GroupBounds& gb, int32_t chunk_steps, int32_t horizon,
                       int iters, float alive, float fall, float gate, float af, float ad, float* fitness,
                       float* steps, hipStream_t s) {
  hipLaunchKernelGGL(set_count_kernel, dim3(1), dim3(1), 0, s, dst.count, 0u);
  hipLaunchKernelGGL((rollout_chunk_kernel<C, HID, false>), dim3((unsigned)grid), dim3(64), 0, s, state0, theta0, p,
                     src, dst, cap, chunk_steps, horizon, iters, alive, fall, gate, af, ad, fitness, steps,
                     gb.group_max);
  if constexpr (kGroupChunks<C>) {
    if (gb.group_max > gb.wide_max)
      hipLaunchKernelGGL((rollout_group_chunk_kernel<C, HID, kChunkGroupLanes>), dim3((unsigned)gb.group_grid), dim3(64), 0,
                         s, src, dst, cap, chunk_steps, horizon, iters, alive, fall, gate, af, ad, fitness, steps,
                         gb.wide_max, gb.group_max);
  }
  hipLaunchKernelGGL((rollout_tail_kernel<C, HID>), dim3((unsigned)gb.tail_grid), dim3(64), 0, s, src, cap, horizon,
                     iters, alive, fall, gate, af, ad, fitness, steps, gb.wide_max);
  return launch_status();
}

// Tag of the per-device occupancy cache of rollout_chunk_kernel<C, HID, false>.
template <int C, int HID>
struct ChunkTag {};

#ifndef LEGGED_SMALL_POP_TAIL
#define LEGGED_SMALL_POP_TAIL 1
#endif
template <int C, int HID, bool kRows>
int launch_chunked(const float* state, const float* theta0, int64_t p, int32_t horizon, int iters,
                   int32_t chunk_steps, float alive, float fall, float gate, double assist, float* fitness,
                   float* steps, void* workspace, hipStream_t s) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  const int64_t cap = round_to_tile(p);
  // carve the workspace: two packed sets, then two counters
  char* ws = static_cast<char*>(workspace);
  Packed set[2];
  for (int b = 0; b < 2; ++b) {
    set[b].state = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * 2 * N * cap;
    set[b].theta = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * (int64_t)D * cap;
    set[b].acc = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * 2 * cap;
    set[b].meta = reinterpret_cast<int32_t*>(ws);
    ws += sizeof(int32_t) * 2 * cap;
  }
  set[0].count = reinterpret_cast<uint32_t*>(ws);
  set[1].count = set[0].count + 1;
  int cus = 0, per_cu = 0;
  int query = device_cus(&cus);
  if (query == HIPENVS_OK)
    query = resident_blocks_per_cu<ChunkTag<C, HID>>(rollout_chunk_kernel<C, HID, false>, &per_cu);
  if (query != HIPENVS_OK) return query;
  const int64_t needed = (p + 63) / 64;
  int64_t resident = (int64_t)cus * (per_cu > 0 ? per_cu : 1);
  const float af = (float)assist, ad = (float)(0.1 * assist);
  const GroupBounds gb = group_bounds<C>(p, cus);
  // first chunk: the caller's arrays -> set 0. A population the group tail holds at once
  // (at most wide_max members) takes no step in it: the chunk only packs the members, and the
  // tail runs them from step 0 instead of one lane per member stepping the first chunk
  // (ES rollout, C = 4, 500 steps: P = 1,024, H = 16 12.6 -> 11.7 ms; P = 4,096, H = 64
  // 13.0 -> 12.0 ms; at C = 2 within +-2 %).
  const int32_t first_steps = (LEGGED_SMALL_POP_TAIL && p <= gb.wide_max) ? 0 : first_chunk_steps<C>(chunk_steps);
  hipLaunchKernelGGL(set_count_kernel, dim3(1), dim3(1), 0, s, set[0].count, 0u);
  hipLaunchKernelGGL((rollout_chunk_kernel<C, HID, true, kRows>), dim3((unsigned)needed), dim3(64), 0, s, state, theta0,
                     p, set[1], set[0], cap, first_steps, horizon, iters, alive, fall, gate, af, ad, fitness, steps,
                     gb.group_max);
  int status = launch_status();
  int cur = 0;
  const int64_t grid = resident < needed ? resident : needed;
  for (int64_t done = first_steps; status == HIPENVS_OK && done < horizon; done += chunk_steps) {
    status = launch_later_chunk<C, HID>(state, theta0, p, set[cur], set[1 - cur], cap, grid, gb, chunk_steps,
                                        horizon, iters, alive, fall, gate, af, ad, fitness, steps, s);
    cur = 1 - cur;
  }
  return status;
}

// The seeded rollout. Above the group tail's bound, seed_pairs_kernel writes the pair tiles and
// rollout_pairs_first_kernel runs the first chunk from them; at or below it, seed_set_kernel
// writes set 0 (every member, weights formed in place) and the tail takes it from step 0.
// The later chunks run in the compacted form, with the group tail after each. Members run the
// same arithmetic as in launch_chunked on theta + sigma * [eps; -eps].
#ifndef LEGGED_SEEDED_PAIRS
#define LEGGED_SEEDED_PAIRS 1
#endif
template <int C, int HID>
int launch_chunked_seeded(const float* state, const float* theta, int64_t p, uint32_t seed, float sigma,
                          int32_t horizon, int iters, int32_t chunk_steps, float alive, float fall, float gate,
                          double assist, float* fitness, float* steps, void* workspace, hipStream_t s) {
  constexpr int N = 3 + C, OBS = 5 + 2 * C, OUT = 3 * C;
  constexpr int D = OBS * HID + HID + HID * OUT + OUT;
  const int64_t cap = round_to_tile(p);
  char* ws = static_cast<char*>(workspace);
  Packed set[2];
  for (int b = 0; b < 2; ++b) {
    set[b].state = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * 2 * N * cap;
    set[b].theta = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * (int64_t)D * cap;
    set[b].acc = reinterpret_cast<float*>(ws);
    ws += sizeof(float) * 2 * cap;
    set[b].meta = reinterpret_cast<int32_t*>(ws);
    ws += sizeof(int32_t) * 2 * cap;
  }
  set[0].count = reinterpret_cast<uint32_t*>(ws);
  set[1].count = set[0].count + 1;
  int cus = 0, per_cu = 0;
  int query = device_cus(&cus);
  if (query == HIPENVS_OK)
    query = resident_blocks_per_cu<ChunkTag<C, HID>>(rollout_chunk_kernel<C, HID, false>, &per_cu);
  if (query != HIPENVS_OK) return query;
  const int64_t needed = (p + 63) / 64;
  const int64_t resident = (int64_t)cus * (per_cu > 0 ? per_cu : 1);
  const int64_t grid = resident < needed ? resident : needed;
  const GroupBounds gb = group_bounds<C>(p, cus);
  const float af = (float)assist, ad = (float)(0.1 * assist);
  int status, cur;
  int64_t done = 0;
  int32_t len = first_chunk_steps<C>(chunk_steps);
  if (LEGGED_SEEDED_PAIRS && p > gb.wide_max) {
    // the pair tiles (half of set 0's weight space) feed the first chunk, whose survivors go
    // to set 1
    const int64_t tiles = (p / 2 + kPairTile - 1) / kPairTile;
    hipLaunchKernelGGL((seed_pairs_kernel<C, HID>), dim3((unsigned)((p / 2 + 63) / 64)), dim3(64), 0, s, p, seed,
                       sigma, set[0].theta);
    hipLaunchKernelGGL(set_count_kernel, dim3(1), dim3(1), 0, s, set[1].count, 0u);
    hipLaunchKernelGGL((rollout_pairs_first_kernel<C, HID>), dim3((unsigned)tiles), dim3(64), 0, s, state, theta,
                       set[0].theta, p, set[1], cap, len, horizon, iters, alive, fall, gate, af, ad, fitness, steps);
    status = launch_status();
    cur = 1;
    done = len;
    len = chunk_steps;
  } else {
    hipLaunchKernelGGL(set_count_kernel, dim3(1), dim3(1), 0, s, set[0].count, (uint32_t)p);
    hipLaunchKernelGGL((seed_set_kernel<C, HID>), dim3((unsigned)((p / 2 + 63) / 64)), dim3(64), 0, s, state, theta,
                       p, seed, sigma, set[0], cap);
    status = launch_status();
    cur = 0;
  }
  for (; status == HIPENVS_OK && done < horizon; done += len, len = chunk_steps) {
    status = launch_later_chunk<C, HID>(state, theta, p, set[cur], set[1 - cur], cap, grid, gb, len, horizon, iters,
                                        alive, fall, gate, af, ad, fitness, steps, s);
    cur = 1 - cur;
  }
  return status;
}

template <int C>
int dispatch_chunked_seeded(int32_t hidden, const float* state, const float* theta, int64_t p, uint32_t seed,
                            float sigma, int32_t horizon, int iters, int32_t chunk_steps, float alive, float fall,
                            float gate, double assist, float* fitness, float* steps, void* workspace,
                            hipStream_t s) {
  switch (hidden) {
    case 4: return launch_chunked_seeded<C, 4>(state, theta, p, seed, sigma, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 8: return launch_chunked_seeded<C, 8>(state, theta, p, seed, sigma, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 16: return launch_chunked_seeded<C, 16>(state, theta, p, seed, sigma, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 32: return launch_chunked_seeded<C, 32>(state, theta, p, seed, sigma, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 64: return launch_chunked_seeded<C, 64>(state, theta, p, seed, sigma, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

#ifndef LEGGED_EVALUATE_GROUP
#define LEGGED_EVALUATE_GROUP 1
#endif
template <int C>
int launch_evaluate(int32_t hidden, const float* state, const float* theta, int64_t n, int32_t steps, int iters,
                    float eval_bonus, float* fitness, hipStream_t s) {
  const dim3 grid(grid_for(n, 64)), block(64);
  int cus = 0;
  const int query = device_cus(&cus);
  if (query != HIPENVS_OK) return query;
  // a batch that the group form holds at one wave per SIMD takes it (one lane per env would
  // leave most SIMDs idle and step each env at one lane's latency)
  if (LEGGED_EVALUATE_GROUP && n <= (int64_t)4 * kTailWaves<C> * kTailMembers<C> * cus) {
    const dim3 ggrid((unsigned)((n + kTailMembers<C> - 1) / kTailMembers<C>));
    switch (hidden) {
      case 4: hipLaunchKernelGGL((evaluate_group_kernel<C, 4>), ggrid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
      case 8: hipLaunchKernelGGL((evaluate_group_kernel<C, 8>), ggrid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
      case 16: hipLaunchKernelGGL((evaluate_group_kernel<C, 16>), ggrid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
      case 32: hipLaunchKernelGGL((evaluate_group_kernel<C, 32>), ggrid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
      case 64: hipLaunchKernelGGL((evaluate_group_kernel<C, 64>), ggrid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
      default: return HIPENVS_E_UNSUPPORTED;
    }
    return launch_status();
  }
  switch (hidden) {
    case 4: hipLaunchKernelGGL((evaluate_kernel<C, 4>), grid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
    case 8: hipLaunchKernelGGL((evaluate_kernel<C, 8>), grid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
    case 16: hipLaunchKernelGGL((evaluate_kernel<C, 16>), grid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
    case 32: hipLaunchKernelGGL((evaluate_kernel<C, 32>), grid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
    case 64: hipLaunchKernelGGL((evaluate_kernel<C, 64>), grid, block, 0, s, state, theta, n, steps, iters, eval_bonus, fitness); break;
    default: return HIPENVS_E_UNSUPPORTED;
  }
  return launch_status();
}

template <int C, bool kRows>
int dispatch_chunked_layout(int32_t hidden, const float* state, const float* theta0, int64_t p, int32_t horizon,
                            int iters, int32_t chunk_steps, float alive, float fall, float gate, double assist,
                            float* fitness, float* steps, void* workspace, hipStream_t s) {
  switch (hidden) {
    case 4: return launch_chunked<C, 4, kRows>(state, theta0, p, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 8: return launch_chunked<C, 8, kRows>(state, theta0, p, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 16: return launch_chunked<C, 16, kRows>(state, theta0, p, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 32: return launch_chunked<C, 32, kRows>(state, theta0, p, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    case 64: return launch_chunked<C, 64, kRows>(state, theta0, p, horizon, iters, chunk_steps, alive, fall, gate, assist, fitness, steps, workspace, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

// The chunked rollout from the caller's (D, p) columns (rows false) or (p, D) rows (true).
template <int C>
int dispatch_chunked(bool rows, int32_t hidden, const float* state, const float* theta0, int64_t p, int32_t horizon,
                     int iters, int32_t chunk_steps, float alive, float fall, float gate, double assist,
                     float* fitness, float* steps, void* workspace, hipStream_t s) {
  return rows ? dispatch_chunked_layout<C, true>(hidden, state, theta0, p, horizon, iters, chunk_steps, alive, fall,
                                                 gate, assist, fitness, steps, workspace, s)
              : dispatch_chunked_layout<C, false>(hidden, state, theta0, p, horizon, iters, chunk_steps, alive, fall,
                                                  gate, assist, fitness, steps, workspace, s);
}

template <int C>
int launch_step(const float* state, const int32_t* action, uint32_t seed, const float* stand, int iters, double assist,
                float* next, float* reward, uint8_t* done, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(step_kernel<C>, dim3(grid_for(n)), dim3(kBlock), 0, s, state, action, seed, stand, iters,
                     (float)assist, (float)(0.1 * assist), next, reward, done, n);
  return launch_status();
}

template <int C, int HID>
int launch_rollout(bool columns, const float* state, const float* theta, int64_t p, int32_t horizon, int iters,
                   float alive, float fall, float gate, double assist, float* fitness, float* steps, hipStream_t s) {
  const dim3 grid(grid_for(p, 64)), block(64);
  if (columns)
    hipLaunchKernelGGL((rollout_kernel<C, HID, true>), grid, block, 0, s, state, theta, p, horizon, iters, alive, fall,
                       gate, (float)assist, (float)(0.1 * assist), fitness, steps);
  else
    hipLaunchKernelGGL((rollout_kernel<C, HID, false>), grid, block, 0, s, state, theta, p, horizon, iters, alive,
                       fall, gate, (float)assist, (float)(0.1 * assist), fitness, steps);
  return launch_status();
}

template <int C>
int dispatch_hidden(int32_t hidden, bool columns, const float* state, const float* theta, int64_t p, int32_t horizon,
                    int iters, float alive, float fall, float gate, double assist, float* fitness, float* steps,
                    hipStream_t s) {
  switch (hidden) {
    case 4: return launch_rollout<C, 4>(columns, state, theta, p, horizon, iters, alive, fall, gate, assist, fitness, steps, s);
    case 8: return launch_rollout<C, 8>(columns, state, theta, p, horizon, iters, alive, fall, gate, assist, fitness, steps, s);
    case 16: return launch_rollout<C, 16>(columns, state, theta, p, horizon, iters, alive, fall, gate, assist, fitness, steps, s);
    case 32: return launch_rollout<C, 32>(columns, state, theta, p, horizon, iters, alive, fall, gate, assist, fitness, steps, s);
    case 64: return launch_rollout<C, 64>(columns, state, theta, p, horizon, iters, alive, fall, gate, assist, fitness, steps, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

}  // namespace lg
}  // namespace hipenvs

using namespace hipenvs;

static constexpr int kMaxIters = 4096;

extern "C" int hipenvs_legged_reset(int32_t c, const float* stand, float* state, int64_t n, uint32_t seed,
                                    hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!stand || !state))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  const dim3 grid(grid_for(n)), block(kBlock);
  switch (c) {
    case 1: hipLaunchKernelGGL(lg::reset_kernel<1>, grid, block, 0, s, stand, state, seed, n); break;
    case 2: hipLaunchKernelGGL(lg::reset_kernel<2>, grid, block, 0, s, stand, state, seed, n); break;
    case 3: hipLaunchKernelGGL(lg::reset_kernel<3>, grid, block, 0, s, stand, state, seed, n); break;
    case 4: hipLaunchKernelGGL(lg::reset_kernel<4>, grid, block, 0, s, stand, state, seed, n); break;
    default: return HIPENVS_E_UNSUPPORTED;
  }
  return launch_status();
}

extern "C" int hipenvs_legged_step(int32_t c, int32_t iters, double assist, const float* state, const int32_t* action,
                                   uint32_t seed, const float* stand, float* next_state, float* reward, uint8_t* done,
                                   int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || iters < 0 || iters > kMaxIters ||
      (n > 0 && (!state || !action || !stand || !next_state || !reward || !done)))
    return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (c) {
    case 1: return lg::launch_step<1>(state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 2: return lg::launch_step<2>(state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 3: return lg::launch_step<3>(state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    case 4: return lg::launch_step<4>(state, action, seed, stand, iters, assist, next_state, reward, done, n, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int hipenvs_legged_es_rollout(int32_t c, int32_t hidden, int32_t iters, int32_t layout, const float* state,
                                         const float* theta, int64_t p, int32_t horizon, float alive_bonus,
                                         float fall_penalty, float height_gate, double assist, float* fitness,
                                         float* steps, hipenvs_stream_t stream) {
  if (p < 0 || horizon < 0 || iters < 0 || iters > kMaxIters || (layout != 0 && layout != 1) ||
      (p > 0 && (!state || !theta || !fitness || !steps)))
    return HIPENVS_E_ARG;
  if (p == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  const bool columns = layout == 1;
  switch (c) {
    case 1: return lg::dispatch_hidden<1>(hidden, columns, state, theta, p, horizon, iters, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, s);
    case 2: return lg::dispatch_hidden<2>(hidden, columns, state, theta, p, horizon, iters, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, s);
    case 3: return lg::dispatch_hidden<3>(hidden, columns, state, theta, p, horizon, iters, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, s);
    case 4: return lg::dispatch_hidden<4>(hidden, columns, state, theta, p, horizon, iters, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int64_t hipenvs_legged_es_rollout_workspace_bytes(int32_t c, int32_t hidden, int64_t p) {
  if (p < 0 || c < 1 || c > 4 || (hidden != 4 && hidden != 8 && hidden != 16 && hidden != 32 &&
                                                hidden != 64))
    return -1;
  const int64_t n = 3 + c, obs = 5 + 2 * c, out = 3 * c;
  const int64_t d = obs * hidden + hidden + hidden * out + out;
  return 2 * (2 * n + d + 4) * lg::round_to_tile(p) * 4 + 64;
}

namespace {
int legged_chunked(bool rows, int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps, const float* state,
                   const float* theta0, int64_t p, int32_t horizon, float alive_bonus, float fall_penalty,
                   float height_gate, double assist, float* fitness, float* steps, void* workspace,
                   int64_t workspace_bytes, hipenvs_stream_t stream) {
  if (p < 0 || horizon < 0 || iters < 0 || iters > kMaxIters || chunk_steps < 1 || p > 0x7fffffffLL ||
      (p > 0 && (!state || !theta0 || !fitness || !steps || !workspace)))
    return HIPENVS_E_ARG;
  if (rows && ((uintptr_t)theta0 & 3u) != 0) return HIPENVS_E_ARG;  // rows are read as dword-aligned vectors
  if (p == 0) return HIPENVS_OK;
  const int64_t need = hipenvs_legged_es_rollout_workspace_bytes(c, hidden, p);
  if (need < 0) return HIPENVS_E_UNSUPPORTED;
  // the rows are read through a buffer resource with 32-bit byte offsets
  const int64_t d = (5 + 2 * (int64_t)c) * hidden + hidden + hidden * 3 * (int64_t)c + 3 * (int64_t)c;
  if (rows && p * d * 4 >= ((int64_t)1 << 31)) return HIPENVS_E_UNSUPPORTED;
  if (workspace_bytes < need) return HIPENVS_E_ARG;
  if (horizon == 0)  // nothing to step: every member scores 0 in 0 steps
    return hipenvs_legged_es_rollout(c, hidden, iters, rows ? 0 : 1, state, theta0, p, 0, alive_bonus, fall_penalty,
                                     height_gate, assist, fitness, steps, stream);
  hipStream_t s = as_stream(stream);
  switch (c) {
    case 1: return lg::dispatch_chunked<1>(rows, hidden, state, theta0, p, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 2: return lg::dispatch_chunked<2>(rows, hidden, state, theta0, p, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 3: return lg::dispatch_chunked<3>(rows, hidden, state, theta0, p, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 4: return lg::dispatch_chunked<4>(rows, hidden, state, theta0, p, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}
}  // namespace

extern "C" int hipenvs_legged_es_rollout_chunked(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                                 const float* state, const float* theta_cols, int64_t p,
                                                 int32_t horizon, float alive_bonus, float fall_penalty,
                                                 float height_gate, double assist, float* fitness, float* steps,
                                                 void* workspace, int64_t workspace_bytes, hipenvs_stream_t stream) {
  return legged_chunked(false, c, hidden, iters, chunk_steps, state, theta_cols, p, horizon, alive_bonus,
                        fall_penalty, height_gate, assist, fitness, steps, workspace, workspace_bytes, stream);
}

extern "C" int hipenvs_legged_es_rollout_chunked_rows(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                                      const float* state, const float* theta_rows, int64_t p,
                                                      int32_t horizon, float alive_bonus, float fall_penalty,
                                                      float height_gate, double assist, float* fitness,
                                                      float* steps, void* workspace, int64_t workspace_bytes,
                                                      hipenvs_stream_t stream) {
  return legged_chunked(true, c, hidden, iters, chunk_steps, state, theta_rows, p, horizon, alive_bonus,
                        fall_penalty, height_gate, assist, fitness, steps, workspace, workspace_bytes, stream);
}

extern "C" int hipenvs_legged_es_rollout_seeded(int32_t c, int32_t hidden, int32_t iters, int32_t chunk_steps,
                                                const float* state, const float* theta, int64_t p, uint32_t seed,
                                                double sigma, int32_t horizon, float alive_bonus,
                                                float fall_penalty, float height_gate, double assist,
                                                float* fitness, float* steps, void* workspace,
                                                int64_t workspace_bytes, hipenvs_stream_t stream) {
  if (p < 2 || (p & 1) || p > 0x7fffffffLL || horizon < 0 || iters < 0 || iters > kMaxIters || chunk_steps < 1 ||
      !state || !theta || !fitness || !steps || !workspace)
    return HIPENVS_E_ARG;
  const int64_t need = hipenvs_legged_es_rollout_workspace_bytes(c, hidden, p);
  if (need < 0) return HIPENVS_E_UNSUPPORTED;
  if (workspace_bytes < need) return HIPENVS_E_ARG;
  hipStream_t s = as_stream(stream);
  if (horizon == 0) {  // nothing to step: every member scores 0 in 0 steps
    hipLaunchKernelGGL(lg::zero_pair_kernel, dim3(grid_for(p)), dim3(kBlock), 0, s, fitness, steps, p);
    return launch_status();
  }
  const float sg = (float)sigma;
  switch (c) {
    case 1: return lg::dispatch_chunked_seeded<1>(hidden, state, theta, p, seed, sg, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 2: return lg::dispatch_chunked_seeded<2>(hidden, state, theta, p, seed, sg, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 3: return lg::dispatch_chunked_seeded<3>(hidden, state, theta, p, seed, sg, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    case 4: return lg::dispatch_chunked_seeded<4>(hidden, state, theta, p, seed, sg, horizon, iters, chunk_steps, alive_bonus, fall_penalty, height_gate, assist, fitness, steps, workspace, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int hipenvs_legged_evaluate(int32_t c, int32_t hidden, int32_t iters, const float* state,
                                       const float* theta, int64_t n, int32_t steps, float eval_bonus,
                                       float* fitness, hipenvs_stream_t stream) {
  if (n < 0 || steps < 0 || iters < 0 || iters > kMaxIters || (n > 0 && (!state || !theta || !fitness)))
    return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipStream_t s = as_stream(stream);
  switch (c) {
    case 1: return lg::launch_evaluate<1>(hidden, state, theta, n, steps, iters, eval_bonus, fitness, s);
    case 2: return lg::launch_evaluate<2>(hidden, state, theta, n, steps, iters, eval_bonus, fitness, s);
    case 3: return lg::launch_evaluate<3>(hidden, state, theta, n, steps, iters, eval_bonus, fitness, s);
    case 4: return lg::launch_evaluate<4>(hidden, state, theta, n, steps, iters, eval_bonus, fitness, s);
    default: return HIPENVS_E_UNSUPPORTED;
  }
}

extern "C" int hipenvs_hopper_reset(float* state, int64_t n, uint32_t seed, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && !state)) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  hipLaunchKernelGGL(lg::hopper_reset_kernel, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, seed, n);
  return launch_status();
}

extern "C" int hipenvs_hopper_step(const float* state, const int32_t* action, uint32_t seed, float* next_state,
                                   float* reward, uint8_t* done, int64_t n, hipenvs_stream_t stream) {
  if (n < 0 || (n > 0 && (!state || !action || !next_state || !reward || !done))) return HIPENVS_E_ARG;
  if (n == 0) return HIPENVS_OK;
  // one exact contact solve per substep: the C = 1 body with one sweep, no assist
  hipLaunchKernelGGL((lg::step_kernel<1, true>), dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), state, action,
                     seed, nullptr, 1, 0.0f, 0.0f, next_state, reward, done, n);
  return launch_status();
}
