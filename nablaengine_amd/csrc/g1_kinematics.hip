// Kinematics outputs of a state and their VJP (the reference's k_kin / k_kin_vjp, g1_engine/kinematics.py:1-45; MuJoCo
// MJX's kinematics + com_pos + com_vel semantics, mujoco 3.17 smooth.py):
//   qpos_n       qpos with the free joint's quaternion normalized;
//   xpos, xquat  the body frames (world body 0 at the origin, identity); the root from qpos; a hinge body composed
//                from its parent: x_b = x_p + R_p p_b, Q_b = Q_p (x) q_b (x) (axis_b, qpos angle);
//   subtree_com  sum over the subtree of m_c xipos_c / its mass, xipos_c = x_c + R_c ipos_c (the torso's ipos + com);
//                the world body's is body 1's;
//   cvel         [W_b; V_b + W_b x (c - x_b)], c = subtree_com[1]: W_b the body's angular velocity, V_b its origin's
//                velocity (root: R_1 qvel[3:6], qvel[0:3]); body 0 zeros.
// One world per wave64, lane b = body b. Each body lane composes its own pose along its chain from the root; the
// subtree and path sums are one loop over the bodies per lane (the subtree and ancestor masks of the tree), reading
// the other lanes' values from LDS.
//
// VJP (reverse mode of the same map; cotangents of the five outputs -> of qpos and qvel): per body the "own"
// cotangents of its origin (x bar: a world force) and of its rotation (tau bar: a world torque; a quaternion cotangent
// g gives 1/2 vec(g Q*)), with the sums over the tree in closed form:
//   cvel:        V bar_b = g_lin, W bar_b = g_ang + (c - x_b) x g_lin, x bar_b += W_b x g_lin, c bar += g_lin x W_b;
//   subtree_com: S bar_b = g_sc_b / m_sub_b; xipos bar_c = m_c sum of S bar over c's path; x bar_c += it,
//                tau bar_c += (xipos_c - x_c) x it;
//   velocities:  V tot_b = sum_sub V bar, W tot_b = sum_sub (W bar_d + x_d x V bar_d) - x_b x V tot_b; hinge rate bar
//                z_b . W tot_b, tau bar_b += qd_b z_b x W tot_b; x bar_b += V tot_b x W_parent - (V tot_b - V bar_b) x W_b;
//                root: qvel[0:3] bar = V tot_1, qvel[3:6] bar = R_1' W tot_1, tau bar_1 += W_1 x W tot_1;
//   poses:       F_b = sum_sub x bar, N_b = sum_sub (tau bar_d + x_d x x bar_d) - x_b x F_b; hinge angle bar z_b . N_b;
//                root position bar F_1; quaternion: a = 2 [0; N_1] (x) u + g_xquat_1 + g_qpos_n[3:7],
//                raw bar = (a - u (u . a)) / |q| (MJX's normalization).
// The incoming cotangents gq_in / gv_in (nullable) are added to the result last.
#include "g1_device.h"

namespace g1k {

struct Kin {
  float q[40], v[36], com[4];
  float X[NB][4], Q[NB][4], Z[NB][4], W[NB][4];  // origin, rotation, world hinge axis, angular velocity
  float P[NB][4];                                 // m xipos (forward); then the VJP's per-body sums
  float R[NB][4], T[NB][4];                       // VJP: per-body own cotangents to sum over subtrees and paths
  float c[4];
  float qnorm;
};

// the forward map on lane b: poses, axes, subtree COMs, twists; leaves X, Q, Z, W of every body in LDS and returns
// this lane's (xipos - x, subtree mass, subtree COM, V)
__device__ __forceinline__ void kin_forward(Kin& s, int lane, const float* __restrict__ qpos,
                                            const float* __restrict__ qvel, const float* __restrict__ com, int w,
                                            float* rip, float* msub, float* sc, float* V) {
  if (lane < NQ) s.q[lane] = qpos[(size_t)w * NQ + lane];
  if (lane < NV) s.v[lane] = qvel[(size_t)w * NV + lane];
  if (lane < 3) s.com[lane] = com[(size_t)w * 3 + lane];
  wsync();
  const int b = lane < NB ? lane : 0;
  float Q[4] = {1.f, 0.f, 0.f, 0.f}, X[3] = {0.f, 0.f, 0.f};
  if (lane >= 1 && lane < NB) {
    const float qq = s.q[3] * s.q[3] + s.q[4] * s.q[4] + s.q[5] * s.q[5] + s.q[6] * s.q[6];
    const float n = 1.f / sqrtf(qq);
    for (int k = 0; k < 4; k++) Q[k] = s.q[3 + k] * n;
    for (int k = 0; k < 3; k++) X[k] = s.q[k];
    if (lane == 1) s.qnorm = sqrtf(qq);
    const int depth = cDepth[b];
    for (int l = 1; l < depth; l++) {  // compose the chain root -> b
      const int k = cTree.path[b][l];
      const float qb[4] = {cQuat[4 * k], cQuat[4 * k + 1], cQuat[4 * k + 2], cQuat[4 * k + 3]};
      const float pb[3] = {cPos[3 * k], cPos[3 * k + 1], cPos[3 * k + 2]};
      float t[3], q0[4], sn, cs;
      qrot(Q, pb, t);
      for (int e = 0; e < 3; e++) X[e] += t[e];
      qmul(Q, qb, q0);
      sincosf(0.5f * s.q[cQadr[k]], &sn, &cs);
      const float ha[4] = {cs, sn * cAxis[3 * k], sn * cAxis[3 * k + 1], sn * cAxis[3 * k + 2]};
      qmul(q0, ha, Q);
    }
  }
  float Z[3] = {0.f, 0.f, 0.f};
  if (lane >= 2 && lane < NB) {
    const float ax[3] = {cAxis[3 * b], cAxis[3 * b + 1], cAxis[3 * b + 2]};
    qrot(Q, ax, Z);
  }
  float ip[3] = {cIpos[3 * b], cIpos[3 * b + 1], cIpos[3 * b + 2]};
  if (b == TORSO_BODY)
    for (int k = 0; k < 3; k++) ip[k] += s.com[k];
  qrot(Q, ip, rip);
  const float m = lane >= 1 && lane < NB ? cMass[b] : 0.f;
  if (lane < NB) {
    for (int k = 0; k < 4; k++) s.Q[lane][k] = Q[k];
    for (int k = 0; k < 3; k++) { s.X[lane][k] = X[k]; s.Z[lane][k] = Z[k]; s.P[lane][k] = m * (X[k] + rip[k]); }
  }
  wsync();
  // subtree sums (body 0: body 1's subtree)
  const unsigned sub = cTree.submask[b < 1 ? 1 : b];
  float S[3] = {0.f, 0.f, 0.f}, ms = 0.f;
  for (int d = 1; d < NB; d++)
    if ((sub >> d) & 1u) {
      ms += cMass[d];
      for (int k = 0; k < 3; k++) S[k] += s.P[d][k];
    }
  *msub = ms;
  for (int k = 0; k < 3; k++) sc[k] = S[k] / ms;
  if (lane == 1)
    for (int k = 0; k < 3; k++) s.c[k] = sc[k];
  // twists: W_b = R_1 w + sum over b's hinges of z_j qd_j; V_b = v + (R_1 w) x (x_b - x_1) + sum (z_j qd_j) x (x_b - x_j)
  float W[3] = {0.f, 0.f, 0.f};
  for (int k = 0; k < 3; k++) V[k] = 0.f;
  if (lane >= 1 && lane < NB) {
    const float q1[4] = {s.Q[1][0], s.Q[1][1], s.Q[1][2], s.Q[1][3]};
    const float wl[3] = {s.v[3], s.v[4], s.v[5]};
    qrot(q1, wl, W);
    float r[3], u[3];
    for (int k = 0; k < 3; k++) r[k] = X[k] - s.X[1][k];
    cross(W, r, u);
    for (int k = 0; k < 3; k++) V[k] = s.v[k] + u[k];
    const int depth = cDepth[b];
    for (int l = 1; l < depth; l++) {
      const int j = cTree.path[b][l];
      const float qd = s.v[cQadr[j] - 1];
      const float zq[3] = {s.Z[j][0] * qd, s.Z[j][1] * qd, s.Z[j][2] * qd};
      for (int k = 0; k < 3; k++) { W[k] += zq[k]; r[k] = X[k] - s.X[j][k]; }
      cross(zq, r, u);
      for (int k = 0; k < 3; k++) V[k] += u[k];
    }
  }
  if (lane < NB)
    for (int k = 0; k < 3; k++) s.W[lane][k] = W[k];
  wsync();
}

__global__ __launch_bounds__(64) void k_kin(int nw, const float* __restrict__ qpos, const float* __restrict__ qvel,
                                            const float* __restrict__ com, float* __restrict__ qn,
                                            float* __restrict__ xpos, float* __restrict__ xquat,
                                            float* __restrict__ cvel, float* __restrict__ osc) {
  __shared__ Kin s;
  const int lane = threadIdx.x, w = blockIdx.x;
  if (w >= nw) return;
  float rip[3], msub, sc[3], V[3];
  kin_forward(s, lane, qpos, qvel, com, w, rip, &msub, sc, V);
  if (lane < NQ) qn[(size_t)w * NQ + lane] = lane >= 3 && lane < 7 ? s.Q[1][lane - 3] : s.q[lane];
  if (lane < NB) {
    const size_t o = (size_t)w * NB + lane;
    float cv[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (lane >= 1) {
      float r[3], u[3];
      const float Wb[3] = {s.W[lane][0], s.W[lane][1], s.W[lane][2]};
      for (int k = 0; k < 3; k++) r[k] = s.c[k] - s.X[lane][k];
      cross(Wb, r, u);
      for (int k = 0; k < 3; k++) { cv[k] = Wb[k]; cv[3 + k] = V[k] + u[k]; }
    }
    for (int k = 0; k < 3; k++) { xpos[3 * o + k] = s.X[lane][k]; osc[3 * o + k] = sc[k]; }
    for (int k = 0; k < 4; k++) xquat[4 * o + k] = s.Q[lane][k];
    for (int k = 0; k < 6; k++) cvel[6 * o + k] = cv[k];
  }
}

__global__ __launch_bounds__(64) void k_kin_vjp(int nw, const float* __restrict__ qpos,
                                                const float* __restrict__ qvel, const float* __restrict__ com,
                                                const float* __restrict__ gqn, const float* __restrict__ gxpos,
                                                const float* __restrict__ gxquat, const float* __restrict__ gcvel,
                                                const float* __restrict__ gsc, const float* __restrict__ gq_in,
                                                const float* __restrict__ gv_in, float* __restrict__ gq,
                                                float* __restrict__ gv) {
  __shared__ Kin s;
  const int lane = threadIdx.x, w = blockIdx.x;
  if (w >= nw) return;
  float rip[3], msub, sc[3], V[3];
  kin_forward(s, lane, qpos, qvel, com, w, rip, &msub, sc, V);
  const int b = lane < NB ? lane : 0;
  const bool body = lane >= 1 && lane < NB;
  const size_t o = (size_t)w * NB + b;
  float X[3], Wb[3], Q[4];
  for (int k = 0; k < 3; k++) { X[k] = s.X[b][k]; Wb[k] = s.W[b][k]; }
  for (int k = 0; k < 4; k++) Q[k] = s.Q[b][k];
  // cvel: own V bar, W bar, x bar; the reference point's cotangent summed over the bodies
  float Vb[3] = {0.f, 0.f, 0.f}, Wbar[3] = {0.f, 0.f, 0.f}, xb[3] = {0.f, 0.f, 0.f}, tb[3] = {0.f, 0.f, 0.f};
  float cc[3] = {0.f, 0.f, 0.f};
  if (body) {
    const float gA[3] = {gcvel[6 * o], gcvel[6 * o + 1], gcvel[6 * o + 2]};
    const float gL[3] = {gcvel[6 * o + 3], gcvel[6 * o + 4], gcvel[6 * o + 5]};
    float r[3], u[3];
    for (int k = 0; k < 3; k++) { Vb[k] = gL[k]; r[k] = s.c[k] - X[k]; }
    cross(r, gL, u);
    for (int k = 0; k < 3; k++) Wbar[k] = gA[k] + u[k];
    cross(Wb, gL, xb);
    cross(gL, Wb, cc);
    for (int k = 0; k < 3; k++) xb[k] += gxpos[3 * o + k];
    if (lane >= 2) {  // a hinge body's quaternion cotangent as a world torque: 1/2 vec(g Q*)
      const float g[4] = {gxquat[4 * o], gxquat[4 * o + 1], gxquat[4 * o + 2], gxquat[4 * o + 3]};
      const float qc[4] = {Q[0], -Q[1], -Q[2], -Q[3]};
      float t[4];
      qmul(g, qc, t);
      for (int k = 0; k < 3; k++) tb[k] = 0.5f * t[1 + k];
    }
  }
  wsum_n<3>(cc);
  // subtree COM cotangents -> S bar_b (body 0's goes to body 1, with the reference point's)
  {
    float g[3] = {0.f, 0.f, 0.f};
    if (body)
      for (int k = 0; k < 3; k++) g[k] = gsc[3 * o + k];
    if (lane == 1)
      for (int k = 0; k < 3; k++) g[k] += gsc[(size_t)w * NB * 3 + k] + cc[k];
    if (lane < NB)
      for (int k = 0; k < 3; k++) s.P[lane][k] = body ? g[k] / msub : 0.f;
  }
  wsync();
  if (body) {  // xipos bar_c = m_c sum of S bar over c's path (root .. c)
    float a[3] = {0.f, 0.f, 0.f};
    const int depth = cDepth[b];
    for (int l = 0; l < depth; l++) {
      const int j = cTree.path[b][l];
      for (int k = 0; k < 3; k++) a[k] += s.P[j][k];
    }
    const float m = cMass[b];
    float u[3];
    for (int k = 0; k < 3; k++) { a[k] *= m; xb[k] += a[k]; }
    cross(rip, a, u);
    for (int k = 0; k < 3; k++) tb[k] += u[k];
  }
  // velocities: subtree sums of V bar and of W bar + x x V bar
  if (lane < NB) {
    float u[3];
    cross(X, Vb, u);
    for (int k = 0; k < 3; k++) { s.R[lane][k] = Vb[k]; s.T[lane][k] = Wbar[k] + u[k]; }
  }
  wsync();
  const unsigned sub = cTree.submask[b];
  float Vt[3] = {0.f, 0.f, 0.f}, Wt[3] = {0.f, 0.f, 0.f};
  if (body) {
    for (int d = 1; d < NB; d++)
      if ((sub >> d) & 1u)
        for (int k = 0; k < 3; k++) { Vt[k] += s.R[d][k]; Wt[k] += s.T[d][k]; }
    float u[3];
    cross(X, Vt, u);
    for (int k = 0; k < 3; k++) Wt[k] -= u[k];
  }
  float rate = 0.f;  // hinge rate bar, or unused
  if (body) {
    float u[3], dv[3];
    for (int k = 0; k < 3; k++) dv[k] = Vt[k] - Vb[k];
    cross(dv, Wb, u);
    for (int k = 0; k < 3; k++) xb[k] -= u[k];
    if (lane >= 2) {
      const int p = cParent[b];
      const float Wp[3] = {s.W[p][0], s.W[p][1], s.W[p][2]};
      cross(Vt, Wp, u);
      for (int k = 0; k < 3; k++) xb[k] += u[k];
      const float Z[3] = {s.Z[b][0], s.Z[b][1], s.Z[b][2]};
      rate = dot3(Z, Wt);
      const float qd = s.v[cQadr[b] - 1];
      cross(Z, Wt, u);
      for (int k = 0; k < 3; k++) tb[k] += qd * u[k];
    } else {
      cross(Wb, Wt, u);
      for (int k = 0; k < 3; k++) tb[k] += u[k];
    }
  }
  wsync();  // every lane is done reading R, T
  // poses: F_b = sum_sub x bar, N_b = sum_sub (tau bar + x x x bar) - x_b x F_b
  if (lane < NB) {
    float u[3];
    cross(X, xb, u);
    for (int k = 0; k < 3; k++) { s.R[lane][k] = xb[k]; s.T[lane][k] = tb[k] + u[k]; }
  }
  wsync();
  float F[3] = {0.f, 0.f, 0.f}, N[3] = {0.f, 0.f, 0.f};
  if (body) {
    for (int d = 1; d < NB; d++)
      if ((sub >> d) & 1u)
        for (int k = 0; k < 3; k++) { F[k] += s.R[d][k]; N[k] += s.T[d][k]; }
    float u[3];
    cross(X, F, u);
    for (int k = 0; k < 3; k++) N[k] -= u[k];
  }
  // outputs: hinge bodies write their angle's and rate's entries; the root its position, quaternion, velocities
  float* oq = gq + (size_t)w * NQ;
  float* ov = gv + (size_t)w * NV;
  const float* iq = gq_in ? gq_in + (size_t)w * NQ : nullptr;
  const float* iv = gv_in ? gv_in + (size_t)w * NV : nullptr;
  const float* gn = gqn + (size_t)w * NQ;
  if (lane >= 2 && lane < NB) {
    const int qa = cQadr[b], da = qa - 1;
    const float Z[3] = {s.Z[b][0], s.Z[b][1], s.Z[b][2]};
    const float ang = dot3(Z, N) + gn[qa];
    oq[qa] = iq ? ang + iq[qa] : ang;
    ov[da] = iv ? rate + iv[da] : rate;
  }
  if (lane == 1) {
    for (int k = 0; k < 3; k++) {
      const float pq = F[k] + gn[k];
      oq[k] = iq ? pq + iq[k] : pq;
      ov[k] = iv ? Vt[k] + iv[k] : Vt[k];
    }
    float wl[3];
    qrot_inv(Q, Wt, wl);
    for (int k = 0; k < 3; k++) ov[3 + k] = iv ? wl[k] + iv[3 + k] : wl[k];
    const float n4[4] = {0.f, N[0], N[1], N[2]};
    float a[4];
    qmul(n4, Q, a);
    const float* gx = gxquat + (size_t)w * NB * 4 + 4;
    for (int k = 0; k < 4; k++) a[k] = 2.f * a[k] + gx[k] + gn[3 + k];
    const float ua = Q[0] * a[0] + Q[1] * a[1] + Q[2] * a[2] + Q[3] * a[3];
    const float inv = 1.f / s.qnorm;
    for (int k = 0; k < 4; k++) {
      const float g = (a[k] - Q[k] * ua) * inv;
      oq[3 + k] = iq ? g + iq[3 + k] : g;
    }
  }
}

int launch_kinematics(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com, float* qn,
                      float* xpos, float* xquat, float* cvel, float* sc) {
  if (nw <= 0) return 0;
  hipLaunchKernelGGL(k_kin, dim3(nw), dim3(64), 0, st, nw, qpos, qvel, com, qn, xpos, xquat, cvel, sc);
  return (int)hipGetLastError();
}

int launch_kinematics_vjp(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com,
                          const float* gqn, const float* gxpos, const float* gxquat, const float* gcvel,
                          const float* gsc, const float* gq_in, const float* gv_in, float* gq, float* gv) {
  if (nw <= 0) return 0;
  hipLaunchKernelGGL(k_kin_vjp, dim3(nw), dim3(64), 0, st, nw, qpos, qvel, com, gqn, gxpos, gxquat, gcvel, gsc,
                     gq_in, gv_in, gq, gv);
  return (int)hipGetLastError();
}

}  // namespace g1k
