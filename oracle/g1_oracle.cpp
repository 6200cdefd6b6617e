// TEST INFRASTRUCTURE ONLY: the float64 CPU oracle of the G1 control step. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it, as the checker (never as the product path).
//
// A float64 restatement of the reference's batched G1 control step (4 substeps of 5 ms: smooth dynamics, collision,
// constraint rows, Newton solver, implicitfast integration), written from its source as text:
//   smooth dynamics     g1_engine/source.py:186-329 (fwd_body, body_force, accumulate, torques, body_inertia,
//                       apply_inertia, dof_motion, body_ipos) and step.py:1666-1783 (substep_pre's tree passes, CRBA,
//                       actuators, qacc_smooth)
//   collision           step.py:378-554 (make_frame, plane_point, plane_capsule_frame, capsule_end, segment_point,
//                       capcap_*) and step.py:1042-1143 (collide_pair)
//   contact Jacobians   step.py:1830-1878
//   rows, impedance     step.py:1157-1188 (kbimp, limit_dists, contact_invw, efc_D), rows loop step.py:1881-1957
//   Newton              step.py:1974-2137 (warm start, Hessian, exact line search, update, stop test)
//   implicitfast        step.py:2153-2182, integrate_root step.py:1492-1504
// Differences that change no converged result: contacts are kept in (pair, slot) order (the reference's order comes
// from shared-memory atomics), the Jacobian rows are dense, and the Cholesky is a plain textbook LL^T.
// The model (MuJoCo 3.17 g1_train.mjb) is compiled in from ../nablaengine_amd/csrc/g1_model.h.
//
// It is pinned against MuJoCo C float64 truth vectors (benchmarks/data/truth/*.npz out, check_out) by tests/.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../nablaengine_amd/csrc/g1_model.h"

namespace {
using namespace g1;
constexpr int NB = NBODY;
constexpr int MAXCON = 64;
constexpr int NEFC = 192;

struct Contact {
  int pair, slot, b1, b2, dim;
  double dist, pos[3], frame[9], mu;
};

struct World {
  double qpos[NQ], qvel[NV], qacc[NV];
  double com[3], fric;
  double Q[NB][4], X[NB][3], W[NB][3], V[NB][3], AL[NB][3], A[NB][3], F[NB][3], N[NB][3], Jc[NB][10];
  double S[NV][6];  // dof motion subspaces about the root origin O: angular (3), velocity of O (3)
  double O[3];
  double M[NV][NV], qsm[NV], qacc0[NV];
  double gx[NGEOM][3], gq[NGEOM][4];
  int ncon, ncon_raw, flags;
  Contact con[MAXCON];
  int nefc, nlim;
  double efcJ[NEFC][NV], efcD[NEFC], aref[NEFC];
  int niter;
  double Ib[NB][10];  // each body's own spatial inertia about O (before the subtree sums)
  double aadv[NV];    // implicitfast's a_adv of the last substep
  bool clamped[NV];   // dofs whose actuator force is at its limit
  double flops;  // algorithmic flops of the world-step so far (the closed-form phase counts, see count_* below)
  double aflops;  // algorithmic flops of the world-step's VJP so far (closed form, VJP_FLOPS_* below)
  // The checker's own hooks, inert at their defaults (no part of the reference's step): qfrc, a generalized force
  // added to qfrc_smooth (NV, or NULL), so that finite differences in it measure the adjoint's lambda; freeze, per
  // capsule-capsule pair (flag, x1, x2): with freeze_mode 1 the forward records the segment parameters of every pair
  // whose both parameters are free, with 2 it uses the recorded ones instead of solving for them (the forward in
  // which the near-parallel rule's held parameters are exact); normal_eps, parallel_eps: the eps of the normal
  // options 2 and 3 (1e-3 m) and the near-parallel rule's sin^2 threshold (1.2e-3), the reference's
  // DK_ADJ_NORMAL_EPS / DK_ADJ_PARALLEL_EPS (adjoint_contact.py:76-95).
  const double* qfrc;
  double (*hfinal)[NV];  // the checker's hook: newton() writes H at its final zones here (or NULL)
  double (*freeze)[3];
  int freeze_mode;
  double normal_eps, parallel_eps;
};

void init_hooks(World& s) {
  s.qfrc = nullptr;
  s.hfinal = nullptr;
  s.freeze = nullptr;
  s.freeze_mode = 0;
  s.normal_eps = 1e-3;
  s.parallel_eps = 1.2e-3;
}

inline void qmul(const double* a, const double* b, double* o) {
  double w = a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3];
  double x = a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2];
  double y = a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1];
  double z = a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0];
  o[0] = w; o[1] = x; o[2] = y; o[3] = z;
}
inline void qrot(const double* q, const double* v, double* o) {  // o = q v q^-1
  double tx = 2 * (q[2] * v[2] - q[3] * v[1]), ty = 2 * (q[3] * v[0] - q[1] * v[2]), tz = 2 * (q[1] * v[1] - q[2] * v[0]);
  o[0] = v[0] + q[0] * tx + q[2] * tz - q[3] * ty;
  o[1] = v[1] + q[0] * ty + q[3] * tx - q[1] * tz;
  o[2] = v[2] + q[0] * tz + q[1] * ty - q[2] * tx;
}
inline void qrot_inv(const double* q, const double* v, double* o) {
  double qc[4] = {q[0], -q[1], -q[2], -q[3]};
  qrot(qc, v, o);
}
inline void cross(const double* a, const double* b, double* o) {
  double x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  o[0] = x; o[1] = y; o[2] = z;
}
inline double dot3(const double* a, const double* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }

// ---------------------------------------------------------------------------------------------- smooth dynamics
// body b from its parent (source.py:186-235 fwd_body; qacc = 0 in the bias pass, so AL, A carry only the velocity
// product terms and gravity)
void fwd_body(World& s, int b, const double* qacc) {
  if (b == 1) {
    const double* q = s.qpos + 3;
    double n = 1.0 / std::sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    for (int k = 0; k < 4; k++) s.Q[1][k] = q[k] * n;
    for (int k = 0; k < 3; k++) { s.X[1][k] = s.qpos[k]; s.V[1][k] = s.qvel[k]; s.A[1][k] = qacc[k] - GRAVITY[k]; }
    qrot(s.Q[1], s.qvel + 3, s.W[1]);
    qrot(s.Q[1], qacc + 3, s.AL[1]);
    return;
  }
  int p = BODY_PARENT[b];
  double q0[4], t[3], ha[4], aw[3], r[3], awd[3], u[3], wr[3], u2[3];
  qmul(s.Q[p], BODY_QUAT + 4 * b, q0);
  qrot(s.Q[p], BODY_POS + 3 * b, t);
  for (int k = 0; k < 3; k++) s.X[b][k] = s.X[p][k] + t[k];
  double ang = s.qpos[BODY_QADR[b]], qd = s.qvel[BODY_DADR[b]], qdd = qacc[BODY_DADR[b]];
  const double* ax = BODY_AXIS + 3 * b;
  double sn = std::sin(0.5 * ang), cs = std::cos(0.5 * ang);
  ha[0] = cs; ha[1] = sn * ax[0]; ha[2] = sn * ax[1]; ha[3] = sn * ax[2];
  qmul(q0, ha, s.Q[b]);
  qrot(s.Q[b], ax, aw);
  for (int k = 0; k < 3; k++) {
    r[k] = s.X[b][k] - s.X[p][k];
    awd[k] = aw[k] * qd;
    s.W[b][k] = s.W[p][k] + awd[k];
  }
  cross(s.W[p], r, u);
  for (int k = 0; k < 3; k++) s.V[b][k] = s.V[p][k] + u[k];
  cross(s.W[p], awd, u);
  for (int k = 0; k < 3; k++) s.AL[b][k] = s.AL[p][k] + aw[k] * qdd + u[k];
  cross(s.AL[p], r, u);
  cross(s.W[p], r, wr);
  cross(s.W[p], wr, u2);
  for (int k = 0; k < 3; k++) s.A[b][k] = s.A[p][k] + u[k] + u2[k];
}

void body_ipos(const World& s, int b, double* out) {
  for (int k = 0; k < 3; k++) out[k] = BODY_IPOS[3 * b + k] + (b == TORSO_BODY ? s.com[k] : 0.0);
}

// Newton-Euler force and moment about the body origin (source.py:238-258)
void body_force(World& s, int b) {
  double ip[3], c[3], u[3], wc[3], u2[3];
  body_ipos(s, b, ip);
  qrot(s.Q[b], ip, c);
  cross(s.AL[b], c, u);
  cross(s.W[b], c, wc);
  cross(s.W[b], wc, u2);
  double m = BODY_MASS[b];
  for (int k = 0; k < 3; k++) s.F[b][k] = m * (s.A[b][k] + u[k] + u2[k]);
  double qi[4], l[3], Iw[3], Ia[3], cf[3];
  qmul(s.Q[b], BODY_IQUAT + 4 * b, qi);
  qrot_inv(qi, s.W[b], l);
  for (int k = 0; k < 3; k++) l[k] *= BODY_INERTIA[3 * b + k];
  qrot(qi, l, Iw);
  qrot_inv(qi, s.AL[b], l);
  for (int k = 0; k < 3; k++) l[k] *= BODY_INERTIA[3 * b + k];
  qrot(qi, l, Ia);
  cross(s.W[b], Iw, u);
  cross(c, s.F[b], cf);
  for (int k = 0; k < 3; k++) s.N[b][k] = Ia[k] + u[k] + cf[k];
}

// spatial inertia about O packed as (xx yy zz xy xz yz, h = m c, m) (source.py:280-302)
void body_inertia(World& s, int b) {
  double qi[4], R[9], c[3], t[3], ip[3];
  qmul(s.Q[b], BODY_IQUAT + 4 * b, qi);
  for (int k = 0; k < 3; k++) {
    double e[3] = {0, 0, 0};
    e[k] = 1;
    qrot(qi, e, R + 3 * k);
  }
  const double* I = BODY_INERTIA + 3 * b;
  double* J = s.Jc[b];
  J[0] = I[0] * R[0] * R[0] + I[1] * R[3] * R[3] + I[2] * R[6] * R[6];
  J[1] = I[0] * R[1] * R[1] + I[1] * R[4] * R[4] + I[2] * R[7] * R[7];
  J[2] = I[0] * R[2] * R[2] + I[1] * R[5] * R[5] + I[2] * R[8] * R[8];
  J[3] = I[0] * R[0] * R[1] + I[1] * R[3] * R[4] + I[2] * R[6] * R[7];
  J[4] = I[0] * R[0] * R[2] + I[1] * R[3] * R[5] + I[2] * R[6] * R[8];
  J[5] = I[0] * R[1] * R[2] + I[1] * R[4] * R[5] + I[2] * R[7] * R[8];
  body_ipos(s, b, ip);
  qrot(s.Q[b], ip, t);
  for (int k = 0; k < 3; k++) c[k] = s.X[b][k] + t[k] - s.O[k];
  double m = BODY_MASS[b], cc = dot3(c, c);
  J[0] += m * (cc - c[0] * c[0]); J[1] += m * (cc - c[1] * c[1]); J[2] += m * (cc - c[2] * c[2]);
  J[3] -= m * c[0] * c[1]; J[4] -= m * c[0] * c[2]; J[5] -= m * c[1] * c[2];
  J[6] = m * c[0]; J[7] = m * c[1]; J[8] = m * c[2]; J[9] = m;
}

void apply_inertia(const double* J, const double* w, const double* v, double* n, double* f) {
  double hv[3], hw[3];
  cross(J + 6, v, hv);
  cross(J + 6, w, hw);
  n[0] = J[0] * w[0] + J[3] * w[1] + J[4] * w[2] + hv[0];
  n[1] = J[3] * w[0] + J[1] * w[1] + J[5] * w[2] + hv[1];
  n[2] = J[4] * w[0] + J[5] * w[1] + J[2] * w[2] + hv[2];
  for (int k = 0; k < 3; k++) f[k] = J[9] * v[k] - hw[k];
}

void chol_solve(const double (*A)[NV], const double* b, double* x) {  // x = A^-1 b, A symmetric positive definite
  static thread_local double L[NV][NV];
  for (int i = 0; i < NV; i++)
    for (int j = 0; j <= i; j++) {
      double acc = A[i][j];
      for (int k = 0; k < j; k++) acc -= L[i][k] * L[j][k];
      if (i == j) L[i][i] = std::sqrt(std::fmax(acc, 1e-300));
      else L[i][j] = acc / L[j][j];
    }
  double y[NV];
  for (int i = 0; i < NV; i++) {
    double acc = b[i];
    for (int k = 0; k < i; k++) acc -= L[i][k] * y[k];
    y[i] = acc / L[i][i];
  }
  for (int i = NV - 1; i >= 0; i--) {
    double acc = y[i];
    for (int k = i + 1; k < NV; k++) acc -= L[k][i] * x[k];
    x[i] = acc / L[i][i];
  }
}

void smooth(World& s, const double* ctrl) {
  const double zero[NV] = {0};
  for (int k = 0; k < 4; k++) s.Q[0][k] = k == 0 ? 1 : 0;
  for (int k = 0; k < 3; k++) s.X[0][k] = s.W[0][k] = s.V[0][k] = s.AL[0][k] = s.A[0][k] = 0;
  for (int b = 1; b < NB; b++) fwd_body(s, b, zero);  // bodies are in topological order
  for (int k = 0; k < 3; k++) s.O[k] = s.X[1][k];
  for (int b = 1; b < NB; b++) {
    body_force(s, b);
    body_inertia(s, b);
    std::memcpy(s.Ib[b], s.Jc[b], sizeof(s.Ib[b]));
  }
  for (int b = NB - 1; b >= 2; b--) {  // subtree sums (children have larger indices)
    int p = BODY_PARENT[b];
    double r[3], u[3];
    for (int k = 0; k < 3; k++) r[k] = s.X[b][k] - s.X[p][k];
    cross(r, s.F[b], u);
    for (int k = 0; k < 3; k++) { s.F[p][k] += s.F[b][k]; s.N[p][k] += s.N[b][k] + u[k]; }
    for (int k = 0; k < 10; k++) s.Jc[p][k] += s.Jc[b][k];
  }
  double bias[NV];
  {
    double l[3];
    qrot_inv(s.Q[1], s.N[1], l);
    for (int k = 0; k < 3; k++) { bias[k] = s.F[1][k]; bias[3 + k] = l[k]; }
    for (int b = 2; b < NB; b++) {
      double aw[3];
      qrot(s.Q[b], BODY_AXIS + 3 * b, aw);
      bias[BODY_DADR[b]] = dot3(aw, s.N[b]);
    }
  }
  // motion subspaces about O (source.py:316-329 dof_motion)
  for (int t = 0; t < 6; t++) {
    double e[3] = {0, 0, 0};
    e[t % 3] = 1;
    if (t < 3) { for (int k = 0; k < 3; k++) { s.S[t][k] = 0; s.S[t][3 + k] = e[k]; } }
    else { qrot(s.Q[1], e, s.S[t]); for (int k = 0; k < 3; k++) s.S[t][3 + k] = 0; }
  }
  for (int b = 2; b < NB; b++) {
    int d = BODY_DADR[b];
    double r[3];
    for (int k = 0; k < 3; k++) r[k] = s.O[k] - s.X[b][k];
    qrot(s.Q[b], BODY_AXIS + 3 * b, s.S[d]);
    cross(s.S[d], r, s.S[d] + 3);
  }
  // CRBA: M[i][j] = S_i . I^c_{body(i)} S_j for j an ancestor dof (or a root dof) of i
  std::memset(s.M, 0, sizeof(s.M));
  for (int i = 0; i < NV; i++) {
    int bi = DOF_BODY[i];
    double n[3], f[3];
    apply_inertia(s.Jc[bi], s.S[i], s.S[i] + 3, n, f);
    for (int j = 0; j <= i; j++) {
      int bj = DOF_BODY[j];
      if (!((BODY_ANCMASK[bi] >> bj) & 1u)) continue;  // j's body is not an ancestor of i's body
      double v = dot3(s.S[j], n) + dot3(s.S[j] + 3, f);
      s.M[i][j] = s.M[j][i] = v;
    }
    s.M[i][i] += DOF_ARMATURE[i];
  }
  // clamped PD actuators (step.py:1762-1778): qfrc_smooth = actuator force - bias
  for (int i = 0; i < NV; i++) {
    double act = 0;
    if (i >= 6) {
      act = DOF_KP[i] * (ctrl[i - 6] - s.qpos[i + 1]) - DOF_KV[i] * s.qvel[i];
      act = std::fmin(std::fmax(act, -DOF_FRCLIM[i]), DOF_FRCLIM[i]);
      s.clamped[i] = act <= -DOF_FRCLIM[i] || act >= DOF_FRCLIM[i];
    } else {
      s.clamped[i] = false;
    }
    s.qsm[i] = act - bias[i] + (s.qfrc ? s.qfrc[i] : 0.0);
  }
  chol_solve(s.M, s.qsm, s.qacc0);
}

// ---------------------------------------------------------------------------------------------- collision
void normalize3(double* v) {
  double n = std::sqrt(dot3(v, v));
  if (n > 0) { v[0] /= n; v[1] /= n; v[2] /= n; }
}
void make_frame(const double* n, double* fr) {  // step.py:378-387
  double b[3] = {0, 0, 0};
  if (-0.5 < n[1] && n[1] < 0.5) b[1] = 1; else b[2] = 1;
  double d = dot3(n, b);
  for (int k = 0; k < 3; k++) b[k] -= n[k] * d;
  normalize3(b);
  double c[3];
  cross(n, b, c);
  for (int k = 0; k < 3; k++) { fr[k] = n[k]; fr[3 + k] = b[k]; fr[6 + k] = c[k]; }
}
void zaxis(const double* q, double* a) {
  const double ez[3] = {0, 0, 1};
  qrot(q, ez, a);
}

void add_contact(World& s, int pair, int slot, double dist, const double* pos, const double* fr) {
  s.ncon_raw++;
  if (s.ncon >= MAXCON) { s.flags |= 4; return; }
  Contact& c = s.con[s.ncon++];
  c.pair = pair; c.slot = slot; c.dist = dist; c.dim = PAIR_DIM[pair];
  c.b1 = GEOM_BODY[PAIR_G1[pair]]; c.b2 = GEOM_BODY[PAIR_G2[pair]];
  for (int k = 0; k < 3; k++) c.pos[k] = pos[k];
  for (int k = 0; k < 9; k++) c.frame[k] = fr[k];
  c.mu = PAIR_FOOT[pair] ? s.fric : PAIR_MU[pair];
}

double sphere_sphere(const double* p1, double r1, const double* p2, double r2, double* dist, double* pos, double* n) {
  double dir[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
  double d = std::sqrt(dot3(dir, dir));
  if (d == 0) { n[0] = 1; n[1] = 0; n[2] = 0; } else { for (int k = 0; k < 3; k++) n[k] = dir[k] / d; }
  *dist = d - (r1 + r2);
  double hp = 0.5 * *dist + r1;
  for (int k = 0; k < 3; k++) pos[k] = p1[k] + n[k] * hp;
  return d;
}
double plane_point(const double* p1, const double* n, const double* c, double r, double* pos) {
  double dist = (dot3(c, n) - dot3(p1, n)) - r, hp = 0.5 * dist + r;
  for (int k = 0; k < 3; k++) pos[k] = c[k] - n[k] * hp;
  return dist;
}

void collide_pair(World& s, int pair) {
  int g1 = PAIR_G1[pair], g2 = PAIR_G2[pair], t1 = GEOM_TYPE[g1], t2 = GEOM_TYPE[g2];
  const double *p1 = s.gx[g1], *q1 = s.gq[g1], *p2 = s.gx[g2], *q2 = s.gq[g2];
  const double *sz1 = GEOM_SIZE + 3 * g1, *sz2 = GEOM_SIZE + 3 * g2;
  if (t1 == 0) {  // plane (the floor)
    double n[3];
    zaxis(q1, n);
    double dif[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
    if (dot3(dif, n) > GEOM_RBOUND[g2]) return;
    if (t2 == 2) {
      double pos[3], fr[9];
      double dist = plane_point(p1, n, p2, sz2[0], pos);
      make_frame(n, fr);
      if (dist < 0) add_contact(s, pair, 0, dist, pos, fr);
    } else {
      double axis[3], fr[9];
      zaxis(q2, axis);
      // plane_capsule_frame (step.py:461-474)
      double na = dot3(n, axis), b[3];
      for (int k = 0; k < 3; k++) b[k] = axis[k] - n[k] * na;
      double bn = std::sqrt(dot3(b, b));
      if (bn > 0) for (int k = 0; k < 3; k++) b[k] /= bn;
      if (bn < 0.5) {
        b[0] = b[1] = b[2] = 0;
        if (-0.5 < n[1] && n[1] < 0.5) b[1] = 1; else b[2] = 1;
      }
      double c[3];
      cross(n, b, c);
      for (int k = 0; k < 3; k++) { fr[k] = n[k]; fr[3 + k] = b[k]; fr[6 + k] = c[k]; }
      for (int e = 0; e < 2; e++) {
        double ce[3], pos[3];
        for (int k = 0; k < 3; k++) ce[k] = e == 0 ? p2[k] + axis[k] * sz2[1] : p2[k] - axis[k] * sz2[1];
        double dist = plane_point(p1, n, ce, sz2[0], pos);
        if (dist < 0) add_contact(s, pair, e, dist, pos, fr);
      }
    }
    return;
  }
  {
    double dif[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]}, rb = GEOM_RBOUND[g1] + GEOM_RBOUND[g2];
    if (dot3(dif, dif) > rb * rb) return;
  }
  double dist, pos[3], n[3], fr[9];
  if (t1 == 2 && t2 == 2) {
    sphere_sphere(p1, sz1[0], p2, sz2[0], &dist, pos, n);
    if (dist < 0) { make_frame(n, fr); add_contact(s, pair, 0, dist, pos, fr); }
    return;
  }
  if (t1 == 2 && t2 == 3) {  // sphere-capsule: closest point of the segment (step.py:487-497)
    double axis[3], a[3], ab[3], ap[3], pt[3];
    zaxis(q2, axis);
    for (int k = 0; k < 3; k++) { a[k] = p2[k] - axis[k] * sz2[1]; ab[k] = 2 * axis[k] * sz2[1]; ap[k] = p1[k] - a[k]; }
    double gam = dot3(ab, ab) + 1e-6, t = std::fmin(std::fmax(dot3(ap, ab) / gam, 0.0), 1.0);
    for (int k = 0; k < 3; k++) pt[k] = a[k] + t * ab[k];
    sphere_sphere(p1, sz1[0], pt, sz2[0], &dist, pos, n);
    if (dist < 0) { make_frame(n, fr); add_contact(s, pair, 0, dist, pos, fr); }
    return;
  }
  // capsule-capsule (step.py:501-554)
  double a1[3], a2[3], d[3];
  zaxis(q1, a1);
  zaxis(q2, a2);
  for (int k = 0; k < 3; k++) { a1[k] *= sz1[1]; a2[k] *= sz2[1]; d[k] = p1[k] - p2[k]; }
  double ma = dot3(a1, a1), mb = -dot3(a1, a2), mc = dot3(a2, a2), u = -dot3(a1, d), v = dot3(a2, d);
  double det = ma * mc - mb * mb;
  auto core = [&](double x1, double x2, int slot, bool strict_only) {
    double v1[3], v2[3];
    for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; }
    sphere_sphere(v1, sz1[0], v2, sz2[0], &dist, pos, n);
    (void)strict_only;
    if (dist < 0) { make_frame(n, fr); add_contact(s, pair, slot, dist, pos, fr); }
    return dist;
  };
  if (std::fabs(det) >= 1e-15) {
    double x1 = (mc * u - mb * v) / det, x2 = (ma * v - mb * u) / det;
    if (s.freeze && x1 >= -1 && x1 <= 1 && x2 >= -1 && x2 <= 1) {  // both free: the checker's freeze hook
      double* fz = s.freeze[pair];
      if (s.freeze_mode == 1) { fz[0] = 1; fz[1] = x1; fz[2] = x2; }
      else if (s.freeze_mode == 2 && fz[0] != 0) { x1 = fz[1]; x2 = fz[2]; }
    }
    if (x1 > 1) { x1 = 1; x2 = (v - mb) / mc; }
    else if (x1 < -1) { x1 = -1; x2 = (v + mb) / mc; }
    if (x2 > 1 || x2 < -1) {
      bool hi = x2 > 1;
      x2 = hi ? 1 : -1;
      double raw = hi ? (u - mb) / ma : (u + mb) / ma;
      x1 = std::fmin(std::fmax(raw, -1.0), 1.0);
    }
    core(x1, x2, 0, false);
  } else {
    int cnt = 0;
    for (int e = 0; e < 4 && cnt < 2; e++) {
      double x1, x2;
      if (e < 2) {
        x1 = e == 0 ? 1 : -1;
        double raw = e == 0 ? (v - mb) / mc : (v + mb) / mc;
        x2 = std::fmin(std::fmax(raw, -1.0), 1.0);
      } else {
        x2 = e == 2 ? 1 : -1;
        double raw = e == 2 ? (u - mb) / ma : (u + mb) / ma;
        x1 = std::fmin(std::fmax(raw, -1.0), 1.0);
      }
      double v1[3], v2[3];
      for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; }
      sphere_sphere(v1, sz1[0], v2, sz2[0], &dist, pos, n);
      if (dist <= 0) {
        cnt++;
        if (dist < 0) { make_frame(n, fr); add_contact(s, pair, e, dist, pos, fr); }
      }
    }
  }
}

void collision(World& s) {
  for (int g = 0; g < NGEOM; g++) {
    int b = GEOM_BODY[g];
    double t[3];
    qrot(s.Q[b], GEOM_POS + 3 * g, t);
    for (int k = 0; k < 3; k++) s.gx[g][k] = s.X[b][k] + t[k];
    qmul(s.Q[b], GEOM_QUAT + 4 * g, s.gq[g]);
  }
  s.ncon = 0;
  s.ncon_raw = 0;
  for (int p = 0; p < NPAIR; p++) collide_pair(s, p);
}

// ---------------------------------------------------------------------------------------------- constraint rows
void kbimp(const double* solref, const double* solimp, double pos, double h, double* k, double* b, double* imp) {
  double tc = std::fmax(solref[0], 2 * h), dr = solref[1];
  double dmin = std::fmin(std::fmax(solimp[0], 1e-4), 0.9999), dmax = std::fmin(std::fmax(solimp[1], 1e-4), 0.9999);
  double width = std::fmax(1e-15, solimp[2]), mid = std::fmin(std::fmax(solimp[3], 1e-4), 0.9999);
  double power = std::fmax(1.0, solimp[4]);
  *k = 1.0 / std::fmax(1e-15, dmax * dmax * tc * tc * dr * dr);
  *b = 2.0 / std::fmax(1e-15, dmax * tc);
  double x = std::fabs(pos) / width;
  if (dmin == dmax || solimp[2] <= 1e-15) *imp = 0.5 * (dmin + dmax);
  else if (x <= 0) *imp = dmin;
  else if (x >= 1) *imp = dmax;
  else if (power == 1) *imp = dmin + x * (dmax - dmin);
  else {
    double y = x <= mid ? std::pow(x, power) / std::pow(mid, power - 1)
                        : 1 - std::pow(1 - x, power) / std::pow(1 - mid, power - 1);
    *imp = std::fmin(std::fmax(dmin + y * (dmax - dmin), dmin), dmax);
  }
}

// support size k_c of a contact: the dofs on exactly one of its bodies' chains
int support_size(const Contact& c) {
  int k = 0;
  for (int i = 0; i < NV; i++) {
    int bi = DOF_BODY[i];
    k += ((BODY_ANCMASK[c.b1] >> bi) & 1u) != ((BODY_ANCMASK[c.b2] >> bi) & 1u);
  }
  return k;
}

void rows(World& s) {
  const double h = TIMESTEP;
  int r = 0;
  std::memset(s.efcJ, 0, sizeof(s.efcJ));
  s.nlim = 0;
  for (int i = 6; i < NV; i++) {  // hinge limits (dof order)
    double q = s.qpos[i + 1], dmin = q - DOF_RANGE[2 * i], dmax = DOF_RANGE[2 * i + 1] - q;
    if (!(std::fmin(dmin, dmax) < 0)) continue;
    if (r >= NEFC) { s.flags |= 16; continue; }
    double sg = dmin < dmax ? 1 : -1, pos = std::fmin(dmin, dmax), k, b, imp;
    kbimp(JNT_SOLREF, JNT_SOLIMP, pos, h, &k, &b, &imp);
    double iw = DOF_INVWEIGHT0[i];
    s.efcJ[r][i] = sg;
    s.efcD[r] = 1.0 / std::fmax(iw * (1 - imp) / imp, 1e-15);
    s.aref[r] = -k * imp * pos - b * (sg * s.qvel[i]);
    r++;
    s.nlim++;
  }
  for (int c = 0; c < s.ncon; c++) {
    const Contact& ct = s.con[c];
    // contact Jacobian frame rows (step.py:1830-1878): J(body2, pos) - J(body1, pos) on the dofs of exactly one chain
    double Jf[3][NV];
    std::memset(Jf, 0, sizeof(Jf));
    double rr[3];
    for (int k = 0; k < 3; k++) rr[k] = ct.pos[k] - s.O[k];
    for (int i = 0; i < NV; i++) {
      int bi = DOF_BODY[i];
      int in1 = (BODY_ANCMASK[ct.b1] >> bi) & 1, in2 = (BODY_ANCMASK[ct.b2] >> bi) & 1;
      if (in1 == in2) continue;
      double u[3], jp[3], sg = in2 ? 1 : -1;
      cross(s.S[i], rr, u);
      for (int k = 0; k < 3; k++) jp[k] = sg * (s.S[i][3 + k] + u[k]);
      for (int d = 0; d < 3; d++) Jf[d][i] = dot3(ct.frame + 3 * d, jp);
    }
    double k, b, imp, mu = ct.mu;
    kbimp(PAIR_SOLREF, PAIR_SOLIMP, ct.dist, h, &k, &b, &imp);
    double iw = BODY_INVWEIGHT0[ct.b1] + BODY_INVWEIGHT0[ct.b2];
    if (ct.dim == 3) iw = (mu * mu * iw + iw) * 2 * mu * mu / IMPRATIO;  // contact_invw (step.py:1181-1185)
    double D = 1.0 / std::fmax(iw * (1 - imp) / imp, 1e-15);
    int nr = ct.dim == 3 ? 4 : 1;
    s.flops += 200.0 + 25.0 * support_size(ct) + 60.0 * nr;  // narrowphase, Jacobian, rows of one contact
    for (int t = 0; t < nr; t++) {
      if (r >= NEFC) { s.flags |= 16; break; }
      double sg = (t & 1) ? -1 : 1;
      double vel = 0;
      for (int i = 0; i < NV; i++) {
        double j = ct.dim == 3 ? Jf[0][i] + sg * mu * Jf[1 + (t >> 1)][i] : Jf[0][i];
        s.efcJ[r][i] = j;
        vel += j * s.qvel[i];
      }
      s.efcD[r] = D;
      s.aref[r] = -k * imp * ct.dist - b * vel;
      r++;
    }
  }
  s.nefc = r;
}

// ---------------------------------------------------------------------------------------------- Newton solver
struct Solver {
  World& s;
  double Ma[NV], jar[NEFC], grad[NV];
  explicit Solver(World& w) : s(w) {}
  void refresh(const double* qacc) {
    for (int i = 0; i < NV; i++) { double a = 0; for (int j = 0; j < NV; j++) a += s.M[i][j] * qacc[j]; Ma[i] = a; }
    for (int r = 0; r < s.nefc; r++) {
      double a = 0;
      for (int i = 0; i < NV; i++) a += s.efcJ[r][i] * qacc[i];
      jar[r] = a - s.aref[r];
    }
  }
  double cost(const double* qacc) const {
    double g = 0;
    for (int i = 0; i < NV; i++) g += 0.5 * (Ma[i] - s.qsm[i]) * (qacc[i] - s.qacc0[i]);
    for (int r = 0; r < s.nefc; r++) if (jar[r] < 0) g += 0.5 * s.efcD[r] * jar[r] * jar[r];
    return g;
  }
  double gradient() {
    double gn = 0;
    for (int i = 0; i < NV; i++) {
      double jtf = 0;
      for (int r = 0; r < s.nefc; r++) if (jar[r] < 0) jtf -= s.efcJ[r][i] * s.efcD[r] * jar[r];
      grad[i] = Ma[i] - s.qsm[i] - jtf;
      gn += grad[i] * grad[i];
    }
    return std::sqrt(gn);
  }
};

void newton(World& s, int iterations, double tol, int ls_max, double ls_tol) {
  Solver v(s);
  const double scale = 1.0 / (MEANINERTIA * NV);
  double warm[NV], Mw[NV], jw[NEFC];
  std::memcpy(warm, s.qacc, sizeof(warm));
  v.refresh(s.qacc);
  double cost = v.cost(s.qacc);
  std::memcpy(Mw, v.Ma, sizeof(Mw));
  std::memcpy(jw, v.jar, sizeof(jw));
  std::memcpy(s.qacc, s.qacc0, sizeof(warm));
  v.refresh(s.qacc);
  double cost0 = v.cost(s.qacc);
  if (cost0 > cost) {
    std::memcpy(s.qacc, warm, sizeof(warm));
    std::memcpy(v.Ma, Mw, sizeof(Mw));
    std::memcpy(v.jar, jw, sizeof(jw));
  } else {
    cost = cost0;
  }
  v.gradient();
  int it = 0;
  static thread_local double H[NV][NV];
  int ksum = 0;
  for (int c = 0; c < s.ncon; c++) ksum += support_size(s.con[c]);
  bool zsame = false;
  while (it < iterations) {
    // algorithmic flops of the iteration (closed form): Hessian assembly over the contacts with a quadratic row and a
    // factorization (or a re-solve with the kept factor when no row changed its zone), J p and J' f over the supports,
    // M p; the line search's 6 R flops per evaluation are added below
    if (!zsame) {
      int r = s.nlim;
      for (int c = 0; c < s.ncon; c++) {
        int nr = s.con[c].dim == 3 ? 4 : 1;
        bool act = false;
        for (int t = 0; t < nr && r + t < s.nefc; t++) act |= v.jar[r + t] < 0;
        r += nr;
        int k = support_size(s.con[c]);
        if (act) s.flops += 6.0 * k * (k + 1) / 2 + 12.0 * k;
      }
      s.flops += 2.86e4;
    } else {
      s.flops += 2.45e3;
    }
    s.flops += 12.0 * ksum + 2.45e3;
    for (int i = 0; i < NV; i++)
      for (int j = 0; j < NV; j++) H[i][j] = s.M[i][j];
    for (int r = 0; r < s.nefc; r++) {
      if (!(v.jar[r] < 0)) continue;
      for (int i = 0; i < NV; i++) {
        double ji = s.efcJ[r][i] * s.efcD[r];
        if (ji == 0) continue;
        for (int j = 0; j < NV; j++) H[i][j] += ji * s.efcJ[r][j];
      }
    }
    double p[NV], mg[NV];
    for (int i = 0; i < NV; i++) mg[i] = -v.grad[i];
    chol_solve(H, mg, p);
    // exact line search on the piecewise-quadratic cost along p (step.py:2032-2084)
    double Mp[NV], jv[NEFC], a1 = 0, a2 = 0;
    for (int i = 0; i < NV; i++) { double a = 0; for (int j = 0; j < NV; j++) a += s.M[i][j] * p[j]; Mp[i] = a; }
    for (int r = 0; r < s.nefc; r++) { double a = 0; for (int i = 0; i < NV; i++) a += s.efcJ[r][i] * p[i]; jv[r] = a; }
    for (int i = 0; i < NV; i++) { a1 += (v.Ma[i] - s.qsm[i]) * p[i]; a2 += p[i] * Mp[i]; }
    double alpha = 0, lo = 0, hi = 1e300, d0 = 0;
    bool newton_step = false;
    bool zprev_valid = false;
    static thread_local unsigned char zprev[NEFC], z[NEFC];
    for (int k = 0; k <= ls_max; k++) {
      s.flops += 6.0 * s.nefc;
      double fd = 0, fdd = 0;
      for (int r = 0; r < s.nefc; r++) {
        double x = v.jar[r] + alpha * jv[r];
        z[r] = x < 0;
        if (x < 0) { fd += s.efcD[r] * x * jv[r]; fdd += s.efcD[r] * jv[r] * jv[r]; }
      }
      if (newton_step && zprev_valid && std::memcmp(z, zprev, s.nefc) == 0) break;
      if (k == ls_max) break;
      fd += a1 + alpha * a2;
      fdd += a2;
      if (k == 0) { d0 = fd; if (d0 >= 0) break; }
      if (std::fabs(fd) <= ls_tol * std::fabs(d0)) break;
      if (fd < 0) lo = alpha; else hi = alpha;
      double nx = alpha - fd / fdd;
      newton_step = nx > lo && nx < hi;
      if (!newton_step) nx = hi < 1e299 ? 0.5 * (lo + hi) : 2 * std::fmax(alpha, 1e-6);
      std::memcpy(zprev, z, s.nefc);
      zprev_valid = true;
      alpha = nx;
    }
    for (int i = 0; i < NV; i++) { s.qacc[i] += alpha * p[i]; v.Ma[i] += alpha * Mp[i]; }
    bool chg = false;
    for (int r = 0; r < s.nefc; r++) {
      double xn = v.jar[r] + alpha * jv[r];
      chg |= (v.jar[r] < 0) != (xn < 0);
      v.jar[r] = xn;
    }
    zsame = !chg;
    double newcost = v.cost(s.qacc);
    double gn = v.gradient();
    double improvement = scale * (cost - newcost);
    cost = newcost;
    it++;
    if (improvement < tol || scale * gn < tol) break;
  }
  s.niter = it;
  if (s.hfinal) {  // the checker's hook: H = M + J' D J on the rows in the quadratic zone at the final a*
    for (int i = 0; i < NV; i++)
      for (int j = 0; j < NV; j++) s.hfinal[i][j] = s.M[i][j];
    for (int r = 0; r < s.nefc; r++) {
      if (!(v.jar[r] < 0)) continue;
      for (int i = 0; i < NV; i++)
        for (int j = 0; j < NV; j++) s.hfinal[i][j] += s.efcJ[r][i] * s.efcD[r] * s.efcJ[r][j];
    }
  }
}

// ---------------------------------------------------------------------------------------------- integration
void integrate(World& s) {
  const double h = TIMESTEP;
  static thread_local double Q[NV][NV];
  double Ma[NV], adv[NV];
  for (int i = 0; i < NV; i++) {
    double a = 0;
    for (int j = 0; j < NV; j++) { a += s.M[i][j] * s.qacc[j]; Q[i][j] = s.M[i][j]; }
    Ma[i] = a;
    Q[i][i] += h * DOF_KV[i];
  }
  chol_solve(Q, Ma, adv);
  std::memcpy(s.aadv, adv, sizeof(adv));
  for (int i = 0; i < NV; i++) s.qvel[i] += h * adv[i];
  for (int k = 0; k < 3; k++) s.qpos[k] += h * s.qvel[k];
  double w[3] = {s.qvel[3], s.qvel[4], s.qvel[5]}, nw = std::sqrt(dot3(w, w));
  if (nw > 0) {
    double ang = h * nw, sa = std::sin(0.5 * ang), ca = std::cos(0.5 * ang);
    double dq[4] = {ca, sa * w[0] / nw, sa * w[1] / nw, sa * w[2] / nw}, q[4], o[4];
    std::memcpy(q, s.qpos + 3, sizeof(q));
    qmul(q, dq, o);
    double on = 1.0 / std::sqrt(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
    for (int k = 0; k < 4; k++) s.qpos[3 + k] = o[k] * on;
  }
  for (int i = 6; i < NV; i++) s.qpos[i + 1] += h * s.qvel[i];
}


// ---------------------------------------------------------------------------------------------- adjoint (float64)
// The VJP of a control step, restated in spatial algebra about the fixed point O (the root origin at the substep's
// input state). Per substep, in reverse: the integrator's VJP in the tangent space (root rotation q (+) exp(h w' / 2):
// t = R(dq) t', w' bar += h J_r(h w')' t'), y = Q^-1 a_adv bar with Q = M + h kv, a* bar = a_adv bar - h kv y, the
// IFT of Newton's optimum lambda = H^-1 a* bar (H at the final zones), then the gradient of
//   Psi(q, v) = y' M(q) a~ - lambda' [RNE(q, v, a*) - f_act(q, v, u) + sum_active D_r J_r' (J_r a* - aref_r)]
// (a~ = a* - a_adv). The derivative of a term in q_j follows from moving the subtree of dof j rigidly by its motion
// subspace S_j: quantities attached to that subtree change covariantly, the others (the joint's outside: parent body,
// gravity) do not, so every q-derivative is a subtree sum of force vectors dotted with S_j plus terms with the joint's
// outside quantities. Contacts enter as wrenches (pose cotangents of the collision primitives, and the change of the
// bodies' twists at the contact point); limit rows through their distance.
struct Sv { double w[3], v[3]; };  // a spatial vector (motion: angular, linear at O; force: moment about O, force)

inline Sv sv0() { Sv r; for (int k = 0; k < 3; k++) r.w[k] = r.v[k] = 0; return r; }
inline Sv sv_add(const Sv& a, const Sv& b, double s = 1) {
  Sv r;
  for (int k = 0; k < 3; k++) { r.w[k] = a.w[k] + s * b.w[k]; r.v[k] = a.v[k] + s * b.v[k]; }
  return r;
}
inline Sv sv_scale(const Sv& a, double s) { return sv_add(sv0(), a, s); }
inline double sv_dot(const Sv& m, const Sv& f) { return dot3(m.w, f.w) + dot3(m.v, f.v); }
inline Sv cross_mm(const Sv& x, const Sv& y) {  // motion x motion
  Sv r;
  double a[3], b[3];
  cross(x.w, y.w, r.w);
  cross(x.w, y.v, a);
  cross(x.v, y.w, b);
  for (int k = 0; k < 3; k++) r.v[k] = a[k] + b[k];
  return r;
}
inline Sv cross_mf(const Sv& x, const Sv& f) {  // motion x* force
  Sv r;
  double a[3], b[3];
  cross(x.w, f.w, a);
  cross(x.v, f.v, b);
  for (int k = 0; k < 3; k++) r.w[k] = a[k] + b[k];
  cross(x.w, f.v, r.v);
  return r;
}
inline Sv inertia_apply(const double* J, const Sv& x) {
  Sv r;
  apply_inertia(J, x.w, x.v, r.w, r.v);
  return r;
}
inline Sv dof_sv(const World& s, int d) {
  Sv r;
  for (int k = 0; k < 3; k++) { r.w[k] = s.S[d][k]; r.v[k] = s.S[d][3 + k]; }
  return r;
}
inline bool in_sub(int b, int root) { return b > 0 && ((BODY_ANCMASK[b] >> root) & 1u); }  // b in root's subtree

// chain twists: W[b] = sum over the dofs d moving b of S_d w_d
void chain_twists(const World& s, const double* w, Sv* W) {
  for (int b = 0; b < NB; b++) {
    W[b] = sv0();
    if (b == 0) continue;
    for (int d = 0; d < NV; d++)
      if ((BODY_ANCMASK[b] >> DOF_BODY[d]) & 1u) W[b] = sv_add(W[b], dof_sv(s, d), w[d]);
  }
}

// impedance and its derivative in the distance: imp, dimp / dpos (kbimp's curve; 0 where clamped)
void imp_d(const double* solimp, double pos, double* imp, double* dimp) {
  double dmin = std::fmin(std::fmax(solimp[0], 1e-4), 0.9999), dmax = std::fmin(std::fmax(solimp[1], 1e-4), 0.9999);
  double width = std::fmax(1e-15, solimp[2]), mid = std::fmin(std::fmax(solimp[3], 1e-4), 0.9999);
  double x = std::fabs(pos) / width, sg = pos < 0 ? -1.0 : 1.0;
  *dimp = 0;
  if (x <= 0) { *imp = dmin; return; }
  if (x >= 1) { *imp = dmax; return; }
  double y, dy;
  if (x <= mid) { y = x * x / mid; dy = 2 * x / mid; }
  else { y = 1 - (1 - x) * (1 - x) / (1 - mid); dy = 2 * (1 - x) / (1 - mid); }
  double v = dmin + y * (dmax - dmin);
  if (v < dmin || v > dmax) { *imp = std::fmin(std::fmax(v, dmin), dmax); return; }
  *imp = v;
  *dimp = dy * (dmax - dmin) * sg / width;
}

// the normal derivative's factor kappa(nu) (1 / nu exact; the reference's options 1-3: frozen, regularized, frozen
// below eps = 1e-3 m; adjoint_contact.py:239-249 adj_kappa)
double kappa(double nu, int normal, double eps) {
  if (normal == 0) return 1.0 / nu;
  if (normal == 1) return 0.0;
  if (normal == 2) return 1.0 / std::fmax(nu, eps);
  return nu < eps ? 0.0 : 1.0 / nu;
}

// make_frame VJP: cotangents of the frame rows (n, b, c) -> n bar
void make_frame_vjp(const double* n, const double* frb, double* nb) {
  double e[3] = {0, 0, 0};
  if (-0.5 < n[1] && n[1] < 0.5) e[1] = 1; else e[2] = 1;
  double ne = dot3(n, e), b0[3];
  for (int k = 0; k < 3; k++) b0[k] = e[k] - n[k] * ne;
  double bl = std::sqrt(dot3(b0, b0)), b[3];
  for (int k = 0; k < 3; k++) b[k] = b0[k] / bl;
  const double* cbar = frb + 6;
  double bbar[3], t[3];
  cross(b, cbar, t);  // c = n x b: n bar += b x c bar, b bar += c bar x n
  for (int k = 0; k < 3; k++) nb[k] += frb[k] + t[k];
  cross(cbar, n, t);
  for (int k = 0; k < 3; k++) bbar[k] = frb[3 + k] + t[k];
  double bb = dot3(b, bbar), b0bar[3];
  for (int k = 0; k < 3; k++) b0bar[k] = (bbar[k] - b[k] * bb) / bl;
  double nb0 = dot3(n, b0bar);
  for (int k = 0; k < 3; k++) nb[k] += -ne * b0bar[k] - nb0 * e[k];
}

// sphere core VJP: (dist, pos, n) = sphere_sphere(p1, r1, p2, r2) with cotangents db, posb, nb -> p1b, p2b
void sphere_core_vjp(const double* p1, double r1, const double* p2, double r2, double db, const double* posb,
                     const double* nb, int normal, double eps, double* p1b, double* p2b) {
  double dl[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
  double l = std::sqrt(dot3(dl, dl));
  double dlb[3] = {0, 0, 0};
  for (int k = 0; k < 3; k++) { p1b[k] += posb[k]; dlb[k] += 0.5 * posb[k]; }
  if (l > 0) {
    double n[3] = {dl[0] / l, dl[1] / l, dl[2] / l}, nt[3];
    for (int k = 0; k < 3; k++) nt[k] = nb[k] + 0.5 * (r1 - r2) * posb[k];
    double nn = dot3(n, nt), kap = kappa(l, normal, eps);
    for (int k = 0; k < 3; k++) dlb[k] += kap * (nt[k] - n[k] * nn) + n[k] * db;
  }
  for (int k = 0; k < 3; k++) { p1b[k] -= dlb[k]; p2b[k] += dlb[k]; }
}

// geometry VJP of contact c: cotangents of (dist, pos, frame) -> world position / rotation cotangents of its geoms
void contact_geom_vjp(const World& s, const Contact& c, double db, const double* posb, const double* frb, int normal,
                      double* x1b, double* t1b, double* x2b, double* t2b) {
  int g1 = PAIR_G1[c.pair], g2 = PAIR_G2[c.pair], ty1 = GEOM_TYPE[g1], ty2 = GEOM_TYPE[g2];
  const double *p1 = s.gx[g1], *q1 = s.gq[g1], *p2 = s.gx[g2], *q2 = s.gq[g2];
  const double *sz1 = GEOM_SIZE + 3 * g1, *sz2 = GEOM_SIZE + 3 * g2;
  for (int k = 0; k < 3; k++) x1b[k] = t1b[k] = x2b[k] = t2b[k] = 0;
  if (ty1 == 0) {  // the floor: n constant; pos = ce - n (r + d / 2), d = (ce - p1) . n - r
    double n[3];
    zaxis(q1, n);
    double ceb[3], pn = dot3(n, posb);
    for (int k = 0; k < 3; k++) ceb[k] = posb[k] - 0.5 * n[k] * pn + n[k] * db;
    if (ty2 == 2) {
      for (int k = 0; k < 3; k++) x2b[k] += ceb[k];
    } else {
      double axis[3], axb[3] = {0, 0, 0};
      zaxis(q2, axis);
      double sg = c.slot == 0 ? 1 : -1;
      for (int k = 0; k < 3; k++) { x2b[k] += ceb[k]; axb[k] += sg * sz2[1] * ceb[k]; }
      // plane_capsule_frame: b = normalize(axis - n (n . axis)) when that is >= 0.5 long
      double na = dot3(n, axis), b0[3];
      for (int k = 0; k < 3; k++) b0[k] = axis[k] - n[k] * na;
      double bn = std::sqrt(dot3(b0, b0));
      if (bn >= 0.5) {
        double b[3], bbar[3], t[3];
        for (int k = 0; k < 3; k++) b[k] = b0[k] / bn;
        cross(frb + 6, n, t);  // c = n x b: b bar += c bar x n
        for (int k = 0; k < 3; k++) bbar[k] = frb[3 + k] + t[k];
        double bb = dot3(b, bbar), b0b[3];
        for (int k = 0; k < 3; k++) b0b[k] = (bbar[k] - b[k] * bb) / bn;
        double nb0 = dot3(n, b0b);
        for (int k = 0; k < 3; k++) axb[k] += b0b[k] - n[k] * nb0;
      }
      cross(axis, axb, t2b);  // a rotation dth of the capsule moves its axis by dth x axis
    }
    return;
  }
  double nb[3] = {0, 0, 0};
  make_frame_vjp(c.frame, frb, nb);
  if (ty1 == 2 && ty2 == 2) {
    sphere_core_vjp(p1, sz1[0], p2, sz2[0], db, posb, nb, normal, s.normal_eps, x1b, x2b);
    return;
  }
  if (ty1 == 2 && ty2 == 3) {
    double axis[3], a[3], ab[3], ap[3], pt[3];
    zaxis(q2, axis);
    for (int k = 0; k < 3; k++) { a[k] = p2[k] - axis[k] * sz2[1]; ab[k] = 2 * axis[k] * sz2[1]; ap[k] = p1[k] - a[k]; }
    double gam = dot3(ab, ab) + 1e-6, raw = dot3(ap, ab) / gam, t = std::fmin(std::fmax(raw, 0.0), 1.0);
    for (int k = 0; k < 3; k++) pt[k] = a[k] + t * ab[k];
    double ptb[3] = {0, 0, 0};
    sphere_core_vjp(p1, sz1[0], pt, sz2[0], db, posb, nb, normal, s.normal_eps, x1b, ptb);
    double abb[3], apb[3] = {0, 0, 0}, axb[3], tb = dot3(ptb, ab);
    for (int k = 0; k < 3; k++) abb[k] = t * ptb[k];
    double ab_a[3];
    for (int k = 0; k < 3; k++) ab_a[k] = ptb[k];  // a bar
    if (raw > 0 && raw < 1) {
      for (int k = 0; k < 3; k++) { apb[k] += tb * ab[k] / gam; abb[k] += tb * ap[k] / gam - tb * raw / gam * 2 * ab[k]; }
    }
    for (int k = 0; k < 3; k++) { x1b[k] += apb[k]; ab_a[k] -= apb[k]; }
    for (int k = 0; k < 3; k++) { x2b[k] += ab_a[k]; axb[k] = -sz2[1] * ab_a[k] + 2 * sz2[1] * abb[k]; }
    cross(axis, axb, t2b);
    return;
  }
  // capsule-capsule: x1, x2 from the segments' normal equations with the forward's clamp cascade
  double z1[3], z2[3], a1[3], a2[3], d[3];
  zaxis(q1, z1);
  zaxis(q2, z2);
  const double h1 = sz1[1], h2 = sz2[1];
  for (int k = 0; k < 3; k++) { a1[k] = z1[k] * h1; a2[k] = z2[k] * h2; d[k] = p1[k] - p2[k]; }
  double ma = dot3(a1, a1), mb = -dot3(a1, a2), mc = dot3(a2, a2), u = -dot3(a1, d), v = dot3(a2, d);
  double det = ma * mc - mb * mb;
  double x1, x2;
  int mode;  // 0 both free, 1 x1 fixed (x2 free), 2 x2 fixed (x1 free), 3 both fixed
  if (std::fabs(det) >= 1e-15) {
    x1 = (mc * u - mb * v) / det; x2 = (ma * v - mb * u) / det;
    mode = 0;
    if (x1 > 1) { x1 = 1; x2 = (v - mb) / mc; mode = 1; }
    else if (x1 < -1) { x1 = -1; x2 = (v + mb) / mc; mode = 1; }
    if (x2 > 1 || x2 < -1) {
      bool hi = x2 > 1;
      x2 = hi ? 1 : -1;
      double raw = hi ? (u - mb) / ma : (u + mb) / ma;
      x1 = std::fmin(std::fmax(raw, -1.0), 1.0);
      mode = (raw >= -1 && raw < 1) ? 2 : 3;
    }
  } else {
    int e = c.slot;
    if (e < 2) {
      x1 = e == 0 ? 1 : -1;
      double raw = e == 0 ? (v - mb) / mc : (v + mb) / mc;
      x2 = std::fmin(std::fmax(raw, -1.0), 1.0);
      mode = (raw >= -1 && raw < 1) ? 1 : 3;
    } else {
      x2 = e == 2 ? 1 : -1;
      double raw = e == 2 ? (u - mb) / ma : (u + mb) / ma;
      x1 = std::fmin(std::fmax(raw, -1.0), 1.0);
      mode = (raw >= -1 && raw < 1) ? 2 : 3;
    }
  }
  double v1[3], v2[3], v1b[3] = {0, 0, 0}, v2b[3] = {0, 0, 0}, dl[3], w[3], a1b[3], a2b[3], x1bar, x2bar;
  for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; dl[k] = v2[k] - v1[k]; }
  cross(a1, a2, w);
  const double ww = dot3(w, w);  // = det without its cancellation
  const bool wok = ww > 1e-12 * ma * mc;
  // near-parallel rule (normal options != 0; adjoint_contact.py:436-448): both parameters held where
  // sin^2(theta) < 1.2e-3
  const bool held = mode == 0 && normal != 0 && ww < s.parallel_eps * ma * mc;
  const double nu = std::sqrt(dot3(dl, dl));
  if (mode == 0 && !held && wok && nu > 0) {
    // both parameters free (adjoint_contact.py:449-465): v2 - v1 is normal to both axes, so the normal is
    // n = sg w / |w| of the axes alone (dn = sg (I - n n') dw / |w|), the distance is stationary in x1, x2, and
    // pos = v1 + n (r1 + dist / 2) moves with x1 through v1 only; the normal options scale this normal path by
    // kappa(nu) nu (the exact derivative: 1). For the exact derivative this equals the general chain below; for the
    // options it is the reference's definition
    double n[3], t[3], tau[3], u1[3], u2[3];
    for (int k = 0; k < 3; k++) n[k] = dl[k] / nu;
    const double dist = nu - sz1[0] - sz2[0], hp = sz1[0] + 0.5 * dist, dt = db + 0.5 * dot3(n, posb);
    for (int k = 0; k < 3; k++) t[k] = nb[k] + hp * posb[k];
    const double nt = dot3(n, t);
    const double knu = normal == 0 ? 1.0 : kappa(nu, normal, s.normal_eps) * nu;
    double f = knu / std::sqrt(ww);
    if (dot3(n, w) < 0) f = -f;
    for (int k = 0; k < 3; k++) tau[k] = f * (t[k] - n[k] * nt);
    cross(a2, tau, u1);
    cross(tau, a1, u2);
    for (int k = 0; k < 3; k++) { v2b[k] = n[k] * dt; v1b[k] = posb[k] - v2b[k]; }
    for (int k = 0; k < 3; k++) {
      x1b[k] += v1b[k]; x2b[k] += v2b[k];
      a1b[k] = x1 * v1b[k] + u1[k]; a2b[k] = x2 * v2b[k] + u2[k];
    }
    x1bar = dot3(a1, posb);
    x2bar = 0;
  } else {
    sphere_core_vjp(v1, sz1[0], v2, sz2[0], db, posb, nb, normal, s.normal_eps, v1b, v2b);
    for (int k = 0; k < 3; k++) { x1b[k] += v1b[k]; x2b[k] += v2b[k]; a1b[k] = x1 * v1b[k]; a2b[k] = x2 * v2b[k]; }
    x1bar = held ? 0 : dot3(a1, v1b);
    x2bar = held ? 0 : dot3(a2, v2b);
  }
  double mab = 0, mbb = 0, mcb = 0, ub = 0, vb = 0, db3[3] = {0, 0, 0};
  if (mode == 0) {  // G's determinant as |a1 x a2|^2 where that is not rounding noise (adjoint_contact.py:472)
    const double g = wok ? ww : det;
    double N1b = x1bar / g, N2b = x2bar / g, detb = -x1bar * x1 / g - x2bar * x2 / g;
    mcb += N1b * u; ub += N1b * mc; mbb -= N1b * v; vb -= N1b * mb;
    mab += N2b * v; vb += N2b * ma; mbb -= N2b * u; ub -= N2b * mb;
    mab += detb * mc; mcb += detb * ma; mbb -= 2 * mb * detb;
  } else if (mode == 1) {  // x2 = (v - mb x1) / mc
    vb += x2bar / mc; mbb -= x2bar * x1 / mc; mcb -= x2bar * x2 / mc;
  } else if (mode == 2) {  // x1 = (u - mb x2) / ma
    ub += x1bar / ma; mbb -= x1bar * x2 / ma; mab -= x1bar * x1 / ma;
  }
  for (int k = 0; k < 3; k++) {
    a1b[k] += 2 * mab * a1[k] - mbb * a2[k] - ub * d[k];
    a2b[k] += 2 * mcb * a2[k] - mbb * a1[k] + vb * d[k];
    db3[k] += -ub * a1[k] + vb * a2[k];
  }
  for (int k = 0; k < 3; k++) { x1b[k] += db3[k]; x2b[k] -= db3[k]; a1b[k] *= h1; a2b[k] *= h2; }
  cross(z1, a1b, t1b);
  cross(z2, a2b, t2b);
}

struct Rec { double qpos[NQ], qvel[NV], astar[NV], aadv[NV]; };

// Algorithmic flops of one substep's VJP (closed form, FMA = 2; counted by substep_vjp as step counts the forward's):
// what the adjoint computes from the substep's record, not this restatement's recomputation of the record.
//  - pose replay (forward kinematics of the 30 hinge bodies: the hinge rotation's sincos ~20, two quaternion products
//    56, the body offset rotated into the world and added 33): 30 x 110 = 3.3e3
//  - integrator VJP (the root's exp map: a rotation 30, J_r' t with two cross products ~80; v bar += h q bar 70): 2e2
//  - implicitfast and IFT solves: two triangular solve pairs with 35 x 35 factors, 2 x 2 x 35^2 = 4.9e3, and
//    a* bar = a_adv bar - h kv y, 70: 4.97e3
//  - twists of v, lambda, y, a*, a~ down the tree (12 per body and channel) and the RNE acceleration's velocity
//    products (30 per body for each of the 2 channels that carry them): 30 x (5 x 12 + 2 x 30) = 3.6e3
//  - per-body force vectors f1, P, Q, R, T, f2, P2 (inertia products ~60, cross products ~30): 30 x 350 = 1.05e4
//  - subtree sums of 12 spatial vectors (72 floats per body): 30 x 72 = 2.2e3
//  - per dof projections (3 motion cross products 90, 12 six-vector dot products 132, 3 force cross products 90,
//    sums 48): 35 x 360 = 1.26e4
//  - actuators: 29 x 8 = 2.3e2
// plus VJP_FLOPS_LIMIT per limit row in the quadratic zone, and per contact with a row in it VJP_FLOPS_CONTACT
// (impedance and its derivative 40, relative twists 18, the three wrench channels onto both bodies 228, the primitive
// and frame VJP 250, the geom wrenches 34) and VJP_FLOPS_ROW per such row (its direction and moment, dot products,
// the D terms, Psi's cotangent of the row).
constexpr double VJP_FLOPS_SUBSTEP = 3.3e3 + 2e2 + 4.97e3 + 3.6e3 + 1.05e4 + 2.2e3 + 1.26e4 + 2.3e2;
constexpr double VJP_FLOPS_LIMIT = 25, VJP_FLOPS_CONTACT = 570, VJP_FLOPS_ROW = 90;

// one substep's VJP: (qb tangent, vb) of its output -> of its input; ub accumulates the ctrl gradient
void substep_vjp(World& s, const Rec& rec, const double* ctrl, double* qb, double* vb, double* ub, int clamp_kv,
                 int normal, double clamp_soft) {
  const double h = TIMESTEP;
  std::memcpy(s.qpos, rec.qpos, sizeof(rec.qpos));
  std::memcpy(s.qvel, rec.qvel, sizeof(rec.qvel));
  smooth(s, ctrl);
  collision(s);
  rows(s);
  const double* as = rec.astar;
  s.aflops += VJP_FLOPS_SUBSTEP;
  // 1. integrator: v' = v + h a_adv, q' = q (+) h v'
  double vt[NV], qn[NV];
  for (int i = 0; i < NV; i++) { vt[i] = vb[i]; qn[i] = qb[i]; }
  for (int i = 0; i < 3; i++) vt[i] += h * qb[i];
  for (int i = 6; i < NV; i++) vt[i] += h * qb[i];
  {
    double w[3], phi[3];
    for (int k = 0; k < 3; k++) { w[k] = rec.qvel[3 + k] + h * rec.aadv[3 + k]; phi[k] = h * w[k]; }
    double th = std::sqrt(dot3(phi, phi));
    double dq[4];
    if (th > 0) {
      double sn = std::sin(0.5 * th) / th;
      dq[0] = std::cos(0.5 * th); dq[1] = sn * phi[0]; dq[2] = sn * phi[1]; dq[3] = sn * phi[2];
    } else { dq[0] = 1; dq[1] = dq[2] = dq[3] = 0; }
    double t[3] = {qb[3], qb[4], qb[5]}, rt[3];
    qrot(dq, t, rt);  // t = R(dq) t'
    for (int k = 0; k < 3; k++) qn[3 + k] = rt[k];
    // J_r(phi)' t' = t' + c1 phi x t' + c2 phi x (phi x t')  (J_r = I - c1 [phi] + c2 [phi]^2), c1 = (1 - cos th) /
    // th^2, c2 = (th - sin th) / th^3: their Taylor series through th^8 below th = 0.5 (truncation < 5e-12 relative;
    // the closed forms cancel at small th, in the float32 build of this text most), the closed forms above
    double c1, c2;
    if (th < 0.5) {
      const double x = th * th;
      c1 = 0.5 + x * (-1.0 / 24 + x * (1.0 / 720 + x * (-1.0 / 40320 + x * (1.0 / 3628800))));
      c2 = 1.0 / 6 + x * (-1.0 / 120 + x * (1.0 / 5040 + x * (-1.0 / 362880 + x * (1.0 / 39916800))));
    } else { c1 = (1 - std::cos(th)) / (th * th); c2 = (th - std::sin(th)) / (th * th * th); }
    double pt[3], ppt[3];
    cross(phi, t, pt);
    cross(phi, pt, ppt);
    for (int k = 0; k < 3; k++) vt[3 + k] += h * (t[k] + c1 * pt[k] + c2 * ppt[k]);
  }
  // 2. implicitfast: y = Q^-1 a_adv bar, a* bar = a_adv bar - h kv y
  static thread_local double Qm[NV][NV], H[NV][NV];
  double aab[NV], y[NV], asb[NV], lam[NV], at[NV];
  for (int i = 0; i < NV; i++) {
    aab[i] = h * vt[i];
    for (int j = 0; j < NV; j++) Qm[i][j] = s.M[i][j];
    Qm[i][i] += h * DOF_KV[i];
  }
  chol_solve(Qm, aab, y);
  for (int i = 0; i < NV; i++) { asb[i] = aab[i] - h * DOF_KV[i] * y[i]; at[i] = as[i] - rec.aadv[i]; }
  // 3. IFT: lambda = H^-1 a* bar, H = M + J' D J on the rows with J a* - aref < 0
  double jar[NEFC];
  for (int r = 0; r < s.nefc; r++) {
    double a = 0;
    for (int i = 0; i < NV; i++) a += s.efcJ[r][i] * as[i];
    jar[r] = a - s.aref[r];
  }
  for (int i = 0; i < NV; i++)
    for (int j = 0; j < NV; j++) H[i][j] = s.M[i][j];
  for (int r = 0; r < s.nefc; r++)
    if (jar[r] < 0)
      for (int i = 0; i < NV; i++)
        for (int j = 0; j < NV; j++) H[i][j] += s.efcD[r] * s.efcJ[r][i] * s.efcJ[r][j];
  chol_solve(H, asb, lam);
  // 4. gradients of Psi
  double gq[NV] = {0}, gv[NV] = {0};
  static thread_local Sv V[NB], Lm[NB], Yt[NB], Aw[NB], A1[NB], A2[NB];
  chain_twists(s, s.qvel, V);
  chain_twists(s, lam, Lm);
  chain_twists(s, y, Yt);
  chain_twists(s, as, Aw);
  chain_twists(s, at, A2);
  Sv grav = sv0();
  for (int k = 0; k < 3; k++) grav.v[k] = -GRAVITY[k];
  for (int b = 1; b < NB; b++) {  // RNE acceleration: gravity, S a*, and V_c(d) x S_d v_d for the non-translation dofs
    A1[b] = sv_add(grav, Aw[b]);
    for (int d = 3; d < NV; d++)
      if ((BODY_ANCMASK[b] >> DOF_BODY[d]) & 1u) A1[b] = sv_add(A1[b], cross_mm(V[DOF_BODY[d]], dof_sv(s, d)), s.qvel[d]);
  }
  // per-body force vectors; Psi's contact wrenches
  static thread_local Sv f1[NB], P[NB], Qs[NB], Rs[NB], Ts[NB], f2[NB], P2[NB], E[NB], OL[NB], OA[NB], OV[NB], G[NB];
  for (int b = 0; b < NB; b++) {
    f1[b] = P[b] = Qs[b] = Rs[b] = Ts[b] = f2[b] = P2[b] = E[b] = OL[b] = OA[b] = OV[b] = G[b] = sv0();
    if (b == 0) continue;
    const double* I = s.Ib[b];
    Sv IV = inertia_apply(I, V[b]), IL = inertia_apply(I, Lm[b]);
    f1[b] = sv_add(inertia_apply(I, A1[b]), cross_mf(V[b], IV));
    P[b] = IL;
    Qs[b] = cross_mf(V[b], IL);
    Rs[b] = cross_mf(Lm[b], IV);
    Ts[b] = inertia_apply(I, cross_mm(V[b], Lm[b]));
    f2[b] = inertia_apply(I, A2[b]);
    P2[b] = inertia_apply(I, Yt[b]);
  }
  // limit rows
  int r = 0;
  for (int i = 6; i < NV; i++) {
    double q = s.qpos[i + 1], dmin = q - DOF_RANGE[2 * i], dmax = DOF_RANGE[2 * i + 1] - q;
    if (!(std::fmin(dmin, dmax) < 0)) continue;
    if (r >= s.nefc) break;
    if (jar[r] < 0) {
      s.aflops += VJP_FLOPS_LIMIT;
      double sg = dmin < dmax ? 1 : -1, pos = std::fmin(dmin, dmax), k, b, imp, dimp;
      kbimp(JNT_SOLREF, JNT_SOLIMP, pos, h, &k, &b, &imp);
      imp_d(JNT_SOLIMP, pos, &imp, &dimp);
      double iw = DOF_INVWEIGHT0[i], D = s.efcD[r], dD = dimp / (iw * (1 - imp) * (1 - imp));
      double jl = sg * lam[i], x = jar[r];
      double dbar = -(dD * jl * x + D * jl * k * (dimp * pos + imp));
      gq[i] += dbar * sg;
      gv[i] += -D * jl * b * sg;
    }
    r++;
  }
  // contacts
  for (int c = 0; c < s.ncon && r < s.nefc; c++) {
    const Contact& ct = s.con[c];
    int nr = ct.dim == 3 ? 4 : 1, r0 = r;
    r += nr;
    bool act = false;
    for (int t = 0; t < nr && r0 + t < s.nefc; t++) act |= jar[r0 + t] < 0;
    if (!act) continue;
    s.aflops += VJP_FLOPS_CONTACT;
    double k, b, imp, dimp;
    kbimp(PAIR_SOLREF, PAIR_SOLIMP, ct.dist, h, &k, &b, &imp);
    imp_d(PAIR_SOLIMP, ct.dist, &imp, &dimp);
    double mu = ct.mu, iw = BODY_INVWEIGHT0[ct.b1] + BODY_INVWEIGHT0[ct.b2];
    if (ct.dim == 3) iw = (mu * mu * iw + iw) * 2 * mu * mu / IMPRATIO;
    double D = 1.0 / (iw * (1 - imp) / imp), dD = dimp / (iw * (1 - imp) * (1 - imp));
    double rr[3];
    for (int q = 0; q < 3; q++) rr[q] = ct.pos[q] - s.O[q];
    Sv Lc = sv_add(Lm[ct.b2], Lm[ct.b1], -1), Ac = sv_add(Aw[ct.b2], Aw[ct.b1], -1), Vc = sv_add(V[ct.b2], V[ct.b1], -1);
    double dbar = 0, rb[3] = {0, 0, 0}, frb[9] = {0};
    Sv OmL = sv0(), OmA = sv0();
    for (int t = 0; t < nr && r0 + t < s.nefc; t++) {
      if (!(jar[r0 + t] < 0)) continue;
      s.aflops += VJP_FLOPS_ROW;
      double sg = (t & 1) ? -1 : 1, u[3];
      const double* tk = ct.frame + 3 * (1 + (t >> 1));
      for (int q = 0; q < 3; q++) u[q] = ct.dim == 3 ? ct.frame[q] + sg * mu * tk[q] : ct.frame[q];
      Sv Ph;
      cross(rr, u, Ph.w);
      for (int q = 0; q < 3; q++) Ph.v[q] = u[q];
      double jl = sv_dot(Lc, Ph), x = jar[r0 + t];
      dbar += -(dD * jl * x + D * jl * k * (dimp * ct.dist + imp));
      OmL = sv_add(OmL, Ph, -D * x);
      OmA = sv_add(OmA, Ph, -D * jl);
      Sv Pb = sv_add(sv_scale(Lc, -D * x), sv_add(Ac, Vc, b), -D * jl);  // Psi's cotangent of Phi
      double ubar[3], t3[3];
      cross(Pb.w, rr, t3);
      for (int q = 0; q < 3; q++) ubar[q] = Pb.v[q] + t3[q];
      cross(u, Pb.w, t3);
      for (int q = 0; q < 3; q++) rb[q] += t3[q];
      for (int q = 0; q < 3; q++) {
        frb[q] += ubar[q];
        if (ct.dim == 3) frb[3 * (1 + (t >> 1)) + q] += sg * mu * ubar[q];
      }
    }
    Sv OmV = sv_scale(OmA, b);
    const int bs[2] = {ct.b1, ct.b2};
    for (int side = 0; side < 2; side++) {
      int bb = bs[side];
      if (bb == 0) continue;
      double sgn = side ? 1 : -1;
      Sv e = sv_add(sv_add(cross_mf(Lm[bb], OmL), cross_mf(Aw[bb], OmA)), cross_mf(V[bb], OmV));
      E[bb] = sv_add(E[bb], e, sgn);
      OL[bb] = sv_add(OL[bb], OmL, sgn);
      OA[bb] = sv_add(OA[bb], OmA, sgn);
      OV[bb] = sv_add(OV[bb], OmV, sgn);
    }
    double x1b[3], t1b[3], x2b[3], t2b[3];
    contact_geom_vjp(s, ct, dbar, rb, frb, normal, x1b, t1b, x2b, t2b);
    const int gs[2] = {PAIR_G1[ct.pair], PAIR_G2[ct.pair]};
    const double* xb[2] = {x1b, x2b};
    const double* tb[2] = {t1b, t2b};
    for (int side = 0; side < 2; side++) {
      int g = gs[side], bb = GEOM_BODY[g];
      if (bb == 0) continue;
      Sv w;
      double xo[3], m[3];
      for (int q = 0; q < 3; q++) xo[q] = s.gx[g][q] - s.O[q];
      cross(xo, xb[side], m);
      for (int q = 0; q < 3; q++) { w.w[q] = tb[side][q] + m[q]; w.v[q] = xb[side][q]; }
      G[bb] = sv_add(G[bb], w);
    }
  }
  // per dof: subtree sums and the joint's outside quantities
  for (int j = 0; j < NV; j++) {
    const int bj = DOF_BODY[j];
    Sv F1s = sv0(), Ps = sv0(), Qss = sv0(), Rss = sv0(), Tss = sv0(), F2s = sv0(), P2s = sv0(), Es = sv0(), Gs = sv0(),
       OLs = sv0(), OAs = sv0(), OVs = sv0();
    for (int b = 1; b < NB; b++) {
      if (!in_sub(b, bj)) continue;
      F1s = sv_add(F1s, f1[b]); Ps = sv_add(Ps, P[b]); Qss = sv_add(Qss, Qs[b]); Rss = sv_add(Rss, Rs[b]);
      Tss = sv_add(Tss, Ts[b]); F2s = sv_add(F2s, f2[b]); P2s = sv_add(P2s, P2[b]); Es = sv_add(Es, E[b]);
      Gs = sv_add(Gs, G[b]); OLs = sv_add(OLs, OL[b]); OAs = sv_add(OAs, OA[b]); OVs = sv_add(OVs, OV[b]);
    }
    Sv Vo = sv0(), Lo = sv0(), Yo = sv0(), Awo = sv0(), A1o = grav, A2o = sv0();
    if (j >= 3 && j < 6) {
      for (int k = 0; k < 3; k++) {
        Vo.v[k] = s.qvel[k]; Lo.v[k] = lam[k]; Yo.v[k] = y[k]; Awo.v[k] = as[k]; A1o.v[k] += as[k]; A2o.v[k] = at[k];
      }
    } else if (j >= 6) {
      int p = BODY_PARENT[bj];
      Vo = V[p]; Lo = Lm[p]; Yo = Yt[p]; Awo = Aw[p]; A1o = A1[p]; A2o = A2[p];
    }
    Sv Sj = dof_sv(s, j);
    Sv sig = cross_mm(Sj, Vo), alp = cross_mm(Sj, A1o), ell = cross_mm(Sj, Lo);
    double dq1 = -sv_dot(ell, F1s) - sv_dot(alp, Ps) - sv_dot(sig, Qss) + sv_dot(cross_mm(sig, Vo), Ps)
                 + sv_dot(sig, Rss) + sv_dot(sig, Tss);
    Sv rho = sv0();
    if (j >= 3) rho = sv_add(sig, cross_mm(Sj, V[bj]));
    double dv1 = sv_dot(Sj, sv_add(sv_add(Qss, Rss, -1), Tss, -1)) - sv_dot(rho, Ps);
    double dq2 = -sv_dot(cross_mm(Sj, Yo), F2s) - sv_dot(cross_mm(Sj, A2o), P2s);
    double dqc = sv_dot(Sj, sv_add(Es, Gs)) - sv_dot(Sj, sv_add(sv_add(cross_mf(Lo, OLs), cross_mf(Awo, OAs)),
                                                               cross_mf(Vo, OVs)));
    gq[j] += dq2 - dq1 + dqc;
    gv[j] += -dv1 + sv_dot(Sj, OVs);
  }
  // actuators (the PD force kp (u - q) - kv v, clamped at +-frclim)
  for (int i = 6; i < NV; i++) {
    double wq = 1, wv = 1;
    if (s.clamped[i]) {
      if (clamp_kv == 0) { wq = 0; wv = 1; }
      else if (clamp_kv == 1) { wq = wv = 0; }
      else {
        double raw = DOF_KP[i] * (ctrl[i - 6] - s.qpos[i + 1]) - DOF_KV[i] * s.qvel[i];
        // the relative overshoot, floored at 0 (adjoint.py:822-829 lam_soft): w <= 1
        double o = std::fmax((std::fabs(raw) - DOF_FRCLIM[i]) / DOF_FRCLIM[i], 0.0);
        wq = wv = clamp_soft > 0 ? std::exp(-o / clamp_soft) : 0.0;
      }
    }
    gq[i] -= wq * DOF_KP[i] * lam[i];
    gv[i] -= wv * DOF_KV[i] * lam[i];
    ub[i - 6] += wq * DOF_KP[i] * lam[i];
  }
  for (int i = 0; i < NV; i++) { qb[i] = qn[i] + gq[i]; vb[i] = vt[i] + gv[i]; }
}

}  // namespace

extern "C" {

// One control step of nsub substeps for each of nw worlds, float64 (row-major world-major arrays as the engine's).
// iterations / tol: Newton's iteration cap and tolerance (the engine: 10, the model's 1e-8; MuJoCo C truth: 2000,
// 1e-13); ls_max / ls_tol: the line search's evaluation cap and relative derivative tolerance (40, 1e-7).
// info (nw, 4): last substep's Newton iterations, contacts (found, before the cap), rows, flags (4 contacts over
// capacity, 16 rows over capacity). flops (nw) or NULL: the world-step's algorithmic flops by the closed-form phase
// counts (smooth 2.5e4, each factor + solve 3.1e4, broadphase 5e3 per substep; per contact 200 + 25 k + 60 rows;
// per Newton iteration the Hessian assembly 6 k (k + 1) / 2 + 12 k over the contacts with a quadratic row and a
// factorization 2.86e4, or 2.45e3 for a re-solve, plus 12 sum k + 2.45e3 and 6 R per line-search evaluation), k the
// contact's support size and R the rows. Returns 0.
int g1o_step_ex(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
                const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub,
                double* oqpos, double* oqvel, double* owarm, int* info, double* flops, const double* qfrc,
                double* freeze, int freeze_mode) {
  World* s = new World;
  init_hooks(*s);
  s->freeze = reinterpret_cast<double (*)[3]>(freeze);
  s->freeze_mode = freeze ? freeze_mode : 0;
  for (int w = 0; w < nw; w++) {
    std::memcpy(s->qpos, qpos + (size_t)w * NQ, sizeof(double) * NQ);
    std::memcpy(s->qvel, qvel + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->qacc, warm + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->com, com + (size_t)w * 3, sizeof(double) * 3);
    s->fric = fric[w];
    s->flags = 0;
    s->flops = 0;
    s->qfrc = qfrc ? qfrc + (size_t)w * NV : nullptr;
    for (int k = 0; k < nsub; k++) {
      // smooth dynamics 2.5e4, qacc_smooth factor + solve 3.1e4, implicitfast factor + solve 3.1e4, broadphase 5e3
      s->flops += 2.5e4 + 3.1e4 + 3.1e4 + 5e3;
      smooth(*s, ctrl + (size_t)w * NU);
      collision(*s);
      rows(*s);
      newton(*s, iterations, tol, ls_max, ls_tol);
      integrate(*s);
    }
    std::memcpy(oqpos + (size_t)w * NQ, s->qpos, sizeof(double) * NQ);
    std::memcpy(oqvel + (size_t)w * NV, s->qvel, sizeof(double) * NV);
    std::memcpy(owarm + (size_t)w * NV, s->qacc, sizeof(double) * NV);
    if (info) {
      info[4 * w] = s->niter; info[4 * w + 1] = s->ncon_raw; info[4 * w + 2] = s->nefc; info[4 * w + 3] = s->flags;
    }
    if (flops) flops[w] = s->flops;
  }
  delete s;
  return 0;
}

int g1o_step(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
             const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub,
             double* oqpos, double* oqvel, double* owarm, int* info, double* flops) {
  return g1o_step_ex(nw, qpos, qvel, warm, ctrl, fric, com, iterations, tol, ls_max, ls_tol, nsub, oqpos, oqvel, owarm,
                     info, flops, nullptr, nullptr, 0);
}

// g1o_step on nthreads host threads, each taking a contiguous share of the worlds (the CPU baseline's all-threads
// leg; results identical to g1o_step's, every world being independent).
int g1o_step_mt(int nthreads, int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
                const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub,
                double* oqpos, double* oqvel, double* owarm, int* info) {
  if (nthreads < 1) nthreads = 1;
  if (nthreads > nw) nthreads = nw > 0 ? nw : 1;
  std::vector<std::thread> pool;
  for (int t = 0; t < nthreads; t++) {
    const int a = (int)((long long)nw * t / nthreads), b = (int)((long long)nw * (t + 1) / nthreads);
    pool.emplace_back([=] {
      g1o_step(b - a, qpos + (size_t)a * NQ, qvel + (size_t)a * NV, warm + (size_t)a * NV, ctrl + (size_t)a * NU,
               fric + a, com + (size_t)a * 3, iterations, tol, ls_max, ls_tol, nsub, oqpos + (size_t)a * NQ,
               oqvel + (size_t)a * NV, owarm + (size_t)a * NV, info ? info + 4 * (size_t)a : nullptr, nullptr);
    });
  }
  for (auto& th : pool) th.join();
  return 0;
}

// One substep of one world (the checker's view of a tape record): M (NV x NV) at the input state, and H = M + J'DJ at
// Newton's final zones (NV x NV), with the given warm start and solver settings.
int g1o_substep_hessian(const double* qpos, const double* qvel, const double* warm, const double* ctrl, double fric,
                        const double* com, int iterations, double tol, int ls_max, double ls_tol, double* M,
                        double* H) {
  World* s = new World;
  init_hooks(*s);
  std::memcpy(s->qpos, qpos, sizeof(double) * NQ);
  std::memcpy(s->qvel, qvel, sizeof(double) * NV);
  std::memcpy(s->qacc, warm, sizeof(double) * NV);
  std::memcpy(s->com, com, sizeof(double) * 3);
  s->fric = fric;
  s->flags = 0;
  s->flops = 0;
  s->hfinal = reinterpret_cast<double (*)[NV]>(H);
  smooth(*s, ctrl);
  std::memcpy(M, s->M, sizeof(s->M));
  collision(*s);
  rows(*s);
  newton(*s, iterations, tol, ls_max, ls_tol);
  delete s;
  return 0;
}

// Smooth dynamics of one state (tests): M (NV x NV dense), qfrc_smooth (NV), qacc_smooth (NV), body poses
// (xpos (NB, 3), xquat (NB, 4)).
int g1o_smooth(const double* qpos, const double* qvel, const double* ctrl, const double* com, double* M, double* qsm,
               double* qacc0, double* xpos, double* xquat) {
  World* s = new World;
  init_hooks(*s);
  std::memcpy(s->qpos, qpos, sizeof(double) * NQ);
  std::memcpy(s->qvel, qvel, sizeof(double) * NV);
  std::memcpy(s->com, com, sizeof(double) * 3);
  smooth(*s, ctrl);
  std::memcpy(M, s->M, sizeof(s->M));
  std::memcpy(qsm, s->qsm, sizeof(double) * NV);
  std::memcpy(qacc0, s->qacc0, sizeof(double) * NV);
  std::memcpy(xpos, s->X, sizeof(s->X));
  std::memcpy(xquat, s->Q, sizeof(s->Q));
  delete s;
  return 0;
}

// Kinematics outputs of nw states (g1_engine/kinematics.py:1-45: MuJoCo MJX's kinematics + com_pos + com_vel, mujoco
// 3.17 smooth.py), float64:
//   qn    qpos with the free joint's quaternion normalized (smooth.py 49, 67-70);
//   xpos, xquat (nw, NB, 3 / 4)  the body frames, world body 0 at the origin with the identity quaternion; the root
//         from qpos; a hinge body from its parent as fwd_body composes it (hinge at the body origin, angle qpos);
//   sc    (nw, NB, 3) subtree COMs: sum of m_b xipos_b over the subtree / its mass, xipos_b = xpos_b + R_b ipos_b
//         (ipos of the torso + com); the world body's is body 1's (smooth.py 150-165);
//   cvel  (nw, NB, 6) [angular; linear] twist of each body at the point sc[1] (body 0: zeros): angular W_b (world),
//         linear V_b + W_b x (sc[1] - xpos_b), V_b the velocity of the body origin (smooth.py 415-457).
int g1o_kinematics(int nw, const double* qpos, const double* qvel, const double* com, double* qn, double* xpos,
                   double* xquat, double* cvel, double* sc) {
  World* s = new World;
  init_hooks(*s);
  const double zero[NV] = {0};
  for (int w = 0; w < nw; w++) {
    std::memcpy(s->qpos, qpos + (size_t)w * NQ, sizeof(double) * NQ);
    std::memcpy(s->qvel, qvel + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->com, com + (size_t)w * 3, sizeof(double) * 3);
    for (int b = 1; b < NB; b++) fwd_body(*s, b, zero);  // parents before children in the body order
    double* o = qn + (size_t)w * NQ;
    std::memcpy(o, s->qpos, sizeof(double) * NQ);
    for (int k = 0; k < 4; k++) o[3 + k] = s->Q[1][k];
    double* xp = xpos + (size_t)w * NB * 3;
    double* xq = xquat + (size_t)w * NB * 4;
    for (int k = 0; k < 3; k++) xp[k] = 0.0;
    xq[0] = 1.0; xq[1] = xq[2] = xq[3] = 0.0;
    for (int b = 1; b < NB; b++) {
      for (int k = 0; k < 3; k++) xp[3 * b + k] = s->X[b][k];
      for (int k = 0; k < 4; k++) xq[4 * b + k] = s->Q[b][k];
    }
    double ms[NB] = {0}, ws[NB][3] = {{0}};  // subtree mass and sum of m xipos, leaf to root
    for (int b = NB - 1; b >= 1; b--) {
      double ip[3], r[3];
      body_ipos(*s, b, ip);
      qrot(s->Q[b], ip, r);
      ms[b] += BODY_MASS[b];
      for (int k = 0; k < 3; k++) ws[b][k] += BODY_MASS[b] * (s->X[b][k] + r[k]);
      const int p = BODY_PARENT[b];
      if (p >= 1) {
        ms[p] += ms[b];
        for (int k = 0; k < 3; k++) ws[p][k] += ws[b][k];
      }
    }
    double* c = sc + (size_t)w * NB * 3;
    for (int b = 1; b < NB; b++)
      for (int k = 0; k < 3; k++) c[3 * b + k] = ws[b][k] / ms[b];
    for (int k = 0; k < 3; k++) c[k] = c[3 + k];
    double* cv = cvel + (size_t)w * NB * 6;
    for (int k = 0; k < 6; k++) cv[k] = 0.0;
    for (int b = 1; b < NB; b++) {
      double r[3], u[3];
      for (int k = 0; k < 3; k++) r[k] = c[3 + k] - s->X[b][k];
      cross(s->W[b], r, u);
      for (int k = 0; k < 3; k++) { cv[6 * b + k] = s->W[b][k]; cv[6 * b + 3 + k] = s->V[b][k] + u[k]; }
    }
  }
  delete s;
  return 0;
}

// Contacts of one state (tests): returns the count kept (<= 64); per contact (pair, slot, dist, pos[3], frame[9]) as
// 15 doubles in out.
int g1o_contacts(const double* qpos, const double* qvel, const double* ctrl, const double* com, double fric,
                 double* out) {
  World* s = new World;
  init_hooks(*s);
  std::memcpy(s->qpos, qpos, sizeof(double) * NQ);
  std::memcpy(s->qvel, qvel, sizeof(double) * NV);
  std::memcpy(s->com, com, sizeof(double) * 3);
  s->fric = fric;
  s->flags = 0;
  smooth(*s, ctrl);
  collision(*s);
  for (int c = 0; c < s->ncon; c++) {
    double* o = out + 15 * c;
    o[0] = s->con[c].pair; o[1] = s->con[c].slot; o[2] = s->con[c].dist;
    for (int k = 0; k < 3; k++) o[3 + k] = s->con[c].pos[k];
    for (int k = 0; k < 9; k++) o[6 + k] = s->con[c].frame[k];
  }
  int n = s->ncon;
  delete s;
  return n;
}


// VJP of one control step (float64): the forward as g1o_step, then the substeps' VJPs in reverse. Cotangents of the
// outputs gq_out (nw, 36) qpos form, gv_out (nw, 35); gradients gq_in (nw, 36) qpos form (its quaternion part
// 2 q (x) (0, t) of the tangent cotangent t), gv_in (nw, 35), gu (nw, 29). clamp_kv 0 / 1 / 2, normal 0..3 as the
// reference's adjoint options; clamp_soft the soft clamp's delta.
// g1o_vjp_ex with the algorithmic flops of each world-step's VJP (closed form, VJP_FLOPS_*) in flops (nw) or NULL
int g1o_vjp_count(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
                  const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol,
                  int nsub, const double* gq_out, const double* gv_out, int clamp_kv, int normal, double clamp_soft,
                  double normal_eps, double parallel_eps, double* gq_in, double* gv_in, double* gu, double* flops) {
  World* s = new World;
  init_hooks(*s);
  s->normal_eps = normal_eps;
  s->parallel_eps = parallel_eps;
  Rec* rec = new Rec[nsub];
  for (int w = 0; w < nw; w++) {
    std::memcpy(s->qpos, qpos + (size_t)w * NQ, sizeof(double) * NQ);
    std::memcpy(s->qvel, qvel + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->qacc, warm + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->com, com + (size_t)w * 3, sizeof(double) * 3);
    s->fric = fric[w];
    s->flags = 0;
    s->aflops = 0;
    const double* u = ctrl + (size_t)w * NU;
    for (int k = 0; k < nsub; k++) {
      std::memcpy(rec[k].qpos, s->qpos, sizeof(rec[k].qpos));
      std::memcpy(rec[k].qvel, s->qvel, sizeof(rec[k].qvel));
      smooth(*s, u);
      collision(*s);
      rows(*s);
      newton(*s, iterations, tol, ls_max, ls_tol);
      integrate(*s);
      std::memcpy(rec[k].astar, s->qacc, sizeof(rec[k].astar));
      std::memcpy(rec[k].aadv, s->aadv, sizeof(rec[k].aadv));
    }
    // output cotangent in the tangent space at q'
    double qb[NV], vb[NV], ub[NU] = {0};
    const double* g = gq_out + (size_t)w * NQ;
    const double* q1 = s->qpos + 3;
    for (int k = 0; k < 3; k++) qb[k] = g[k];
    for (int k = 0; k < 3; k++) {
      double e[4] = {0, 0, 0, 0}, t[4];
      e[1 + k] = 1;
      qmul(q1, e, t);
      qb[3 + k] = 0.5 * (t[0] * g[3] + t[1] * g[4] + t[2] * g[5] + t[3] * g[6]);
    }
    for (int i = 6; i < NV; i++) qb[i] = g[i + 1];
    std::memcpy(vb, gv_out + (size_t)w * NV, sizeof(double) * NV);
    for (int k = nsub - 1; k >= 0; k--) substep_vjp(*s, rec[k], u, qb, vb, ub, clamp_kv, normal, clamp_soft);
    double* o = gq_in + (size_t)w * NQ;
    for (int k = 0; k < 3; k++) o[k] = qb[k];
    {
      const double* q0 = qpos + (size_t)w * NQ + 3;
      double qn = std::sqrt(q0[0] * q0[0] + q0[1] * q0[1] + q0[2] * q0[2] + q0[3] * q0[3]);
      double qq[4] = {q0[0] / qn, q0[1] / qn, q0[2] / qn, q0[3] / qn}, t[4] = {0, qb[3], qb[4], qb[5]}, r[4];
      qmul(qq, t, r);
      for (int k = 0; k < 4; k++) o[3 + k] = 2 * r[k];
    }
    for (int i = 6; i < NV; i++) o[i + 1] = qb[i];
    std::memcpy(gv_in + (size_t)w * NV, vb, sizeof(double) * NV);
    std::memcpy(gu + (size_t)w * NU, ub, sizeof(double) * NU);
    if (flops) flops[w] = s->aflops;
  }
  delete[] rec;
  delete s;
  return 0;
}

int g1o_vjp_ex(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
               const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub,
               const double* gq_out, const double* gv_out, int clamp_kv, int normal, double clamp_soft,
               double normal_eps, double parallel_eps, double* gq_in, double* gv_in, double* gu) {
  return g1o_vjp_count(nw, qpos, qvel, warm, ctrl, fric, com, iterations, tol, ls_max, ls_tol, nsub, gq_out, gv_out,
                       clamp_kv, normal, clamp_soft, normal_eps, parallel_eps, gq_in, gv_in, gu, nullptr);
}

int g1o_vjp(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl, const double* fric,
            const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub, const double* gq_out,
            const double* gv_out, int clamp_kv, int normal, double clamp_soft, double* gq_in, double* gv_in,
            double* gu) {
  return g1o_vjp_ex(nw, qpos, qvel, warm, ctrl, fric, com, iterations, tol, ls_max, ls_tol, nsub, gq_out, gv_out,
                    clamp_kv, normal, clamp_soft, 1e-3, 1.2e-3, gq_in, gv_in, gu);
}

}  // extern "C"
