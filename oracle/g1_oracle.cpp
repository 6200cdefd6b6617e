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
};

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
  for (int b = 1; b < NB; b++) { body_force(s, b); body_inertia(s, b); }
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
    }
    s.qsm[i] = act - bias[i];
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
  while (it < iterations) {
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
    for (int r = 0; r < s.nefc; r++) v.jar[r] += alpha * jv[r];
    double newcost = v.cost(s.qacc);
    double gn = v.gradient();
    double improvement = scale * (cost - newcost);
    cost = newcost;
    it++;
    if (improvement < tol || scale * gn < tol) break;
  }
  s.niter = it;
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

}  // namespace

extern "C" {

// One control step of nsub substeps for each of nw worlds, float64 (row-major world-major arrays as the engine's).
// iterations / tol: Newton's iteration cap and tolerance (the engine: 10, the model's 1e-8; MuJoCo C truth: 2000,
// 1e-13); ls_max / ls_tol: the line search's evaluation cap and relative derivative tolerance (40, 1e-7).
// info (nw, 4): last substep's Newton iterations, contacts (found, before the cap), rows, flags (4 contacts over
// capacity, 16 rows over capacity). Returns 0.
int g1o_step(int nw, const double* qpos, const double* qvel, const double* warm, const double* ctrl,
             const double* fric, const double* com, int iterations, double tol, int ls_max, double ls_tol, int nsub,
             double* oqpos, double* oqvel, double* owarm, int* info) {
  World* s = new World;
  for (int w = 0; w < nw; w++) {
    std::memcpy(s->qpos, qpos + (size_t)w * NQ, sizeof(double) * NQ);
    std::memcpy(s->qvel, qvel + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->qacc, warm + (size_t)w * NV, sizeof(double) * NV);
    std::memcpy(s->com, com + (size_t)w * 3, sizeof(double) * 3);
    s->fric = fric[w];
    s->flags = 0;
    for (int k = 0; k < nsub; k++) {
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
  }
  delete s;
  return 0;
}

// Smooth dynamics of one state (tests): M (NV x NV dense), qfrc_smooth (NV), qacc_smooth (NV), body poses
// (xpos (NB, 3), xquat (NB, 4)).
int g1o_smooth(const double* qpos, const double* qvel, const double* ctrl, const double* com, double* M, double* qsm,
               double* qacc0, double* xpos, double* xquat) {
  World* s = new World;
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

// Contacts of one state (tests): returns the count kept (<= 64); per contact (pair, slot, dist, pos[3], frame[9]) as
// 15 doubles in out.
int g1o_contacts(const double* qpos, const double* qvel, const double* ctrl, const double* com, double fric,
                 double* out) {
  World* s = new World;
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

}  // extern "C"
