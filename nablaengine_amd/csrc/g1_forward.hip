// The G1 control step, forward: one wave64 per world, all substeps in one launch.
//
// Per substep (the reference's substep_pre / substep_post, g1_engine/step.py:1650-2184, restated for wave64):
//   smooth     FK by each body walking its own chain (no level barriers), RNE bias and composite inertias by subtree
//              masks, CRBA, clamped PD actuators, qacc_smooth = M^-1 qfrc_smooth (register Cholesky)
//   collision  geom poses, bounding-sphere broadphase over the 502 pairs (ballot compaction in pair order),
//              narrowphase one candidate per lane, contacts compacted in (pair, slot) order by a wave prefix sum
//   rows       limits on their dof's lane, contact rows (4 pyramid edges or 1 normal row) on the contact's lane, all
//              in registers; impedance from solref / solimp (step.py:1157-1188)
//   Newton     cost 0.5 (a - a_s)' M (a - a_s) + sum s(J a - aref), warm start vs a_s, H = M + J'DJ, exact line
//              search (step.py:1974-2137)
//   implicit   (M + h kv) a_adv = M a*, qvel += h a_adv, qpos integrated (step.py:2153-2182)
//
// Contact Jacobians are never stored. J v is the contact point's relative velocity in the contact frame, from the
// bodies' spatial velocities (sum of the motion subspaces S_d v_d along each body's chain); J' f is the sum of the
// contacts' spatial forces projected on the dofs whose subtree holds the contact's bodies; J' C J enters the
// Hessian as a 6x6 contact stiffness K_c = Phi' C Phi composited over subtrees exactly as CRBA composites inertia,
// plus the cross-chain terms of contacts between two robot bodies.
#include "g1_forward.h"
#include "g1_collide.h"
#include "g1_diag.h"
#include "g1_tape.h"

#define PROF(k) PROF_MARK(s.prof_acc, s.prof_t, k)

namespace g1k {

// factor the packed matrix in s.L in place as L' L; dense when a contact couples two robot bodies (cross-branch
// entries), else with the tree's sparsity
// pattern: 0 the tree's sparsity, 1 with the common self-contact fill, 2 dense (hessian()'s classification)
__device__ __forceinline__ void factor_L(Sim& s, int lane, int pattern = 0) {
#ifdef G1_PROFILE
  if (pattern != 0 && lane == 0) s.prof_acc[PH_DENSE] += 1;
#endif
  if (pattern == 0) ltl_factor<0>(s.L, lane);
  else if (pattern == 1) ltl_factor<1>(s.L, lane);
  else ltl_factor<2>(s.L, lane);
  wsync();
}

// ============================================================================================== smooth dynamics
// motion subspace S_i of dof i about O: angular w (world), velocity of the point O (source.py:316-329 dof_motion)
__device__ __forceinline__ void dof_motion(const Sim& s, int i, float* w, float* v) {
  if (i < 3) {
    w[0] = w[1] = w[2] = 0.f;
    v[0] = i == 0; v[1] = i == 1; v[2] = i == 2;
  } else if (i < 6) {
    const float e[3] = {(float)(i == 3), (float)(i == 4), (float)(i == 5)};
    qrot(s.Q[1], e, w);
    v[0] = v[1] = v[2] = 0.f;
  } else {
    int b = i - 4;
    float r[3] = {s.O[0] - s.X[b][0], s.O[1] - s.X[b][1], s.O[2] - s.X[b][2]};
    const float ax[3] = {cAxis[3 * b], cAxis[3 * b + 1], cAxis[3 * b + 2]};
    qrot(s.Q[b], ax, w);
    cross(w, r, v);
  }
}

// Entry t of a chain-table row (the dofs moving a body, ascending; padding 255) for the row of dof `lane`, clamped to
// lane: a chain's entries are lane's ancestor dofs and lane itself, so the clamp maps the padding and a root dof past
// lane (the root rows' chains hold all 6 root dofs) to the diagonal. A row assembly then stores every entry
// unconditionally: the clamped ones store the diagonal's value again.
__device__ __forceinline__ int chain_dof_row(const unsigned* ch, int t, int lane) {
  return (int)min((ch[t >> 2] >> (8 * (t & 3))) & 255u, (unsigned)lane);
}

// (n, f) = I (w, v) for a packed spatial inertia about O: n = J w + h x v, f = m v - h x w (source.py:305-313)
__device__ __forceinline__ void apply_inertia(const float* J, const float* w, const float* v, float* n, float* f) {
  float hv[3], hw[3];
  cross(J + 6, v, hv);
  cross(J + 6, w, hw);
  n[0] = J[0] * w[0] + J[3] * w[1] + J[4] * w[2] + hv[0];
  n[1] = J[3] * w[0] + J[1] * w[1] + J[5] * w[2] + hv[1];
  n[2] = J[4] * w[0] + J[5] * w[1] + J[2] * w[2] + hv[2];
  for (int k = 0; k < 3; k++) f[k] = J[9] * v[k] - hw[k];
}

// the packed lower triangle of M + dg diag(kv) into s.L for the factorization: zeros, then each dof lane's chain
// entries (M has the tree's sparsity: its nonzeros in row i are on the chain of dof i's body)
__device__ __forceinline__ void m_to_L(Sim& s, int lane, float dg) {
  for (int e = lane; e < NTRI + 2; e += WL) s.L[e] = 0.f;
  if (lane < NV) {
    const int bi = lane < 6 ? 1 : lane - 4;
    unsigned ch[4];
    for (int k = 0; k < 4; k++) ch[k] = s.chain[bi][k];
    float* row = s.L + tri(lane, 0);
#pragma unroll
    for (int t = 0; t < MAXCHAIN; t++) {
      const int j = chain_dof_row(ch, t, lane);
      row[j] = s.M[lane][j];
    }
    row[lane] = s.M[lane][lane] + dg * cKv[lane];  // after the entries (same wave, program order)
  }
  wsync();
}

__device__ void smooth(Sim& s, int lane) {
  // each hinge body's local transform, one lane per body: q_l = quat (x) hinge rotation, the body's offset in its
  // parent's frame p_b, and the hinge axis in the parent's frame a_l = quat a (the hinge rotation keeps its own axis)
  if (lane >= 2 && lane < NB) {
    float sn, cs;
    sincosf(0.5f * s.qpos[lane + 5], &sn, &cs);
    const float qb[4] = {cQuat[4 * lane], cQuat[4 * lane + 1], cQuat[4 * lane + 2], cQuat[4 * lane + 3]};
    const float ax[3] = {cAxis[3 * lane], cAxis[3 * lane + 1], cAxis[3 * lane + 2]};
    const float ha[4] = {cs, sn * ax[0], sn * ax[1], sn * ax[2]};
    float* h = s.u.sm.hl[lane];
    qmul(qb, ha, h);
    for (int c = 0; c < 3; c++) h[4 + c] = cPos[3 * lane + c];
    qrot(qb, ax, h + 8);
  }
  wsync();
  // FK: each body lane walks its own chain from the root: pose, velocity, and the bias acceleration (qacc = 0;
  // gravity as the root's -g) (source.py:186-235 fwd_body). The chain's bodies come from the LDS chain table (the
  // hinge dofs past the root's 6, body = dof - 4), their local transforms from the table above.
  float Q[4], X[3], W[3], V[3], AL[3], A[3];
  {
    float n = rsqrtf(s.qpos[3] * s.qpos[3] + s.qpos[4] * s.qpos[4] + s.qpos[5] * s.qpos[5] + s.qpos[6] * s.qpos[6]);
    for (int k = 0; k < 4; k++) Q[k] = s.qpos[3 + k] * n;
    for (int k = 0; k < 3; k++) { X[k] = s.qpos[k]; V[k] = s.qvel[k]; A[k] = -kGrav[k]; AL[k] = 0.f; }
    qrot(Q, s.qvel + 3, W);
  }
  const int b = lane < NB ? lane : 0;
  unsigned ch[4];
  for (int k = 0; k < 4; k++) ch[k] = s.chain[b][k];
#pragma unroll
  for (int l = 1; l < MAXDEPTH; l++) {
    bool on;
    const int d = chain_dof(ch, 5 + l, &on);  // the hinge dof of the body at depth l + 1 on b's chain
    if (on) {
      const int k = d - 4;
      const float* h = s.u.sm.hl[k];
      const float ql[4] = {h[0], h[1], h[2], h[3]}, pb[3] = {h[4], h[5], h[6]}, al[3] = {h[8], h[9], h[10]};
      float t[3], aw[3], awd[3], u[3], wr[3], u2[3], q1[4];
      qrot(Q, pb, t);  // X_child - X_parent
      qrot(Q, al, aw);
      qmul(Q, ql, q1);
      for (int c = 0; c < 4; c++) Q[c] = q1[c];
      const float qd = s.qvel[d];
      for (int c = 0; c < 3; c++) awd[c] = aw[c] * qd;
      // from the parent's W, AL (in registers): A, V, AL, then W
      cross(AL, t, u);
      cross(W, t, wr);
      cross(W, wr, u2);
      for (int c = 0; c < 3; c++) { A[c] += u[c] + u2[c]; V[c] += wr[c]; X[c] += t[c]; }
      cross(W, awd, u);
      for (int c = 0; c < 3; c++) { AL[c] += u[c]; W[c] += awd[c]; }
    }
  }
  PROF(PH_SFK);
  if (lane < NB) {
    for (int k = 0; k < 4; k++) s.Q[lane][k] = lane == 0 ? (k == 0 ? 1.f : 0.f) : Q[k];
    for (int k = 0; k < 3; k++) s.X[lane][k] = lane == 0 ? 0.f : X[k];
  }
  if (lane < 3) s.O[lane] = s.qpos[lane];  // O: the root body's origin, the point of M and of the spatial vectors
  // body force F, moment about O T = N + (X - O) x F, composite-ready spatial inertia about O
  if (lane >= 1 && lane < NB) {
    float ip[3], c[3], u[3], wc[3], u2[3], F[3], N[3];
    for (int k = 0; k < 3; k++) ip[k] = cIpos[3 * lane + k] + (lane == TORSO_BODY ? s.com[k] : 0.f);
    qrot(Q, ip, c);
    cross(AL, c, u);
    cross(W, c, wc);
    cross(W, wc, u2);
    const float m = cMass[lane];
    for (int k = 0; k < 3; k++) F[k] = m * (A[k] + u[k] + u2[k]);
    float qi[4], l[3], Iw[3], Ia[3], cf[3];
    const float iq[4] = {cIquat[4 * lane], cIquat[4 * lane + 1], cIquat[4 * lane + 2], cIquat[4 * lane + 3]};
    const float In[3] = {cInert[3 * lane], cInert[3 * lane + 1], cInert[3 * lane + 2]};
    qmul(Q, iq, qi);
    qrot_inv(qi, W, l);
    for (int k = 0; k < 3; k++) l[k] *= In[k];
    qrot(qi, l, Iw);
    qrot_inv(qi, AL, l);
    for (int k = 0; k < 3; k++) l[k] *= In[k];
    qrot(qi, l, Ia);
    cross(W, Iw, u);
    cross(c, F, cf);
    for (int k = 0; k < 3; k++) N[k] = Ia[k] + u[k] + cf[k];
    // moment about O
    float xo[3] = {X[0] - s.qpos[0], X[1] - s.qpos[1], X[2] - s.qpos[2]}, xf[3];
    cross(xo, F, xf);
    for (int k = 0; k < 3; k++) { s.u.sm.V[lane][SM_F + k] = F[k]; s.u.sm.V[lane][SM_T + k] = N[k] + xf[k]; }
    // spatial inertia about O (source.py:280-302 body_inertia)
    float R[9];
    for (int k = 0; k < 3; k++) {
      float e[3] = {(float)(k == 0), (float)(k == 1), (float)(k == 2)};
      qrot(qi, e, R + 3 * k);
    }
    float* J = s.u.sm.V[lane] + SM_I;
    J[0] = In[0] * R[0] * R[0] + In[1] * R[3] * R[3] + In[2] * R[6] * R[6];
    J[1] = In[0] * R[1] * R[1] + In[1] * R[4] * R[4] + In[2] * R[7] * R[7];
    J[2] = In[0] * R[2] * R[2] + In[1] * R[5] * R[5] + In[2] * R[8] * R[8];
    J[3] = In[0] * R[0] * R[1] + In[1] * R[3] * R[4] + In[2] * R[6] * R[7];
    J[4] = In[0] * R[0] * R[2] + In[1] * R[3] * R[5] + In[2] * R[6] * R[8];
    J[5] = In[0] * R[1] * R[2] + In[1] * R[4] * R[5] + In[2] * R[7] * R[8];
    float cc3[3];
    for (int k = 0; k < 3; k++) cc3[k] = xo[k] + c[k];
    float cc = dot3(cc3, cc3);
    J[0] += m * (cc - cc3[0] * cc3[0]); J[1] += m * (cc - cc3[1] * cc3[1]); J[2] += m * (cc - cc3[2] * cc3[2]);
    J[3] -= m * cc3[0] * cc3[1]; J[4] -= m * cc3[0] * cc3[2]; J[5] -= m * cc3[1] * cc3[2];
    J[6] = m * cc3[0]; J[7] = m * cc3[1]; J[8] = m * cc3[2]; J[9] = m;
  }
  wsync();
  PROF(PH_SBF);
  // subtree sums per body B of the force, the moment about O and the spatial inertia (16 floats), a column per lane:
  // lane c < 16 loads column c of every body and adds each body into its parent, highest id first (a body's id is
  // above its parent's, so each body is complete when it is added), then stores the sums in place. The tree is
  // compile-time: 29 adds a lane, no masks. Lanes past the columns compute a copy of the last one and do not store.
  {
    const int c = lane < 16 ? lane : 15;
    float* col = &s.u.sm.V[0][c < 3 ? SM_F + c : (c < 6 ? SM_T + c - 3 : SM_I + c - 6)];
    float v[NB];
#pragma unroll
    for (int b = 1; b < NB; b++) v[b] = col[b * SMW];
    static_for<NB - 1, 1, -1>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      static_assert(BODY_PARENT[b] >= 1 && BODY_PARENT[b] < b, "bodies numbered parents first");
      v[BODY_PARENT[b]] += v[b];
    });
    if (lane < 16)
#pragma unroll
      for (int b = 1; b < NB; b++) col[b * SMW] = v[b];
  }
  PROF(PH_SSUB);
  // motion subspaces
  if (lane < NV) {
    float w[3], v[3];
    dof_motion(s, lane, w, v);
    for (int k = 0; k < 3; k++) { s.S[lane][k] = w[k]; s.S[lane][4 + k] = v[k]; }
  }
  wsync();
  // bias forces (qfrc_bias) projected on the dofs, CRBA row of dof `lane`, actuators
  for (int e = lane; e < NV * MSTRIDE; e += WL) (&s.M[0][0])[e] = 0.f;
  float bias = 0.f;
  if (lane < NV) {
    const int bi = lane < 6 ? 1 : lane - 4;
    const float w[3] = {s.S[lane][0], s.S[lane][1], s.S[lane][2]}, v[3] = {s.S[lane][4], s.S[lane][5], s.S[lane][6]};
    // subtree force / moment about the body origin X_b: N_b = T - (X_b - O) x F; the projection on a dof through O:
    // S . (T, F) with S = (w, w x (O - X_b)) equals w . N_b
    float Fb[3], Tb[3];
    for (int k = 0; k < 3; k++) { Fb[k] = s.u.sm.V[bi][SM_F + k]; Tb[k] = s.u.sm.V[bi][SM_T + k]; }
    bias = dot3(w, Tb) + dot3(v, Fb);
    float Jb[10], n[3], f[3];
    for (int k = 0; k < 10; k++) Jb[k] = s.u.sm.V[bi][SM_I + k];
    apply_inertia(Jb, w, v, n, f);
    // M[i][j] = S_j . I_c(body i) S_i on the chain of dof i's body (its ancestor dofs j <= i), both halves; the
    // rest of M is zero (zero-filled above, earlier in this wave's LDS order). Two lanes never store the same entry:
    // lane i writes row i and column i at j <= i (the entry (i, i) twice)
    unsigned ch[4];
    for (int k = 0; k < 4; k++) ch[k] = s.chain[bi][k];
    const float arm = cArm[lane];
#pragma unroll
    for (int t = 0; t < MAXCHAIN; t++) {
      const int j = chain_dof_row(ch, t, lane);
      const float mij = s.S[j][0] * n[0] + s.S[j][1] * n[1] + s.S[j][2] * n[2] + s.S[j][4] * f[0] + s.S[j][5] * f[1]
                        + s.S[j][6] * f[2] + (j == lane ? arm : 0.f);
      s.M[lane][j] = mij;  // j <= lane: both halves (the clamped entries store the diagonal again)
      s.M[j][lane] = mij;
    }
    float act = 0.f;
    if (lane >= 6) {
      act = cKp[lane] * (s.ctrl[lane - 6] - s.qpos[lane + 1]) - cKv[lane] * s.qvel[lane];
      act = fminf(fmaxf(act, -cFrclim[lane]), cFrclim[lane]);
    }
    s.qsm[lane] = act - bias;
  }
  {  // the clamp mask: the force at its limit (MuJoCo Warp's actuator_lam test, step.py:1773-1775)
    float act = lane >= 6 && lane < NV ? cKp[lane] * (s.ctrl[lane - 6] - s.qpos[lane + 1]) - cKv[lane] * s.qvel[lane]
                                       : 0.f;
    const bool clamp = lane >= 6 && lane < NV &&
                       (fminf(fmaxf(act, -cFrclim[lane]), cFrclim[lane]) <= -cFrclim[lane] ||
                        fminf(fmaxf(act, -cFrclim[lane]), cFrclim[lane]) >= cFrclim[lane]);
    const unsigned long long cm = ballot(clamp);
    if (lane == 0) { s.clampm[0] = (unsigned)cm; s.clampm[1] = (unsigned)(cm >> 32); }
  }
  wsync();
  PROF(PH_SCRBA);
  // qacc_smooth = M^-1 qfrc_smooth
  m_to_L(s, lane, 0.f);
  factor_L(s, lane);
  float x = ltl_solve(s.L, lane < NV ? s.qsm[lane] : 0.f, lane);
  if (lane < NV) s.qacc0[lane] = x;
  wsync();
}

}  // namespace g1k

namespace g1k {

// ============================================================================================== collision
// geom poses, broadphase, narrowphase; contacts in (pair, slot) order into s.u.col.stage
__device__ void collision(Sim& s, int lane) {
  if (lane < NGEOM) {
    const int b = cGbody[lane];
    float t[3], qb[4] = {s.Q[b][0], s.Q[b][1], s.Q[b][2], s.Q[b][3]};
    const float gp[3] = {cGpos[3 * lane], cGpos[3 * lane + 1], cGpos[3 * lane + 2]};
    const float gq[4] = {cGquat[4 * lane], cGquat[4 * lane + 1], cGquat[4 * lane + 2], cGquat[4 * lane + 3]};
    qrot(qb, gp, t);
    for (int k = 0; k < 3; k++) s.u.col.gx[lane][k] = s.X[b][k] + t[k];
    qmul(qb, gq, s.u.col.gq[lane]);
  }
  wsync();
  float fn[3];  // the floor's normal, then the broadphase
  {
    const float q0[4] = {s.u.col.gq[0][0], s.u.col.gq[0][1], s.u.col.gq[0][2], s.u.col.gq[0][3]};
    zaxis(q0, fn);
  }
  const int ncand = broadphase(s.u.col.gx, fn, s.u.col.cand, lane);
  wsync();
  // narrowphase: one candidate per lane; contacts placed by a prefix sum of the per-lane counts (pair order)
  int total = 0;
  for (int c0 = 0; c0 < ncand; c0 += WL) {
    Cand o;
    o.has[0] = o.has[1] = false;
    int pr = -1;
    if (c0 + lane < ncand) {
      pr = s.u.col.cand[c0 + lane];
      collide_pair(s.u.col.gx, s.u.col.gq, pr, o);
    }
    const int n = (int)o.has[0] + (int)o.has[1];
    int tn;
    const int off = total + wscan_bits<2>(n, lane, &tn);
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const int idx = off + (e == 1 ? (int)o.has[0] : 0);
      if (o.has[e] && idx < MAXCON) {
        float* st = s.u.col.stage[idx];
        st[0] = o.d[e];
        for (int k = 0; k < 3; k++) st[1 + k] = o.pos[e][k];
        for (int k = 0; k < 9; k++) st[4 + k] = o.fr[e][k];
        st[13] = __int_as_float(pr);
        st[14] = __int_as_float(o.slot[e]);
      }
    }
    total += tn;
  }
  if (lane == 0) {
    s.ncon_raw = total;
    s.ncon = total < MAXCON ? total : MAXCON;
    if (total > MAXCON) s.flags |= 4;
  }
  wsync();
}

// ============================================================================================== rows
// impedance (k, b, imp) of a row at distance pos, solref / solimp with refsafe (step.py:1157-1171 kbimp); the model's
// solimp power is 2
__device__ __forceinline__ void kbimp(const float* solref, const float* solimp, float pos, float* k, float* b,
                                      float* imp) {
  float tc = fmaxf(solref[0], 2.f * kH), dr = solref[1];
  float dmin = fminf(fmaxf(solimp[0], 1e-4f), 0.9999f), dmax = fminf(fmaxf(solimp[1], 1e-4f), 0.9999f);
  float width = fmaxf(1e-15f, solimp[2]), mid = fminf(fmaxf(solimp[3], 1e-4f), 0.9999f);
  *k = 1.f / fmaxf(1e-15f, dmax * dmax * tc * tc * dr * dr);
  *b = 2.f / fmaxf(1e-15f, dmax * tc);
  float x = fabsf(pos) / width;
  if (dmin == dmax || solimp[2] <= 1e-15f) *imp = 0.5f * (dmin + dmax);
  else if (x <= 0.f) *imp = dmin;
  else if (x >= 1.f) *imp = dmax;
  else {
    float y = x <= mid ? (x * x) / mid : 1.f - ((1.f - x) * (1.f - x)) / (1.f - mid);
    *imp = fminf(fmaxf(dmin + y * (dmax - dmin), dmin), dmax);
  }
}

__constant__ inline Arr<float, 2> cJSolref = to_float(JNT_SOLREF);
__constant__ inline Arr<float, 5> cJSolimp = to_float(JNT_SOLIMP);
__constant__ inline Arr<float, 2> cPSolref = to_float(PAIR_SOLREF);
__constant__ inline Arr<float, 5> cPSolimp = to_float(PAIR_SOLIMP);
static_assert(JNT_SOLIMP[4] == 2.0 && PAIR_SOLIMP[4] == 2.0, "kbimp assumes the solimp power 2");

// body spatial velocities of the dof vector v (LDS): bw[b] = sum over b's chain of S_d v_d, down the tree: the root
// body's from the root's 6 dofs (S_0..2 = (0; e_k), S_3..5 = (w_k; 0): v[0..2] and 3 columns), then each hinge body's
// is its parent's plus S_d v_d of its one dof d = b + 4. Four groups of 16 lanes walk the four paths from the root to
// the leaves (PATHS), lane c < 6 of a group carrying component c: the sums of each body's chain in its order, 10 steps
// of 2 loads, an FMA and a store, every address a per-lane base plus a compile-time offset. Both arm groups compute
// the waist's bodies (the same values); the legs' groups run 4 steps past their 6 bodies, and lanes c >= 6 every
// step, into a sink (the Hessian's self-contact staging, unused outside the Hessian). The world body gets 0.
__device__ __forceinline__ void body_vel(Sim& s, const float* v, int lane) {
  const int g = lane >> 4, c = lane & 15;
  const bool comp = c < 6;
  const int so = comp ? (c < 3 ? c : c + 1) : 0;  // the component's place in a row of S and bw: w 0..2, v 4..6
  const int lo = g == 0 ? PATHS.lo[0] : g == 1 ? PATHS.lo[1] : g == 2 ? PATHS.lo[2] : PATHS.lo[3];
  const int hi = g == 0 ? PATHS.hi[0] : g == 1 ? PATHS.hi[1] : g == 2 ? PATHS.hi[2] : PATHS.hi[3];
  float* sink = &s.u.nt.h.psi[0][0] + (lane & 7);  // 8 * PATH_STEPS + 7 floats: inside psi
  static_assert(8 * PATH_STEPS + 8 <= 16 * 8, "the sink inside psi");
  const float rw = s.S[3][so] * v[3] + s.S[4][so] * v[4] + s.S[5][so] * v[5];
  float T = c < 3 ? rw : v[comp ? c - 3 : 0];
  (comp && g < 2 ? &s.u.nt.bw[1 - g][so] : sink)[0] = g == 0 ? T : 0.f;  // the root body; the world body 0
  const float *Sa = &s.S[4 + lo][so], *Sb = &s.S[4 + hi][so], *va = v + 4 + lo, *vb = v + 4 + hi;
  float* oa = comp ? &s.u.nt.bw[lo][so] : sink;
  float* ob = comp ? &s.u.nt.bw[hi][so] : sink;
  float* oc = comp && g >= 2 ? ob : sink;  // past the legs' 6 bodies only the arm groups' are real
#pragma unroll
  for (int i = 0; i < PATH_STEPS; i++) {
    T = fmaf((i < 3 ? Sa : Sb)[8 * i], (i < 3 ? va : vb)[i], T);
    (i < 3 ? oa : i < 6 ? ob : oc)[8 * i] = T;
  }
  wsync();
}

// relative velocity of body2 against body1 at the contact point, in the contact frame (J_c v): needs body_vel(v)
__device__ __forceinline__ void contact_dots(const Sim& s, const Rows& R, float* dot) {
  float dw[3], dv[3], u[3], rel[3];
  for (int k = 0; k < 3; k++) {
    dw[k] = s.u.nt.bw[R.b2][k] - s.u.nt.bw[R.b1][k];
    dv[k] = s.u.nt.bw[R.b2][4 + k] - s.u.nt.bw[R.b1][4 + k];
  }
  cross(dw, R.r, u);
  for (int k = 0; k < 3; k++) rel[k] = dv[k] + u[k];
  dot[0] = dot3(R.fr, rel);
  dot[1] = dot3(R.fr + 3, rel);
  dot[2] = dot3(R.fr + 6, rel);
}

// J v of this lane's rows: contact rows (pyramid edges n +- mu t1, n +- mu t2, or the normal) and the limit row
__device__ __forceinline__ void rows_jv(Sim& s, const Rows& R, const float* v, int lane, bool con, float* jv,
                                        float* ljv) {
  body_vel(s, v, lane);
  float dot[3] = {0.f, 0.f, 0.f};
  if (con) contact_dots(s, R, dot);
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const float sg = (t & 1) ? -1.f : 1.f;
    jv[t] = R.dim == 3 ? dot[0] + sg * R.mu * dot[1 + (t >> 1)] : dot[0];
  }
  *ljv = lane < NV ? R.lsg * v[lane] : 0.f;
  wsync();
}

// out = M v (M full in LDS, v in LDS: both 16-byte aligned), lane i < NV: row i as 8 four-float loads and 3 scalars,
// v's entries as broadcast loads; every load independent of the others
__device__ __forceinline__ float matvec(const Sim& s, const float* v, int lane_) {
  const int lane = opaque_lane(lane_);
  const int i = lane < NV ? lane : NV - 1;
  const float4* row = reinterpret_cast<const float4*>(s.M[i]);
  const float4* vv = reinterpret_cast<const float4*>(v);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const float4 m = row[c], x = vv[c];
    acc[0] = fmaf(m.x, x.x, acc[0]);
    acc[1] = fmaf(m.y, x.y, acc[1]);
    acc[2] = fmaf(m.z, x.z, acc[2]);
    acc[3] = fmaf(m.w, x.w, acc[3]);
  }
  acc[0] = fmaf(s.M[i][32], v[32], acc[0]);
  acc[1] = fmaf(s.M[i][33], v[33], acc[1]);
  acc[2] = fmaf(s.M[i][34], v[34], acc[2]);
  return lane < NV ? (acc[0] + acc[1]) + (acc[2] + acc[3]) : 0.f;
}

// ============================================================================================== Newton
struct NewtonOut { int it; bool conv, fresh; };  // fresh: s.L holds H's factor at the final zones

// The floor contacts are the contact lanes [0, nf) sorted by body (the floor pairs come first in pair order, sorted by
// body, and contacts are compacted in pair order), and the bodies a dof moves are one run of body ids
// [ctz(dsub), 32 - clz(dsub)) (bodies in depth-first order); both orders are checked at compile time. So the floor
// contacts on the bodies dof i moves are one lane run [flo, fhi): from the last lane of each contact body's run, the
// lanes up to the last body below the dof's first body, and up to the last body inside its range.
__device__ __forceinline__ void floor_run(const Sim& s, Rows& R, int lane) {
  const bool floorl = lane < s.ncon && R.b1 == 0;
  const unsigned long long fl = ballot(floorl);
  const int nf = __popcll(fl);
  const int bnext = __shfl_down(R.b2, 1, WL);
  const unsigned long long ends = ballot(floorl && (lane == nf - 1 || bnext != R.b2));
  const unsigned dm = s.dsub[lane];
  const int bs = dm ? __builtin_ctz(dm) : NB, be = dm ? 32 - __builtin_clz(dm) : NB;
  int lo = 0, hi = 0;
  for (unsigned long long m = ends; m; m &= m - 1ull) {  // one contact body a step, in body order (all lanes)
    const int e = __builtin_ctzll(m), B = rdli(R.b2, e);
    lo = B < bs ? e + 1 : lo;
    hi = B < be ? e + 1 : hi;
  }
  R.nf = nf;
  R.flo = lo;
  R.fhi = hi;
  R.fcl = (lo > 0 || hi == 0) ? 1.f : 0.f;
}
// the sum of x over the lanes [flo, fhi) of this lane's dof, from x's inclusive prefix sums over the floor lanes:
// P[fhi - 1] - P[flo - 1], both read by ds_bpermute; P[-1] reads lane 63 and is weighted by 0 (for fhi = 0 both reads
// are lane 63 and cancel)
__device__ __forceinline__ float run_sum(float p, const Rows& R) {
  return fmaf(-lane_of(p, (R.flo - 1) & (WL - 1)), R.fcl, lane_of(p, (R.fhi - 1) & (WL - 1)));
}

// gradient at the current jar: grad = M a - qfrc_smooth - J' f, f = -D x on the rows with x < 0; returns |grad|
__device__ float newton_grad(Sim& s, const Rows& R, int lane, bool con) {
  // J' f: the contact's frame force f = -D x (rows with x < 0) as a world force F and its moment T about O; dof i adds
  // S_i . (T, F) summed over the contacts on the bodies it moves
  float T[3] = {0.f, 0.f, 0.f}, F[3] = {0.f, 0.f, 0.f};
  bool act = false;
  if (con) {
    float f[4];
#pragma unroll
    for (int t = 0; t < 4; t++) f[t] = (t < R.nr && R.jar[t] < 0.f) ? -R.D * R.jar[t] : 0.f;
    float fn, f1 = 0.f, f2 = 0.f;
    if (R.dim == 3) { fn = f[0] + f[1] + f[2] + f[3]; f1 = R.mu * (f[0] - f[1]); f2 = R.mu * (f[2] - f[3]); }
    else fn = f[0];
    for (int k = 0; k < 3; k++) F[k] = fn * R.fr[k] + f1 * R.fr[3 + k] + f2 * R.fr[6 + k];
    cross(R.r, F, T);
    act = fn != 0.f;
  }
  const unsigned dm = s.dsub[lane];
  const int il = lane < NV ? lane : 0;
  const float w[3] = {s.S[il][0], s.S[il][1], s.S[il][2]}, v[3] = {s.S[il][4], s.S[il][5], s.S[il][6]};
  float tau = 0.f;
  if (R.nf) {  // floor contacts: the run of the bodies dof i moves (floor_run), from prefix sums over the lanes
    float x[6] = {T[0], T[1], T[2], F[0], F[1], F[2]};
    wscan_nw<6>(x, R.nf);
#pragma unroll
    for (int e = 0; e < 6; e++) x[e] = run_sum(x[e], R);
    tau = w[0] * x[0] + w[1] * x[1] + w[2] * x[2] + v[0] * x[3] + v[1] * x[4] + v[2] * x[5];
  }
  // contacts between two robot bodies, one at a time: the contact's (T, F) broadcast to every lane, each dof adding
  // it with the sign of the body it moves (body 2 +, body 1 -; neither or both 0)
  const bool selfc = act && R.b1 != 0;
  for (unsigned long long m = ballot(selfc); m; m &= m - 1ull) {
    const int c = __builtin_ctzll(m);
    const int b1 = rdli(R.b1, c), b2 = rdli(R.b2, c);
    const float sg = (float)((int)((dm >> b2) & 1u) - (int)((dm >> b1) & 1u));
    tau += sg * (w[0] * rdl(T[0], c) + w[1] * rdl(T[1], c) + w[2] * rdl(T[2], c) + v[0] * rdl(F[0], c)
                 + v[1] * rdl(F[1], c) + v[2] * rdl(F[2], c));
  }
  float g = 0.f;
  if (lane < NV) {
    if (R.lsg != 0.f && R.ljar < 0.f) tau += R.lsg * (-R.lD * R.ljar);
    g = s.Ma[lane] - s.qsm[lane] - tau;
    s.grad[lane] = g;
  }
  wsync();
  return sqrtf(wsum(g * g));
}

__device__ __forceinline__ float lane_cost(const Sim& s, const Rows& R, int lane) {
  float g = 0.f;
  if (lane < NV) g = 0.5f * (s.Ma[lane] - s.qsm[lane]) * (s.qacc[lane] - s.qacc0[lane]);
#pragma unroll
  for (int t = 0; t < 4; t++)
    if (t < R.nr && R.jar[t] < 0.f) g += 0.5f * R.D * R.jar[t] * R.jar[t];
  if (R.lsg != 0.f && R.ljar < 0.f) g += 0.5f * R.lD * R.ljar * R.ljar;
  return g;
}

// Ma = M qacc and jar = J qacc - aref; at qacc = qacc_smooth (smooth), M qacc is qfrc_smooth (qacc_smooth solves
// M qacc_smooth = qfrc_smooth), taken as it is
__device__ void refresh(Sim& s, Rows& R, int lane, bool con, bool smooth = false) {
  const float ma = smooth ? (lane < NV ? s.qsm[lane] : 0.f) : matvec(s, s.qacc, lane);
  if (lane < NV) s.Ma[lane] = ma;
  float jv[4], ljv;
  rows_jv(s, R, s.qacc, lane, con, jv, &ljv);
#pragma unroll
  for (int t = 0; t < 4; t++) R.jar[t] = jv[t] - R.aref[t];
  R.ljar = ljv - R.laref;
}

constexpr int SELF_BATCH = 4;  // contacts between two robot bodies per outer-product batch (4 edge rows each)

// a floor contact's 6x6 stiffness K = Phi' C Phi about O (21 floats: Kaa 6, Kal 9, Kf 6), C from the curvatures d of
// its pyramid rows in the frame basis; zero where !on
__device__ __forceinline__ void contact_stiffness(const Rows& R, const float* dd, bool on, float* K) {
  float d[4];
  for (int t = 0; t < 4; t++) d[t] = on ? dd[t] : 0.f;
  float Cnn, Cn1 = 0.f, C11 = 0.f, Cn2 = 0.f, C22 = 0.f;
  if (R.dim == 3) {
    Cnn = d[0] + d[1] + d[2] + d[3];
    Cn1 = R.mu * (d[0] - d[1]); C11 = R.mu * R.mu * (d[0] + d[1]);
    Cn2 = R.mu * (d[2] - d[3]); C22 = R.mu * R.mu * (d[2] + d[3]);
  } else Cnn = d[0];
  const float *n = R.fr, *t1 = R.fr + 3, *t2 = R.fr + 6;
  float Kf[3][3];
  for (int a = 0; a < 3; a++)
    for (int b = 0; b < 3; b++)
      Kf[a][b] = Cnn * n[a] * n[b] + Cn1 * (n[a] * t1[b] + t1[a] * n[b]) + C11 * t1[a] * t1[b]
                 + Cn2 * (n[a] * t2[b] + t2[a] * n[b]) + C22 * t2[a] * t2[b];
  float Kal[3][3], Kaa[3][3];
  for (int b = 0; b < 3; b++) {  // column b of r^ Kf = r x Kf[:, b]
    float col[3] = {Kf[0][b], Kf[1][b], Kf[2][b]}, o[3];
    cross(R.r, col, o);
    for (int a = 0; a < 3; a++) Kal[a][b] = o[a];
  }
  for (int a = 0; a < 3; a++) {  // row a of r^ Kf r^' = r x (row a of Kal)
    float row[3] = {Kal[a][0], Kal[a][1], Kal[a][2]}, o[3];
    cross(R.r, row, o);
    for (int b = 0; b < 3; b++) Kaa[a][b] = o[b];
  }
  K[0] = Kaa[0][0]; K[1] = Kaa[1][1]; K[2] = Kaa[2][2]; K[3] = Kaa[0][1]; K[4] = Kaa[0][2]; K[5] = Kaa[1][2];
  for (int a = 0; a < 3; a++) for (int b = 0; b < 3; b++) K[6 + 3 * a + b] = Kal[a][b];
  K[15] = Kf[0][0]; K[16] = Kf[1][1]; K[17] = Kf[2][2]; K[18] = Kf[0][1]; K[19] = Kf[0][2]; K[20] = Kf[1][2];
}

// H = M + J' D J on the rows with x < 0, packed into s.L (lane i writes row i); returns the factorization pattern its
// contacts between robot bodies need (factor_L: 0 the tree's sparsity, 1 the common self-contact fill, 2 dense).
//   Floor contacts: J'CJ of a contact on body B is S_i' K S_j on every pair of dofs moving B, with K = Phi' C Phi its
//   6x6 stiffness about O. Dof i takes the sum of K over the floor contacts on the bodies it moves, one lane run
//   (floor_run) read from the prefix sums of K over the lanes, accumulates (n, f) = (that sum) S_i, and
//   H[i][j] = S_j . (n, f) on i's ancestor dofs j (the composite stiffness of i's subtree, as CRBA composites inertia).
//   Contacts between two robot bodies: J'CJ = sum over the active pyramid edges t of u_t u_t', u_t = sqrt(D) J' e_t,
//   u_t[d] = sigma_d S_d . (r x e_t, e_t) with sigma_d = (dof d moves body 2) - (dof d moves body 1); added as
//   U U' on the matrix cores (fp32 MFMA), SELF_BATCH contacts (4 edges each) a batch.
//   clear: zero s.L first. Not needed when s.L holds a factor with the tree's sparsity (of M or of an earlier H
//   without contacts between robot bodies): such a factor is exactly 0 off the pattern, and the rows below overwrite
//   every entry on it.
__device__ __forceinline__ int hessian(Sim& s, const Rows& R, int lane, bool con, bool clear) {
  float d[4];
#pragma unroll
  for (int t = 0; t < 4; t++) d[t] = (con && t < R.nr && R.jar[t] < 0.f) ? R.D : 0.f;
  const bool act = (d[0] + d[1]) + (d[2] + d[3]) != 0.f;
  const bool floorc = act && R.b1 == 0;
  const unsigned long long selfm = ballot(act && R.b1 != 0);
  PROF(PH_HK);
  const unsigned dm = s.dsub[lane];
  const int il = lane < NV ? lane : 0;
  const float w[3] = {s.S[il][0], s.S[il][1], s.S[il][2]}, v[3] = {s.S[il][4], s.S[il][5], s.S[il][6]};
  float n[3] = {0.f, 0.f, 0.f}, f[3] = {0.f, 0.f, 0.f};
  float K[21];
  contact_stiffness(R, d, floorc, K);  // exactly 0 off the active floor contacts (Rows are zero past the contacts)
  if (R.nf) {
    // the floor contacts' stiffness sum over the bodies dof i moves: prefix sums P of K over the lanes, then
    // P[fhi - 1] - P[flo - 1] (floor_run)
    wscan_nw<21>(K, R.nf);
    float k[21];
#pragma unroll
    for (int e = 0; e < 21; e++) k[e] = run_sum(K[e], R);
    // n = Kaa w + Kal v, f = Kal' w + Kll v
    n[0] = k[0] * w[0] + k[3] * w[1] + k[4] * w[2] + k[6] * v[0] + k[7] * v[1] + k[8] * v[2];
    n[1] = k[3] * w[0] + k[1] * w[1] + k[5] * w[2] + k[9] * v[0] + k[10] * v[1] + k[11] * v[2];
    n[2] = k[4] * w[0] + k[5] * w[1] + k[2] * w[2] + k[12] * v[0] + k[13] * v[1] + k[14] * v[2];
    f[0] = k[6] * w[0] + k[9] * w[1] + k[12] * w[2] + k[15] * v[0] + k[18] * v[1] + k[19] * v[2];
    f[1] = k[7] * w[0] + k[10] * w[1] + k[13] * w[2] + k[18] * v[0] + k[16] * v[1] + k[20] * v[2];
    f[2] = k[8] * w[0] + k[11] * w[1] + k[14] * w[2] + k[19] * v[0] + k[20] * v[1] + k[17] * v[2];
  }
  PROF(PH_HCOMP);
  // rows of H: zero, then M[i][j] + S_j . (n, f) on the ancestor dofs j of i (M's nonzeros are on these chains)
  if (clear)
    for (int e = lane; e < NTRI + 2; e += WL) s.L[e] = 0.f;
  if (lane < NV) {
    const int bi = lane < 6 ? 1 : lane - 4;
    // the chain of dof i's body: its ancestor dofs (and the root's j <= i). Every load first (S rows, M entries:
    // independent of the stores into L), then the stores of the chain's entries
    unsigned ch[4];
    for (int k = 0; k < 4; k++) ch[k] = s.chain[bi][k];
    float* row = s.L + tri(lane, 0);
#pragma unroll
    for (int t0 = 0; t0 < MAXCHAIN; t0 += 8) {  // 8 entries a batch
      float hv[8];
      int hj[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int j = chain_dof_row(ch, t0 + e, lane);
        hj[e] = j;
        hv[e] = s.M[lane][j] + (s.S[j][0] * n[0] + s.S[j][1] * n[1] + s.S[j][2] * n[2] + s.S[j][4] * f[0]
                                + s.S[j][5] * f[1] + s.S[j][6] * f[2]);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) row[hj[e]] = hv[e];  // the clamped entries store the diagonal's value again
    }
    if (R.lsg != 0.f && R.ljar < 0.f) s.L[tri(lane, lane)] += R.lD;
  }
  PROF(PH_HROWS);
  for (unsigned long long m = selfm; m;) {  // contacts between two robot bodies, SELF_BATCH a batch
    unsigned long long bm = 0ull;
    for (int q = 0; q < SELF_BATCH && m; q++) { bm |= m & (~m + 1ull); m &= m - 1ull; }
    if (lane < 4 * SELF_BATCH)
      for (int k = 0; k < 8; k++) s.u.nt.h.psi[lane][k] = 0.f;
    if ((bm >> lane) & 1ull) {  // this contact's 4 edge rows: sqrt(D) (r x e_t, e_t), e_t = n +- mu t1, n +- mu t2
      const int q = prefix_count(bm, lane);
      const float sd = sqrtf(R.D);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        float e[3];
        const float sg = (t & 1) ? -R.mu : R.mu;
        const float* ta = R.fr + 3 * (1 + (t >> 1));
        for (int k = 0; k < 3; k++) e[k] = R.dim == 3 ? R.fr[k] + sg * ta[k] : (t == 0 ? R.fr[k] : 0.f);
        const float sc = d[t] != 0.f ? sd : 0.f;
        float re[3];
        cross(R.r, e, re);
        float* o = s.u.nt.h.psi[4 * q + t];
        for (int k = 0; k < 3; k++) { o[k] = sc * re[k]; o[3 + k] = sc * e[k]; }
        o[6] = __int_as_float(R.b1);
        o[7] = __int_as_float(R.b2);
      }
    }
    wsync();
    {  // U[i][r] = sigma_r(i) S_i . psi_r (rows past the dofs zero): S Psi' (48 x 8 x 16, S's rows with its two
       // unused slots 3 and 7 as zero columns) on the matrix cores, 3 row tiles x 2 k-steps, then the signs
      const int ln = opaque_lane(lane);
      const int lr = ln & 15, lk = ln >> 4;
      const float* pr = s.u.nt.h.psi[lr];  // this lane's column r = lr
      const int b1r = __float_as_int(pr[6]), b2r = __float_as_int(pr[7]);
      float bv[2];
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        const int k = 4 * kk + lk;  // S's slot; psi's 0..5 are S's 0..2, 4..6
        const float x = pr[k < 3 ? k : (k < 7 ? k - 1 : 0)];
        bv[kk] = (k == 3 || k == 7) ? 0.f : x;
      }
#pragma unroll
      for (int t = 0; t < 3; t++) {
        const int ia = 16 * t + lr, ic = ia < NV ? ia : 0;
        mfma4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
          const int k = 4 * kk + lk;
          const float x = s.S[ic][k];
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ia < NV && k != 3 && k != 7 ? x : 0.f, bv[kk], acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 16 * t + 4 * lk + e;
          const unsigned di = s.dsub[i];  // 0 past the dofs
          const float sg = (float)((int)((di >> b2r) & 1u) - (int)((di >> b1r) & 1u));
          s.u.nt.h.U[i][lr] = sg * acc[e];
        }
      }
    }
    wsync();
    {  // H += U U' on the matrix cores: 16 x 16 tiles (ti, tj <= ti) of the 48-row padding, k = the batch's edge rows
      // in steps of 4 (v_mfma_f32_16x16x4f32: lane l gives A[l % 16][l / 16] and B[l / 16][l % 16], holds
      // C[4 (l / 16) + e][l % 16]). Step kk takes U's columns 4 kk .. 4 kk + 3, contact kk's 4 edge rows, so a batch
      // of nb contacts needs nb steps: the 6 tiles' chains are nb deep, not SELF_BATCH
      const int lr = lane & 15, lk = lane >> 4;
      const int nb = __popcll(bm);
      mfma4 acc[6];
#pragma unroll
      for (int n = 0; n < 6; n++) acc[n] = mfma4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
      for (int kk = 0; kk < nb; kk++) {
        float op[3];
#pragma unroll
        for (int t = 0; t < 3; t++) op[t] = s.u.nt.h.U[16 * t + lr][4 * kk + lk];
        int n = 0;
#pragma unroll
        for (int ti = 0; ti < 3; ti++)
#pragma unroll
          for (int tj = 0; tj <= ti; tj++, n++)
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(op[ti], op[tj], acc[n], 0, 0, 0);
      }
      int n = 0;
#pragma unroll
      for (int ti = 0; ti < 3; ti++)
#pragma unroll
        for (int tj = 0; tj <= ti; tj++, n++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int i = 16 * ti + 4 * lk + e, j = 16 * tj + lr;
            s.L[i < NV && j <= i ? tri(i, j) : LSINK + lane] += acc[n][e];  // off the triangle: the lane's sink
          }
    }
    wsync();
  }
  wsync();
  // the factorization's pattern from the active contacts between robot bodies (body x < y): none when x is y's
  // ancestor (the coupling stays on y's chain); the common fill for a leg against the waist or its own arm, or the two
  // legs; else dense
  int cls = 0;
  if (act && R.b1 != 0) {
    const int x = min(R.b1, R.b2), y = max(R.b1, R.b2);
    const bool anc = x == 1 || ((s.dsub[x + 4] >> y) & 1u);  // body x >= 2 has the one dof x + 4
    const bool legl = x >= 2 && x <= 7, legr = x >= 8 && x <= 13;
    const bool common = (legl && y >= 8 && y <= 23) || (legr && ((y >= 14 && y <= 16) || y >= 24));
    cls = anc ? 0 : common ? 1 : 2;
  }
  const unsigned all = wor((unsigned)cls);
  return all == 0u ? 0 : (all & 2u) ? 2 : 1;
}


__device__ __forceinline__ NewtonOut newton(Sim& s, Rows& R, int lane, bool con, int iterations) {
  // warm start against qacc_smooth: keep the cheaper (step.py:1974-1988)
  refresh(s, R, lane, con);
  float cost = wsum(lane_cost(s, R, lane));
  float wq = lane < NV ? s.qacc[lane] : 0.f, wma = lane < NV ? s.Ma[lane] : 0.f, wj[4], wl = R.ljar;
  for (int t = 0; t < 4; t++) wj[t] = R.jar[t];
  if (lane < NV) s.qacc[lane] = s.qacc0[lane];
  wsync();
  refresh(s, R, lane, con, true);
  const float cost0 = wsum(lane_cost(s, R, lane));
  if (cost0 > cost) {
    if (lane < NV) { s.qacc[lane] = wq; s.Ma[lane] = wma; }
    for (int t = 0; t < 4; t++) R.jar[t] = wj[t];
    R.ljar = wl;
    wsync();
  } else {
    cost = cost0;
  }
  newton_grad(s, R, lane, con);
  int it = 0, lpat = 0;  // lpat: the pattern of the factor in s.L (the smooth dynamics leave M's, the tree's)
  bool conv = false, zsame = false;
  while (it < iterations) {
    // a compiler barrier: LDS values are loaded where they are used inside the iteration, not hoisted out of the loop
    // into registers held across all of it
    asm volatile("" ::: "memory");
    float p;
    PROF(PH_NINIT);
    if (zsame) {  // no row changed its zone in the last step: H, and so its factor in s.L, are unchanged
      p = ltl_solve(s.L, lane < NV ? -s.grad[lane] : 0.f, lane);
    } else {
      const int pattern = hessian(s, R, lane, con, lpat != 0);
      PROF(PH_HESS);
      factor_L(s, lane, pattern);
      lpat = pattern;
      PROF(PH_FACTOR);
      p = ltl_solve(s.L, lane < NV ? -s.grad[lane] : 0.f, lane);
    }
    PROF(PH_SOLVE);
#ifdef G1_PROFILE
    if (lane == 0) s.prof_acc[PH_ITERS] += 1;
#endif
    if (lane < NV) s.p[lane] = p;
    wsync();
    // exact line search along p on the piecewise-quadratic cost (step.py:2032-2084)
    float jv[4], ljv;
    rows_jv(s, R, s.p, lane, con, jv, &ljv);
    PROF(PH_LSJV);
    const float mp = matvec(s, s.p, lane);
    if (lane < NV) s.Mp[lane] = mp;
    // per row: x(alpha) = jar + alpha jv; rows past the kept ones start at +1e30 (never in the quadratic zone)
    float xr[5], vr[5], dr[5];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      xr[t] = t < R.nr ? R.jar[t] : 1e30f;
      vr[t] = t < R.nr ? jv[t] : 0.f;
      dr[t] = R.D;
    }
    xr[4] = R.lsg != 0.f ? R.ljar : 1e30f;
    vr[4] = R.lsg != 0.f ? ljv : 0.f;
    dr[4] = R.lD;
    // the slope and curvature of the rows' cost at alpha (the quadratic-zone rows), and the zone pattern
    auto rows_at = [&](float alpha, float* fd, float* fdd, unsigned* z) {
      float a = 0.f, b = 0.f;
      unsigned zz = 0u;
#pragma unroll
      for (int t = 0; t < 5; t++) {
        const float x = fmaf(alpha, vr[t], xr[t]);
        const bool q = x < 0.f;
        const float dv = q ? dr[t] * vr[t] : 0.f;
        a = fmaf(dv, x, a);
        b = fmaf(dv, vr[t], b);
        zz |= q ? 1u << t : 0u;
      }
      *fd = a; *fdd = b; *z = zz;
    };
    // the Gauss term's coefficients a1 = (M a - f) . p, a2 = p . M p and the rows at alpha = 0: one reduction
    float fd0, fdd0;
    unsigned zprev;
    rows_at(0.f, &fd0, &fdd0, &zprev);
    float r4[4] = {lane < NV ? (s.Ma[lane] - s.qsm[lane]) * p : 0.f, lane < NV ? p * mp : 0.f, fd0, fdd0};
    wsum_n<4>(r4);
    const float a1 = r4[0], a2 = r4[1];
    PROF(PH_LSMV);
    // exact 1-D Newton with bracketing on the piecewise-quadratic cost (step.py:2032-2084)
    float alpha = 0.f, lo = 0.f, hi = 1e30f;
    const float d0 = r4[2] + a1;
    if (d0 < 0.f) {
      float fd = d0, fdd = r4[3] + a2;
      for (int k = 1; k <= 40; k++) {
        if (fabsf(fd) <= 1e-7f * fabsf(d0)) break;
        if (fd < 0.f) lo = alpha; else hi = alpha;
        float nx = fmaf(-fd, __builtin_amdgcn_rcpf(fdd), alpha);
        const bool newton_step = nx > lo && nx < hi;
        if (!newton_step) nx = hi < 1e29f ? 0.5f * (lo + hi) : 2.f * fmaxf(alpha, 1e-6f);
        alpha = nx;
        float f1, f2;
        unsigned z;
        rows_at(alpha, &f1, &f2, &z);
        if (ballot(!(newton_step && z == zprev)) == 0ull) break;  // the Newton step kept every row on its piece
        if (k == 40) break;
#ifdef G1_PROFILE
        if (lane == 0) s.prof_acc[PH_LSEVAL] += 1;
#endif
        const float2 ff = wsum2(f1, f2);
        fd = ff.x + fmaf(alpha, a2, a1);
        fdd = ff.y + a2;
        zprev = z;
      }
    }
    PROF(PH_LSEARCH);
    // move along p
    if (lane < NV) {
      s.qacc[lane] += alpha * p;
      s.Ma[lane] += alpha * mp;
    }
    bool chg = false;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float xn = R.jar[t] + alpha * jv[t];
      chg |= t < R.nr && ((R.jar[t] < 0.f) != (xn < 0.f));
      R.jar[t] = xn;
    }
    {
      const float xn = R.ljar + alpha * ljv;
      chg |= R.lsg != 0.f && ((R.ljar < 0.f) != (xn < 0.f));
      R.ljar = xn;
    }
    zsame = ballot(chg) == 0ull;
    wsync();
    const float newcost = wsum(lane_cost(s, R, lane));
    PROF(PH_UPDATE);
    const float gn = newton_grad(s, R, lane, con);
    PROF(PH_GRAD);
    const float improvement = kScale * (cost - newcost);
    cost = newcost;
    it++;
    conv = improvement < kTol || kScale * gn < kTol;
    if (conv) break;
  }
  return NewtonOut{it, conv, it > 0 && zsame};
}

// ============================================================================================== one substep
// tape store helper: n words of src (LDS) into the record and zeros up to the field's end (the padding: a record
// does not depend on what the buffer held), lane-strided (coalesced)
__device__ __forceinline__ void tape_put(float* dst, const float* src, int n, int end, int lane) {
  for (int i = lane; i < end; i += WL) dst[i] = i < n ? src[i] : 0.f;
}

// Inlined into the kernel's substep loop. The library is built with machine LICM off (-mllvm -disable-machine-licm):
// with it on, uniform values derived from the constant tables (the contact impedance parameters) are hoisted out of
// the substep loop into registers held across the Newton loop, and spilled there; a call per substep instead would
// save and restore about 112 callee-saved VGPRs through scratch each time (0.5 GB of HBM traffic per launch).
__device__ __forceinline__ void substep(Sim& s, int lane_, int iterations, float* rec, float* ocon) {
  const int lane = opaque_lane(lane_);  // nothing lane-dependent is hoisted out of the substep loop
  Rows R;
  if (rec) {
    tape_put(rec + REC_QPOS, s.qpos, NQ, REC_QVEL - REC_QPOS, lane);
    tape_put(rec + REC_QVEL, s.qvel, NV, REC_ASTAR - REC_QVEL, lane);
  }
  PROF(PH_TAPE);
  smooth(s, lane);
  PROF(PH_SMOOTH);
  collision(s, lane);
  PROF(PH_COLLIDE);
  if (rec) {  // the contact table (pair | slot << 9), two per word, in contact (= row) order
    const int nc = s.ncon;
    if (lane < MAXCON / 2) {
      unsigned e[2];
      for (int t = 0; t < 2; t++) {
        const int c = 2 * lane + t;
        e[t] = c < nc ? ((unsigned)__float_as_int(s.u.col.stage[c][13]) | (unsigned)__float_as_int(s.u.col.stage[c][14]) << 9)
                      : TAPE_CON_NONE;
      }
      rec[REC_CON + lane] = __uint_as_float(e[0] | e[1] << 16);
    }
    if (lane < 2) rec[REC_CLAMP + lane] = __uint_as_float(s.clampm[lane]);
  }
  const int ncon = s.ncon;
  const bool con = lane < ncon;
  // this lane's contact
  int pair = -1;
  R.nr = 0; R.b1 = 0; R.b2 = 0; R.dim = 1; R.mu = 0.f; R.D = 0.f;
  for (int k = 0; k < 3; k++) R.r[k] = 0.f;
  for (int k = 0; k < 9; k++) R.fr[k] = 0.f;
  float dist = 0.f, piw = 0.f;
  if (con) {
    const float* st = s.u.col.stage[lane];
    dist = st[0];
    for (int k = 0; k < 3; k++) R.r[k] = st[1 + k] - s.O[k];
    for (int k = 0; k < 9; k++) R.fr[k] = st[4 + k];
    pair = __float_as_int(st[13]);
    const PairC pc = cPair[pair];
    const PairRow prow = cPairRow[pair];
    const unsigned w = pc.w;
    R.b1 = pc.bodies & 255u;
    R.b2 = pc.bodies >> 8;
    R.dim = (w >> 16) & 15u;
    R.mu = ((w >> 20) & 1u) ? s.fric : prow.mu;
    piw = prow.iw;
  }
  floor_run(s, R, lane);
  wsync();
  // limit rows (dof order), then the contacts' rows (contact order) up to the row capacity
  R.lsg = 0.f; R.lD = 0.f; R.laref = 0.f; R.ljar = 0.f;
  float lpos = 0.f;
  if (lane >= 6 && lane < NV) {
    const float q = s.qpos[lane + 1], dmin = q - cRange[2 * lane], dmax = cRange[2 * lane + 1] - q;
    if (fminf(dmin, dmax) < 0.f) { R.lsg = dmin < dmax ? 1.f : -1.f; lpos = fminf(dmin, dmax); }
  }
  const unsigned long long lm = ballot(R.lsg != 0.f);
  const int nlim = __popcll(lm);
  const int nrf = con ? (R.dim == 3 ? 4 : 1) : 0;
  int trf;
  const int r0 = nlim + wscan_bits<3>(nrf, lane, &trf);
  R.nr = con ? max(0, min(nrf, NEFC - r0)) : 0;
  const int need = nlim + trf;
  if (lane == 0) {
    s.nlim = nlim;
    s.nefc = need < NEFC ? need : NEFC;
    if (need > NEFC) s.flags |= 16;
  }
  // impedance, D, aref (velocities J qvel from the bodies' velocities)
  float vdot[3] = {0.f, 0.f, 0.f};
  body_vel(s, s.qvel, lane);
  if (con) contact_dots(s, R, vdot);
  if (R.lsg != 0.f) {
    float k, b, imp;
    kbimp(cJSolref.v, cJSolimp.v, lpos, &k, &b, &imp);
    const float iw = cDinvw[lane];
    R.lD = 1.f / fmaxf(iw * (1.f - imp) / imp, 1e-15f);
    R.laref = -k * imp * lpos - b * (R.lsg * s.qvel[lane]);
  }
  if (con) {
    float k, b, imp;
    kbimp(cPSolref.v, cPSolimp.v, dist, &k, &b, &imp);
    float iw = piw;
    if (R.dim == 3) iw = (R.mu * R.mu * iw + iw) * 2.f * R.mu * R.mu / kImpratio;
    R.D = 1.f / fmaxf(iw * (1.f - imp) / imp, 1e-15f);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const float sg = (t & 1) ? -1.f : 1.f;
      const float vel = R.dim == 3 ? vdot[0] + sg * R.mu * vdot[1 + (t >> 1)] : vdot[0];
      R.aref[t] = -k * imp * dist - b * vel;
    }
  } else {
    for (int t = 0; t < 4; t++) R.aref[t] = 0.f;
  }
  wsync();
  PROF(PH_ROWS);
  // a self contact between nearly meeting geom centres / axes (its distance plus both radii: the centre or axis
  // distance of the sphere / capsule primitives)
  bool sing = false;
  if (rec) {
    float nu = 1e30f;
    if (con && R.b1 != 0) {
      const PairSz psz = cPairSz[pair];
      nu = dist + psz.r1 + psz.r2;
    }
    sing = ballot(nu < SINGULAR_NU) != 0ull;
  }
  const NewtonOut no = newton(s, R, lane, con, iterations);
  PROF(PH_NINIT);
  if (lane == 0) s.niter = no.it;
  if (rec) {  // the final zones, and H's factor at them (assembled again when the last step changed a zone)
    if (!no.fresh) {
      const int pattern = hessian(s, R, lane, con, true);
      factor_L(s, lane, pattern);
    }
    tape_put(rec + REC_LH, s.L, NTRI, REC_LQ - REC_LH, lane);
    unsigned cz = 0u;
    for (int t = 0; t < 4; t++) cz |= (t < R.nr && R.jar[t] < 0.f) ? 1u << t : 0u;
    // 4 bits per contact: lanes 8 w .. 8 w + 7 into word w (gathered by shuffles)
    unsigned word = 0u;
    for (int k = 0; k < 8; k++) word |= (unsigned)__shfl(cz, (lane & 7) * 8 + k, 64) << (4 * k);
    if (lane < 8) rec[REC_CZONE + lane] = __uint_as_float(word);
    const unsigned long long lz = ballot(R.lsg != 0.f && R.ljar < 0.f), lr = ballot(R.lsg != 0.f);
    if (lane < 2) {
      rec[REC_LIMZONE + lane] = __uint_as_float((unsigned)(lane ? lz >> 32 : lz));
      rec[REC_LIMROW + lane] = __uint_as_float((unsigned)(lane ? lr >> 32 : lr));
    }
    tape_put(rec + REC_ASTAR, s.qacc, NV, REC_AADV - REC_ASTAR, lane);
    // the adjoint's dispatch cost of this substep: its contacts, the distinct robot bodies they touch and the contacts
    // between two robot bodies (4 each: the per-body wrench sums, the two-body contact VJPs), and the primitive classes
    // present (8 each: a lane's class branches run for the whole wave), in units of 4 (measured on config-1 worlds:
    // the adjoint's launch in this order ends 3.4% earlier than ordered by the records' constraint rows)
    const unsigned pwc = cPair[con ? pair : 0].w;
    const unsigned cbod = wor(con ? (1u << R.b1) | (1u << R.b2) : 0u) & ~1u;
    const unsigned ccls = wor(con ? 1u << ((pwc >> 21) & 7u) : 0u);
    const int cself = wsumi(con && R.b1 != 0 ? 1 : 0);
    if (lane == 0) {
      s.acost += s.ncon + 4 * (__popc(cbod) + cself) + 8 * __popc(ccls);
      rec[REC_ADJCOST] = __int_as_float(min(s.acost >> 2, COST_BUCKETS - 1));
      rec[REC_HDR] = __uint_as_float((unsigned)s.ncon | (unsigned)s.nefc << 8 | (unsigned)s.nlim << 16
                                     | (unsigned)min(no.it, 255) << 24);
      rec[REC_FLAGS] = __uint_as_float((unsigned)(s.flags & 20) | (no.fresh ? 0u : (unsigned)FLAG_REFACT)
                                       | (no.conv ? 0u : (unsigned)FLAG_NONCONV) | (sing ? (unsigned)FLAG_SINGULAR : 0u));
      s.dcnt += (no.fresh ? 0 : 1) | (no.conv ? 0 : 1 << 8) | (sing ? 1 << 16 : 0);
    }
    wsync();
  }
  PROF(PH_TAPE);
  // implicitfast: (M + h kv) a_adv = M a*
  {
    m_to_L(s, lane, kH);
    factor_L(s, lane);
    const float adv = ltl_solve(s.L, lane < NV ? s.Ma[lane] : 0.f, lane);
    if (lane < NV) s.qvel[lane] += kH * adv;
    if (rec) {
      // L_Q, its off-pattern positions carrying the body frames FK left at the substep's start (g1_tape.h): they
      // are written into the factor's zeros in LDS first (s.L is factored afresh before its next use); a position's
      // fourth word, which nothing writes in s.X, as 0
      for (int q = lane; q < POSE_WORDS; q += WL)
        s.L[cPoseSlots.pos[q]] = q >= 4 * NB && (q & 3) == 3 ? 0.f : (&s.Q[0][0])[q];
      wsync();
      tape_put(rec + REC_LQ, s.L, NTRI, REC_ADJCOST - REC_LQ, lane);
      if (lane < REC_LH - REC_AADV) rec[REC_AADV + lane] = lane < NV ? adv : 0.f;
    }
    wsync();
  }
  if (lane == 0) {  // the free joint: position, then the orientation rotated by h times the local angular velocity
    for (int k = 0; k < 3; k++) s.qpos[k] += kH * s.qvel[k];
    float w[3] = {s.qvel[3], s.qvel[4], s.qvel[5]}, nw = sqrtf(dot3(w, w));
    if (nw > 0.f) {
      float sa, ca;
      sincosf(0.5f * kH * nw, &sa, &ca);
      const float sw = sa / nw;  // the adjoint replays this rotation with the same products
      float dq[4] = {ca, sw * w[0], sw * w[1], sw * w[2]};
      float q[4] = {s.qpos[3], s.qpos[4], s.qpos[5], s.qpos[6]}, o[4];
      qmul(q, dq, o);
      float on = rsqrtf(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
      for (int k = 0; k < 4; k++) s.qpos[3 + k] = o[k] * on;
    }
  }
  if (lane >= 6 && lane < NV) s.qpos[lane + 1] += kH * s.qvel[lane];
  PROF(PH_IMPLICIT);
  if (ocon) {  // this substep's contacts: pair, dist, pos, normal (pair -1 past the count)
    float* o = ocon + 8 * lane;
    o[0] = con ? (float)pair : -1.f;
    o[1] = con ? dist : 0.f;
    for (int k = 0; k < 3; k++) { o[2 + k] = con ? R.r[k] + s.O[k] : 0.f; o[5 + k] = con ? R.fr[k] : 0.f; }
  }
  wsync();
}

// The wave's issue priority (s_setprio, 0..3; it changes which of a SIMD's two waves issues first, never a result)
// from the cycles the world is expected still to need: its mean cycles per substep so far (s_memtime, the shader
// clock) times the substeps left, one level per PRIO_STEP. The longest remaining work goes first, as the dispatch
// order's heaviest-first does at launch: a world whose cost the launch's estimate missed (a self contact appearing
// within the step, more Newton iterations) catches up on its co-resident light world instead of finishing last.
// 4e5 cycles (about two mean substeps) was the best of 2e5 .. 1e6 at 4096 worlds, and 3e5 .. 4e5 again on the later
// build with PRIO_START.
constexpr float PRIO_STEP = 4e5f;
// A world's level for its first substep, before it has a rate of its own: a world dispatched into the launch's second
// round then has all its substeps left (at the mean rate about 2 PRIO_STEP), where its co-resident wave has part of
// one world left. Starting at level 0 held it behind that wave for a substep: 1.5% slower forward at 4096 worlds than
// starting at 1, 2 or 3, which measured alike.
constexpr int PRIO_START = 2;
__device__ __forceinline__ void set_priority_by_remaining(unsigned long long t_start, int k, int nsub) {
  const float rem = (float)(__builtin_amdgcn_s_memtime() - t_start) * (float)(nsub - k) / (float)k;
  if (rem > 3.f * PRIO_STEP) __builtin_amdgcn_s_setprio(3);
  else if (rem > 2.f * PRIO_STEP) __builtin_amdgcn_s_setprio(2);
  else if (rem > PRIO_STEP) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// one world per wave64 (one workgroup of 64 lanes)
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_forward(int nw, const float* __restrict__ qpos, const float* __restrict__ qvel,
                                                const float* __restrict__ warm, const float* __restrict__ ctrl,
                                                const float* __restrict__ fric, const float* __restrict__ com,
                                                int iterations, int nsub, float* __restrict__ oqpos,
                                                float* __restrict__ oqvel, float* __restrict__ owarm,
                                                int* __restrict__ info, float* __restrict__ ocon,
                                                float* __restrict__ tape, const int* __restrict__ perm,
                                                unsigned long long* __restrict__ diag) {
  __shared__ Sim s;
  const int lane = threadIdx.x;
  if ((int)blockIdx.x >= nw) return;
  const int w = perm ? perm[blockIdx.x] : (int)blockIdx.x;  // heaviest worlds first (g1_order.hip)
  // the world's inputs: every load issued at once, on every lane (a lane past a row reads a word inside it and drops
  // it), one memory round trip
  const int lq = min(lane, NQ - 1), lv = min(lane, NV - 1), lu = min(lane, NU - 1), lc = min(lane, 2);
  const float iq = qpos[(size_t)w * NQ + lq], iv = qvel[(size_t)w * NV + lv], iw = warm[(size_t)w * NV + lv];
  const float iu = ctrl[(size_t)w * NU + lu], ic = com[(size_t)w * 3 + lc], ifr = fric[w];
  if (lane < NQ) s.qpos[lane] = iq;
  if (lane < NV) { s.qvel[lane] = iv; s.qacc[lane] = iw; }
  if (lane < NU) s.ctrl[lane] = iu;
  if (lane < 3) s.com[lane] = ic;
  if (lane == 0) { s.fric = ifr; s.flags = 0; s.niter = 0; s.dcnt = 0; s.acost = 0; }
  s.dsub[lane] = lane < NV ? cTree.dofmask32[lane] : 0u;
  chain_table(s.chain, lane);
#ifdef G1_PROFILE
  if (lane < NPHASE) s.prof_acc[lane] = 0;
  if (lane == 0) {
    s.prof_t = __builtin_amdgcn_s_memtime();
    s.prof_acc[PH_T0] = __builtin_amdgcn_s_memrealtime();  // the world's start and end on the 100 MHz clock, and where
    s.prof_acc[PH_HWID] = (unsigned long long)__builtin_amdgcn_s_getreg(0xF804)  // HW_ID: wave, SIMD, CU, SE
                          | (unsigned long long)__builtin_amdgcn_s_getreg(0xF814) << 32;  // XCC_ID
  }
#endif
  wsync();
  const unsigned long long t_start = __builtin_amdgcn_s_memtime();
  for (int k = 0; k < nsub; k++) {
    if (k > 0) set_priority_by_remaining(t_start, k, nsub);
    else __builtin_amdgcn_s_setprio(PRIO_START);
    substep(s, lane, iterations, tape ? tape + ((size_t)w * nsub + k) * REC_WORDS : nullptr,
            ocon && k == nsub - 1 ? ocon + (size_t)w * MAXCON * 8 : nullptr);
  }
  if (lane < NQ) oqpos[(size_t)w * NQ + lane] = s.qpos[lane];
  if (lane < NV) { oqvel[(size_t)w * NV + lane] = s.qvel[lane]; owarm[(size_t)w * NV + lane] = s.qacc[lane]; }
#ifdef G1_PROFILE
  wsync();
  if (lane == 0) s.prof_acc[PH_T1] = __builtin_amdgcn_s_memrealtime();
  wsync();
  if (lane < NPHASE && w < PROF_WORLDS) g_prof[w][lane] = s.prof_acc[lane];
#endif
  if (lane == 0) {
    info[4 * w] = s.niter;
    info[4 * w + 1] = s.ncon_raw;
    info[4 * w + 2] = s.nefc;
    info[4 * w + 3] = s.flags;
    if (diag) {  // this world's part of the diagnostic counters (what k_diag_fwd counts from info and the tape)
      const int f = s.flags, dc = s.dcnt;
      if (f) atomicAdd(&diag[D_FWD_UNSUPPORTED], 1ull);
      if (f & 4) atomicAdd(&diag[D_CONTACT_OVERFLOW], 1ull);
      if (f & 16) atomicAdd(&diag[D_ROW_OVERFLOW], 1ull);
      if (s.niter >= iterations) atomicAdd(&diag[D_FWD_ITER_LIMIT], 1ull);
      if (dc & 255) atomicAdd(&diag[D_REFACT], (unsigned long long)(dc & 255));
      if ((dc >> 8) & 255) atomicAdd(&diag[D_NONCONV], (unsigned long long)((dc >> 8) & 255));
      if (dc >> 16) atomicAdd(&diag[D_SINGULAR], (unsigned long long)(dc >> 16));
      if (blockIdx.x == 0) {
        atomicAdd(&diag[D_FWD_CALLS], 1ull);
        atomicAdd(&diag[D_FWD_WORLDS], (unsigned long long)nw);
        if (tape) atomicAdd(&diag[D_TAPE_RECORDS], (unsigned long long)nw * (unsigned long long)nsub);
      }
    }
  }
}

}  // namespace g1k

namespace g1k {
int launch_order_fwd(hipStream_t st, int nw, const float* qpos, void* work);
int resident_worlds();
// order: 0 index order (work unused), 1 compute the order into work first (index order when the batch fits the
// GPU's resident slots at once: the order cannot change the makespan there), 2 the order already in work; diag: the
// diagnostic counters added to by each world at its end, or NULL
int launch_forward(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm, const float* ctrl,
                   const float* fric, const float* com, int iterations, int nsub, float* oq, float* ov, float* ow,
                   int* info, float* ocon, float* tape, void* work, int order, unsigned long long* diag) {
  if (nw <= 0) return 0;
  const int* perm = nullptr;
  if (order == 1 && nw <= resident_worlds()) order = 0;
  if (work && order) {  // the dispatch order, heaviest worlds first
    if (order == 1) {
      const int rc = launch_order_fwd(st, nw, qpos, work);
      if (rc) return rc;
    }
    perm = (const int*)work;
  }
  hipLaunchKernelGGL(k_forward, dim3(nw), dim3(64), 0, st, nw, qpos, qvel, warm, ctrl, fric, com, iterations, nsub,
                     oq, ov, ow, info, ocon, tape, perm, diag);
  return (int)hipGetLastError();
}
size_t forward_lds_bytes() { return sizeof(Sim); }
int prof_read(unsigned long long* out, int nw) {  // the G1_PROFILE build's per-world phase cycles (nw x NPHASE)
#ifdef G1_PROFILE
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof), sizeof(unsigned long long) * NPHASE * (size_t)nw);
#else
  (void)out; (void)nw;
  return -1;
#endif
}
}  // namespace g1k
