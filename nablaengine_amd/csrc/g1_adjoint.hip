// The G1 control step's adjoint: the VJP of one control step from its forward tape, one wave64 per world, the
// substeps in reverse. Per substep (the reference's k_adjoint phases A0-A8, adjoint.py:1-83, restated):
//   record    the substep's input state, a*, a_adv, the contact table, zones, clamp mask (tape)
//   poses     FK at the input state (each body walks its chain), motion subspaces S about O, own spatial inertias
//   integ.    the integrator's VJP in the tangent space: hinges and root position q' = q + h v'; root rotation
//             q' = q (x) exp(h w' / 2): t = R(dq) t', w' bar += h J_r(h w')' t'
//   solves    y = Q^-1 (h v' bar) with L_Q, a* bar = h v' bar - h kv y; lambda = H^-1 a* bar with L_H (IFT)
//   gradient  of Psi(q, v) = y' M(q) a~ - lambda' [RNE(q, v, a*) - f_act + sum_active D J' (J a* - aref)]:
//             every q-derivative is a subtree sum of force vectors dotted with S_j plus the joint's outside terms
//             (moving dof j's subtree rigidly by S_j: attached quantities change covariantly, the outside does not);
//             contacts as wrenches (the primitives' pose cotangents, the twist changes at the contact point), limit
//             rows through their distance; actuators kp / kv on the unclamped dofs (clamp_kv 0 / 1 / 2)
// Determinism: every sum has a fixed order (lane = body sums over contacts in contact order; lane = dof sums over
// bodies in body order); no atomics.
#include "g1_collide.h"
#include "g1_diag.h"
#include "g1_tape.h"

namespace g1k {

struct Sv { float w[3], v[3]; };

__device__ __forceinline__ Sv sv0() { Sv r; for (int k = 0; k < 3; k++) r.w[k] = r.v[k] = 0.f; return r; }
__device__ __forceinline__ Sv sv_add(const Sv& a, const Sv& b, float s = 1.f) {
  Sv r;
  for (int k = 0; k < 3; k++) { r.w[k] = a.w[k] + s * b.w[k]; r.v[k] = a.v[k] + s * b.v[k]; }
  return r;
}
__device__ __forceinline__ float sv_dot(const Sv& m, const Sv& f) { return dot3(m.w, f.w) + dot3(m.v, f.v); }
__device__ __forceinline__ Sv cross_mm(const Sv& x, const Sv& y) {
  Sv r;
  float a[3], b[3];
  cross(x.w, y.w, r.w);
  cross(x.w, y.v, a);
  cross(x.v, y.w, b);
  for (int k = 0; k < 3; k++) r.v[k] = a[k] + b[k];
  return r;
}
__device__ __forceinline__ Sv cross_mf(const Sv& x, const Sv& f) {
  Sv r;
  float a[3], b[3];
  cross(x.w, f.w, a);
  cross(x.v, f.v, b);
  for (int k = 0; k < 3; k++) r.w[k] = a[k] + b[k];
  cross(x.w, f.v, r.v);
  return r;
}
// (n, f) = I (w, v) for a packed spatial inertia about O
__device__ __forceinline__ Sv inertia_apply(const float* J, const Sv& x) {
  float hv[3], hw[3];
  cross(J + 6, x.v, hv);
  cross(J + 6, x.w, hw);
  Sv r;
  r.w[0] = J[0] * x.w[0] + J[3] * x.w[1] + J[4] * x.w[2] + hv[0];
  r.w[1] = J[3] * x.w[0] + J[1] * x.w[1] + J[5] * x.w[2] + hv[1];
  r.w[2] = J[4] * x.w[0] + J[5] * x.w[1] + J[2] * x.w[2] + hv[2];
  for (int k = 0; k < 3; k++) r.v[k] = J[9] * x.v[k] - hw[k];
  return r;
}
__device__ __forceinline__ Sv ld_sv(const float* p) {
  Sv r;
  for (int k = 0; k < 3; k++) { r.w[k] = p[k]; r.v[k] = p[4 + k]; }
  return r;
}

enum { TW_V = 0, TW_L, TW_Y, TW_AW, TW_A2, TW_A1, NTW };  // per-body twists
enum { FB_F1 = 0, FB_P, FB_X1, FB_F2, FB_P2, FB_EG, FB_OL, FB_OA, FB_OV, NFB };  // per-body force vectors
__device__ __forceinline__ Sv ld_sv6(const float* p) {  // a spatial vector packed as 6 floats (8-byte aligned)
  Sv r;
  for (int k = 0; k < 3; k++) { r.w[k] = p[k]; r.v[k] = p[3 + k]; }
  return r;
}
__device__ __forceinline__ void st_sv6(float* p, const Sv& x) {
  for (int k = 0; k < 3; k++) { p[k] = x.w[k]; p[3 + k] = x.v[k]; }
}

struct __align__(16) Adj {
  float qpos[40], qvel[36], astar[36], aadv[36], at[36];
  float qb[36], vb[36], vt[36], qn[36], y[36], lam[36], ub[32], ctrl[32], com[4];
  float S[NV + 1][8];                 // dof motion subspaces about O (row NV unused); qvel[NV] = 0 pads the chains
  float Q[NB][4], X[NB][4];          // the body frames, copied from the record (X's fourth words 0)
  unsigned short pslot[POSE_WORDS];  // L_Q's packed positions that carry the frames (cPoseSlots, loaded at start)
  unsigned chain[NB][MAXCHAIN / 4];  // the dofs moving each body, ascending, one byte each; 255 past the chain
  float O[4];
  float fric;
  // 16-byte aligned after the scalar above, and with it tw, gx, gq (their sizes are multiples of 16 bytes): the
  // compiler merges their float loads and stores into 64- to 128-bit LDS accesses only where it knows the alignment
  __align__(16) float Ib[NB][12];
  float tw[NB][NTW][6];              // per-body twists (6 floats each)
  float gx[NGEOM][4], gq[NGEOM][4];
  union {
    struct __align__(16) {
      float q[768], h[768];    // the taped factors L_Q and L_H (630 words each, then the last copy's slack)
    } lt;
    float fb[NB][NFB][6];      // then the per-body force vectors (6 floats each)
  };
  int ncon, flags;
  unsigned clampm[2], limzone[2], limrow[2], czone[8];
  unsigned short con[MAXCON];
#ifdef G1_PROFILE
  unsigned long long prof_t, prof_acc[NPHASE];
#endif
};
// 8 worlds per CU: the LDS of one world must stay within 160 KB / 8
static_assert(sizeof(Adj) <= 20480, "Adj outgrew the LDS of 8 worlds per CU");
static_assert(offsetof(Adj, lt) % 16 == 0 && 3 * 256 <= 768 && NTRI <= 3 * 256, "the factors' LDS copies");
static_assert(offsetof(Adj, X) == offsetof(Adj, Q) + 16 * NB, "the body frames Q, X as one array (the tape's copy)");

// L_Q and L_H of a record copied into LDS by the memory unit (global_load_lds_dwordx4: lane l's 16 bytes land 16 l
// bytes past the instruction's LDS base), 3 x 1024 bytes each; lanes past the factor's end load its start again into
// the slack. Issued with the record's other loads, they arrive with them; no registers hold them. (The compiler waits
// for these copies at the next LDS access, as it cannot tell their LDS writes apart; and any later global load's
// wait covers them too, vmcnt counting in issue order, so they cannot be left in flight across the poses, whose
// per-body constants are global loads.)
__device__ __forceinline__ void load_factors(Adj& s, const float* __restrict__ rec, int lane) {
#pragma unroll
  for (int c = 0; c < 3; c++) {
    const int f = 256 * c + 4 * lane;  // the lane's first word (f + 3 <= 631: inside the record for both factors)
    const int fo = f < NTRI ? f : 0;
    __builtin_amdgcn_global_load_lds((const void*)(rec + REC_LQ + fo),
                                     (__attribute__((address_space(3))) void*)(s.lt.q + 256 * c), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(rec + REC_LH + fo),
                                     (__attribute__((address_space(3))) void*)(s.lt.h + 256 * c), 16, 0, 0);
  }
}

// The adjoint's phase profile (a G1_PROFILE build only; g_prof_adj, read by dk_prof_read_adj): s_memtime
// cycles per phase summed over the substeps, then the world's start and end on the 100 MHz clock.
enum { AP_RECORD = 0, AP_POSES, AP_SOLVE, AP_TWIST, AP_CONTACT, AP_BODYSUM, AP_FORCES, AP_DOF, AP_T0, AP_T1,
       AP_SUBTREE, NAPHASE };
static_assert(NAPHASE <= NPHASE, "the adjoint's phases fit g_prof_adj's rows");
#ifdef G1_PROFILE
__device__ unsigned long long g_prof_adj[PROF_WORLDS][NPHASE];
#define APROF(k) PROF_MARK(s.prof_acc, s.prof_t, k)
#else
#define APROF(k) do { } while (0)
#endif

// impedance and its derivative in the distance (kbimp's curve, solimp power 2; 0 where the curve is clamped)
__device__ __forceinline__ void imp_d(const float* solimp, float pos, float* imp, float* dimp) {
  const float dmin = fminf(fmaxf(solimp[0], 1e-4f), 0.9999f), dmax = fminf(fmaxf(solimp[1], 1e-4f), 0.9999f);
  const float width = fmaxf(1e-15f, solimp[2]), mid = fminf(fmaxf(solimp[3], 1e-4f), 0.9999f);
  const float iwd = 1.f / width, x = fabsf(pos) * iwd, sg = pos < 0.f ? -1.f : 1.f;
  *dimp = 0.f;
  if (x <= 0.f) { *imp = dmin; return; }
  if (x >= 1.f) { *imp = dmax; return; }
  float y, dy;
  if (x <= mid) { const float im = 1.f / mid; y = x * x * im; dy = 2.f * x * im; }
  else { const float im = 1.f / (1.f - mid); y = 1.f - (1.f - x) * (1.f - x) * im; dy = 2.f * (1.f - x) * im; }
  const float v = dmin + y * (dmax - dmin);
  if (v < dmin || v > dmax) { *imp = fminf(fmaxf(v, dmin), dmax); return; }
  *imp = v;
  *dimp = dy * (dmax - dmin) * sg * iwd;
}
__device__ __forceinline__ void kb_consts(const float* solref, const float* solimp, float* k, float* b) {
  const float tc = fmaxf(solref[0], 2.f * kH), dr = solref[1];
  const float dmax = fminf(fmaxf(solimp[1], 1e-4f), 0.9999f);
  *k = 1.f / fmaxf(1e-15f, dmax * dmax * tc * tc * dr * dr);
  *b = 2.f / fmaxf(1e-15f, dmax * tc);
}

__constant__ inline Arr<float, 2> caJSolref = to_float(JNT_SOLREF);
__constant__ inline Arr<float, 5> caJSolimp = to_float(JNT_SOLIMP);
__constant__ inline Arr<float, 2> caPSolref = to_float(PAIR_SOLREF);
__constant__ inline Arr<float, 5> caPSolimp = to_float(PAIR_SOLIMP);

// the normal derivative's factor kappa(nu): 1 / nu exact (0), frozen (1), 1 / max(nu, eps) (2), frozen below eps (3)
__device__ __forceinline__ float kappa(float nu, int normal) {
  const float eps = 1e-3f;
  if (normal == 0) return 1.f / nu;
  if (normal == 1) return 0.f;
  if (normal == 2) return 1.f / fmaxf(nu, eps);
  return nu < eps ? 0.f : 1.f / nu;
}

// make_frame VJP: cotangents of the frame rows (n, b, c) -> n bar (added)
__device__ __forceinline__ void make_frame_vjp(const float* n, const float* frb, float* nb) {
  float e[3] = {0.f, 0.f, 0.f};
  if (-0.5f < n[1] && n[1] < 0.5f) e[1] = 1.f; else e[2] = 1.f;
  const float ne = dot3(n, e);
  float b0[3];
  for (int k = 0; k < 3; k++) b0[k] = e[k] - n[k] * ne;
  const float bl = sqrtf(dot3(b0, b0));
  float b[3], bbar[3], t[3];
  const float ibl = 1.f / bl;
  for (int k = 0; k < 3; k++) b[k] = b0[k] * ibl;
  cross(b, frb + 6, t);
  for (int k = 0; k < 3; k++) nb[k] += frb[k] + t[k];
  cross(frb + 6, n, t);
  for (int k = 0; k < 3; k++) bbar[k] = frb[3 + k] + t[k];
  const float bb = dot3(b, bbar);
  float b0b[3];
  for (int k = 0; k < 3; k++) b0b[k] = (bbar[k] - b[k] * bb) * ibl;
  const float nb0 = dot3(n, b0b);
  for (int k = 0; k < 3; k++) nb[k] += -ne * b0b[k] - nb0 * e[k];
}

// sphere core VJP: (dist, pos, n) of two spheres with cotangents db, posb, nb -> p1b, p2b (added)
// kappa(nu) nu, the factor of the normal's derivative where it is written without 1 / nu (capsule-capsule with both
// parameters free): exactly 1 for the exact derivative
__device__ __forceinline__ float kappa_nu(float nu, int normal) {
  const float eps = 1e-3f;
  if (normal == 0) return 1.f;
  if (normal == 1) return 0.f;
  if (normal == 2) return nu / fmaxf(nu, eps);
  return nu < eps ? 0.f : 1.f;
}
__device__ __forceinline__ void sphere_core_vjp(const float* p1, float r1, const float* p2, float r2, float db,
                                                const float* posb, const float* nb, int normal, float* p1b, float* p2b) {
  const float dl[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
  const float l = sqrtf(dot3(dl, dl));
  float dlb[3];
  for (int k = 0; k < 3; k++) { p1b[k] += posb[k]; dlb[k] = 0.5f * posb[k]; }
  if (l > 0.f) {
    float n[3], nt[3];
    const float il = 1.f / l;
    for (int k = 0; k < 3; k++) { n[k] = dl[k] * il; nt[k] = nb[k] + 0.5f * (r1 - r2) * posb[k]; }
    const float nn = dot3(n, nt), kap = kappa(l, normal);
    for (int k = 0; k < 3; k++) dlb[k] += kap * (nt[k] - n[k] * nn) + n[k] * db;
  }
  for (int k = 0; k < 3; k++) { p1b[k] -= dlb[k]; p2b[k] += dlb[k]; }
}

// the contact geometry's VJP (pair pr, its contact `slot`, normal frame fr): cotangents of (dist, pos, frame) -> the
// geoms' world position and rotation cotangents
__device__ void contact_geom_vjp(const Adj& s, int pr, int slot, const float* fr, float db, const float* posb,
                                 const float* frb, int normal, float* x1b, float* t1b, float* x2b, float* t2b) {
  const unsigned w = cPair[pr].w;
  const PairSz psz = cPairSz[pr];
  const int g1 = w & 255u, g2 = (w >> 8) & 255u, cls = (w >> 21) & 7u;
  float p1[3], q1[4], p2[3], q2[4];
  for (int k = 0; k < 3; k++) { p1[k] = s.gx[g1][k]; p2[k] = s.gx[g2][k]; }
  for (int k = 0; k < 4; k++) { q1[k] = s.gq[g1][k]; q2[k] = s.gq[g2][k]; }
  const float r1 = psz.r1, h1 = psz.hl1, r2 = psz.r2, h2 = psz.hl2;
  for (int k = 0; k < 3; k++) x1b[k] = t1b[k] = x2b[k] = t2b[k] = 0.f;
  if (cls == 0 || cls == 4) {  // the floor: n constant
    float n[3];
    zaxis(q1, n);
    const float pn = dot3(n, posb);
    float ceb[3];
    for (int k = 0; k < 3; k++) ceb[k] = posb[k] - 0.5f * n[k] * pn + n[k] * db;
    if (cls == 0) {
      for (int k = 0; k < 3; k++) x2b[k] += ceb[k];
    } else {
      float axis[3], axb[3];
      zaxis(q2, axis);
      const float sg = slot == 0 ? 1.f : -1.f;
      for (int k = 0; k < 3; k++) { x2b[k] += ceb[k]; axb[k] = sg * h2 * ceb[k]; }
      const float na = dot3(n, axis);
      float b0[3];
      for (int k = 0; k < 3; k++) b0[k] = axis[k] - n[k] * na;
      const float bn = sqrtf(dot3(b0, b0));
      if (bn >= 0.5f) {
        float b[3], bbar[3], t[3];
        const float ibn = 1.f / bn;
        for (int k = 0; k < 3; k++) b[k] = b0[k] * ibn;
        cross(frb + 6, n, t);
        for (int k = 0; k < 3; k++) bbar[k] = frb[3 + k] + t[k];
        const float bb = dot3(b, bbar);
        float b0b[3];
        for (int k = 0; k < 3; k++) b0b[k] = (bbar[k] - b[k] * bb) * ibn;
        const float nb0 = dot3(n, b0b);
        for (int k = 0; k < 3; k++) axb[k] += b0b[k] - n[k] * nb0;
      }
      cross(axis, axb, t2b);
    }
    return;
  }
  float nb[3] = {0.f, 0.f, 0.f};
  make_frame_vjp(fr, frb, nb);
  if (cls == 1) {
    sphere_core_vjp(p1, r1, p2, r2, db, posb, nb, normal, x1b, x2b);
    return;
  }
  if (cls == 2) {
    float axis[3], a[3], ab[3], ap[3], pt[3], ptb[3] = {0.f, 0.f, 0.f};
    zaxis(q2, axis);
    for (int k = 0; k < 3; k++) { a[k] = p2[k] - axis[k] * h2; ab[k] = 2.f * axis[k] * h2; ap[k] = p1[k] - a[k]; }
    const float gam = dot3(ab, ab) + 1e-6f, raw = dot3(ap, ab) / gam, t = fminf(fmaxf(raw, 0.f), 1.f);
    for (int k = 0; k < 3; k++) pt[k] = a[k] + t * ab[k];
    sphere_core_vjp(p1, r1, pt, r2, db, posb, nb, normal, x1b, ptb);
    const float tb = dot3(ptb, ab);
    float abb[3], apb[3] = {0.f, 0.f, 0.f}, aab[3], axb[3];
    for (int k = 0; k < 3; k++) { abb[k] = t * ptb[k]; aab[k] = ptb[k]; }
    if (raw > 0.f && raw < 1.f) {
      const float ig = tb / gam;
      for (int k = 0; k < 3; k++) {
        apb[k] = ig * ab[k];
        abb[k] += ig * ap[k] - ig * raw * 2.f * ab[k];
      }
    }
    for (int k = 0; k < 3; k++) { x1b[k] += apb[k]; aab[k] -= apb[k]; }
    for (int k = 0; k < 3; k++) { x2b[k] += aab[k]; axb[k] = -h2 * aab[k] + 2.f * h2 * abb[k]; }
    cross(axis, axb, t2b);
    return;
  }
  // capsule-capsule: the segment parameters' clamp cascade, then the sphere core on the closest points
  float z1[3], z2[3], a1[3], a2[3], d[3];
  zaxis(q1, z1);
  zaxis(q2, z2);
  for (int k = 0; k < 3; k++) { a1[k] = z1[k] * h1; a2[k] = z2[k] * h2; d[k] = p1[k] - p2[k]; }
  const float ma = dot3(a1, a1), mb = -dot3(a1, a2), mc = dot3(a2, a2), u = -dot3(a1, d), v = dot3(a2, d);
  const float det = ma * mc - mb * mb;
  float x1, x2;
  int mode;  // 0 both free, 1 x2 free (x1 fixed), 2 x1 free (x2 fixed), 3 both fixed
  const float idet = 1.f / det;  // used only where |det| >= 1e-15 (the forward's capcap: the same products)
  if (fabsf(det) >= 1e-15f) {
    x1 = (mc * u - mb * v) * idet;
    x2 = (ma * v - mb * u) * idet;
    mode = 0;
    if (x1 > 1.f) { x1 = 1.f; x2 = (v - mb) / mc; mode = 1; }
    else if (x1 < -1.f) { x1 = -1.f; x2 = (v + mb) / mc; mode = 1; }
    if (x2 > 1.f || x2 < -1.f) {
      const bool hi = x2 > 1.f;
      x2 = hi ? 1.f : -1.f;
      const float raw = hi ? (u - mb) / ma : (u + mb) / ma;
      x1 = fminf(fmaxf(raw, -1.f), 1.f);
      mode = (raw >= -1.f && raw < 1.f) ? 2 : 3;
    }
  } else if (slot < 2) {
    x1 = slot == 0 ? 1.f : -1.f;
    const float raw = slot == 0 ? (v - mb) / mc : (v + mb) / mc;
    x2 = fminf(fmaxf(raw, -1.f), 1.f);
    mode = (raw >= -1.f && raw < 1.f) ? 1 : 3;
  } else {
    x2 = slot == 2 ? 1.f : -1.f;
    const float raw = slot == 2 ? (u - mb) / ma : (u + mb) / ma;
    x1 = fminf(fmaxf(raw, -1.f), 1.f);
    mode = (raw >= -1.f && raw < 1.f) ? 2 : 3;
  }
  float v1[3], v2[3], v1b[3] = {0.f, 0.f, 0.f}, v2b[3] = {0.f, 0.f, 0.f}, dl[3], wv[3], a1b[3], a2b[3], x1bar, x2bar;
  for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; dl[k] = v2[k] - v1[k]; }
  cross(a1, a2, wv);
  const float ww = dot3(wv, wv);  // ma mc - mb^2 without its cancellation
  const bool wok = ww > 1e-12f * ma * mc;
  // near-parallel capsules (normal options != 0): both parameters held where sin^2(theta) < 1.2e-3
  const bool held = mode == 0 && normal != 0 && ww < 1.2e-3f * ma * mc;
  const float nu = sqrtf(dot3(dl, dl));
  if (mode == 0 && !held && wok && nu > 0.f) {
    // both parameters free: v2 - v1 is normal to both axes at the optimum, so n = sg w / |w| depends on the axes
    // alone (w = a1 x a2: dn = sg (I - n n') dw / |w|, dw = da1 x a2 + a1 x da2) and the distance is stationary in x1, x2; pos =
    // v1 + n (r1 + dist / 2) moves with x1 through v1 only. No term of order 1 / nu appears (the general chain below
    // sums such terms that cancel to order 1, losing up to 1e-3 relative in float32 at nu = 5 mm). The normal path is
    // scaled by kappa(nu) nu (1 for the exact derivative).
    float n[3], t[3], tau[3], u1[3], u2[3];
    const float inu = 1.f / nu;
    for (int k = 0; k < 3; k++) n[k] = dl[k] * inu;
    const float dist = nu - r1 - r2, hp = r1 + 0.5f * dist, dt = db + 0.5f * dot3(n, posb);
    for (int k = 0; k < 3; k++) t[k] = nb[k] + hp * posb[k];
    const float nt = dot3(n, t);
    float f = kappa_nu(nu, normal) * rsqrtf(ww);
    if (dot3(n, wv) < 0.f) f = -f;
    for (int k = 0; k < 3; k++) tau[k] = f * (t[k] - n[k] * nt);
    cross(a2, tau, u1);
    cross(tau, a1, u2);
    for (int k = 0; k < 3; k++) { v2b[k] = n[k] * dt; v1b[k] = posb[k] - v2b[k]; }
    for (int k = 0; k < 3; k++) {
      x1b[k] += v1b[k]; x2b[k] += v2b[k];
      a1b[k] = x1 * v1b[k] + u1[k]; a2b[k] = x2 * v2b[k] + u2[k];
    }
    x1bar = dot3(a1, posb);
    x2bar = 0.f;
  } else {
    sphere_core_vjp(v1, r1, v2, r2, db, posb, nb, normal, v1b, v2b);
    for (int k = 0; k < 3; k++) { x1b[k] += v1b[k]; x2b[k] += v2b[k]; a1b[k] = x1 * v1b[k]; a2b[k] = x2 * v2b[k]; }
    x1bar = held ? 0.f : dot3(a1, v1b);
    x2bar = held ? 0.f : dot3(a2, v2b);
  }
  float mab = 0.f, mbb = 0.f, mcb = 0.f, ub = 0.f, vb = 0.f;
  if (mode == 0) {  // G's determinant as |a1 x a2|^2 where that is not rounding noise (the forward's det otherwise)
    const float ig = wok ? 1.f / ww : idet;
    const float N1b = x1bar * ig, N2b = x2bar * ig, detb = -(x1bar * x1 + x2bar * x2) * ig;
    mcb += N1b * u; ub += N1b * mc; mbb -= N1b * v; vb -= N1b * mb;
    mab += N2b * v; vb += N2b * ma; mbb -= N2b * u; ub -= N2b * mb;
    mab += detb * mc; mcb += detb * ma; mbb -= 2.f * mb * detb;
  } else if (mode == 1) {
    const float g = x2bar / mc;
    vb += g; mbb -= g * x1; mcb -= g * x2;
  } else if (mode == 2) {
    const float g = x1bar / ma;
    ub += g; mbb -= g * x2; mab -= g * x1;
  }
  float dbv[3];
  for (int k = 0; k < 3; k++) {
    a1b[k] += 2.f * mab * a1[k] - mbb * a2[k] - ub * d[k];
    a2b[k] += 2.f * mcb * a2[k] - mbb * a1[k] + vb * d[k];
    dbv[k] = -ub * a1[k] + vb * a2[k];
  }
  for (int k = 0; k < 3; k++) { x1b[k] += dbv[k]; x2b[k] -= dbv[k]; a1b[k] *= h1; a2b[k] *= h2; }
  cross(z1, a1b, t1b);
  cross(z2, a2b, t2b);
}

// ---------------------------------------------------------------------------------------------- one substep
// A substep's VJP in phases. The record, the poses and the twists of v, a* and a~ depend on the tape alone; the
// integrator's VJP, the solves, the twists of lambda and y and every phase after them on the running cotangent
// (s.qb, s.vb, s.ub). k_adjoint runs them in turn; k_adjoint_sets runs the first group once per substep and the
// second once per cotangent set, the same functions in the same order, so each set's result is bitwise k_adjoint's.

// the record: every field's load issued at once, on every lane (a lane past a field reads a word inside it and drops
// it; a field loaded under its own lane test waited for each load in turn), with the factors' copies into LDS
// (load_factors): one memory round trip
__device__ __forceinline__ void adj_record(Adj& s, const float* __restrict__ rec, int lane) {
  const int lq = min(lane, NQ - 1), lv = min(lane, NV - 1);
  const float rq = rec[REC_QPOS + lq], rv = rec[REC_QVEL + lv], ra = rec[REC_ASTAR + lv], rd = rec[REC_AADV + lv];
  const unsigned rc = __float_as_uint(rec[REC_CLAMP + (lane & 1)]), rz = __float_as_uint(rec[REC_LIMZONE + (lane & 1)]);
  const unsigned rr = __float_as_uint(rec[REC_LIMROW + (lane & 1)]), rcz = __float_as_uint(rec[REC_CZONE + (lane & 7)]);
  const unsigned rcon = __float_as_uint(rec[REC_CON + (lane & (MAXCON / 2 - 1))]), hdr = __float_as_uint(rec[REC_HDR]);
  const unsigned rfl = __float_as_uint(rec[REC_FLAGS]);  // the records' flags, summed into the backward's info
  load_factors(s, rec, lane);
  if (lane < NQ) s.qpos[lane] = rq;
  if (lane < NV) {
    s.qvel[lane] = rv;
    s.astar[lane] = ra;
    s.aadv[lane] = rd;
    s.at[lane] = ra - rd;
  }
  if (lane < 2) {
    s.clampm[lane] = rc;
    s.limzone[lane] = rz;
    s.limrow[lane] = rr;
  }
  if (lane < 8) s.czone[lane] = rcz;
  if (lane < MAXCON / 2) {
    s.con[2 * lane] = (unsigned short)(rcon & 0xFFFFu);
    s.con[2 * lane + 1] = (unsigned short)(rcon >> 16);
  }
  if (lane == 0) { s.ncon = min((int)(hdr & 255u), MAXCON); s.flags |= (int)rfl; }
  // the body frames from L_Q's off-pattern positions (g1_tape.h), which get the factor's zeros back
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the factors' copies have landed in LDS
  wsync();
  float* frames = &s.Q[0][0];
  for (int q = lane; q < POSE_WORDS; q += WL) {
    const int p = s.pslot[q];
    frames[q] = s.lt.q[p];
    s.lt.q[p] = 0.f;
  }
  wsync();
}

// L_Q's off-pattern positions set to 0 again in a new copy of the factors (the frames were taken from the first)
__device__ __forceinline__ void clear_pose_slots(Adj& s, int lane) {
  for (int q = lane; q < POSE_WORDS; q += WL) s.lt.q[s.pslot[q]] = 0.f;
}

// poses: the body frames came with the record (the forward's FK of the substep's qpos); per body lane its spatial
// inertia about O, then the motion subspaces and geom poses, with no barrier after them (the caller's next phase
// shares their interval)
__device__ __forceinline__ void adj_poses(Adj& s, int lane) {
  if (lane < 3) s.O[lane] = s.qpos[lane];
  if (lane >= 1 && lane < NB) {  // own spatial inertia about O
    const float Q[4] = {s.Q[lane][0], s.Q[lane][1], s.Q[lane][2], s.Q[lane][3]};
    const float X[3] = {s.X[lane][0], s.X[lane][1], s.X[lane][2]};
    float ip[3], c[3], qi[4], R[9];
    for (int k = 0; k < 3; k++) ip[k] = cIpos[3 * lane + k] + (lane == TORSO_BODY ? s.com[k] : 0.f);
    qrot(Q, ip, c);
    const float iq[4] = {cIquat[4 * lane], cIquat[4 * lane + 1], cIquat[4 * lane + 2], cIquat[4 * lane + 3]};
    const float In[3] = {cInert[3 * lane], cInert[3 * lane + 1], cInert[3 * lane + 2]};
    qmul(Q, iq, qi);
    for (int k = 0; k < 3; k++) {
      float e[3] = {(float)(k == 0), (float)(k == 1), (float)(k == 2)};
      qrot(qi, e, R + 3 * k);
    }
    float* J = s.Ib[lane];
    J[0] = In[0] * R[0] * R[0] + In[1] * R[3] * R[3] + In[2] * R[6] * R[6];
    J[1] = In[0] * R[1] * R[1] + In[1] * R[4] * R[4] + In[2] * R[7] * R[7];
    J[2] = In[0] * R[2] * R[2] + In[1] * R[5] * R[5] + In[2] * R[8] * R[8];
    J[3] = In[0] * R[0] * R[1] + In[1] * R[3] * R[4] + In[2] * R[6] * R[7];
    J[4] = In[0] * R[0] * R[2] + In[1] * R[3] * R[5] + In[2] * R[6] * R[8];
    J[5] = In[0] * R[1] * R[2] + In[1] * R[4] * R[5] + In[2] * R[7] * R[8];
    float cc3[3];
    for (int k = 0; k < 3; k++) cc3[k] = X[k] - s.qpos[k] + c[k];
    const float m = cMass[lane], cc = dot3(cc3, cc3);
    J[0] += m * (cc - cc3[0] * cc3[0]); J[1] += m * (cc - cc3[1] * cc3[1]); J[2] += m * (cc - cc3[2] * cc3[2]);
    J[3] -= m * cc3[0] * cc3[1]; J[4] -= m * cc3[0] * cc3[2]; J[5] -= m * cc3[1] * cc3[2];
    J[6] = m * cc3[0]; J[7] = m * cc3[1]; J[8] = m * cc3[2]; J[9] = m;
  }
  wsync();
  if (lane < NV) {  // motion subspaces about O
    float w[3], v[3];
    if (lane < 3) {
      w[0] = w[1] = w[2] = 0.f;
      v[0] = lane == 0; v[1] = lane == 1; v[2] = lane == 2;
    } else if (lane < 6) {
      const float e[3] = {(float)(lane == 3), (float)(lane == 4), (float)(lane == 5)};
      qrot(s.Q[1], e, w);
      v[0] = v[1] = v[2] = 0.f;
    } else {
      const int b = lane - 4;
      const float r[3] = {s.O[0] - s.X[b][0], s.O[1] - s.X[b][1], s.O[2] - s.X[b][2]};
      const float ax[3] = {cAxis[3 * b], cAxis[3 * b + 1], cAxis[3 * b + 2]};
      qrot(s.Q[b], ax, w);
      cross(w, r, v);
    }
    for (int k = 0; k < 3; k++) { s.S[lane][k] = w[k]; s.S[lane][4 + k] = v[k]; }
  }
  if (lane < NGEOM) {  // geom poses
    const int b = geom_body(lane);
    float t[3], qb[4] = {s.Q[b][0], s.Q[b][1], s.Q[b][2], s.Q[b][3]};
    const float gp[3] = {cGpos[3 * lane], cGpos[3 * lane + 1], cGpos[3 * lane + 2]};
    const float gq[4] = {cGquat[4 * lane], cGquat[4 * lane + 1], cGquat[4 * lane + 2], cGquat[4 * lane + 3]};
    qrot(qb, gp, t);
    for (int k = 0; k < 3; k++) s.gx[lane][k] = s.X[b][k] + t[k];
    qmul(qb, gq, s.gq[lane]);
  }
}

// the integrator's VJP (tangent space): hinges and root position directly; the root rotation on lane 0
__device__ __forceinline__ void adj_integrator(Adj& s, int lane) {
  if (lane < NV) {
    const bool dir = lane < 3 || lane >= 6;
    s.vt[lane] = s.vb[lane] + (dir ? kH * s.qb[lane] : 0.f);
    s.qn[lane] = s.qb[lane];
  }
  wsync();
  if (lane == 0) {
    float phi[3], t[3] = {s.qb[3], s.qb[4], s.qb[5]};
    for (int k = 0; k < 3; k++) phi[k] = kH * (s.qvel[3 + k] + kH * s.aadv[3 + k]);
    const float th = sqrtf(dot3(phi, phi));
    float dq[4] = {1.f, 0.f, 0.f, 0.f}, sn = 0.f, cs = 1.f;
    if (th > 0.f) {
      sincosf(0.5f * th, &sn, &cs);
      const float st = sn / th;
      dq[0] = cs; dq[1] = st * phi[0]; dq[2] = st * phi[1]; dq[3] = st * phi[2];
    }
    float rt[3];
    qrot(dq, t, rt);  // t = R(dq) t'
    for (int k = 0; k < 3; k++) s.qn[3 + k] = rt[k];
    // J_r(phi)' t' = t' + c1 phi x t' + c2 phi x (phi x t'), c1 = (1 - cos th) / th^2, c2 = (th - sin th) / th^3.
    // Below th = 0.5 both are their Taylor series through th^8 (what is left out is below 5e-12 relative).
    // Above it, cos th and sin th come from the half angle's sine and cosine: 1 - cos th = 2 sin^2(th / 2) has no
    // cancellation, and th - sin th >= th^3 / 6 - th^5 / 120 keeps c2's rounding error below 2e-6 relative there.
    float c1, c2;
    if (th < 0.5f) {
      const float x = th * th;
      c1 = 0.5f + x * (-1.f / 24.f + x * (1.f / 720.f + x * (-1.f / 40320.f + x * (1.f / 3628800.f))));
      c2 = 1.f / 6.f + x * (-1.f / 120.f + x * (1.f / 5040.f + x * (-1.f / 362880.f + x * (1.f / 39916800.f))));
    } else {
      const float i2 = 1.f / (th * th);
      c1 = 2.f * sn * sn * i2;
      c2 = (th - 2.f * sn * cs) * i2 / th;
    }
    float pt[3], ppt[3];
    cross(phi, t, pt);
    cross(phi, pt, ppt);
    for (int k = 0; k < 3; k++) s.vt[3 + k] += kH * (t[k] + c1 * pt[k] + c2 * ppt[k]);
  }
  wsync();
}

// y = Q^-1 a_adv bar (L_Q), a* bar = a_adv bar - h kv y; lambda = H^-1 a* bar (L_H)
// clear: L_Q's frame slots set to 0 first (a copy of the factors made after the record's, whose frames were taken)
__device__ __forceinline__ void adj_solves(Adj& s, int lane, bool clear) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the factors' copies have landed in LDS
  wsync();
  if (clear) {
    clear_pose_slots(s, lane);
    wsync();
  }
  const float aab = lane < NV ? kH * s.vt[lane] : 0.f;
  const float y = ltl_solve(s.lt.q, aab, lane);
  if (lane < NV) s.y[lane] = y;
  wsync();
  const float asb = lane < NV ? aab - kH * cKv[lane] * y : 0.f;
  const float lam = ltl_solve(s.lt.h, asb, lane);
  if (lane < NV) s.lam[lane] = lam;
  wsync();
}

// A cotangent set's values between its passes in k_adjoint_sets: the integrator's results, the running control
// cotangent and the solves' results (LDS of its own, beside the Adj of the world)
struct __align__(16) SetStage { float vt[36], qn[36], y[36], lam[36], ub[32]; };
constexpr int SET_CHUNK = 2;  // cotangent sets whose solves run together (two right-hand sides a pass)

// adj_solves for the staged sets st[0 .. nc) at once (nc <= 2): the same expressions for each set, the pair of
// right-hand sides through ltl_solve2, so each set's y and lambda are bitwise adj_solves' for it
__device__ __forceinline__ void adj_solves_sets(Adj& s, SetStage* st, int nc, int lane, bool clear) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the factors' copies have landed in LDS
  wsync();
  if (clear) {
    clear_pose_slots(s, lane);
    wsync();
  }
  const float aab0 = lane < NV ? kH * st[0].vt[lane] : 0.f, aab1 = lane < NV && nc > 1 ? kH * st[1].vt[lane] : 0.f;
  float y0, y1;
  ltl_solve2(s.lt.q, aab0, aab1, lane, &y0, &y1);
  if (lane < NV) { st[0].y[lane] = y0; st[1].y[lane] = y1; }
  wsync();
  const float asb0 = lane < NV ? aab0 - kH * cKv[lane] * y0 : 0.f, asb1 = lane < NV ? aab1 - kH * cKv[lane] * y1 : 0.f;
  float l0, l1;
  ltl_solve2(s.lt.h, asb0, asb1, lane, &l0, &l1);
  if (lane < NV) { st[0].lam[lane] = l0; st[1].lam[lane] = l1; }
  wsync();
}

// chain twists of v, lambda, y, a*, a~ and the RNE acceleration (gravity, S a*, V_c(d) x S_d v_d) per body.
// The twist of a dof vector x is T[b] = T[parent(b)] + S_d x_d down the tree (d = b + 4, a hinge body's one dof)
// from the root body's T[1] = (sum_k S_{3+k}.w x_{3+k}; x_0..2) (S_0..2 = (0; e_k), S_3..5 = (w_k; 0)): a column per
// lane, lane 6 k + e holding component e of kind k for every body in registers, 2 loads and an FMA a body in
// ascending id order (a body's id is above its parent's; the parent table is compile-time). These are the sums
// along each body's chain in its order, root first. The RNE acceleration's velocity-product term is
// Ac[b] = (0; u x w) + sum over b's hinge chain of (V[body(d)] x S_d) v_d, V = (w; u) the root's velocity twist in
// the first term: each body lane stages its own cross product once, then sums its chain's in chain order; the
// padding byte 255 clamps to dof NV, whose entry of v is zero (its staged product is the last body's, finite).
// STATE: the twists of v, a*, a~ and the RNE acceleration (the record's); COT: those of lambda and y (the
// cotangent's). Each twist is its own chain of sums in the same order either way, so the results are the same with
// either part alone, and the same as adj_twists_cot's.
template <bool STATE, bool COT>
__device__ __forceinline__ void adj_twists(Adj& s, int lane) {
  constexpr int NK = (STATE ? 3 : 0) + (COT ? 2 : 0);  // kinds: STATE's v, a*, a~, then COT's lambda, y
  static_assert(6 * NK <= WL, "a column per lane");
  if (lane < 6 * NK) {
    const int k = lane / 6, e = lane - 6 * k;
    const int kk = STATE ? k : k + 3;  // 0 v, 1 a*, 2 a~, 3 lambda, 4 y
    const float* x = kk == 0 ? s.qvel : kk == 1 ? s.astar : kk == 2 ? s.at : kk == 3 ? s.lam : s.y;
    const int slot = kk == 0 ? TW_V : kk == 1 ? TW_AW : kk == 2 ? TW_A2 : kk == 3 ? TW_L : TW_Y;
    const int so = e < 3 ? e : e + 1;  // the component's place in a row of S: w at 0..2, v at 4..6
    float T[NB];
    const float tw = s.S[3][so] * x[3] + s.S[4][so] * x[4] + s.S[5][so] * x[5];
    T[1] = e < 3 ? tw : x[e < 3 ? 0 : e - 3];
    static_for<2, NB, 1>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      static_assert(BODY_PARENT[b] >= 1 && BODY_PARENT[b] < b, "bodies numbered parents first");
      T[b] = fmaf(s.S[b + 4][so], x[b + 4], T[BODY_PARENT[b]]);
    });
    float* out = &s.tw[0][slot][e];
    out[0] = 0.f;  // the world body
#pragma unroll
    for (int b = 1; b < NB; b++) out[b * NTW * 6] = T[b];
  }
  if (STATE) {
    if (lane == 0) st_sv6(s.tw[0][TW_A1], sv0());
    wsync();  // the velocity twists stored
    if (lane >= 1 && lane < NB) {  // this body's term of the chain sums: (V[b] x S_d) for its dof d, the root's (0; u x w)
      const Sv V = ld_sv6(s.tw[lane][TW_V]);
      Sv c = sv0();
      if (lane == 1) cross(V.v, V.w, c.v);
      else c = cross_mm(V, ld_sv(s.S[lane + 4]));
      st_sv6(s.tw[lane][TW_A1], c);
    }
    wsync();
    if (lane >= 1 && lane < NB) {
      unsigned ch[4];
      for (int k = 0; k < 4; k++) ch[k] = s.chain[lane][k];
      Sv Ac = ld_sv6(s.tw[1][TW_A1]);
#pragma unroll
      for (int t = NROOT; t < MAXCHAIN; t++) {
        const unsigned b = (ch[t >> 2] >> (8 * (t & 3))) & 255u;
        const int d = (int)min(b, (unsigned)NV);
        Ac = sv_add(Ac, ld_sv6(s.tw[min(d - 4, NB - 1)][TW_A1]), s.qvel[d]);
      }
      Sv A1 = sv_add(ld_sv6(s.tw[lane][TW_AW]), Ac);
      for (int k = 0; k < 3; k++) A1.v[k] -= kGrav[k];
      st_sv6(s.tw[lane][TW_A1], A1);  // after every lane's reads of the staged terms (one wave, program order)
    }
  }
  wsync();
}

// The twists of lambda and y alone (the cotangent passes of k_adjoint_sets) down the tree along the G1's four
// root-to-leaf paths (the two legs; the waist and then either arm), one group of 16 lanes a path, lane c < 12 of a
// group carrying component c % 6 of lambda's (c < 6) or y's twist: from the root body's (as in adj_twists) each
// path's bodies in order, an FMA of the body's one dof each (2 loads, an FMA and a store a step, every address a
// per-lane base plus a compile-time offset): the same sums in the same order as adj_twists. Both arm groups compute
// the waist's bodies (the same values); the legs' groups run 4 steps past their 6 bodies, and lanes c >= 12 every
// step, into a sink (the factors' copies, read by the solves before this).
__device__ __forceinline__ void adj_twists_cot(Adj& s, int lane) {
  const int g = lane >> 4, c = lane & 15;
  const bool comp = c < 12;
  const int e = c < 6 ? c : (comp ? c - 6 : 0);
  const float* x = c < 6 ? s.lam : s.y;
  const int slot = c < 6 ? TW_L : TW_Y;
  const int so = e < 3 ? e : e + 1;  // the component's place in a row of S: w at 0..2, v at 4..6
  const int lo = g == 0 ? PATHS.lo[0] : g == 1 ? PATHS.lo[1] : g == 2 ? PATHS.lo[2] : PATHS.lo[3];
  const int hi = g == 0 ? PATHS.hi[0] : g == 1 ? PATHS.hi[1] : g == 2 ? PATHS.hi[2] : PATHS.hi[3];
  constexpr int TWB = NTW * 6;  // a body's twist row
  float* sink = s.lt.q + (lane & 7);
  static_assert(TWB * (PATH_STEPS - 1) + 8 <= 768, "the sink inside the factors' copy");
  const float rw = s.S[3][so] * x[3] + s.S[4][so] * x[4] + s.S[5][so] * x[5];
  float T = e < 3 ? rw : x[e < 3 ? 0 : e - 3];
  (comp && g < 2 ? &s.tw[1 - g][slot][e] : sink)[0] = g == 0 ? T : 0.f;  // the root body; the world body 0
  const float *Sa = &s.S[4 + lo][so], *Sb = &s.S[4 + hi][so], *xa = x + 4 + lo, *xb = x + 4 + hi;
  float* oa = comp ? &s.tw[lo][slot][e] : sink;
  float* ob = comp ? &s.tw[hi][slot][e] : sink;
  float* oc = comp && g >= 2 ? ob : sink;  // past the legs' 6 bodies only the arm groups' are real
#pragma unroll
  for (int i = 0; i < PATH_STEPS; i++) {
    T = fmaf((i < 3 ? Sa : Sb)[8 * i], (i < 3 ? xa : xb)[i], T);
    (i < 3 ? oa : i < 6 ? ob : oc)[TWB * i] = T;
  }
  wsync();
}

// One substep's VJP. STATE: the phases that depend on the record alone (the record, the poses, the twists of v, a*
// and a~); COT: those on the running cotangent (s.qb, s.vb, s.ub at the substep's end -> at its start): the
// integrator's VJP, the solves, the twists of lambda and y, then the limit rows, the contacts (replayed from the
// record's contact table), the per-body wrench sums, body forces and subtree sums, and the dof terms. COT alone needs
// the factors' copies issued (load_factors) after the last COT pass, which overwrote them; recopied: they were, so
// L_Q's frame slots are set to 0 again before the solves. SOLVED (COT alone): the caller ran the integrator's VJP and
// the solves (s.vt, s.qn, s.y, s.lam in place), so the pass starts at the twists. (The phases after the twists stay
// in this body: as a function of their own they were optimized before inlining and k_adjoint grew by 69 v_movs.)
template <bool STATE, bool COT, bool SOLVED = false>
__device__ void adj_substep(Adj& s, const float* __restrict__ rec, int lane, int clamp_kv, int normal,
                            float clamp_soft, bool recopied = false) {
  static_assert(!(SOLVED && STATE), "SOLVED is a cotangent pass alone");
  if (STATE) {
    adj_record(s, rec, lane);
    APROF(AP_RECORD);
    adj_poses(s, lane);
  }
  if (COT && !SOLVED)
    adj_integrator(s, lane);
  else
    wsync();
  APROF(AP_POSES);
  if (COT && !SOLVED) {
    adj_solves(s, lane, recopied);
    APROF(AP_SOLVE);
  }
  if constexpr (STATE) adj_twists<STATE, COT>(s, lane);
  else adj_twists_cot(s, lane);
  APROF(AP_TWIST);
  if (!COT) return;
  // limit rows (their dof's lane): through the distance only (J constant)
  float lgq = 0.f, lgv = 0.f;
  if (lane >= 6 && lane < NV) {
    const unsigned long long lr = (unsigned long long)s.limrow[0] | (unsigned long long)s.limrow[1] << 32;
    const unsigned long long lz = (unsigned long long)s.limzone[0] | (unsigned long long)s.limzone[1] << 32;
    if ((lz >> lane) & 1ull && (lr >> lane) & 1ull) {
      const float q = s.qpos[lane + 1], dmin = q - cRange[2 * lane], dmax = cRange[2 * lane + 1] - q;
      const float sg = dmin < dmax ? 1.f : -1.f, pos = fminf(dmin, dmax);
      float k, b, imp, dimp;
      kb_consts(caJSolref.v, caJSolimp.v, &k, &b);
      imp_d(caJSolimp.v, pos, &imp, &dimp);
      const float iw = cDinvw[lane];
      const float D = 1.f / fmaxf(iw * (1.f - imp) / imp, 1e-15f), dD = dimp / (iw * (1.f - imp) * (1.f - imp));
      const float jl = sg * s.lam[lane], x = sg * s.astar[lane] + k * imp * pos + b * sg * s.qvel[lane];
      const float dbar = -(dD * jl * x + D * jl * k * (dimp * pos + imp));
      lgq = dbar * sg;
      lgv = -D * jl * b * sg;
    }
  }
  // contacts (lane = contact of the tape's table): replay, row terms, geometry VJP -> wrenches
  const int ncon = s.ncon;
  Sv cOmL = sv0(), cOmA = sv0(), cW1 = sv0(), cW2 = sv0();  // this lane's contact: row sums, the sides' wrenches
  float cbb = 0.f;
  int cb1 = 0, cb2 = 0;
  bool cact = false;
  if (lane < ncon) {
    const unsigned zc = (s.czone[lane >> 3] >> (4 * (lane & 7))) & 15u;
    const int pr = min((int)(s.con[lane] & 511u), NPAIR - 1), slot = s.con[lane] >> 9;
    const PairC pc = cPair[pr];
    const PairRow prow = cPairRow[pr];
    const unsigned w = pc.w;
    const int b1 = pc.bodies & 255u, b2 = pc.bodies >> 8, dim = (w >> 16) & 15u;
    cb1 = b1;
    cb2 = b2;
    if (zc) {
      Cand cd;
      collide_pair(s.gx, s.gq, pr, cd);
      const int which = (cd.has[0] && cd.slot[0] == slot) ? 0 : 1;
      if (!cd.has[which] || cd.slot[which] != slot) {
        s.flags |= 1 << 13;  // the replay does not find the tape's contact (a benign race on the same bit)
      } else {
        const float dist = cd.d[which];
        float pos[3], fr[9];
        for (int k = 0; k < 3; k++) pos[k] = which ? cd.pos[1][k] : cd.pos[0][k];
        for (int k = 0; k < 9; k++) fr[k] = which ? cd.fr[1][k] : cd.fr[0][k];
        const float mu = ((w >> 20) & 1u) ? s.fric : prow.mu;
        float k, b, imp, dimp;
        kb_consts(caPSolref.v, caPSolimp.v, &k, &b);
        imp_d(caPSolimp.v, dist, &imp, &dimp);
        float iw = prow.iw;
        if (dim == 3) iw = (mu * mu * iw + iw) * 2.f * mu * mu / kImpratio;
        const float D = 1.f / fmaxf(iw * (1.f - imp) / imp, 1e-15f), dD = dimp / (iw * (1.f - imp) * (1.f - imp));
        float rr[3];
        for (int q = 0; q < 3; q++) rr[q] = pos[q] - s.O[q];
        const Sv Lc = sv_add(ld_sv6(s.tw[b2][TW_L]), ld_sv6(s.tw[b1][TW_L]), -1.f);
        const Sv Ac = sv_add(ld_sv6(s.tw[b2][TW_AW]), ld_sv6(s.tw[b1][TW_AW]), -1.f);
        const Sv Vc = sv_add(ld_sv6(s.tw[b2][TW_V]), ld_sv6(s.tw[b1][TW_V]), -1.f);
        float dbar = 0.f, rb[3] = {0.f, 0.f, 0.f}, frb[9];
        for (int q = 0; q < 9; q++) frb[q] = 0.f;
        Sv OmL = sv0(), OmA = sv0();
        const int nr = dim == 3 ? 4 : 1;
#pragma unroll
        for (int t = 0; t < 4; t++) {
          if (t >= nr || !((zc >> t) & 1u)) continue;
          const float sg = (t & 1) ? -1.f : 1.f;
          const float* tk = fr + 3 * (1 + (t >> 1));
          float u[3];
          for (int q = 0; q < 3; q++) u[q] = dim == 3 ? fr[q] + sg * mu * tk[q] : fr[q];
          Sv Ph;
          cross(rr, u, Ph.w);
          for (int q = 0; q < 3; q++) Ph.v[q] = u[q];
          const float jl = sv_dot(Lc, Ph), x = sv_dot(Ph, Ac) + k * imp * dist + b * sv_dot(Ph, Vc);
          dbar += -(dD * jl * x + D * jl * k * (dimp * dist + imp));
          OmL = sv_add(OmL, Ph, -D * x);
          OmA = sv_add(OmA, Ph, -D * jl);
          const Sv Pb = sv_add(sv_add(sv0(), Lc, -D * x), sv_add(Ac, Vc, b), -D * jl);
          float ubar[3], t3[3];
          cross(Pb.w, rr, t3);
          for (int q = 0; q < 3; q++) ubar[q] = Pb.v[q] + t3[q];
          cross(u, Pb.w, t3);
          for (int q = 0; q < 3; q++) rb[q] += t3[q];
          for (int q = 0; q < 3; q++) {
            frb[q] += ubar[q];
            if (dim == 3) frb[3 * (1 + (t >> 1)) + q] += sg * mu * ubar[q];
          }
        }
        const Sv OmV = sv_add(sv0(), OmA, b);
        // the bodies' twist changes at the contact (side b2 +, b1 -)
        const Sv e1 = sv_add(sv_add(cross_mf(ld_sv6(s.tw[b1][TW_L]), OmL), cross_mf(ld_sv6(s.tw[b1][TW_AW]), OmA)),
                             cross_mf(ld_sv6(s.tw[b1][TW_V]), OmV));
        const Sv e2 = sv_add(sv_add(cross_mf(ld_sv6(s.tw[b2][TW_L]), OmL), cross_mf(ld_sv6(s.tw[b2][TW_AW]), OmA)),
                             cross_mf(ld_sv6(s.tw[b2][TW_V]), OmV));
        float x1b[3], t1b[3], x2b[3], t2b[3];
        contact_geom_vjp(s, pr, slot, fr, dbar, rb, frb, normal, x1b, t1b, x2b, t2b);
        const int g1 = w & 255u, g2 = (w >> 8) & 255u;
        Sv G1, G2;
        {
          float xo[3], m[3];
          for (int q = 0; q < 3; q++) xo[q] = s.gx[g1][q] - s.O[q];
          cross(xo, x1b, m);
          for (int q = 0; q < 3; q++) { G1.w[q] = t1b[q] + m[q]; G1.v[q] = x1b[q]; }
          for (int q = 0; q < 3; q++) xo[q] = s.gx[g2][q] - s.O[q];
          cross(xo, x2b, m);
          for (int q = 0; q < 3; q++) { G2.w[q] = t2b[q] + m[q]; G2.v[q] = x2b[q]; }
        }
        cOmL = OmL;
        cOmA = OmA;
        cW1 = sv_add(G1, e1, -1.f);  // the b1 side's wrench (its twists enter with -)
        cW2 = sv_add(G2, e2);        // the b2 side's wrench
        cbb = b;
        cact = true;
      }
    }
  }
  APROF(AP_CONTACT);
  // per body: the contacts' wrenches and row sums (body 2 +, body 1 -); body lane B keeps its totals. The floor
  // contacts (body 1 the world) summed over the contact lanes once per distinct body they touch (masked wave sums,
  // a fixed order); a contact between two robot bodies taken one at a time, its values broadcast to every lane and
  // added by the two body lanes (a wave sum per body it touches cost 24 sums of up to 6 steps each)
  Sv EG = sv0(), OL = sv0(), OA = sv0(), OV = sv0();
  const bool cself = cact && cb1 != 0;
  for (unsigned m = wor(cact && !cself ? 1u << cb2 : 0u) & ~1u; m; m &= m - 1u) {
    const int B = __builtin_ctz(m);
    const bool on = cact && !cself && cb2 == B;
    float x[24];
    for (int k = 0; k < 3; k++) {
      x[k] = on ? cW2.w[k] : 0.f;
      x[3 + k] = on ? cW2.v[k] : 0.f;
      x[6 + k] = on ? cOmL.w[k] : 0.f;
      x[9 + k] = on ? cOmL.v[k] : 0.f;
      x[12 + k] = on ? cOmA.w[k] : 0.f;
      x[15 + k] = on ? cOmA.v[k] : 0.f;
      x[18 + k] = on ? cbb * cOmA.w[k] : 0.f;
      x[21 + k] = on ? cbb * cOmA.v[k] : 0.f;
    }
    wsum_nw<24>(x, ncon);  // contact lanes only
    if (lane == B)
      for (int k = 0; k < 3; k++) {
        EG.w[k] = x[k]; EG.v[k] = x[3 + k]; OL.w[k] = x[6 + k]; OL.v[k] = x[9 + k];
        OA.w[k] = x[12 + k]; OA.v[k] = x[15 + k]; OV.w[k] = x[18 + k]; OV.v[k] = x[21 + k];
      }
  }
  for (unsigned long long m = ballot(cself); m; m &= m - 1ull) {
    const int c = __builtin_ctzll(m);
    const int b1 = rdli(cb1, c), b2 = rdli(cb2, c);
    const float s2 = lane == b2 ? 1.f : 0.f, s1 = lane == b1 ? 1.f : 0.f, sd = s2 - s1;
    const float bb = rdl(cbb, c);
    for (int k = 0; k < 3; k++) {
      EG.w[k] += s2 * rdl(cW2.w[k], c) + s1 * rdl(cW1.w[k], c);
      EG.v[k] += s2 * rdl(cW2.v[k], c) + s1 * rdl(cW1.v[k], c);
      OL.w[k] += sd * rdl(cOmL.w[k], c);
      OL.v[k] += sd * rdl(cOmL.v[k], c);
      const float aw = rdl(cOmA.w[k], c), av = rdl(cOmA.v[k], c);
      OA.w[k] += sd * aw;
      OA.v[k] += sd * av;
      OV.w[k] += sd * (bb * aw);
      OV.v[k] += sd * (bb * av);
    }
  }
  APROF(AP_BODYSUM);
  if (lane >= 1 && lane < NB) {
    const float* I = s.Ib[lane];
    const Sv V = ld_sv6(s.tw[lane][TW_V]), Lm = ld_sv6(s.tw[lane][TW_L]);
    const Sv IV = inertia_apply(I, V), IL = inertia_apply(I, Lm);
    const Sv F1 = sv_add(inertia_apply(I, ld_sv6(s.tw[lane][TW_A1])), cross_mf(V, IV));
    const Sv Qs = cross_mf(V, IL), Rs = cross_mf(Lm, IV), Ts = inertia_apply(I, cross_mm(V, Lm));
    const Sv X1 = sv_add(sv_add(Rs, Ts), Qs, -1.f);
    st_sv6(s.fb[lane][FB_F1], F1);
    st_sv6(s.fb[lane][FB_P], IL);
    st_sv6(s.fb[lane][FB_X1], X1);
    st_sv6(s.fb[lane][FB_F2], inertia_apply(I, ld_sv6(s.tw[lane][TW_A2])));
    st_sv6(s.fb[lane][FB_P2], inertia_apply(I, ld_sv6(s.tw[lane][TW_Y])));
    st_sv6(s.fb[lane][FB_EG], EG);
    st_sv6(s.fb[lane][FB_OL], OL);
    st_sv6(s.fb[lane][FB_OA], OA);
    st_sv6(s.fb[lane][FB_OV], OV);
  }
  wsync();
  APROF(AP_FORCES);
  // per body B: the subtree sums T[B] = sum of fb[b] over the bodies b of B's subtree (54 floats each), a column per
  // lane: lane c < 54 loads column c of every body and adds each body into its parent, highest id first (a body's id
  // is above its parent's, so each body is complete when it is added), then stores the sums in place. The tree is
  // compile-time: 29 adds a lane, no masks. Lanes past the columns compute a copy of the last one and do not store.
  {
    constexpr int NF = NFB * 6;
    static_assert(NF <= WL, "a column per lane");
    float* F = &s.fb[0][0][0] + (lane < NF ? lane : NF - 1);
    float v[NB];
#pragma unroll
    for (int b = 1; b < NB; b++) v[b] = F[b * NF];
    static_for<NB - 1, 1, -1>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      static_assert(BODY_PARENT[b] >= 1 && BODY_PARENT[b] < b, "bodies numbered parents first");
      v[BODY_PARENT[b]] += v[b];
    });
    if (lane < NF)
#pragma unroll
      for (int b = 1; b < NB; b++) F[b * NF] = v[b];
  }
  wsync();
  APROF(AP_SUBTREE);
  // per dof: subtree sums and the joint's outside terms
  if (lane < NV) {
    const int j = lane;
    const int bj = j < 6 ? 1 : j - 4;
    const Sv F1 = ld_sv6(s.fb[bj][FB_F1]), P = ld_sv6(s.fb[bj][FB_P]), X1 = ld_sv6(s.fb[bj][FB_X1]);  // subtree sums
    const Sv F2 = ld_sv6(s.fb[bj][FB_F2]), P2 = ld_sv6(s.fb[bj][FB_P2]), EGs = ld_sv6(s.fb[bj][FB_EG]);
    const Sv OLs = ld_sv6(s.fb[bj][FB_OL]), OAs = ld_sv6(s.fb[bj][FB_OA]), OVs = ld_sv6(s.fb[bj][FB_OV]);
    Sv Vo = sv0(), Lo = sv0(), Yo = sv0(), Awo = sv0(), A1o = sv0(), A2o = sv0();
    for (int k = 0; k < 3; k++) A1o.v[k] = -kGrav[k];
    if (j >= 3 && j < 6) {
      for (int k = 0; k < 3; k++) {
        Vo.v[k] = s.qvel[k]; Lo.v[k] = s.lam[k]; Yo.v[k] = s.y[k]; Awo.v[k] = s.astar[k];
        A1o.v[k] += s.astar[k]; A2o.v[k] = s.at[k];
      }
    } else if (j >= 6) {
      const int p = body_parent(bj);
      Vo = ld_sv6(s.tw[p][TW_V]); Lo = ld_sv6(s.tw[p][TW_L]); Yo = ld_sv6(s.tw[p][TW_Y]);
      Awo = ld_sv6(s.tw[p][TW_AW]); A1o = ld_sv6(s.tw[p][TW_A1]); A2o = ld_sv6(s.tw[p][TW_A2]);
    }
    const Sv Sj = ld_sv(s.S[j]);
    const Sv sig = cross_mm(Sj, Vo), alp = cross_mm(Sj, A1o), ell = cross_mm(Sj, Lo);
    const float dq1 = -sv_dot(ell, F1) - sv_dot(alp, P) + sv_dot(cross_mm(sig, Vo), P) + sv_dot(sig, X1);
    Sv rho = sv0();
    if (j >= 3) rho = sv_add(sig, cross_mm(Sj, ld_sv6(s.tw[bj][TW_V])));
    const float dv1 = -sv_dot(Sj, X1) - sv_dot(rho, P);
    const float dq2 = -sv_dot(cross_mm(Sj, Yo), F2) - sv_dot(cross_mm(Sj, A2o), P2);
    const float dqc = sv_dot(Sj, EGs) - sv_dot(Sj, sv_add(sv_add(cross_mf(Lo, OLs), cross_mf(Awo, OAs)),
                                                          cross_mf(Vo, OVs)));
    float gq = dq2 - dq1 + dqc + lgq, gv = -dv1 + sv_dot(Sj, OVs) + lgv;
    if (j >= 6) {  // the PD actuator kp (u - q) - kv v, clamped at +-frclim
      float wq = 1.f, wv = 1.f;
      const unsigned long long cm = (unsigned long long)s.clampm[0] | (unsigned long long)s.clampm[1] << 32;
      if ((cm >> j) & 1ull) {
        if (clamp_kv == 0) { wq = 0.f; wv = 1.f; }
        else if (clamp_kv == 1) { wq = wv = 0.f; }
        else {
          // w = exp(-o / delta), o = max((|f| - tau) / tau, 0) the relative overshoot of the unclamped PD force
          // (adjoint.py:811-829): a dof the tape marks clamped whose recomputed f rounds to inside its bound gets
          // o = 0, w = 1, never w > 1
          const float raw = cKp[j] * (s.ctrl[j - 6] - s.qpos[j + 1]) - cKv[j] * s.qvel[j];
          const float ov = fmaxf((fabsf(raw) - cFrclim[j]) / cFrclim[j], 0.f);
          wq = wv = clamp_soft > 0.f ? expf(-ov / clamp_soft) : 0.f;
        }
      }
      gq -= wq * cKp[j] * s.lam[j];
      gv -= wv * cKv[j] * s.lam[j];
      s.ub[j - 6] += wq * cKp[j] * s.lam[j];
    }
    s.qb[j] = s.qn[j] + gq;
    s.vb[j] = s.vt[j] + gv;
  }
  wsync();
  APROF(AP_DOF);
}

// the rotation part of a set's output cotangent in the tangent space at the output state, on one lane: the output
// root quaternion is the last substep's integration of its record's qvel, a_adv and qpos rows, replayed; g the
// cotangent's 4 quaternion entries
__device__ __forceinline__ void seed_rotation(Adj& s, const float* qvel, const float* aadv, const float* qpos,
                                              const float* g) {
  float wv[3], q[4];
  for (int k = 0; k < 3; k++) wv[k] = qvel[3 + k] + kH * aadv[3 + k];
  for (int k = 0; k < 4; k++) q[k] = qpos[3 + k];
  const float nw = sqrtf(dot3(wv, wv));
  if (nw > 0.f) {
    float sa, ca, o[4];
    sincosf(0.5f * kH * nw, &sa, &ca);
    const float sw = sa / nw;
    const float dq[4] = {ca, sw * wv[0], sw * wv[1], sw * wv[2]};
    qmul(q, dq, o);
    const float on = rsqrtf(o[0] * o[0] + o[1] * o[1] + o[2] * o[2] + o[3] * o[3]);
    for (int k = 0; k < 4; k++) q[k] = o[k] * on;
  }
  for (int k = 0; k < 3; k++) {
    float e[4] = {0.f, 0.f, 0.f, 0.f}, t[4];
    e[1 + k] = 1.f;
    qmul(q, e, t);
    s.qb[3 + k] = 0.5f * (t[0] * g[0] + t[1] * g[1] + t[2] * g[2] + t[3] * g[3]);
  }
}

// a set's gradients from s.qb, s.vb, s.ub: qpos form into oq (36), qvel into ov (35), ctrl into ou (29). The
// quaternion's entries 2 q0 (x) (0, t), q0 the step's input quaternion (the first record's qpos row, qpos), are
// computed on every lane and written by lanes 3..6; every other entry by the lane of its dof, so no entry of the
// three rows is written by two lanes. Returns the non-finite bits of the values written (check) or 0.
__device__ __forceinline__ int adj_emit(const Adj& s, const float* qpos, float* __restrict__ oq,
                                        float* __restrict__ ov, float* __restrict__ ou, int lane, bool check) {
  bool nq = false;  // a non-finite entry among those this lane writes
  if (lane < 3 || (lane >= 6 && lane < NV)) {
    oq[lane < 3 ? lane : lane + 1] = s.qb[lane];
    nq = !__builtin_isfinite(s.qb[lane]);
  }
  {
    const float* q0 = qpos + 3;
    const float n = rsqrtf(q0[0] * q0[0] + q0[1] * q0[1] + q0[2] * q0[2] + q0[3] * q0[3]);
    const float qq[4] = {q0[0] * n, q0[1] * n, q0[2] * n, q0[3] * n}, t[4] = {0.f, s.qb[3], s.qb[4], s.qb[5]};
    float r[4];
    qmul(qq, t, r);
    if (lane >= 3 && lane < 7) {
      const float o = 2.f * (lane == 3 ? r[0] : lane == 4 ? r[1] : lane == 5 ? r[2] : r[3]);
      oq[lane] = o;
      nq |= !__builtin_isfinite(o);
    }
  }
  const float xv = s.vb[min(lane, NV - 1)], xu = s.ub[min(lane, NU - 1)];
  if (lane < NV) ov[lane] = xv;
  if (lane < NU) ou[lane] = xu;
  if (!check) return 0;
  return (ballot(nq) ? NONFINITE_QPOS : 0) | (ballot(!__builtin_isfinite(xv)) ? NONFINITE_QVEL : 0) |
         (ballot(!__builtin_isfinite(xu)) ? NONFINITE_CTRL : 0);
}

// a set's part of the counters, from its info word f, on one lane; once per set (one backward call each) by the
// workgroup of the set's first dispatched world
__device__ __forceinline__ void adj_count(unsigned long long* __restrict__ diag, int f, bool first, int nw) {
  const int b = f >> NONFINITE_SHIFT;
  if (b & 7) atomicAdd(&diag[D_NONFINITE], 1ull);
  if (b & NONFINITE_QPOS) atomicAdd(&diag[D_NONFINITE_QPOS], 1ull);
  if (b & NONFINITE_QVEL) atomicAdd(&diag[D_NONFINITE_QVEL], 1ull);
  if (b & NONFINITE_CTRL) atomicAdd(&diag[D_NONFINITE_CTRL], 1ull);
  if (b & NONFINITE_COT) atomicAdd(&diag[D_NONFINITE_COT], 1ull);
  if (f & ADJ_REPLAY_MISMATCH) atomicAdd(&diag[D_REPLAY_MISMATCH], 1ull);
  if (first) {
    atomicAdd(&diag[D_BWD_CALLS], 1ull);
    atomicAdd(&diag[D_BWD_ROWS], (unsigned long long)nw);
  }
}

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_adjoint(int nw, int nsub, const float* __restrict__ tape,
                                                const float* __restrict__ fric, const float* __restrict__ com,
                                                const float* __restrict__ gq_out, const float* __restrict__ gv_out,
                                                float* __restrict__ gq_in, float* __restrict__ gv_in,
                                                float* __restrict__ gctrl, int* __restrict__ info,
                                                const float* __restrict__ ctrl, float clamp_soft, int clamp_kv,
                                                int normal, const int* __restrict__ perm,
                                                unsigned long long* __restrict__ diag, int ncot) {
  __shared__ Adj s;
  const int lane = threadIdx.x;
  if ((int)blockIdx.x >= nw * ncot) return;
  // ncot sets of output cotangents on one tape, set-major: workgroup b takes set b / nw; within a set the worlds run
  // heaviest first (g1_order.hip). wr: the world's row in its set's cotangents, gradients and info
  const int kc = (int)blockIdx.x / nw, wi = (int)blockIdx.x - kc * nw;
  const int w = perm ? perm[wi] : wi, wr = kc * nw + w;
  const float* wt = tape + (size_t)w * nsub * REC_WORDS;
  // the world's inputs: every load issued at once, on every lane (a lane past a row reads a word inside it and drops
  // it), one memory round trip
  const int lc = min(lane, 2), lu = min(lane, NU - 1), lv = min(lane, NV - 1);
  const int lqo = min(lane < 3 ? lane : lane + 1, NQ - 1);  // qpos-form entry of tangent dof lane (< 3 or >= 6)
  const float ic = com[(size_t)w * 3 + lc], iu = ctrl ? ctrl[(size_t)w * NU + lu] : 0.f, ifr = fric[w];
  const float igv = gv_out[(size_t)wr * NV + lv], igq = gq_out[(size_t)wr * NQ + lqo];
  if (lane < 3) s.com[lane] = ic;
  if (lane < NU) { s.ub[lane] = 0.f; s.ctrl[lane] = iu; }
  bool cbad = false;  // with the counters: a non-finite entry in the output cotangents (every entry of both rows)
  if (diag) {
    const float icq = gq_out[(size_t)wr * NQ + min(lane, NQ - 1)];
    cbad = ballot(!(__builtin_isfinite(icq) && __builtin_isfinite(igv))) != 0ull;
  }
  if (lane == 0) { s.fric = ifr; s.flags = cbad ? NONFINITE_COT << NONFINITE_SHIFT : 0; }
#ifdef G1_PROFILE
  if (lane < NPHASE) s.prof_acc[lane] = 0;
  if (lane == 0) {
    s.prof_t = __builtin_amdgcn_s_memtime();
    s.prof_acc[AP_T0] = __builtin_amdgcn_s_memrealtime();
  }
#endif
  chain_table(s.chain, lane);
  for (int q = lane; q < POSE_WORDS; q += WL) s.pslot[q] = (unsigned short)cPoseSlots.pos[q];
  if (lane == 0) s.qvel[NV] = 0.f;  // the chain padding's entry (adj_twists' velocity-product walk)
  // the output cotangents in the tangent space at the output state
  if (lane < NV) s.vb[lane] = igv;
  if (lane < NV && (lane < 3 || lane >= 6)) s.qb[lane] = igq;
  if (lane == 0) {
    const float* rec = wt + (size_t)(nsub - 1) * REC_WORDS;
    seed_rotation(s, rec + REC_QVEL, rec + REC_AADV, rec + REC_QPOS, gq_out + (size_t)wr * NQ + 3);
  }
  wsync();
  for (int k = nsub - 1; k >= 0; k--) adj_substep<true, true>(s, wt + (size_t)k * REC_WORDS, lane, clamp_kv, normal, clamp_soft);
  // gradients, and with the counters the non-finite bits of the values written (k_diag_bwd's)
  const int nb = adj_emit(s, wt + REC_QPOS, gq_in + (size_t)wr * NQ, gv_in + (size_t)wr * NV,
                          gctrl + (size_t)wr * NU, lane, diag != nullptr);
  if (lane == 0) {
    const int f = s.flags | nb << NONFINITE_SHIFT;
    info[wr] = f;
    if (diag) adj_count(diag, f, wi == 0, nw);
  }
#ifdef G1_PROFILE
  wsync();
  if (lane == 0) s.prof_acc[AP_T1] = __builtin_amdgcn_s_memrealtime();
  wsync();
  if (lane < NPHASE && w < PROF_WORLDS) g_prof_adj[w][lane] = s.prof_acc[lane];
#endif
}

// ncot sets of output cotangents on one tape, one workgroup per (world, group of per consecutive sets): per substep
// the record's phases once, then each set's cotangent phases, the same code as k_adjoint's in the same order (each
// set's gradients and info are bitwise k_adjoint's for it). Workgroup b takes the sets [per g, per (g + 1)) of the
// world dispatched b - g nw-th, g = b / nw. Between substeps a set's running cotangent waits in its own output rows,
// each entry in a slot one lane alone writes and reads: qb[d] in gq_in's slot d (d < 6) or d + 1, vb[d] in gv_in's d,
// ub[d] in gctrl's d, and the set's non-finite-cotangent bit in its info word; the last substep writes the gradients
// over them (adj_emit writes gq_in's slots 3..6 from lanes 3..6).
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_adjoint_sets(
    int nw, int nsub, const float* __restrict__ tape, const float* __restrict__ fric, const float* __restrict__ com,
    const float* __restrict__ gq_out, const float* __restrict__ gv_out, float* __restrict__ gq_in,
    float* __restrict__ gv_in, float* __restrict__ gctrl, int* __restrict__ info, const float* __restrict__ ctrl,
    float clamp_soft, int clamp_kv, int normal, const int* __restrict__ perm, unsigned long long* __restrict__ diag,
    int ncot, int per) {
  __shared__ Adj s;
  __shared__ SetStage st[SET_CHUNK];
  const int lane = threadIdx.x;
  const int ngrp = (ncot + per - 1) / per;
  if ((int)blockIdx.x >= nw * ngrp) return;
  const int g = (int)blockIdx.x / nw, wi = (int)blockIdx.x - g * nw;
  const int w = perm ? perm[wi] : wi;
  const int c0 = g * per, c1 = min(ncot, c0 + per);
  const float* wt = tape + (size_t)w * nsub * REC_WORDS;
  const int lc = min(lane, 2), lu = min(lane, NU - 1), lv = min(lane, NV - 1);
  const int lqo = min(lane < 3 ? lane : lane + 1, NQ - 1);  // qpos-form entry of tangent dof lane (< 3 or >= 6)
  const int lqs = min(lane < 6 ? lane : lane + 1, NQ - 1);  // the running qb's slot of dof lane
  const float ic = com[(size_t)w * 3 + lc], iu = ctrl ? ctrl[(size_t)w * NU + lu] : 0.f, ifr = fric[w];
  if (lane < 3) s.com[lane] = ic;
  if (lane < NU) s.ctrl[lane] = iu;
  if (lane == 0) { s.fric = ifr; s.flags = 0; }  // the tape's flags, the same for every set
#ifdef G1_PROFILE
  if (lane < NPHASE) s.prof_acc[lane] = 0;
  if (lane == 0) s.prof_t = __builtin_amdgcn_s_memtime();
#endif
  chain_table(s.chain, lane);
  for (int q = lane; q < POSE_WORDS; q += WL) s.pslot[q] = (unsigned short)cPoseSlots.pos[q];
  if (lane == 0) s.qvel[NV] = 0.f;  // the chain padding's entry (adj_twists' velocity-product walk)
  wsync();
#pragma unroll 1
  for (int k = nsub - 1; k >= 0; k--) {
    const float* rec = wt + (size_t)k * REC_WORDS;
    adj_substep<true, false>(s, rec, lane, clamp_kv, normal, clamp_soft);
#pragma unroll 1
    for (int cc = c0; cc < c1; cc += SET_CHUNK) {
      const int nc = min(SET_CHUNK, c1 - cc);
      // each set's running cotangent and the integrator's VJP, staged
#pragma unroll 1
      for (int q = 0; q < nc; q++) {
        const int c = cc + q;
        const size_t wr = (size_t)c * nw + w;
        if (k == nsub - 1) {  // the set's output cotangents in the tangent space at the output state
          const float igv = gv_out[wr * NV + lv], igq = gq_out[wr * NQ + lqo];
          bool cbad = false;  // with the counters: a non-finite entry in the output cotangents
          if (diag) {
            const float icq = gq_out[wr * NQ + min(lane, NQ - 1)];
            cbad = ballot(!(__builtin_isfinite(icq) && __builtin_isfinite(igv))) != 0ull;
          }
          if (lane < NU) s.ub[lane] = 0.f;
          if (lane < NV) s.vb[lane] = igv;
          if (lane < NV && (lane < 3 || lane >= 6)) s.qb[lane] = igq;
          if (lane == 0) {
            info[wr] = cbad ? NONFINITE_COT << NONFINITE_SHIFT : 0;
            seed_rotation(s, s.qvel, s.aadv, s.qpos, gq_out + wr * NQ + 3);  // s holds the last record
          }
        } else {
          const float rq = gq_in[wr * NQ + lqs], rv = gv_in[wr * NV + lv], ru = gctrl[wr * NU + lu];
          if (lane < NV) { s.qb[lane] = rq; s.vb[lane] = rv; }
          if (lane < NU) s.ub[lane] = ru;
        }
        wsync();
        adj_integrator(s, lane);
        if (lane < NV) { st[q].vt[lane] = s.vt[lane]; st[q].qn[lane] = s.qn[lane]; }
        if (lane < NU) st[q].ub[lane] = s.ub[lane];
        wsync();
      }
      // the sets' solves together: the substep's first chunk on the record's copies of the factors, a later one on a
      // fresh copy (the previous chunk's tails overwrote them)
      if (cc > c0) load_factors(s, rec, lane);
      adj_solves_sets(s, st, nc, lane, cc > c0);
      // each set's remaining phases
#pragma unroll 1
      for (int q = 0; q < nc; q++) {
        const int c = cc + q;
        const size_t wr = (size_t)c * nw + w;
        float* oq = gq_in + wr * NQ;
        float* ov = gv_in + wr * NV;
        float* ou = gctrl + wr * NU;
        if (lane < NV) { s.vt[lane] = st[q].vt[lane]; s.qn[lane] = st[q].qn[lane]; s.y[lane] = st[q].y[lane]; s.lam[lane] = st[q].lam[lane]; }
        if (lane < NU) s.ub[lane] = st[q].ub[lane];
        adj_substep<false, true, true>(s, rec, lane, clamp_kv, normal, clamp_soft);
        if (k > 0) {
          if (lane < NV) { oq[lqs] = s.qb[lane]; ov[lane] = s.vb[lane]; }
          if (lane < NU) ou[lane] = s.ub[lane];
        } else {  // s holds the first record: its qpos row is the step's input
          const int nb = adj_emit(s, s.qpos, oq, ov, ou, lane, diag != nullptr);
          if (lane == 0) {
            const int f = s.flags | info[wr] | nb << NONFINITE_SHIFT;
            info[wr] = f;
            if (diag) adj_count(diag, f, wi == 0, nw);
          }
        }
        wsync();
      }
    }
  }
}

int launch_order_adj(hipStream_t st, int nw, int nsub, const float* tape, void* work);
int resident_worlds();

// k_adjoint_sets' sets per workgroup: groups small enough that nw x groups makes G1_SETS_WAVES waves, and at least
// two groups (a workgroup of all of a world's sets is a long wave, whose tail shows at 16384 worlds: 1.3% there).
// Of 2048 resident waves (2 per SIMD on 256 CUs), 16384 makes 8 rounds: the launch's tail is a few sets long, and the
// record phases repeated per group cost under 2% (measured at 1024, 4096 and 16384 worlds with 4096 to 32768 waves:
// 16384 the best at 4096 worlds and within 0.5% at 1024)
#ifndef G1_SETS_WAVES
#define G1_SETS_WAVES 16384
#endif
int sets_per_group(int nw, int ncot) {
  const long long ngrp = std::min<long long>(ncot, std::max<long long>(2, (G1_SETS_WAVES + nw - 1) / nw));
  return (int)((ncot + ngrp - 1) / ngrp);
}
int launch_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                   const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                   const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work, int order,
                   unsigned long long* diag, int ncot) {
  if (nw <= 0) return 0;
  if (reinterpret_cast<uintptr_t>(tape) & 15u) return (int)hipErrorInvalidValue;  // 16-byte copies of the factors
  const int* perm = nullptr;
  // one set of a batch that fits the resident slots at once: every world starts at the launch, index order
  if (order == 1 && ncot == 1 && nw <= resident_worlds()) order = 0;
  if (work && order) {  // the dispatch order, heaviest worlds first (order 1: computed here; 2: already in work)
    if (order == 1) {
      const int rc = launch_order_adj(st, nw, nsub, tape, work);
      if (rc) return rc;
    }
    perm = (const int*)work;
  }
  if (ncot == 1) {
    hipLaunchKernelGGL(k_adjoint, dim3(nw), dim3(64), 0, st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in,
                       gctrl, info, ctrl, clamp_soft, clamp_kv, normal, perm, diag, 1);
  } else {
    const int per = sets_per_group(nw, ncot), ngrp = (ncot + per - 1) / per;
    hipLaunchKernelGGL(k_adjoint_sets, dim3(nw * ngrp), dim3(64), 0, st, nw, nsub, tape, fric, com, gq_out, gv_out,
                       gq_in, gv_in, gctrl, info, ctrl, clamp_soft, clamp_kv, normal, perm, diag, ncot, per);
  }
  return (int)hipGetLastError();
}
size_t adjoint_lds_bytes() { return sizeof(Adj); }

// k_adjoint's resident workgroups (worlds) per CU on device dev, the current device restored afterwards
int adjoint_occupancy(int dev, int* n) {
  int old = -1;
  hipError_t e = hipGetDevice(&old);
  if (e != hipSuccess) return (int)e;
  if ((e = hipSetDevice(dev)) != hipSuccess) return (int)e;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(n, k_adjoint, 64, 0);
  const hipError_t e2 = hipSetDevice(old);
  return (int)(e != hipSuccess ? e : e2);
}

int prof_read_adj(unsigned long long* out, int nw) {  // the G1_PROFILE build's adjoint phase cycles (nw x NPHASE)
#ifdef G1_PROFILE
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prof_adj), sizeof(unsigned long long) * NPHASE * (size_t)nw);
#else
  (void)out;
  (void)nw;
  return -1;
#endif
}

}  // namespace g1k
