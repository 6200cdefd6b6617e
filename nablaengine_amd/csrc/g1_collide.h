// Collision primitives of the G1 pairs (plane-sphere, plane-capsule, sphere-sphere, sphere-capsule, capsule-capsule)
// at zero margin, shared by the forward's narrowphase and the adjoint's replay: restated from the reference's
// step.py:378-554 (make_frame, plane_point, plane_capsule_frame, capsule_end, segment_point, capcap_*) and
// step.py:1042-1143 (collide_pair), which follow MuJoCo Warp's collision_primitive_core.
#pragma once
#include "g1_device.h"

namespace g1k {

// MuJoCo's frame from a normal n: rows n, b, n x b with b the unit vector e_y (|n_y| < 0.5) or e_z made orthogonal to
// n (step.py:378-387 make_frame)
__device__ __forceinline__ void make_frame(const float* n, float* fr) {
  float b[3] = {0.f, 0.f, 0.f};
  if (-0.5f < n[1] && n[1] < 0.5f) b[1] = 1.f; else b[2] = 1.f;
  float d = dot3(n, b);
  for (int k = 0; k < 3; k++) b[k] -= n[k] * d;
  float bn = sqrtf(dot3(b, b));
  if (bn > 0.f) {
    const float ib = 1.f / bn;  // one division, three products
    for (int k = 0; k < 3; k++) b[k] *= ib;
  }
  float c[3];
  cross(n, b, c);
  for (int k = 0; k < 3; k++) { fr[k] = n[k]; fr[3 + k] = b[k]; fr[6 + k] = c[k]; }
}

__device__ __forceinline__ void sphere_sphere(const float* p1, float r1, const float* p2, float r2, float* dist,
                                              float* pos, float* n) {
  float dir[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
  float d = sqrtf(dot3(dir, dir));
  if (d == 0.f) { n[0] = 1.f; n[1] = 0.f; n[2] = 0.f; } else {
    const float id = 1.f / d;
    for (int k = 0; k < 3; k++) n[k] = dir[k] * id;
  }
  *dist = d - (r1 + r2);
  float hp = 0.5f * *dist + r1;
  for (int k = 0; k < 3; k++) pos[k] = p1[k] + n[k] * hp;
}

__device__ __forceinline__ float plane_point(const float* p1, const float* n, const float* c, float r, float* pos) {
  float dist = (dot3(c, n) - dot3(p1, n)) - r, hp = 0.5f * dist + r;
  for (int k = 0; k < 3; k++) pos[k] = c[k] - n[k] * hp;
  return dist;
}

__device__ __forceinline__ void zaxis(const float* q, float* a) {
  const float ez[3] = {0.f, 0.f, 1.f};
  qrot(q, ez, a);
}

struct Cand {  // up to two contacts of one pair: A then B
  float d[2], pos[2][3], fr[2][9];
  int slot[2];
  bool has[2];
};

__device__ __forceinline__ void put(Cand& o, int which, int slot, float dist, const float* pos, const float* fr) {
  // which is a compile-time 0 / 1 at every call site
  o.has[which] = true;
  o.d[which] = dist;
  o.slot[which] = slot;
  for (int k = 0; k < 3; k++) o.pos[which][k] = pos[k];
  for (int k = 0; k < 9; k++) o.fr[which][k] = fr[k];
}

// broadphase over the 502 pairs (step.py:1789-1826): the narrowphase's first test with a relative slack of 1e-5 (the
// plane's normal distance against the bounding radius, else the bounding spheres), candidates compacted into cand in
// pair order; returns their count. Branch-free and unrolled (a clamped pair index, the spare slot cand[NPAIR + 1]
// for the dropped ones), so every iteration's table loads are issued together.
__device__ __forceinline__ int broadphase(const float (*gx)[4], const float* fn, unsigned short* cand, int lane) {
  int ncand = 0;
#pragma unroll
  for (int k = 0; k < (NPAIR + WL - 1) / WL; k++) {
    const int pr = lane + WL * k;
    const PairC pc = cPair[pr < NPAIR ? pr : NPAIR - 1];
    const unsigned w = pc.w;
    const int g1 = w & 255u, g2 = (w >> 8) & 255u;
    const float dif[3] = {gx[g2][0] - gx[g1][0], gx[g2][1] - gx[g1][1], gx[g2][2] - gx[g1][2]};
    const unsigned cls = (w >> 21) & 7u;
    const float r2 = pc.rb2, rb = pc.rb;
    const bool plane = cls == 0u || cls == 4u;
    const bool keep = pr < NPAIR && (plane ? dot3(dif, fn) <= r2 * (1.f + 1e-5f) + 1e-6f
                                           : dot3(dif, dif) <= rb * rb * (1.f + 1e-5f) + 1e-12f);
    const unsigned long long bal = ballot(keep);
    cand[keep ? ncand + prefix_count(bal, lane) : NPAIR + 1] = (unsigned short)pr;
    ncand += __popcll(bal);
  }
  return ncand;
}

// narrowphase of pair pr (step.py:1042-1143 collide_pair), zero margin
__device__ void collide_pair(const float (*gx)[4], const float (*gq)[4], int pr, Cand& o) {
  o.has[0] = o.has[1] = false;
  const PairC pc = cPair[pr];
  const PairSz psz = cPairSz[pr];
  const unsigned w = pc.w;
  const int g1 = w & 255u, g2 = (w >> 8) & 255u, cls = (w >> 21) & 7u;
  float p1[3], q1[4], p2[3], q2[4];
  for (int k = 0; k < 3; k++) { p1[k] = gx[g1][k]; p2[k] = gx[g2][k]; }
  for (int k = 0; k < 4; k++) { q1[k] = gq[g1][k]; q2[k] = gq[g2][k]; }
  const float r1 = psz.r1, hl1 = psz.hl1, r2 = psz.r2, hl2 = psz.hl2;
  float pos[3], fr[9], n[3], dist;
  if (cls == 0 || cls == 4) {  // plane (the floor) against a sphere or a capsule
    zaxis(q1, n);
    float dif[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]};
    if (dot3(dif, n) > pc.rb2) return;
    if (cls == 0) {
      dist = plane_point(p1, n, p2, r2, pos);
      make_frame(n, fr);
      if (dist < 0.f) put(o, 0, 0, dist, pos, fr);
    } else {
      float axis[3];
      zaxis(q2, axis);
      // plane_capsule_frame (step.py:461-474): b = axis projected on the plane, normalized; make_frame's basis
      // vector where the projection is shorter than 0.5
      float na = dot3(n, axis), b[3];
      for (int k = 0; k < 3; k++) b[k] = axis[k] - n[k] * na;
      float bn = sqrtf(dot3(b, b));
      if (bn > 0.f) {
        const float ib = 1.f / bn;
        for (int k = 0; k < 3; k++) b[k] *= ib;
      }
      if (bn < 0.5f) {
        b[0] = b[1] = b[2] = 0.f;
        if (-0.5f < n[1] && n[1] < 0.5f) b[1] = 1.f; else b[2] = 1.f;
      }
      float c[3];
      cross(n, b, c);
      for (int k = 0; k < 3; k++) { fr[k] = n[k]; fr[3 + k] = b[k]; fr[6 + k] = c[k]; }
      float ce[3];
      for (int k = 0; k < 3; k++) ce[k] = p2[k] + axis[k] * hl2;
      dist = plane_point(p1, n, ce, r2, pos);
      if (dist < 0.f) put(o, 0, 0, dist, pos, fr);
      for (int k = 0; k < 3; k++) ce[k] = p2[k] - axis[k] * hl2;
      dist = plane_point(p1, n, ce, r2, pos);
      if (dist < 0.f) put(o, 1, 1, dist, pos, fr);
    }
    return;
  }
  {
    float dif[3] = {p2[0] - p1[0], p2[1] - p1[1], p2[2] - p1[2]}, rb = pc.rb;
    if (dot3(dif, dif) > rb * rb) return;
  }
  if (cls == 1) {  // sphere-sphere
    sphere_sphere(p1, r1, p2, r2, &dist, pos, n);
    if (dist < 0.f) { make_frame(n, fr); put(o, 0, 0, dist, pos, fr); }
    return;
  }
  if (cls == 2) {  // sphere-capsule: the capsule segment's closest point (step.py:487-497 segment_point)
    float axis[3], a[3], ab[3], ap[3], pt[3];
    zaxis(q2, axis);
    for (int k = 0; k < 3; k++) { a[k] = p2[k] - axis[k] * hl2; ab[k] = 2.f * axis[k] * hl2; ap[k] = p1[k] - a[k]; }
    float gam = dot3(ab, ab) + 1e-6f, t = fminf(fmaxf(dot3(ap, ab) / gam, 0.f), 1.f);
    for (int k = 0; k < 3; k++) pt[k] = a[k] + t * ab[k];
    sphere_sphere(p1, r1, pt, r2, &dist, pos, n);
    if (dist < 0.f) { make_frame(n, fr); put(o, 0, 0, dist, pos, fr); }
    return;
  }
  // capsule-capsule (step.py:501-554 capcap_setup / capcap_params / capcap_candidate)
  float a1[3], a2[3], d[3];
  zaxis(q1, a1);
  zaxis(q2, a2);
  for (int k = 0; k < 3; k++) { a1[k] *= hl1; a2[k] *= hl2; d[k] = p1[k] - p2[k]; }
  const float ma = dot3(a1, a1), mb = -dot3(a1, a2), mc = dot3(a2, a2), u = -dot3(a1, d), v = dot3(a2, d);
  const float det = ma * mc - mb * mb;
  if (fabsf(det) >= 1e-15f) {
    const float idet = 1.f / det;
    float x1 = (mc * u - mb * v) * idet, x2 = (ma * v - mb * u) * idet;
    if (x1 > 1.f) { x1 = 1.f; x2 = (v - mb) / mc; }
    else if (x1 < -1.f) { x1 = -1.f; x2 = (v + mb) / mc; }
    if (x2 > 1.f || x2 < -1.f) {
      bool hi = x2 > 1.f;
      x2 = hi ? 1.f : -1.f;
      float raw = hi ? (u - mb) / ma : (u + mb) / ma;
      x1 = fminf(fmaxf(raw, -1.f), 1.f);
    }
    float v1[3], v2[3];
    for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; }
    sphere_sphere(v1, r1, v2, r2, &dist, pos, n);
    if (dist < 0.f) { make_frame(n, fr); put(o, 0, 0, dist, pos, fr); }
  } else {
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if (cnt >= 2) break;
      float x1, x2;
      if (e < 2) {
        x1 = e == 0 ? 1.f : -1.f;
        float raw = e == 0 ? (v - mb) / mc : (v + mb) / mc;
        x2 = fminf(fmaxf(raw, -1.f), 1.f);
      } else {
        x2 = e == 2 ? 1.f : -1.f;
        float raw = e == 2 ? (u - mb) / ma : (u + mb) / ma;
        x1 = fminf(fmaxf(raw, -1.f), 1.f);
      }
      float v1[3], v2[3];
      for (int k = 0; k < 3; k++) { v1[k] = p1[k] + a1[k] * x1; v2[k] = p2[k] + a2[k] * x2; }
      sphere_sphere(v1, r1, v2, r2, &dist, pos, n);
      if (dist <= 0.f) {
        if (dist < 0.f) {
          make_frame(n, fr);
          if (!o.has[0]) put(o, 0, e, dist, pos, fr); else put(o, 1, e, dist, pos, fr);
        }
        cnt++;
      }
    }
  }
}


}  // namespace g1k
