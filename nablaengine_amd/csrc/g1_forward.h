// LDS state of one world (one wave64) for the G1 forward control step.
#pragma once
#include "g1_device.h"

namespace g1k {

constexpr int MSTRIDE = 36;
// the smooth dynamics' per-body row: force, moment about O, spatial inertia (10 of 12), each 16-byte aligned
constexpr int SM_F = 0, SM_T = 4, SM_I = 8, SMW = 20;

struct __align__(16) Sim {
  // the dof vectors padded to 36 entries (16-byte multiples; matvec reads them as float4s)
  float qpos[40], qvel[36], qacc[36], ctrl[32], com[4];
  float qsm[36], qacc0[36], Ma[36], grad[36], p[36], Mp[36];
  float M[NV][MSTRIDE];  // the mass matrix, full and symmetric, row-major (rows 16-byte aligned; column 35 unused)
  float L[LSINK + 64];  // the packed factor (NTRI + 2 padding), then the per-lane sink of masked stores
  float S[NV + 1][8];         // dof motion subspaces about O: angular (0..2), velocity of O (4..6); row NV unused
  float Q[NB][4], X[NB][4];   // body poses
  unsigned chain[NB][MAXCHAIN / 4];  // the dofs moving each body, ascending, one byte each; 255 past the chain
  unsigned dsub[WL];                 // bodies moved by dof i (bit b), 0 past the dofs
  float O[4];
  float fric;
  int ncon, ncon_raw, nlim, nefc, flags, niter;
  int dcnt;  // the records' flags counted over the substeps: refactored | not converged << 8 | singular << 16
  int acost;  // the adjoint's dispatch cost summed over the substeps so far (taped forward)
  unsigned clampm[2];  // dofs whose actuator force is at its limit (tape)
#ifdef G1_PROFILE
  unsigned long long prof_t, prof_acc[NPHASE];
#endif
  union __align__(16) {  // 16-byte aligned whatever the scalars above add up to (its rows are read as float4s)
    // smooth dynamics: per body its force (SM_F + 0..2), moment about O (SM_T + 0..2) and spatial inertia about O
    // (SM_I + 0..9), summed over its subtree in place; the bodies' local transforms
    struct { float V[NB][SMW], hl[NB][12]; } sm;
    struct { float gx[NGEOM][4], gq[NGEOM][4]; float stage[MAXCON][16]; unsigned short cand[NPAIR + 2]; } col;
    struct {
      float bw[NB][8];  // body spatial velocity of a dof vector: angular (0..2), velocity of O (4..6)
      struct { float psi[16][8]; float U[48][17]; } h;  // Hessian: a batch of self-contact rows (<= 16);
                                                         // U's rows past the dofs zero (MFMA tiles of 16); rows
                                                         // padded to 17 floats: no LDS bank conflicts down a column
    } nt;
  } u;
};

// 8 worlds per CU: the LDS of one world must stay within 160 KB / 8 (the profile build's counters excepted)
#ifndef G1_PROFILE
static_assert(sizeof(Sim) <= 20480, "Sim outgrew the LDS of 8 worlds per CU");
#endif
static_assert(offsetof(Sim, X) == offsetof(Sim, Q) + 16 * NB, "the body frames Q, X as one array (the tape's copy)");

// per-lane register state of the constraint rows: lane l holds contact l's rows and dof l's limit row
struct Rows {
  float r[3], fr[9], mu, D;  // contact point - O; frame rows n, t1, t2; friction; the rows' D
  int b1, b2, nr, dim;       // bodies, kept rows (0..4), condim
  float aref[4], jar[4];     // per pyramid edge (or the normal row)
  float lsg, lD, laref, ljar;  // the limit row of this lane's dof (active when lsg != 0)
  // the floor contacts are the lanes [0, nf) sorted by body; those on the bodies this lane's dof moves are the lanes
  // [flo, fhi), and fcl = (flo > 0 || fhi == 0) weights the prefix sum below the run (floor_run)
  int nf, flo, fhi;
  float fcl;
};

}  // namespace g1k
