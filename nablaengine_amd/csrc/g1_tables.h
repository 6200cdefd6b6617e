// Compile-time tables of the G1 model for the HIP kernels: the model arrays of g1_model.h as float, and the tree
// structure the kernels walk (paths, subtree and ancestor masks, dof chains), all derived by constexpr code so the
// kernels are specialised to the model at compile time.
#pragma once
#include <cstdint>

#include "g1_model.h"

namespace g1t {
using namespace g1;
constexpr int NB = NBODY;
constexpr int NTRI = NV * (NV + 1) / 2;
constexpr int LSINK = NTRI + 2;  // a packed factor buffer's per-lane sink (64 floats after the matrix and its padding):
                                 // lanes without an entry to store write there instead of branching around the store
constexpr int MAXCON = 64;     // contact capacity per world (step.py:70-79 maxcon for 502 pairs)
constexpr int NEFC = 192;      // constraint row capacity (step.py:43)
constexpr int MAXCHAIN = 16;   // dofs on a body's chain: root 6 + at most 10 hinges (waist 3 + arm 7)

__host__ __device__ constexpr int tri(int i, int j) { return i * (i + 1) / 2 + j; }

template <class T, int N>
struct Arr {
  T v[N];
  __host__ __device__ constexpr const T& operator[](int i) const { return v[i]; }
};

template <int N>
constexpr Arr<float, N> to_float(const double (&a)[N]) {
  Arr<float, N> r{};
  for (int i = 0; i < N; i++) r.v[i] = (float)a[i];
  return r;
}

struct Tree {
  int path[NB][MAXDEPTH];       // path[b][l]: the body at depth l + 1 on b's chain (path[b][0] = 1, the root)
  unsigned submask[NB];         // bit c: body c is in b's subtree (b itself included)
  uint64_t dofanc[NV];          // bit j: dof j on dof i's chain (root dofs, hinge ancestors, i itself)
  int chain[NB][MAXCHAIN];      // the dofs that move body b, ascending
  int nchain[NB];
  unsigned dofmask32[NV];       // bodies moved by dof i (its body's subtree), for J^T f sign tests
};

constexpr Tree make_tree() {
  Tree t{};
  for (int b = 0; b < NB; b++) {
    for (int l = 0; l < MAXDEPTH; l++) t.path[b][l] = 0;
    int d = BODY_DEPTH[b];
    int k = b;
    for (int l = d - 1; l >= 0; l--) { t.path[b][l] = k; k = BODY_PARENT[k]; }
    t.submask[b] = 0;
  }
  for (int c = 1; c < NB; c++)
    for (int b = 1; b < NB; b++)
      if ((BODY_ANCMASK[c] >> b) & 1u) t.submask[b] |= 1u << c;
  for (int i = 0; i < NV; i++) {
    uint64_t m = 0;
    for (int j = 0; j <= i; j++) {
      int bi = DOF_BODY[i], bj = DOF_BODY[j];
      bool anc = (BODY_ANCMASK[bi] >> bj) & 1u;  // bj is bi or one of its ancestors
      if (anc) m |= (uint64_t)1 << j;
    }
    t.dofanc[i] = m;
    t.dofmask32[i] = t.submask[DOF_BODY[i]];
  }
  for (int b = 0; b < NB; b++) {
    int n = 0;
    for (int i = 0; i < MAXCHAIN; i++) t.chain[b][i] = 0;
    if (b >= 1)
      for (int i = 0; i < NV; i++)
        if ((BODY_ANCMASK[b] >> DOF_BODY[i]) & 1u) t.chain[b][n++] = i;
    t.nchain[b] = n;
  }
  return t;
}

constexpr Tree TREE = make_tree();

constexpr bool check_tree() {
  for (int b = 1; b < NB; b++)
    if (TREE.nchain[b] > MAXCHAIN) return false;
  return NV <= 64 && NB <= 32 && NGEOM <= 64;
}
static_assert(check_tree(), "the kernels assume <= 64 dofs, <= 32 bodies, <= 16 dofs per chain");

// The Hessian's floor-contact prefix sums rely on two orders: each dof's bodies (its body's subtree) are one run of
// body ids (bodies in depth-first order), and the floor pairs (g1 on the world body) come first in pair order,
// sorted by g2's body, so the contacts, compacted in pair order, put the floor contacts in lanes [0, nf) by body.
constexpr bool check_orders() {
  for (int i = 0; i < NV; i++) {
    const uint64_t m = TREE.dofmask32[i];
    if (m == 0 || ((m + (m & (~m + 1))) & m) != 0) return false;
  }
  bool other = false;
  int last = 0;
  for (int p = 0; p < NPAIR; p++) {
    if (GEOM_BODY[PAIR_G1[p]] == 0) {
      if (other || GEOM_BODY[PAIR_G2[p]] < last || GEOM_BODY[PAIR_G2[p]] == 0) return false;
      last = GEOM_BODY[PAIR_G2[p]];
    } else {
      other = true;
    }
  }
  return true;
}
static_assert(check_orders(), "dofs' subtrees as body-id runs; floor pairs first, sorted by body");

// The tree as four root-to-leaf paths below the root body 1 (the two legs; the waist and then either arm), for the
// kernels' path walks (body velocities, twists): group g's step i is body i < 3 ? lo + i : hi + i for i < len, and
// each step's parent is the step before it (the first's the root). The two arm paths share the waist's 3 bodies.
// Checked against the parent table: every hinge body on a path, and every step's dof b + 4 (also past a path's end,
// where the leg groups' walks run on into a sink) a dof.
struct PathGroups { int lo[4], hi[4], len[4]; };  // group g's step i: body i < 3 ? lo + i : hi + i, for i < len
constexpr int PATH_STEPS = 10;
constexpr PathGroups PATHS = {{2, 8, 14, 14}, {2, 8, 14, 21}, {6, 6, 10, 10}};
constexpr int path_body(int g, int i) { return i < 3 ? PATHS.lo[g] + i : PATHS.hi[g] + i; }
constexpr bool check_paths() {  // each a path from the root body 1, together every hinge body; every read in bounds
  bool seen[NB] = {};
  for (int g = 0; g < 4; g++) {
    if (PATHS.len[g] != (g < 2 ? 6 : PATH_STEPS)) return false;  // the walks store steps 6.. of groups 2, 3 only
    for (int i = 0; i < PATH_STEPS; i++) {
      const int b = path_body(g, i);
      if (b < 2 || b + 4 >= NV) return false;
      if (i < PATHS.len[g]) {
        if (BODY_PARENT[b] != (i == 0 ? 1 : path_body(g, i - 1))) return false;
        seen[b] = true;
      }
    }
  }
  for (int b = 2; b < NB; b++)
    if (!seen[b]) return false;
  return true;
}
static_assert(check_paths(), "the G1's root-to-leaf paths: legs 2..7, 8..13; waist 14..16 then arms 17..23, 24..30");

// geom type codes (mjtGeom): plane 0, sphere 2, capsule 3
constexpr int GPLANE = 0, GSPHERE = 2, GCAPSULE = 3;

// pairs as one word: g1 | g2 << 8 | dim << 16 | foot << 20 | class << 21 (0 plane-sphere, 1 sphere-sphere,
// 2 sphere-capsule, 3 capsule-capsule, 4 plane-capsule); g1 has the lower geom type (MuJoCo's collision table order)
constexpr Arr<unsigned, NPAIR> make_pairs() {
  Arr<unsigned, NPAIR> r{};
  for (int p = 0; p < NPAIR; p++) {
    int g1 = PAIR_G1[p], g2 = PAIR_G2[p], t1 = GEOM_TYPE[g1], t2 = GEOM_TYPE[g2];
    unsigned cls = t1 == GPLANE ? (t2 == GSPHERE ? 0u : 4u)
                                : (t1 == GSPHERE && t2 == GSPHERE) ? 1u : (t1 == GSPHERE) ? 2u : 3u;
    r.v[p] = (unsigned)g1 | (unsigned)g2 << 8 | (unsigned)PAIR_DIM[p] << 16 | (unsigned)PAIR_FOOT[p] << 20 | cls << 21;
  }
  return r;
}
constexpr Arr<unsigned, NPAIR> PAIRW = make_pairs();

}  // namespace g1t
