// The forward tape: one record of REC_WORDS float32 words per world and substep (record w * nsub + k), what the
// adjoint needs to differentiate the substep without re-solving it. Own layout (the reference's is tape.py:28-45):
// integer fields are bit-cast into float words.
#pragma once
#include "g1_device.h"

namespace g1k {
constexpr int REC_HDR = 0;        // ncon | nefc << 8 | nlim << 16 | Newton iterations << 24
constexpr int REC_FLAGS = 1;      // the reference's record flags (tape.py:20-23): 4 contacts beyond capacity, 16 rows
                                  // beyond capacity, FLAG_REFACT, FLAG_NONCONV, FLAG_SINGULAR
constexpr int REC_CLAMP = 2;      // 2 words: dofs whose actuator force is at its limit (bit i: dof i)
constexpr int REC_LIMZONE = 4;    // 2 words: dofs whose limit row is in its quadratic zone at a*
constexpr int REC_LIMROW = 6;     // 2 words: dofs with a limit row
constexpr int REC_CZONE = 8;      // 8 words: 4 bits per contact (bit t: pyramid edge t / the normal row quadratic)
constexpr int REC_CON = 16;       // 32 words: contacts in row order, 16 bits each: pair | slot << 9
constexpr int REC_QPOS = 48;      // 36: the substep's input qpos
constexpr int REC_QVEL = 84;      // 35: input qvel
constexpr int REC_ASTAR = 128;    // 35: Newton's final acceleration a*
constexpr int REC_AADV = 164;     // 35: implicitfast's a_adv = (M + h kv)^-1 M a*
constexpr int REC_LH = 200;       // 630: factor L of H = L' L = M + J'DJ at the final zones (packed lower, row-major)
constexpr int REC_LQ = 832;       // 630: factor L of M + h kv = L' L, with the body frames in its off-pattern positions
constexpr int REC_ADJCOST = 1471; // the adjoint's dispatch cost of the substeps up to this one (g1_order.hip): the last
                                  // record's is the world's, which the adjoint's ordering reads
constexpr int REC_WORDS = 1472;
constexpr int COST_BUCKETS = 128; // dispatch costs are buckets 0 .. COST_BUCKETS - 1
constexpr unsigned TAPE_CON_NONE = 0xFFFFu;
constexpr int FLAG_REFACT = 1 << 8;    // the zones changed after the last Newton factorization: H re-factored for the tape
constexpr int FLAG_NONCONV = 1 << 9;   // the Newton iterations ran out before the stopping test held
constexpr int FLAG_SINGULAR = 1 << 10; // a self contact whose geom centres / axes are nearer than SINGULAR_NU
constexpr float SINGULAR_NU = 5e-3f;   // m

// M + h kv has the tree's sparsity and its leaf-first factor keeps it, so the packed lower triangle of L_Q is 0 off the
// dof chains (289 of its 630 positions). The record keeps the 341 entries on the chains at their packed positions; the
// first POSE_WORDS off-pattern positions (in packed order) carry the body frames at the substep's qpos, as the
// forward's FK leaves them in LDS (NB quaternions, then NB positions, 4 words each; a position's fourth word 0), and
// the rest hold 0. The adjoint takes the frames from its copy of L_Q and writes the factor's zeros back.
constexpr int POSE_WORDS = 8 * NB;
struct PoseSlots {
  short pos[POSE_WORDS];  // the packed position of frame word q
};
constexpr PoseSlots make_pose_slots() {
  PoseSlots t{};
  int q = 0;
  for (int i = 0; i < NV; i++)
    for (int j = 0; j <= i; j++)
      if (!((TREE.dofanc[i] >> j) & 1ull) && q < POSE_WORDS) t.pos[q++] = (short)tri(i, j);
  return t;
}
constexpr int off_pattern_positions() {
  int n = 0;
  for (int i = 0; i < NV; i++)
    for (int j = 0; j <= i; j++) n += ((TREE.dofanc[i] >> j) & 1ull) ? 0 : 1;
  return n;
}
static_assert(off_pattern_positions() >= POSE_WORDS, "L_Q's off-pattern positions hold the body frames");
__constant__ inline PoseSlots cPoseSlots = make_pose_slots();
}  // namespace g1k
