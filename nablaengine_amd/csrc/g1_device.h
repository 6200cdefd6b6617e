// Device-side building blocks of the G1 control step shared by the forward and adjoint kernels: model constants in
// constant memory, quaternion / vector helpers, wave64 cross-lane primitives, and the register Cholesky.
//
// Layout convention: one world per wave64 (64 lanes); lane l is dof l (l < 35), body l (l < 31), contact l
// (l < ncon <= 64), geom l (l < 34) depending on the phase. World state that several lanes read lives in LDS.
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "g1_tables.h"

namespace g1k {
using namespace g1t;

constexpr int WL = 64;  // lanes per world: one wave64

template <int N>
constexpr Arr<int, N> to_int(const int (&a)[N]) {
  Arr<int, N> r{};
  for (int i = 0; i < N; i++) r.v[i] = a[i];
  return r;
}

// model constants (float) in constant memory
__constant__ inline Arr<float, NB * 3> cPos = to_float(BODY_POS);
__constant__ inline Arr<float, NB * 4> cQuat = to_float(BODY_QUAT);
__constant__ inline Arr<float, NB * 3> cAxis = to_float(BODY_AXIS);
__constant__ inline Arr<float, NB * 3> cIpos = to_float(BODY_IPOS);
__constant__ inline Arr<float, NB * 4> cIquat = to_float(BODY_IQUAT);
__constant__ inline Arr<float, NB> cMass = to_float(BODY_MASS);
__constant__ inline Arr<float, NB * 3> cInert = to_float(BODY_INERTIA);
__constant__ inline Arr<int, NB> cParent = to_int(BODY_PARENT);
__constant__ inline Arr<int, NB> cDepth = to_int(BODY_DEPTH);
__constant__ inline Arr<int, NB> cQadr = to_int(BODY_QADR);
__constant__ inline Arr<float, NV> cArm = to_float(DOF_ARMATURE);
__constant__ inline Arr<float, NV> cDinvw = to_float(DOF_INVWEIGHT0);
__constant__ inline Arr<float, NV> cKp = to_float(DOF_KP);
__constant__ inline Arr<float, NV> cKv = to_float(DOF_KV);
__constant__ inline Arr<float, NV> cFrclim = to_float(DOF_FRCLIM);
__constant__ inline Arr<float, NV * 2> cRange = to_float(DOF_RANGE);
__constant__ inline Arr<float, NGEOM * 3> cGpos = to_float(GEOM_POS);
__constant__ inline Arr<float, NGEOM * 4> cGquat = to_float(GEOM_QUAT);
__constant__ inline Arr<int, NGEOM> cGbody = to_int(GEOM_BODY);
// Per pair, the words its tests read together, each table one 16-byte load indexed by the pair (where the pair word
// and then loads indexed by its geoms were two dependent round trips): the pair word (PAIRW), the two geoms' bodies
// (b1 | b2 << 8), the bounding radii's sum (the floats added in float) and the second geom's bounding radius; the
// two geoms' radius and half-length (GEOM_SIZE 0 and 1).
struct __align__(16) PairC { unsigned w, bodies; float rb, rb2; };
struct __align__(16) PairSz { float r1, hl1, r2, hl2; };
constexpr Arr<PairC, NPAIR> make_pairc() {
  Arr<PairC, NPAIR> r{};
  for (int p = 0; p < NPAIR; p++) {
    const int g1 = PAIR_G1[p], g2 = PAIR_G2[p];
    const float a = (float)GEOM_RBOUND[g1], b = (float)GEOM_RBOUND[g2];
    r.v[p] = PairC{PAIRW[p], (unsigned)GEOM_BODY[g1] | (unsigned)GEOM_BODY[g2] << 8, a + b, b};
  }
  return r;
}
constexpr Arr<PairSz, NPAIR> make_pairsz() {
  Arr<PairSz, NPAIR> r{};
  for (int p = 0; p < NPAIR; p++) {
    const int g1 = PAIR_G1[p], g2 = PAIR_G2[p];
    r.v[p] = PairSz{(float)GEOM_SIZE[3 * g1], (float)GEOM_SIZE[3 * g1 + 1], (float)GEOM_SIZE[3 * g2],
                    (float)GEOM_SIZE[3 * g2 + 1]};
  }
  return r;
}
// the rows' per-pair constants: the two bodies' inverse weights summed (in float) and the friction coefficient
struct __align__(8) PairRow { float iw, mu; };
constexpr Arr<PairRow, NPAIR> make_pairrow() {
  Arr<PairRow, NPAIR> r{};
  for (int p = 0; p < NPAIR; p++) {
    const float a = (float)BODY_INVWEIGHT0[GEOM_BODY[PAIR_G1[p]]], b = (float)BODY_INVWEIGHT0[GEOM_BODY[PAIR_G2[p]]];
    r.v[p] = PairRow{a + b, (float)PAIR_MU[p]};
  }
  return r;
}
__constant__ inline Arr<PairC, NPAIR> cPair = make_pairc();
__constant__ inline Arr<PairSz, NPAIR> cPairSz = make_pairsz();
__constant__ inline Arr<PairRow, NPAIR> cPairRow = make_pairrow();
// A small table of 5-bit entries as three 64-bit compile-time words (12 entries a word): a lane's entry by selects
// and a shift, with no memory access (a lane-indexed table in constant memory is a global load, and an LDS address
// taken from it waits for that round trip).
struct Packed5 { uint64_t w[3]; };
template <int N>
constexpr Packed5 pack5(const int (&a)[N]) {
  static_assert(N <= 36, "three words of 12 entries");
  Packed5 p{};
  for (int i = 0; i < N; i++) p.w[i / 12] |= (uint64_t)(a[i] & 31) << (5 * (i % 12));
  return p;
}
template <int N>
constexpr bool fits5(const int (&a)[N]) {
  for (int i = 0; i < N; i++)
    if (a[i] < 0 || a[i] > 31) return false;
  return true;
}
static_assert(fits5(GEOM_BODY) && fits5(BODY_PARENT), "5-bit entries");
constexpr Packed5 GEOM_BODY5 = pack5(GEOM_BODY), BODY_PARENT5 = pack5(BODY_PARENT);
template <const Packed5& P>
__device__ __forceinline__ int unpack5(int i) {
  constexpr uint64_t w0 = P.w[0], w1 = P.w[1], w2 = P.w[2];
  const uint64_t x = i < 12 ? w0 : (i < 24 ? w1 : w2);
  const int sh = 5 * (i < 12 ? i : (i < 24 ? i - 12 : i - 24));
  return (int)((x >> sh) & 31u);
}
__device__ __forceinline__ int geom_body(int g) { return unpack5<GEOM_BODY5>(g); }
__device__ __forceinline__ int body_parent(int b) { return unpack5<BODY_PARENT5>(b); }
// a hinge body's joint angle is qpos[b + 5] (the root's 7 coordinates first, one per hinge body in body order)
constexpr bool check_qadr() {
  for (int b = 2; b < NB; b++)
    if (BODY_QADR[b] != b + 5) return false;
  return true;
}
static_assert(check_qadr(), "one hinge per body, in body order");
__constant__ inline Tree cTree = TREE;
// each body's chain (the dofs moving it, ascending) packed one byte a dof into 4 words, 255 past its end (a 16-byte row
// per body: one load each)
struct __align__(16) ChainWords { unsigned w[NB][MAXCHAIN / 4]; };
constexpr ChainWords make_chain_words() {
  ChainWords c{};
  for (int b = 0; b < NB; b++)
    for (int k = 0; k < MAXCHAIN / 4; k++) {
      unsigned wd = 0u;
      for (int e = 0; e < 4; e++)
        wd |= (4 * k + e < TREE.nchain[b] ? (unsigned)TREE.chain[b][4 * k + e] : 255u) << (8 * e);
      c.w[b][k] = wd;
    }
  return c;
}
__constant__ inline ChainWords cChainW = make_chain_words();
static_assert(MAXCHAIN == 16, "a chain row is one 16-byte load");

constexpr float kH = (float)TIMESTEP;
constexpr float kGrav[3] = {(float)GRAVITY[0], (float)GRAVITY[1], (float)GRAVITY[2]};
constexpr float kImpratio = (float)IMPRATIO;
constexpr float kScale = (float)(1.0 / (MEANINERTIA * NV));  // Newton's cost / gradient scale (step.py:1974)
constexpr float kTol = (float)TOLERANCE;

// ------------------------------------------------------------------------------------------------ lane helpers
// The lane index as a value the compiler cannot see through: lane-dependent addresses and masks computed from it stay
// where they are used. Without this, loop-invariant code motion hoists them out of the solver's loops (dozens of
// per-lane addresses and lane masks), and the register allocator spills them to scratch, putting a scratch reload on
// every step of the factor / solve chains.
__device__ __forceinline__ int opaque_lane(int lane) {
  asm volatile("" : "+v"(lane));
  return lane;
}
__device__ __forceinline__ float rdl(float x, int k) {  // lane k's x, k uniform
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), k));
}
__device__ __forceinline__ int rdli(int x, int k) { return __builtin_amdgcn_readlane(x, k); }
__device__ __forceinline__ unsigned long long ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int prefix_count(unsigned long long m, int lane) {  // set bits of m below lane
  return __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
}
// Sum over the wave's 64 lanes by DPP: an inclusive scan within each row of 16 lanes (row_shr 1, 2, 4, 8), then
// row_bcast 15 / 31 carry the row totals up, so lane 63 holds the total (T3 + T2) + (T1 + T0); v_readlane broadcasts
// it as a wave-uniform scalar. A fixed order on every call (bitwise deterministic); lanes without a DPP source add +0.
// The two broadcasts run on every row (row mask 0xf): only lanes 31 and 63 are read after them, and what the other
// rows add does not reach those lanes, while a row mask other than 0xf keeps each step from folding into one
// v_add_f32_dpp (a zero move, a v_mov_b32_dpp and an add instead). The prefix scans (wscan_nw) need the masks: with
// row 0 enabled, row_bcast 15 changes row 0 too (measured: the scan's first lanes went wrong).
#define G1_DPP(x, ctrl, rmask) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), (ctrl), (rmask), 0xf, false))
// A reduction's input as an opaque value: its first step then stays one v_add_f32_dpp, where otherwise a product
// input is contracted with the first add into an FMA of the DPP-moved value (a zero move, a v_mov_b32_dpp and the FMA)
__device__ __forceinline__ float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float wsum(float v) {
  v = opaque(v);
  v += G1_DPP(v, 0x111, 0xf);  // row_shr:1
  v += G1_DPP(v, 0x112, 0xf);  // row_shr:2
  v += G1_DPP(v, 0x114, 0xf);  // row_shr:4
  v += G1_DPP(v, 0x118, 0xf);  // row_shr:8
  v += G1_DPP(v, 0x142, 0xf);  // row_bcast:15: lane 31 = T1 + T0, lane 63 = T3 + T2
  v += G1_DPP(v, 0x143, 0xf);  // row_bcast:31: lane 63 += lane 31
  return rdl(v, 63);
}
__device__ __forceinline__ float2 wsum2(float a, float b) {
  a = opaque(a);
  b = opaque(b);
  a += G1_DPP(a, 0x111, 0xf); b += G1_DPP(b, 0x111, 0xf);
  a += G1_DPP(a, 0x112, 0xf); b += G1_DPP(b, 0x112, 0xf);
  a += G1_DPP(a, 0x114, 0xf); b += G1_DPP(b, 0x114, 0xf);
  a += G1_DPP(a, 0x118, 0xf); b += G1_DPP(b, 0x118, 0xf);
  a += G1_DPP(a, 0x142, 0xf); b += G1_DPP(b, 0x142, 0xf);
  a += G1_DPP(a, 0x143, 0xf); b += G1_DPP(b, 0x143, 0xf);
  return make_float2(rdl(a, 63), rdl(b, 63));
}
// the wave totals of n values at once (a masked sum passes 0 on the lanes outside the set): wsum's DPP steps with
// the n chains interleaved, so every step's n instructions are independent of each other
template <int N>
__device__ __forceinline__ void wsum_n(float* x) {
#pragma unroll
  for (int e = 0; e < N; e++) x[e] = opaque(x[e]);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x111, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x112, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x114, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x118, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x142, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x143, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] = rdl(x[e], 63);
}
// bitwise OR over the wave's 64 lanes (wsum's DPP steps with OR; lanes without a source OR in 0)
__device__ __forceinline__ unsigned wor(unsigned v) {
#define G1_DPPI(x, ctrl, rmask) (unsigned)__builtin_amdgcn_update_dpp(0, (int)(x), (ctrl), (rmask), 0xf, false)
  v |= G1_DPPI(v, 0x111, 0xf);
  v |= G1_DPPI(v, 0x112, 0xf);
  v |= G1_DPPI(v, 0x114, 0xf);
  v |= G1_DPPI(v, 0x118, 0xf);
  v |= G1_DPPI(v, 0x142, 0xf);
  v |= G1_DPPI(v, 0x143, 0xf);
#undef G1_DPPI
  return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}
// wsum_n over the first `width` lanes only (the other lanes' values are not read): 4 DPP steps for 16 lanes, 5 for
// 32, 6 for 64; width uniform. The same fixed order on every call with the same width.
template <int N>
__device__ __forceinline__ void wsum_nw(float* x, int width) {
#pragma unroll
  for (int e = 0; e < N; e++) x[e] = opaque(x[e]);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x111, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x112, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x114, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x118, 0xf);
  if (width <= 16) {
#pragma unroll
    for (int e = 0; e < N; e++) x[e] = rdl(x[e], 15);
    return;
  }
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x142, 0xf);
  if (width <= 32) {
#pragma unroll
    for (int e = 0; e < N; e++) x[e] = rdl(x[e], 31);
    return;
  }
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x143, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] = rdl(x[e], 63);
}
// inclusive prefix sums of n values over the first `width` lanes (wsum_nw's DPP steps without the broadcast): lane
// l < width holds the sum over lanes 0..l; lanes past width hold partial sums of their own rows
template <int N>
__device__ __forceinline__ void wscan_nw(float* x, int width) {
#pragma unroll
  for (int e = 0; e < N; e++) x[e] = opaque(x[e]);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x111, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x112, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x114, 0xf);
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x118, 0xf);
  if (width <= 16) return;
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x142, 0xa);
  if (width <= 32) return;
#pragma unroll
  for (int e = 0; e < N; e++) x[e] += G1_DPP(x[e], 0x143, 0xc);
}
// lane src's x (src per lane; ds_bpermute: the LDS unit's crossbar, no memory access)
__device__ __forceinline__ float lane_of(float x, int src) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(x)));
}
__device__ __forceinline__ int wsumi(int v) {  // small counts: exact in float
  return (int)wsum((float)v);
}
// exclusive prefix sum and wave total of a count 0 <= v < 2^NBITS, bit by bit from ballots (each bit's lanes below
// this one by v_mbcnt, the total by a scalar popcount): no cross-lane data movement, exact
template <int NBITS>
__device__ __forceinline__ int wscan_bits(int v, int lane, int* total) {
  int r = 0, t = 0;
#pragma unroll
  for (int b = 0; b < NBITS; b++) {
    const unsigned long long m = ballot((v >> b) & 1);
    r += prefix_count(m, lane) << b;
    t += __popcll(m) << b;
  }
  *total = t;
  return r;
}
// The LDS barrier of a workgroup of one wave (every kernel that calls it has 64 threads): a wave's LDS instructions
// execute in issue order, so a lane's LDS write is seen by every later LDS read of the wave with no hardware barrier
// and no wait for the outstanding LDS operations (__syncthreads' workgroup fence drains them). Only the compiler
// must not move memory accesses across this point. LDS written by the memory unit (global_load_lds) is not ordered
// this way: its readers wait for it explicitly (s_waitcnt vmcnt).
__device__ __forceinline__ void wsync() { asm volatile("" ::: "memory"); }

// x with lane L's value replaced by 0 (v_writelane_b32 with the lane an inline constant: one instruction, no compare)
template <int L>
__device__ __forceinline__ float zero_lane(float x) {
  asm("v_writelane_b32 %0, 0, %1" : "+v"(x) : "n"(L));
  return x;
}
// f(std::integral_constant<int, I>) for I = A, A + S, ... while I != B (unrolled, I a compile-time constant)
template <int A, int B, int S, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (A != B) {
    f(std::integral_constant<int, A>{});
    static_for<A + S, B, S>(f);
  }
}

// Phase profile (a G1_PROFILE build only): per world, s_memtime cycles of the forward's phases summed over the substeps
// (lane 0's clock at phase ends, after a barrier), written to g_prof[world][phase] for the first PROF_WORLDS worlds
// and read by dk_prof_read. The production build compiles every mark to nothing.
enum { PH_SMOOTH = 0, PH_COLLIDE, PH_ROWS, PH_NINIT, PH_HESS, PH_FACTOR, PH_SOLVE, PH_LSEARCH, PH_UPDATE, PH_GRAD,
       PH_IMPLICIT, PH_TAPE, PH_ITERS, PH_LSEVAL, PH_DENSE, PH_LSJV, PH_LSMV, PH_HK, PH_HCOMP, PH_HROWS, PH_T0, PH_T1, PH_HWID, PH_SFK, PH_SBF, PH_SSUB, PH_SCRBA, NPHASE };
constexpr int PROF_WORLDS = 16384;
#ifdef G1_PROFILE
__device__ inline unsigned long long g_prof[PROF_WORLDS][NPHASE];
#define PROF_DECL unsigned long long prof_t = __builtin_amdgcn_s_memtime(); unsigned long long prof_acc[NPHASE] = {0};
#define PROF_MARK(acc, t, k) do { wsync(); unsigned long long t_ = __builtin_amdgcn_s_memtime(); (acc)[k] += t_ - (t); (t) = t_; } while (0)
#else
#define PROF_DECL
#define PROF_MARK(acc, t, k) do { } while (0)
#endif

// The chain table of a world (in LDS, built at kernel start by chain_table): per body, the dofs moving it in
// ascending order, one byte each in 4 words, 255 past the chain's end. chain_dof reads entry t of a row: the dof,
// clamped to a valid one past the end (with *on false).
__device__ __forceinline__ int chain_dof(const unsigned* ch, int t, bool* on) {
  const unsigned d = (ch[t >> 2] >> (8 * (t & 3))) & 255u;
  *on = d != 255u;
  return d != 255u ? (int)d : 0;
}
__device__ __forceinline__ void chain_table(unsigned (*chain)[MAXCHAIN / 4], int lane) {
  const uint4 v = reinterpret_cast<const uint4*>(cChainW.w)[lane < NB ? lane : 0];  // every lane's load in bounds
  if (lane < NB) {
    chain[lane][0] = v.x;
    chain[lane][1] = v.y;
    chain[lane][2] = v.z;
    chain[lane][3] = v.w;
  }
}

// ------------------------------------------------------------------------------------------------ 3D helpers
__device__ __forceinline__ void qmul(const float* a, const float* b, float* o) {
  float w = a[0] * b[0] - a[1] * b[1] - a[2] * b[2] - a[3] * b[3];
  float x = a[0] * b[1] + a[1] * b[0] + a[2] * b[3] - a[3] * b[2];
  float y = a[0] * b[2] - a[1] * b[3] + a[2] * b[0] + a[3] * b[1];
  float z = a[0] * b[3] + a[1] * b[2] - a[2] * b[1] + a[3] * b[0];
  o[0] = w; o[1] = x; o[2] = y; o[3] = z;
}
__device__ __forceinline__ void qrot(const float* q, const float* v, float* o) {  // o = q v q^-1
  float tx = 2.f * (q[2] * v[2] - q[3] * v[1]), ty = 2.f * (q[3] * v[0] - q[1] * v[2]);
  float tz = 2.f * (q[1] * v[1] - q[2] * v[0]);
  o[0] = v[0] + q[0] * tx + q[2] * tz - q[3] * ty;
  o[1] = v[1] + q[0] * ty + q[3] * tx - q[1] * tz;
  o[2] = v[2] + q[0] * tz + q[1] * ty - q[2] * tx;
}
__device__ __forceinline__ void qrot_inv(const float* q, const float* v, float* o) {
  float qc[4] = {q[0], -q[1], -q[2], -q[3]};
  qrot(qc, v, o);
}
__device__ __forceinline__ void cross(const float* a, const float* b, float* o) {
  float x = a[1] * b[2] - a[2] * b[1], y = a[2] * b[0] - a[0] * b[2], z = a[0] * b[1] - a[1] * b[0];
  o[0] = x; o[1] = y; o[2] = z;
}
__device__ __forceinline__ float dot3(const float* a, const float* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; }

// ------------------------------------------------------------------------------------------------ LTL factorization
// A = L' L with L lower triangular, eliminated leaf-first (k = NV-1 .. 0), as MuJoCo factors M: with parents before
// children in the dof order, row k of L is nonzero only at k's ancestor dofs (no fill-in) for a matrix with the
// tree's sparsity (M, and H = M + J'DJ when no contact couples two robot bodies). Lane j holds column j of the lower
// triangle in registers (c[m] = A[m][j], m >= j), so row k's entries L[k][j] are lane-local and L[k][m] is one
// v_readlane away: step k is one pivot and, per ancestor m of k, a broadcast and one FMA on every lane.
// SPARSE = false visits every m < k (the dense factor of a matrix with cross-branch entries). In place in Lp (packed
// lower, TRI layout, followed by the 64-float sink at LSINK). Lane j's registers c[m] for m < j hold other entries of the matrix (loaded from in-bounds
// addresses, not zeroed): they are updated from one another only, never broadcast (a broadcast reads lane m's c[k],
// k > m) and never stored, so the valid entries do not depend on them.
// The fill that contacts between robot bodies of the common kinds add to the tree's sparsity: a leg against the
// waist or its own arm, or the two legs. H gains entries between the non-shared dofs of the two chains, and
// eliminating leaf-first spreads them to the rows of the later (higher) chain and of the shared ancestors in
// between: rows 18-27 gain columns 6-11 (left leg against waist / left arm), rows 18-20 and 28-34 gain 12-17 (right
// leg against waist / right arm), rows 12-17 gain 6-11 (the legs; also the fill of both arm kinds together, coupled
// through the waist). Other kinds use the dense routine.
__host__ __device__ constexpr uint64_t fill_bits(int k) {
  uint64_t m = 0;
  if (k >= 18 && k <= 27) m |= 0xFC0ull;                                 // columns 6..11
  if ((k >= 18 && k <= 20) || (k >= 28 && k <= 34)) m |= 0x3F000ull;     // columns 12..17
  if (k >= 12 && k <= 17) m |= 0xFC0ull;                                 // columns 6..11
  return m;
}
static_assert(NV == 35, "the fill rows are the G1's dof ranges");
static_assert(NV * (NV - 1) / 2 + 63 < LSINK + 64, "the unmasked row stores of the last row stay in the factor buffer");

// The hinge dofs are eliminated first; each would update the 6 x 6 root block (rows and columns 0..5) by the outer
// product of its row's root part, 6 broadcasts and FMAs a step that only lanes 0..5 use (174 of the tree pattern's 306
// pairs). These updates are summed instead as one product on the matrix cores, the Schur complement
// D = X' X with X[k][r] = L[k][r] (hinge rows k = 6..34, root columns r < 6; 29 rows padded to 32): 8 steps of
// v_mfma_f32_16x16x4f32, lane l giving A[l % 16][k'] = B[k'][l % 16] = X[6 + k'][l % 16] for k' = 4 t + l / 16 (read
// back from the factor's hinge rows, stored first), lane l holding D[4 (l / 16) + e][l % 16]. Then the root block is
// eliminated as before.
// The elimination order. Any order that eliminates a dof after all its descendants gives the same factor; for the
// tree's pattern the four branches below the root and waist (right arm 34..28, left arm 27..21, right leg 17..12, left
// leg 11..6) are independent chains, interleaved two at a time so that consecutive steps do not wait on each other;
// then the waist (20..18) and the root (5..0). With the self-contact fill (rows 18..27 and 12..17 gain leg columns) and
// dense, the descending order.
typedef float mfma4 __attribute__((ext_vector_type(4)));
constexpr int NROOT = 6;  // the free joint's dofs: every other dof's ancestors
struct Order { int v[NV]; };
constexpr Order elim_order(bool tree) {
  Order o{};
  int n = 0;
  if (tree) {
    for (int t = 0; t < 7; t++) { o.v[n++] = 34 - t; o.v[n++] = 27 - t; }
    for (int t = 0; t < 6; t++) { o.v[n++] = 17 - t; o.v[n++] = 11 - t; }
    for (int k = 20; k >= 18; k--) o.v[n++] = k;
    for (int k = NROOT - 1; k >= 0; k--) o.v[n++] = k;
  } else {
    for (int k = NV - 1; k >= 0; k--) o.v[n++] = k;
  }
  return o;
}
constexpr bool order_ok(const Order& o) {  // a permutation, each dof after all of its descendants (tree pattern)
  bool seen[NV] = {};
  for (int s = 0; s < NV; s++) {
    const int k = o.v[s];
    if (k < 0 || k >= NV || seen[k]) return false;
    for (int d = k + 1; d < NV; d++)
      if (((TREE.dofanc[d] >> k) & 1ull) && !seen[d]) return false;
    seen[k] = true;
  }
  return true;
}
static_assert(order_ok(elim_order(true)) && order_ok(elim_order(false)), "elimination orders");
static_assert(((TREE.dofanc[34] >> 18) & 1) != 0 && ((TREE.dofanc[27] >> 18) & 1) != 0 &&
              ((TREE.dofanc[27] >> 28) & 1) == 0 && ((TREE.dofanc[17] >> 6) & 1) == 0,
              "the G1's branches: arms 21..27 / 28..34 below the waist, legs 6..11 / 12..17");

// The hinge dofs are eliminated first; each would update the 6 x 6 root block (rows and columns 0..5) by the outer
// product of its row's root part, 6 broadcasts and FMAs a step that only lanes 0..5 use (174 of the tree pattern's 306
// pairs). These updates are summed instead as one product on the matrix cores, the Schur complement
// D = X' X with X[k][r] = L[k][r] (hinge rows k = 6..34, root columns r < 6; 29 rows padded to 32): 8 steps of
// v_mfma_f32_16x16x4f32, lane l giving A[l % 16][k'] = B[k'][l % 16] = X[6 + k'][l % 16] for k' = 4 t + l / 16 (read
// back from the factor's hinge rows, stored first), lane l holding D[4 (l / 16) + e][l % 16]. Then the root block is
// eliminated as before.
template <int PATTERN>  // 0: the tree's sparsity; 1: with the common self-contact fill; 2: every pair
__device__ __forceinline__ void ltl_factor(float* Lp, int lane_) {
  constexpr bool SPARSE = PATTERN < 2;
  constexpr Order ORD = elim_order(PATTERN == 0);
  const int lane = opaque_lane(lane_);
  // column j = lane of the lower triangle: A[m][j] = col[tri(m, 0)] for m >= j; every lane's address inside the
  // matrix (lanes past the column select 0), all the loads issued before the elimination
  const float* col = Lp + (lane < NV ? lane : NV - 1);
  float c[NV];
#pragma unroll
  for (int m = 0; m < NV; m++) c[m] = col[tri(m, 0)];
  static_for<0, NV, 1>([&](auto sc) {
    constexpr int k = ORD.v[decltype(sc)::value];
    if constexpr (k == NROOT - 1) {
      // the hinge rows are final: store them, row m at tri(m, 0) + lane on every lane, rows in increasing order. A
      // lane past the row (lane > m, or no column) writes into a later row's slots, which that row's own store
      // overwrites afterwards (a wave's LDS stores land in program order), or for the last row into the padding and
      // the sink (tri(34, 0) + 63 < LSINK + 64): no address arithmetic per store. Then the root block's Schur
      // complement on the matrix cores
      float* rowbase = Lp + lane;
#pragma unroll
      for (int m = NROOT; m < NV; m++) rowbase[tri(m, 0)] = c[m];
      wsync();
      const int r = lane & 15, q = lane >> 4;
      mfma4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const int kk = NROOT + 4 * t + q;
        const bool in = r < NROOT && kk < NV;
        const float x = Lp[tri(in ? kk : NV - 1, in ? r : 0)];
        const float xv = in ? x : 0.f;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xv, xv, acc, 0, 0, 0);
      }
      // lane j < 6: D[0..3][j] in its own acc, D[4][j] and D[5][j] in lane j + 16's acc[0], acc[1]
      const float d4 = __shfl(acc[0], lane + 16, 64), d5 = __shfl(acc[1], lane + 16, 64);
      c[0] -= acc[0]; c[1] -= acc[1]; c[2] -= acc[2]; c[3] -= acc[3]; c[4] -= d4; c[5] -= d5;
    }
    // the pivot, floored at 1e-30 on the lanes before the broadcast: one v_max on a vector register (a max of the
    // broadcast scalar would first canonicalize it, a second instruction on the pivot's dependency chain)
    const float d = rdl(fmaxf(c[k], 1e-30f), k);
    // L[k][j] = A[k][j] / sqrt(d) on lane j; on lane k itself d / sqrt(d) = L[k][k] (the hardware 1/sqrt, 1 ulp)
    c[k] *= __builtin_amdgcn_rsqf(d);
    // every broadcast of the step first, then the updates: a v_readlane's SGPR is not read by the next instruction;
    // a hinge step's updates of the root rows are left to the Schur complement above
    constexpr int m0 = k >= NROOT ? NROOT : 0;
    float bc[NV];
#pragma unroll
    for (int m = m0; m < k; m++)
      if (!SPARSE || (((TREE.dofanc[k] | (PATTERN ? fill_bits(k) : 0ull)) >> m) & 1ull)) bc[m] = rdl(c[k], m);
#pragma unroll
    for (int m = m0; m < k; m++)  // A[m][j] -= L[k][j] L[k][m] (the pattern's test at compile time)
      if (!SPARSE || (((TREE.dofanc[k] | (PATTERN ? fill_bits(k) : 0ull)) >> m) & 1ull)) c[m] = fmaf(-c[k], bc[m], c[m]);
  });
  // lane j stores column j's root rows m >= j; the other lanes store into their sink slot (the hinge rows are stored
  // already: no write past a root row may reach them)
#pragma unroll
  for (int m = 0; m < NROOT; m++) Lp[m >= lane && lane < NV ? tri(m, lane) : LSINK + lane] = c[m];
}

// x = A^-1 b for A = L' L (ltl_factor), b and x on lane i < NV: L' y = b leaf-first (reads row i of L: lane k takes
// L[i][k]), then L x = y root-first (lane k takes L[k][j]); one v_readlane per pivot broadcasts the solved entry.
// Each lane keeps its running value scaled by 1 / L[lane][lane], so the value broadcast at step i is already the
// solved entry, and the entries it is multiplied with are pre-scaled the same way and zeroed on lanes that take no
// update: a step is one v_readlane and one FMA on the dependency chain. The factor entries come from one base address
// per pass plus the step's immediate offset (no address arithmetic per step, and every load independent of the
// chain); the lanes that take no update read an entry of L too (always inside it) and select 0 instead.
__device__ __forceinline__ float ltl_solve(const float* Lp, float b, int lane_) {
  const int lane = opaque_lane(lane_);
  const int r = lane < NV ? lane : NV - 1;
  const float dself = lane < NV ? 1.f / Lp[tri(r, r)] : 0.f;
  float z = b * dself;  // (b - sum of the solved descendants' terms) / L[lane][lane]
  // pass 1, step i: lanes r < i take L[i][r] = col[tri(i, 0)] (every lane's address inside L); the lanes at or past
  // i take 0 through dm, their copy of dself zeroed one lane a step (v_writelane: no compare and select per step)
  const float* col = Lp + r;
  float lv[NV];
#pragma unroll
  for (int i = NV - 1; i >= 1; i--) lv[i] = col[tri(i, 0)];
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the chain
  float dm = dself;
  static_for<NV - 1, 0, -1>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    dm = zero_lane<i>(dm);  // lane i solves at this step
    z = fmaf(-(lv[i] * dm), rdl(z, i), z);
  });
  // z = y; root-first: x[lane] = (y[lane] - sum_{k < lane} L[lane][k] x[k]) / L[lane][lane]
  // pass 2, step k: lanes r > k take L[r][k] = row[k] (every lane's address inside L); lanes up to k take 0 (dm)
  z *= dself;
  const float* row = Lp + tri(r, 0);
#pragma unroll
  for (int k = 0; k < NV - 1; k++) lv[k] = row[k];
  __builtin_amdgcn_sched_barrier(0);
  dm = dself;
  static_for<0, NV - 1, 1>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    dm = zero_lane<k>(dm);  // lane k is solved at this step
    z = fmaf(-(lv[k] * dm), rdl(z, k), z);
  });
  return z;
}

// ltl_solve for two right-hand sides at once (the step Jacobian's cotangent sets): every step's broadcast and FMA
// for each, the coefficients shared, so each result is bitwise ltl_solve's for its right-hand side; the two chains
// are independent, so each step's latency is taken once for both
__device__ __forceinline__ void ltl_solve2(const float* Lp, float b0, float b1, int lane_, float* x0, float* x1) {
  const int lane = opaque_lane(lane_);
  const int r = lane < NV ? lane : NV - 1;
  const float dself = lane < NV ? 1.f / Lp[tri(r, r)] : 0.f;
  float z0 = b0 * dself, z1 = b1 * dself;
  const float* col = Lp + r;
  float lv[NV];
#pragma unroll
  for (int i = NV - 1; i >= 1; i--) lv[i] = col[tri(i, 0)];
  __builtin_amdgcn_sched_barrier(0);
  float dm = dself;
  static_for<NV - 1, 0, -1>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    dm = zero_lane<i>(dm);
    const float cf = -(lv[i] * dm);
    z0 = fmaf(cf, rdl(z0, i), z0);
    z1 = fmaf(cf, rdl(z1, i), z1);
  });
  z0 *= dself;
  z1 *= dself;
  const float* row = Lp + tri(r, 0);
#pragma unroll
  for (int k = 0; k < NV - 1; k++) lv[k] = row[k];
  __builtin_amdgcn_sched_barrier(0);
  dm = dself;
  static_for<0, NV - 1, 1>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    dm = zero_lane<k>(dm);
    const float cf = -(lv[k] * dm);
    z0 = fmaf(cf, rdl(z0, k), z0);
    z1 = fmaf(cf, rdl(z1, k), z1);
  });
  *x0 = z0;
  *x1 = z1;
}

}  // namespace g1k
