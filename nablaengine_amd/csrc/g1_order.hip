// World ordering for the forward and adjoint launches: heaviest worlds first.
//
// A launch of B worlds runs them one wave64 each, and the hardware dispatches workgroups in blockIdx order as slots
// free up. The kernel time is the makespan: a heavy world (many contacts, contacts between two robot bodies) that
// starts late finishes late. Dispatching worlds in decreasing cost is the longest-processing-time-first schedule.
// The reference does the same for its split kernels (host.py:236-264 dk_order_world, row-count buckets).
//
// The cost is estimated per world before the launch, in the caller's work buffer:
//   forward  contacts at the input state (the main kernel's broadphase and narrowphase): their constraint rows, and a
//            weight per contact between two robot bodies (each makes the Newton Hessian dense);
//   adjoint  the taped forward's contacts per substep: their count, the robot bodies they touch, the contacts between
//            two robot bodies and the primitive classes present, summed by the forward itself into its records
//            (REC_ADJCOST, g1_forward.hip), so the adjoint's order needs no pass over the tape of its own.
// Then one workgroup buckets the costs (LDS histogram, descending prefix) into the permutation the main kernel reads
// as blockIdx.x -> world. Results do not depend on the order: every world's computation is the same wherever and
// whenever it runs, so the permutation only moves work in time (its order inside a bucket is free).
//
// A batch that fits the GPU's resident slots at once (8 worlds per CU in both kernels) starts every world at the
// launch: no world waits for a slot, so the order cannot shorten the makespan, and the order's two launches are
// skipped (index order).
#include <atomic>

#include "g1_device.h"
#include "g1_collide.h"
#include "g1_tape.h"

namespace g1k {

constexpr int NBKT = COST_BUCKETS;

// worlds resident at once on the current device: 8 per CU (the forward's and the adjoint's LDS and VGPRs), the CU
// count queried once per device (host threads may race to store the same value: atomics); 0 when the query fails
// (the order is then always computed)
constexpr int WORLDS_PER_CU = 8, MAX_DEVICES = 64;
int resident_worlds() {
  static std::atomic<int> per_dev[MAX_DEVICES];  // 0: not queried yet
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return 0;
  int n = per_dev[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
    n = WORLDS_PER_CU * cus;
    per_dev[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// contacts at the input state: FK of body poses (each body lane walks its chain from the root), geom poses, the main
// kernel's broadphase and narrowphase (the same code); the cost counts the contacts' constraint rows (4 per pyramid
// contact, 1 per frictionless one) plus a weight per contact between two robot bodies (each makes the Newton Hessian
// dense and adds its outer products)
constexpr int COST_SELF = 12;
__global__ __launch_bounds__(64) void k_cost_fwd(int nw, const float* __restrict__ qpos, int* __restrict__ cost) {
  __shared__ float q[40];
  __shared__ float bq[NB][4], bx[NB][4];
  __shared__ float hl[NB][8];  // each hinge body's local rotation (quat (x) hinge rotation) and offset in its parent
  __shared__ float gx[NGEOM][4], gq[NGEOM][4];
  __shared__ unsigned short cand[NPAIR + 2];
  const int lane = threadIdx.x, w = blockIdx.x;
  if (w >= nw) return;
  if (lane < NQ) q[lane] = qpos[(size_t)w * NQ + lane];
  wsync();
  if (lane >= 2 && lane < NB) {  // one hinge rotation per body, then the chain walks use products only
    float sn, cs;
    sincosf(0.5f * q[lane + 5], &sn, &cs);
    const float qb[4] = {cQuat[4 * lane], cQuat[4 * lane + 1], cQuat[4 * lane + 2], cQuat[4 * lane + 3]};
    const float ha[4] = {cs, sn * cAxis[3 * lane], sn * cAxis[3 * lane + 1], sn * cAxis[3 * lane + 2]};
    qmul(qb, ha, hl[lane]);
    for (int c = 0; c < 3; c++) hl[lane][4 + c] = cPos[3 * lane + c];
  }
  wsync();
  if (lane < NB) {
    float Q[4], X[3];
    {
      const float n = rsqrtf(q[3] * q[3] + q[4] * q[4] + q[5] * q[5] + q[6] * q[6]);
      for (int k = 0; k < 4; k++) Q[k] = q[3 + k] * n;
      for (int k = 0; k < 3; k++) X[k] = q[k];
    }
    const int depth = cDepth[lane];
    int pth[MAXDEPTH];  // the path's bodies, all loaded before the walk
#pragma unroll
    for (int l = 1; l < MAXDEPTH; l++) pth[l] = cTree.path[lane][l];
#pragma unroll
    for (int l = 1; l < MAXDEPTH; l++) {
      if (l < depth) {
        const float* h = hl[pth[l]];
        const float ql[4] = {h[0], h[1], h[2], h[3]}, pb[3] = {h[4], h[5], h[6]};
        float t[3], q1[4];
        qrot(Q, pb, t);
        for (int c = 0; c < 3; c++) X[c] += t[c];
        qmul(Q, ql, q1);
        for (int c = 0; c < 4; c++) Q[c] = q1[c];
      }
    }
    for (int k = 0; k < 4; k++) bq[lane][k] = lane == 0 ? (k == 0 ? 1.f : 0.f) : Q[k];
    for (int k = 0; k < 3; k++) bx[lane][k] = lane == 0 ? 0.f : X[k];
  }
  wsync();
  if (lane < NGEOM) {
    const int b = cGbody[lane];
    float t[3];
    const float qb[4] = {bq[b][0], bq[b][1], bq[b][2], bq[b][3]};
    const float gp[3] = {cGpos[3 * lane], cGpos[3 * lane + 1], cGpos[3 * lane + 2]};
    const float gqq[4] = {cGquat[4 * lane], cGquat[4 * lane + 1], cGquat[4 * lane + 2], cGquat[4 * lane + 3]};
    qrot(qb, gp, t);
    for (int k = 0; k < 3; k++) gx[lane][k] = bx[b][k] + t[k];
    qmul(qb, gqq, gq[lane]);
  }
  wsync();
  float fn[3];
  {
    const float q0[4] = {gq[0][0], gq[0][1], gq[0][2], gq[0][3]};
    zaxis(q0, fn);
  }
  const int ncand = broadphase(gx, fn, cand, lane);
  wsync();
  int c = 0;
  for (int c0 = 0; c0 < ncand; c0 += WL) {
    if (c0 + lane < ncand) {
      const int pr = cand[c0 + lane];
      Cand o;
      collide_pair(gx, gq, pr, o);
      const unsigned pw = cPair[pr].w;
      const unsigned cls = (pw >> 21) & 7u;
      const int n = (int)o.has[0] + (int)o.has[1];
      const int rows = ((pw >> 16) & 15u) == 3u ? 4 : 1;
      c += n * (cls == 0u || cls == 4u ? rows : rows + COST_SELF);
    }
  }
  const int tot = wsumi(c) / 2;
  if (lane == 0) cost[w] = tot < NBKT ? tot : NBKT - 1;
}

// one workgroup of ORDER_THREADS: histogram of the costs, descending prefix (a suffix scan on one wave), scatter
// (perm[slot] = world, heaviest first). Each thread takes its worlds ORDER_LOADS at a time, every load issued before
// the first is used (one memory round trip per batch, not per world).
constexpr int ORDER_THREADS = 1024, ORDER_LOADS = 8;
// cost[w * cstride] is world w's bucket
__global__ __launch_bounds__(ORDER_THREADS) void k_order(int nw, const int* __restrict__ cost, size_t cstride,
                                                         int* __restrict__ perm) {
  static_assert(NBKT == 128, "the bucket prefix: two buckets per lane of one wave");
  __shared__ int cnt[NBKT], cur[NBKT];
  const int t = threadIdx.x;
  if (t < NBKT) cnt[t] = 0;
  __syncthreads();
  // the costs of this thread's worlds (the first ORDER_LOADS kept in registers for the scatter: all of them up to
  // ORDER_LOADS x ORDER_THREADS worlds)
  int c0[ORDER_LOADS];
  for (int w0 = t; w0 < nw; w0 += ORDER_LOADS * ORDER_THREADS) {
    int c[ORDER_LOADS];
#pragma unroll
    for (int u = 0; u < ORDER_LOADS; u++) {
      const int w = w0 + u * ORDER_THREADS;
      c[u] = w < nw ? cost[w * cstride] : -1;
    }
#pragma unroll
    for (int u = 0; u < ORDER_LOADS; u++) {
      if (c[u] >= 0) atomicAdd(&cnt[c[u]], 1);
      if (w0 == t) c0[u] = c[u];
    }
  }
  __syncthreads();
  // descending exclusive prefix: cur[b] = the worlds in buckets above b. Lane l of the first wave takes buckets 2l
  // and 2l + 1; a suffix scan of their sums over the lanes (6 shuffle steps)
  if (t < 64) {
    const int lo = cnt[2 * t], hi = cnt[2 * t + 1], sum = lo + hi;
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_down(incl, o, 64);
      if (t + o < 64) incl += v;
    }
    const int above = incl - sum;
    cur[2 * t + 1] = above;
    cur[2 * t] = above + hi;
  }
  __syncthreads();
  for (int w0 = t; w0 < nw; w0 += ORDER_LOADS * ORDER_THREADS) {
    int c[ORDER_LOADS];
#pragma unroll
    for (int u = 0; u < ORDER_LOADS; u++) {
      const int w = w0 + u * ORDER_THREADS;
      c[u] = w0 == t ? c0[u] : (w < nw ? cost[w * cstride] : -1);
    }
#pragma unroll
    for (int u = 0; u < ORDER_LOADS; u++)
      if (c[u] >= 0) perm[atomicAdd(&cur[c[u]], 1)] = w0 + u * ORDER_THREADS;
  }
}
static_assert(NBKT <= ORDER_THREADS, "one thread clears each bucket");

// work buffer: perm (nw int32), cost (nw int32)
size_t order_work_bytes(int nw) { return nw > 0 ? ((8 * (size_t)nw + 255) & ~(size_t)255) : 0; }

int launch_order_fwd(hipStream_t st, int nw, const float* qpos, void* work) {
  int* perm = (int*)work;
  int* cost = perm + nw;
  hipLaunchKernelGGL(k_cost_fwd, dim3(nw), dim3(64), 0, st, nw, qpos, cost);
  hipLaunchKernelGGL(k_order, dim3(1), dim3(ORDER_THREADS), 0, st, nw, (const int*)cost, (size_t)1, perm);
  return (int)hipGetLastError();
}

// the adjoint's costs gathered from the tape into the work buffer, one thread per world: the words lie a world's
// tape apart (23.5 KB at 4 substeps), and the ordering workgroup's 1024 threads alone, loading them where they lie,
// took 42 us at 16384 worlds (this gather and the order from the gathered costs: a fraction of that)
__global__ __launch_bounds__(256) void k_gather_cost(int nw, const int* __restrict__ src, size_t stride,
                                                      int* __restrict__ cost) {
  const int w = blockIdx.x * 256 + threadIdx.x;
  if (w < nw) cost[w] = src[w * stride];
}

int launch_order_adj(hipStream_t st, int nw, int nsub, const float* tape, void* work) {
  int* perm = (int*)work;
  int* cost = perm + nw;
  const int* src = reinterpret_cast<const int*>(tape + (size_t)(nsub - 1) * REC_WORDS + REC_ADJCOST);
  hipLaunchKernelGGL(k_gather_cost, dim3((nw + 255) / 256), dim3(256), 0, st, nw, src, (size_t)nsub * REC_WORDS, cost);
  hipLaunchKernelGGL(k_order, dim3(1), dim3(ORDER_THREADS), 0, st, nw, (const int*)cost, (size_t)1, perm);
  return (int)hipGetLastError();
}

}  // namespace g1k
