// Diagnostic counters of the forward and the backward (the reference's dk_torch_diag_fwd / dk_torch_diag_bwd,
// torch_ffi.py:85-156) as kernels of their own, run after a forward / backward: the counters and their order are in
// g1_diag.h. Integer counts only; each thread tallies its worlds in the counters' own slots and publishes the slots it
// owns once (k_forward / k_adjoint count the same things at each world's end when given the array).
#include "g1_device.h"
#include "g1_diag.h"
#include "g1_tape.h"

namespace g1k {

// A thread's tallies, indexed as the device counters: each kernel adds its worlds' counts into the slots it owns, then
// publish() adds those slots to the device array (a wave sum per slot, one 64-bit atomic add per wave and nonzero sum)
struct Tally {
  int n[NDIAG] = {};
  template <int N>
  __device__ __forceinline__ void publish(unsigned long long* d, const int (&slots)[N]) const {
#pragma unroll
    for (int i = 0; i < N; i++) {
      const int t = wsumi(n[slots[i]]);
      if ((threadIdx.x & 63) == 0 && t) atomicAdd(&d[slots[i]], (unsigned long long)t);
    }
  }
};

// after a forward: one thread per world (grid-stride): the info row's flags and iteration count, and with a tape the
// flags word of each of the world's records (4 records' loads in flight at a time)
__global__ __launch_bounds__(256) void k_diag_fwd(unsigned long long* d, int nw, int nsub, int iterations,
                                                  const int* __restrict__ info, const float* __restrict__ tape) {
  Tally y;
  for (int w = blockIdx.x * blockDim.x + threadIdx.x; w < nw; w += gridDim.x * blockDim.x) {
    const int flags = info[4 * w + 3];
    y.n[D_FWD_UNSUPPORTED] += flags != 0;
    y.n[D_CONTACT_OVERFLOW] += (flags & OVERFLOW_CONTACTS) != 0;
    y.n[D_ROW_OVERFLOW] += (flags & OVERFLOW_ROWS) != 0;
    y.n[D_FWD_ITER_LIMIT] += info[4 * w] >= iterations;
    if (!tape) continue;
    const float* recs = tape + (size_t)w * nsub * REC_WORDS + REC_FLAGS;
    for (int k0 = 0; k0 < nsub; k0 += 4) {
      unsigned rf[4];
#pragma unroll
      for (int u = 0; u < 4; u++) rf[u] = k0 + u < nsub ? __float_as_uint(recs[(size_t)(k0 + u) * REC_WORDS]) : 0u;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        y.n[D_REFACT] += (rf[u] & FLAG_REFACT) != 0;
        y.n[D_NONCONV] += (rf[u] & FLAG_NONCONV) != 0;
        y.n[D_SINGULAR] += (rf[u] & FLAG_SINGULAR) != 0;
      }
    }
  }
  constexpr int kSlots[] = {D_FWD_UNSUPPORTED, D_FWD_ITER_LIMIT, D_REFACT, D_NONCONV, D_SINGULAR, D_CONTACT_OVERFLOW,
                            D_ROW_OVERFLOW};
  y.publish(d, kSlots);
  if (blockIdx.x == 0 && threadIdx.x == 0) {  // the call itself
    atomicAdd(&d[D_FWD_CALLS], 1ull);
    atomicAdd(&d[D_FWD_WORLDS], (unsigned long long)nw);
    if (tape) atomicAdd(&d[D_TAPE_RECORDS], (unsigned long long)nw * (unsigned long long)nsub);
  }
}

// after a backward: one wave per world (4 worlds per workgroup of 256), lane l reading entry l of each gradient and
// cotangent row (coalesced, every load issued at once); the wave's ballots give the world's non-finite bits, which go
// into its info (<< NONFINITE_SHIFT) and, with the replay-mismatch flag, into lane 0's tallies
__global__ __launch_bounds__(256) void k_diag_bwd(unsigned long long* d, int nw, const float* __restrict__ gq,
                                                  const float* __restrict__ gv, const float* __restrict__ gu,
                                                  const float* __restrict__ cq, const float* __restrict__ cv,
                                                  int* __restrict__ info) {
  static_assert(NQ <= 64 && NV <= 64 && NU <= 64, "one row per wave");
  const int lane = threadIdx.x & 63, w = blockIdx.x * 4 + (threadIdx.x >> 6);
  Tally y;
  if (w < nw) {  // wave-uniform
    const int lq = min(lane, NQ - 1), lv = min(lane, NV - 1), lu = min(lane, NU - 1);
    const float xq = gq[(size_t)w * NQ + lq], xv = gv[(size_t)w * NV + lv], xu = gu[(size_t)w * NU + lu];
    const float yq = cq[(size_t)w * NQ + lq], yv = cv[(size_t)w * NV + lv];
    const auto bad = [](bool finite) { return __ballot(!finite) != 0ull; };
    const unsigned bits = (bad(__builtin_isfinite(xq)) ? (unsigned)NONFINITE_QPOS : 0u)
                          | (bad(__builtin_isfinite(xv)) ? (unsigned)NONFINITE_QVEL : 0u)
                          | (bad(__builtin_isfinite(xu)) ? (unsigned)NONFINITE_CTRL : 0u)
                          | (bad(__builtin_isfinite(yq) && __builtin_isfinite(yv)) ? (unsigned)NONFINITE_COT : 0u);
    if (lane == 0) {
      const int prev = info[w];
      info[w] = prev | (int)(bits << NONFINITE_SHIFT);
      y.n[D_NONFINITE] = (bits & (NONFINITE_QPOS | NONFINITE_QVEL | NONFINITE_CTRL)) != 0u;
      y.n[D_NONFINITE_QPOS] = (bits & NONFINITE_QPOS) != 0u;
      y.n[D_NONFINITE_QVEL] = (bits & NONFINITE_QVEL) != 0u;
      y.n[D_NONFINITE_CTRL] = (bits & NONFINITE_CTRL) != 0u;
      y.n[D_NONFINITE_COT] = (bits & NONFINITE_COT) != 0u;
      y.n[D_REPLAY_MISMATCH] = (prev & ADJ_REPLAY_MISMATCH) != 0;
    }
  }
  constexpr int kSlots[] = {D_NONFINITE, D_NONFINITE_QPOS, D_NONFINITE_QVEL, D_NONFINITE_CTRL, D_NONFINITE_COT,
                            D_REPLAY_MISMATCH};
  y.publish(d, kSlots);
  if (blockIdx.x == 0 && threadIdx.x == 0) {  // the call itself
    atomicAdd(&d[D_BWD_CALLS], 1ull);
    atomicAdd(&d[D_BWD_ROWS], (unsigned long long)nw);
  }
}

static unsigned diag_grid(int nw) {
  const int g = (nw + 255) / 256;
  return (unsigned)(g < 1 ? 1 : g > 256 ? 256 : g);
}

int launch_diag_fwd(hipStream_t st, unsigned long long* d, int nw, int nsub, int iterations, const int* info,
                    const float* tape) {
  hipLaunchKernelGGL(k_diag_fwd, dim3(diag_grid(nw)), dim3(256), 0, st, d, nw, nsub, iterations, info, tape);
  return (int)hipGetLastError();
}

int launch_diag_bwd(hipStream_t st, unsigned long long* d, int nw, const float* gq, const float* gv, const float* gu,
                    const float* cq, const float* cv, int* info) {
  hipLaunchKernelGGL(k_diag_bwd, dim3(nw > 0 ? (nw + 3) / 4 : 1), dim3(256), 0, st, d, nw, gq, gv, gu, cq, cv, info);
  return (int)hipGetLastError();
}

}  // namespace g1k
