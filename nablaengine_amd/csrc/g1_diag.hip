// Diagnostic counters of the forward and the backward (the reference's dk_torch_diag_fwd / dk_torch_diag_bwd,
// torch_ffi.py:85-156) as kernels of their own, run after a forward / backward: the counters and their order are in
// g1_diag.h. The forward's counters: one thread per world (grid-stride); the backward's: one wave per world; a wave
// sum per count, one 64-bit atomic add per wave and count; integer counts only.
#include "g1_device.h"
#include "g1_diag.h"
#include "g1_tape.h"

namespace g1k {

__device__ __forceinline__ void diag_add(unsigned long long* d, int k, int v) {
  const int t = wsumi(v);
  if ((threadIdx.x & 63) == 0 && t) atomicAdd(&d[k], (unsigned long long)t);
}

__global__ __launch_bounds__(256) void k_diag_fwd(unsigned long long* d, int nw, int nsub, int iterations,
                                                  const int* __restrict__ info, const float* __restrict__ tape) {
  int unsup = 0, lim = 0, refact = 0, nonconv = 0, sing = 0, ocon = 0, orow = 0;
  for (int w = blockIdx.x * blockDim.x + threadIdx.x; w < nw; w += gridDim.x * blockDim.x) {
    const int f = info[4 * w + 3];
    unsup += f != 0;
    ocon += (f & 4) != 0;
    orow += (f & 16) != 0;
    lim += info[4 * w] >= iterations;
    if (tape)
      for (int k0 = 0; k0 < nsub; k0 += 4) {  // 4 records' flags in flight at a time
        unsigned fl[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
          fl[u] = k0 + u < nsub ? __float_as_uint(tape[((size_t)w * nsub + k0 + u) * REC_WORDS + REC_FLAGS]) : 0u;
#pragma unroll
        for (int u = 0; u < 4; u++) {
          refact += (fl[u] & FLAG_REFACT) != 0;
          nonconv += (fl[u] & FLAG_NONCONV) != 0;
          sing += (fl[u] & FLAG_SINGULAR) != 0;
        }
      }
  }
  diag_add(d, D_FWD_UNSUPPORTED, unsup);
  diag_add(d, D_FWD_ITER_LIMIT, lim);
  diag_add(d, D_REFACT, refact);
  diag_add(d, D_NONCONV, nonconv);
  diag_add(d, D_SINGULAR, sing);
  diag_add(d, D_CONTACT_OVERFLOW, ocon);
  diag_add(d, D_ROW_OVERFLOW, orow);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    atomicAdd(&d[D_FWD_CALLS], 1ull);
    atomicAdd(&d[D_FWD_WORLDS], (unsigned long long)nw);
    if (tape) atomicAdd(&d[D_TAPE_RECORDS], (unsigned long long)nw * (unsigned long long)nsub);
  }
}

// one wave per world (4 worlds per workgroup of 256): lane l reads entry l of each row (the rows' loads coalesced, all
// issued at once), the wave's ballots give the row's non-finite bits
__global__ __launch_bounds__(256) void k_diag_bwd(unsigned long long* d, int nw, const float* __restrict__ gq,
                                                  const float* __restrict__ gv, const float* __restrict__ gu,
                                                  const float* __restrict__ cq, const float* __restrict__ cv,
                                                  int* __restrict__ info) {
  static_assert(NQ <= 64 && NV <= 64 && NU <= 64, "one row per wave");
  const int lane = threadIdx.x & 63, w = blockIdx.x * 4 + (threadIdx.x >> 6);
  int rows = 0, rq = 0, rv = 0, ru = 0, rc = 0, rm = 0;
  if (w < nw) {  // wave-uniform
    const int lq = min(lane, NQ - 1), lv = min(lane, NV - 1), lu = min(lane, NU - 1);
    const float xq = gq[(size_t)w * NQ + lq], xv = gv[(size_t)w * NV + lv], xu = gu[(size_t)w * NU + lu];
    const float yq = cq[(size_t)w * NQ + lq], yv = cv[(size_t)w * NV + lv];
    const bool bq = __ballot(!__builtin_isfinite(xq)) != 0ull, bv = __ballot(!__builtin_isfinite(xv)) != 0ull;
    const bool bu = __ballot(!__builtin_isfinite(xu)) != 0ull;
    const bool bc = __ballot(!(__builtin_isfinite(yq) && __builtin_isfinite(yv))) != 0ull;
    const unsigned b = (bq ? 1u : 0u) | (bv ? 2u : 0u) | (bu ? 4u : 0u) | (bc ? 8u : 0u);
    if (lane == 0) {
      const int f = info[w];
      info[w] = f | (int)(b << NONFINITE_SHIFT);
      rows = (b & 7u) != 0;
      rq = (b & 1u) != 0;
      rv = (b & 2u) != 0;
      ru = (b & 4u) != 0;
      rc = (b & 8u) != 0;
      rm = (f & ADJ_REPLAY_MISMATCH) != 0;
    }
  }
  diag_add(d, D_NONFINITE, rows);
  diag_add(d, D_NONFINITE_QPOS, rq);
  diag_add(d, D_NONFINITE_QVEL, rv);
  diag_add(d, D_NONFINITE_CTRL, ru);
  diag_add(d, D_NONFINITE_COT, rc);
  diag_add(d, D_REPLAY_MISMATCH, rm);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
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
