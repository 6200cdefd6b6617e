// The C ABI (include/nablaengine_g1.h): thin entries over the kernels' launchers.
#include "../../include/nablaengine_g1.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace g1k {
int launch_forward(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm, const float* ctrl,
                   const float* fric, const float* com, int iterations, int nsub, float* oq, float* ov, float* ow,
                   int* info, float* ocon, float* tape, void* work, int order, unsigned long long* diag);
int launch_order_fwd(hipStream_t st, int nw, const float* qpos, void* work);
size_t order_work_bytes(int nw);
size_t forward_lds_bytes();
size_t adjoint_lds_bytes();
int adjoint_occupancy(int dev, int* n);
int prof_read(unsigned long long* out, int nw);
int prof_read_adj(unsigned long long* out, int nw);
int launch_diag_fwd(hipStream_t st, unsigned long long* d, int nw, int nsub, int iterations, const int* info,
                    const float* tape);
int launch_diag_bwd(hipStream_t st, unsigned long long* d, int nw, const float* gq, const float* gv, const float* gu,
                    const float* cq, const float* cv, int* info);
int launch_kinematics(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com, float* qn,
                      float* xpos, float* xquat, float* cvel, float* sc);
int launch_kinematics_vjp(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com,
                          const float* gqn, const float* gxpos, const float* gxquat, const float* gcvel,
                          const float* gsc, const float* gq_in, const float* gv_in, float* gq, float* gv);
int launch_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                   const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                   const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work, int order,
                   unsigned long long* diag, int ncot);
int launch_order_adj(hipStream_t st, int nw, int nsub, const float* tape, void* work);
}  // namespace g1k

namespace {
// The allocation-free forward's scratch (dk_fwd_forward_static): the dispatch order of up to DK_STATIC_MAX_WORLDS
// worlds (a permutation and a cost, 4 bytes each per world) in a file-scope device array, one copy per GPU held until
// the process ends. Host code never passes the array's name to a kernel (on the host it is a stand-in, not a device
// address): each device's address is taken once by hipGetSymbolAddress with that device current and kept in
// g_scratch. The kernels write every word they read (costs, then the permutation), so nothing is cleared.
__device__ __align__(256) unsigned char scratch[8 * (size_t)DK_STATIC_MAX_WORLDS];
constexpr int MAX_DEVICES = 64;
void* g_scratch[MAX_DEVICES];
std::mutex g_scratch_mu;

// the scratch's address on the current device (taken on the first call for that device)
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return 0;
}

int check_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, dev);
  if (e != hipSuccess) return (int)e;
  return p.sharedMemPerBlock >= g1k::forward_lds_bytes() ? 0 : -1;
}
}  // namespace

extern "C" {

int dk_fwd_forward(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm, const float* ctrl,
                   const float* fric, const float* com, int iterations, int nsub, float* oq, float* ov, float* ow,
                   int* info, float* ocon, float* tape, void* work) {
  if (nw < 0 || nsub < 1 || nsub > 32 || iterations < 0) return (int)hipErrorInvalidValue;
  return g1k::launch_forward(st, nw, qpos, qvel, warm, ctrl, fric, com, iterations, nsub, oq, ov, ow, info, ocon, tape,
                             work, 1, nullptr);
}

int dk_fwd_forward_diag(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                        const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                        float* ov, float* ow, int* info, float* ocon, float* tape, void* work, unsigned long long* d) {
  if (nw < 0 || nsub < 1 || nsub > 32 || iterations < 0 || !d) return (int)hipErrorInvalidValue;
  return g1k::launch_forward(st, nw, qpos, qvel, warm, ctrl, fric, com, iterations, nsub, oq, ov, ow, info, ocon, tape,
                             work, 1, d);
}

int dk_fwd_order(hipStream_t st, int nw, const float* qpos, void* work) {
  if (nw < 0 || (nw > 0 && !work)) return (int)hipErrorInvalidValue;
  return nw > 0 ? g1k::launch_order_fwd(st, nw, qpos, work) : 0;
}

int dk_fwd_forward_ordered(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                           const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                           float* ov, float* ow, int* info, float* ocon, float* tape, const void* work) {
  if (nw < 0 || nsub < 1 || nsub > 32 || iterations < 0 || (nw > 0 && !work)) return (int)hipErrorInvalidValue;
  return g1k::launch_forward(st, nw, qpos, qvel, warm, ctrl, fric, com, iterations, nsub, oq, ov, ow, info, ocon, tape,
                             const_cast<void*>(work), 2, nullptr);
}

int dk_fwd_kinematics(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com, float* qn,
                      float* xpos, float* xquat, float* cvel, float* sc) {
  if (nw < 0) return (int)hipErrorInvalidValue;
  return g1k::launch_kinematics(st, nw, qpos, qvel, com, qn, xpos, xquat, cvel, sc);
}

int dk_fwd_kinematics_vjp(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com,
                          const float* gqn, const float* gxpos, const float* gxquat, const float* gcvel,
                          const float* gsc, const float* gq_in, const float* gv_in, float* gq, float* gv) {
  if (nw < 0) return (int)hipErrorInvalidValue;
  return g1k::launch_kinematics_vjp(st, nw, qpos, qvel, com, gqn, gxpos, gxquat, gcvel, gsc, gq_in, gv_in, gq, gv);
}

int dk_torch_diag_fwd(hipStream_t st, unsigned long long* d, int nw, int nsub, int iterations, const int* info,
                      const float* tape) {
  if (nw < 0 || nsub < 1 || !d) return (int)hipErrorInvalidValue;
  return g1k::launch_diag_fwd(st, d, nw, nsub, iterations, info, tape);
}

int dk_torch_diag_bwd(hipStream_t st, unsigned long long* d, int nw, const float* gq, const float* gv, const float* gu,
                      const float* cq, const float* cv, int* info) {
  if (nw < 0 || !d) return (int)hipErrorInvalidValue;
  return g1k::launch_diag_bwd(st, d, nw, gq, gv, gu, cq, cv, info);
}

long long dk_fwd_work_bytes(int nw) { return nw > 0 ? (long long)g1k::order_work_bytes(nw) : 0; }

int dk_fwd_upload(const float* consts, hipStream_t st) {
  (void)consts;
  (void)st;
  const int rc = check_device();
  if (rc) return rc;
  void* p = nullptr;  // the allocation-free forward's scratch address on this device, taken at set-up
  return scratch_ptr(&p);
}

int dk_fwd_forward_static(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                          const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                          float* ov, float* ow, int* info, float* ocon, float* tape) {
  if (nw < 0 || nsub < 1 || nsub > 32 || iterations < 0) return (int)hipErrorInvalidValue;
  if (nw > DK_STATIC_MAX_WORLDS) return DK_ERR_STATIC_CAPACITY;
  if (nw == 0) return 0;
  void* work = nullptr;
  const int rc = scratch_ptr(&work);
  if (rc) return rc;
  return g1k::launch_forward(st, nw, qpos, qvel, warm, ctrl, fric, com, iterations, nsub, oq, ov, ow, info, ocon, tape,
                             work, 1, nullptr);
}

// the profiling build's per-world phase cycles of the last forward (test and measurement helper; -1 in production)
int dk_prof_read(unsigned long long* out, int nw) { return g1k::prof_read(out, nw); }
int dk_prof_read_adj(unsigned long long* out, int nw) { return g1k::prof_read_adj(out, nw); }

int dk_fwd_launch(int dev, long long* o) {
  o[0] = (long long)g1k::adjoint_lds_bytes();
  o[1] = 0;
  int n = 0;
  const int rc = g1k::adjoint_occupancy(dev, &n);
  o[1] = rc ? 0 : n;
  return rc;
}

void dk_fwd_sizes(long long* o) {
  o[0] = (long long)g1k::forward_lds_bytes(); o[1] = (long long)g1k::adjoint_lds_bytes(); o[2] = 1472; o[3] = 36;
  o[4] = 35; o[5] = 64; o[6] = -1; o[7] = -1; o[8] = 1;
}

int dk_adjoint_work(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                    const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                    const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work) {
  if (nw < 0 || nsub < 1 || nsub > 32 || clamp_kv < 0 || clamp_kv > 2 || normal < 0 || normal > 3)
    return (int)hipErrorInvalidValue;
  if (clamp_kv == 2 && !ctrl) return (int)hipErrorInvalidValue;
  return g1k::launch_adjoint(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl,
                             clamp_soft, clamp_kv, normal, work, 1, nullptr, 1);
}

int dk_adjoint_work_diag(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                         const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                         const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work,
                         unsigned long long* d) {
  if (nw < 0 || nsub < 1 || nsub > 32 || clamp_kv < 0 || clamp_kv > 2 || normal < 0 || normal > 3 || !d)
    return (int)hipErrorInvalidValue;
  if (clamp_kv == 2 && !ctrl) return (int)hipErrorInvalidValue;
  return g1k::launch_adjoint(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl,
                             clamp_soft, clamp_kv, normal, work, 1, d, 1);
}

int dk_adjoint_order(hipStream_t st, int nw, int nsub, const float* tape, void* work) {
  if (nw < 0 || nsub < 1 || nsub > 32 || (nw > 0 && !work)) return (int)hipErrorInvalidValue;
  return nw > 0 ? g1k::launch_order_adj(st, nw, nsub, tape, work) : 0;
}

int dk_adjoint_work_ordered(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                            const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl,
                            int* info, const float* ctrl, float clamp_soft, int clamp_kv, int normal, const void* work,
                            unsigned long long* d) {
  if (nw < 0 || nsub < 1 || nsub > 32 || clamp_kv < 0 || clamp_kv > 2 || normal < 0 || normal > 3 ||
      (nw > 0 && !work))
    return (int)hipErrorInvalidValue;
  if (clamp_kv == 2 && !ctrl) return (int)hipErrorInvalidValue;
  return g1k::launch_adjoint(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl,
                             clamp_soft, clamp_kv, normal, const_cast<void*>(work), 2, d, 1);
}

int dk_adjoint_many(hipStream_t st, int nw, int ncot, int nsub, const float* tape, const float* fric, const float* com,
                    const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                    const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work, unsigned long long* d) {
  // one launch of nw * ncot workgroups of 64 work-items: HIP takes fewer than 2^32 work-items a launch
  if (nw < 0 || ncot < 1 || (long long)nw * ncot * 64 >= (1LL << 32) || nsub < 1 || nsub > 32 || clamp_kv < 0 ||
      clamp_kv > 2 || normal < 0 || normal > 3)
    return (int)hipErrorInvalidValue;
  if (clamp_kv == 2 && !ctrl) return (int)hipErrorInvalidValue;
  return g1k::launch_adjoint(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl,
                             clamp_soft, clamp_kv, normal, work, 1, d, ncot);
}

long long dk_adjoint_work_bytes(int nw) { return nw > 0 ? (long long)g1k::order_work_bytes(nw) : 0; }

int dk_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
               const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
               const float* ctrl, float clamp_soft, int clamp_kv, int normal) {
  return dk_adjoint_work(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl, clamp_soft,
                         clamp_kv, normal, nullptr);
}

#define DK_VARIANT_DEF(KV, N)                                                                                        \
  int dk_kv##KV##_n##N##_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric,            \
                                  const float* com, const float* gq_out, const float* gv_out, float* gq_in,          \
                                  float* gv_in, float* gctrl, int* info, const float* ctrl, float clamp_soft) {      \
    return dk_adjoint(st, nw, nsub, tape, fric, com, gq_out, gv_out, gq_in, gv_in, gctrl, info, ctrl, clamp_soft, KV, \
                      N);                                                                                            \
  }                                                                                                                  \
  int dk_kv##KV##_n##N##_upload(const float* consts, hipStream_t st) { return dk_fwd_upload(consts, st); }          \
  int dk_kv##KV##_n##N##_launch(int dev, long long* o) { return dk_fwd_launch(dev, o); }                             \
  void dk_kv##KV##_n##N##_sizes(long long* o) {                                                                      \
    dk_fwd_sizes(o);                                                                                                 \
    o[6] = KV;                                                                                                       \
    o[7] = N;                                                                                                        \
  }
DK_VARIANT_DEF(0, 0) DK_VARIANT_DEF(0, 1) DK_VARIANT_DEF(0, 2) DK_VARIANT_DEF(0, 3)
DK_VARIANT_DEF(1, 0) DK_VARIANT_DEF(1, 1) DK_VARIANT_DEF(1, 2) DK_VARIANT_DEF(1, 3)
DK_VARIANT_DEF(2, 0) DK_VARIANT_DEF(2, 1) DK_VARIANT_DEF(2, 2) DK_VARIANT_DEF(2, 3)

}  // extern "C"
