/* C ABI of the MI355X G1 control-step library (libnablaengine_g1.so): the entry points the reference's FFI binds
 * (ctypes in src/nablaengine/torch_ffi.py:333-366 _bind, XLA FFI in src/nablaengine/jax_ffi.py:486-797), with
 * cudaStream_t -> hipStream_t. Plain pointers and sizes: float32 arrays world-major and row-contiguous, int32 info.
 * Every entry returns 0 on success, else a hipError_t (or -1: the device cannot take the launch; -2: more worlds
 * than dk_fwd_forward_static's scratch holds); nothing is allocated per call (the caller owns every output, the tape and the work buffer); launches go on the given stream. */
#ifndef NABLAENGINE_G1_H
#define NABLAENGINE_G1_H
#include <hip/hip_runtime_api.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Replaces <fwd>_forward (jax_ffi.py:266-278, FWD_SHIM): one control step of nsub substeps for nw worlds.
 * in: qpos (nw, 36), qvel (nw, 35), warm (nw, 35) Newton warm start, ctrl (nw, 29), fric (nw,), com (nw, 3);
 * out: oq (nw, 36), ov (nw, 35), ow (nw, 35) = the last substep's qacc, info (nw, 4) = (Newton iterations of the last
 * substep, contacts found, constraint rows, flags: 4 contacts beyond 64 dropped, 16 rows beyond 192 dropped);
 * ocon (nw, 64, 8) or NULL: the last substep's contacts (pair, dist, pos[3], normal[3]; pair -1 past the count);
 * tape (nw, nsub * DK_REC_WORDS) or NULL: the adjoint's record (its flags word as the reference's: 4 / 16
 * overflow, 1 << 8 refactored at the final zones, 1 << 9 not converged, 1 << 10 near-singular self contact); work:
 * dk_fwd_work_bytes(nw) bytes or NULL when 0, for the dispatch order (heaviest worlds first), which is skipped, and work
 * left unwritten, when the GPU holds all nw worlds at once (8 per CU): every world then starts at the launch. */
int dk_fwd_forward(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm, const float* ctrl,
                   const float* fric, const float* com, int iterations, int nsub, float* oq, float* ov, float* ow,
                   int* info, float* ocon, float* tape, void* work);
/* No counterpart in the reference's ABI (its order is internal to dk_forward_split, host.py:310-330): the dispatch
 * order of dk_fwd_forward on its own, written into work (dk_fwd_work_bytes(nw) bytes) from the input qpos; and the
 * forward launched with an order already in work (no recomputation), for callers that reuse one order across steps
 * (the worlds' costs change slowly) and for timing the forward kernel alone. Results are the same in any order. */
int dk_fwd_order(hipStream_t st, int nw, const float* qpos, void* work);
int dk_fwd_forward_ordered(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                           const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                           float* ov, float* ow, int* info, float* ocon, float* tape, const void* work);
/* No counterpart in the reference (its forward takes the caller's work memory): dk_fwd_forward for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same
 * arguments without work, and the same results; the dispatch order lives in a static device array of the library
 * (1 MiB per GPU, held until the process ends) whose address dk_fwd_upload takes once per device (else the first
 * call on the device does). At most DK_STATIC_MAX_WORLDS worlds: more returns DK_ERR_STATIC_CAPACITY without a
 * launch. Nothing is allocated. Every call on one GPU shares that array, so calls that overlap on one GPU (two
 * streams at once) race; calls in one stream's order do not. */
#define DK_STATIC_MAX_WORLDS 131072
#define DK_ERR_STATIC_CAPACITY (-2)
int dk_fwd_forward_static(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                          const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                          float* ov, float* ow, int* info, float* ocon, float* tape);
/* Replaces <fwd>_work_bytes (jax_ffi.py:265): scratch bytes the forward's work buffer takes for nw worlds (the
 * dispatch order, heaviest worlds first: 8 bytes per world). work = NULL runs the worlds in index order instead; the
 * results are the same either way. */
long long dk_fwd_work_bytes(int nw);
/* Replaces <fwd>_kinematics (jax_ffi.py:281-285; g1_engine/kinematics.py:1-45): the kinematics outputs of nw states
 * (MJX kinematics + com_pos + com_vel). in: qpos (nw, 36), qvel (nw, 35), com (nw, 3); out: qn (nw, 36) qpos with the
 * root quaternion normalized, xpos (nw, 31, 3), xquat (nw, 31, 4) body frames (world body 0 included), cvel (nw, 31, 6)
 * [angular; linear] twists at subtree_com[1], sc (nw, 31, 3) subtree COMs. torch_ffi runs it on a step's output state
 * for step(..., kinematics=True). */
int dk_fwd_kinematics(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com, float* qn,
                      float* xpos, float* xquat, float* cvel, float* sc);
/* Replaces <fwd>_kinematics_vjp (jax_ffi.py:286-292): the VJP of dk_fwd_kinematics at (qpos, qvel, com): the outputs'
 * cotangents gqn, gxpos, gxquat, gcvel, gsc (shapes as the outputs) -> gq (nw, 36), gv (nw, 35); gq_in / gv_in
 * (NULL, or cotangents of the same state, e.g. a step's outputs') are added to the result last. com gets none. */
int dk_fwd_kinematics_vjp(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* com,
                          const float* gqn, const float* gxpos, const float* gxquat, const float* gcvel,
                          const float* gsc, const float* gq_in, const float* gv_in, float* gq, float* gv);
/* Replace dk_torch_diag_fwd / dk_torch_diag_bwd (torch_ffi.py:85-156, 146-155): the diagnostic counters, 18 uint64 in
 * d (the caller's device array; order of torch_ffi.DIAG), added to after a forward (calls, worlds, worlds with info[3]
 * bits, at the iteration cap, tape records and their REFACT / NONCONV / SINGULAR flags, contact / row overflow worlds)
 * and after a backward (calls, rows, rows with non-finite gradients of qpos / qvel / ctrl or non-finite cotangents,
 * replay mismatches). The backward's also ORs the non-finite bits (1 qpos, 2 qvel, 4 ctrl, 8 cotangent) << 16 into
 * its info. */
int dk_torch_diag_fwd(hipStream_t st, unsigned long long* d, int nw, int nsub, int iterations, const int* info,
                      const float* tape);
int dk_torch_diag_bwd(hipStream_t st, unsigned long long* d, int nw, const float* gq, const float* gv, const float* gu,
                      const float* cq, const float* cv, int* info);
/* No counterpart in the reference (its torch_ffi launches the diagnostics kernel after each call): dk_fwd_forward /
 * dk_adjoint_work with dk_torch_diag_fwd / dk_torch_diag_bwd's counting done by the forward / adjoint kernel itself,
 * each world adding its part at its end (one launch fewer per call). The same outputs, the same counters in d (d is
 * required), and for the adjoint the same non-finite bits << 16 in info (the output cotangents gq_out, gv_out are the
 * rows dk_torch_diag_bwd's cq, cv check). */
int dk_fwd_forward_diag(hipStream_t st, int nw, const float* qpos, const float* qvel, const float* warm,
                        const float* ctrl, const float* fric, const float* com, int iterations, int nsub, float* oq,
                        float* ov, float* ow, int* info, float* ocon, float* tape, void* work, unsigned long long* d);
int dk_adjoint_work_diag(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                         const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                         const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work,
                         unsigned long long* d);
/* Replaces <unit>_upload (jax_ffi.py:214-225): the model constants are compiled into this library, so the call only
 * checks that the current device can run the kernels; consts may be NULL. */
int dk_fwd_upload(const float* consts, hipStream_t st);
/* Replaces <unit>_launch (jax_ffi.py:243-254): the adjoint's launch on device dev, o[0] the LDS bytes k_adjoint
 * takes per world (static: the kernel needs no dynamic LDS and no opt-in), o[1] its resident worlds per CU
 * (hipOccupancyMaxActiveBlocksPerMultiprocessor); the current device is restored. Returns 0 or a hipError_t. */
int dk_fwd_launch(int dev, long long* o);
/* Replaces <unit>_sizes (jax_ffi.py:255-258): o[0..8] = LDS bytes of the forward, of the adjoint, tape words per
 * world and substep, nq, nv, max contacts, clamp_kv, normal, the tape's flags word offset (o[6], o[7] -1: runtime). */
void dk_fwd_sizes(long long* o);

/* No counterpart in the reference's ABI (its DK_PROFILE builds read g_prof the same way, host.py:13-17): in a build
 * with -DG1_PROFILE, copies the last forward's per-world phase cycles (s_memtime) of the first nw worlds, nw x 27
 * uint64 (smooth, collision, rows, Newton init, Hessian, factor, solve, line search, update, gradient, implicitfast,
 * tape, Newton iterations, line-search evaluations, dense factorizations, then the cycles of parts of the line
 * search (row velocities J p; M p) and of the Hessian (contact stiffnesses, subtree sums, rows), then the world's start
 * and end (s_memrealtime, 100 MHz) and where it ran (HW_ID | XCC_ID << 32), then the cycles of parts of the smooth
 * dynamics (forward kinematics, body forces, subtree sums, CRBA and bias)); returns -1 in the production build. */
int dk_prof_read(unsigned long long* out, int nw);
/* No counterpart in the reference's ABI (its adjoint's DK_PROFILE phases, adjoint.py:101-107,221-232): in a build with
 * -DG1_PROFILE, copies the last adjoint's per-world phase cycles of the first nw worlds, nw x 27 uint64 (record,
 * poses, solves, twists, contacts, body sums, body forces, dof terms, then the world's start and end on the 100 MHz
 * clock; the rest 0); returns -1 in the production build. */
int dk_prof_read_adj(unsigned long long* out, int nw);

/* Replaces <variant>_adjoint (jax_ffi.py:228-241) for every (clamp_kv, normal) variant at once: the VJP of one control
 * step from its tape. in: tape (nw, nsub * DK_REC_WORDS; 16-byte aligned, else hipErrorInvalidValue), fric, com as
 * the forward's, gq_out (nw, 36), gv_out (nw, 35) the output cotangents, ctrl (nw, 29) (clamp_kv 2 only, else may be
 * NULL), clamp_soft (clamp_kv 2); out: gq_in (nw, 36) qpos-form, gv_in (nw, 35), gctrl (nw, 29), info (nw,): the union
 * of the records' flags, 1 << 13 a replayed contact not found (the reference's ADJ_REPLAY_MISMATCH). */
int dk_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
               const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
               const float* ctrl, float clamp_soft, int clamp_kv, int normal);

/* No counterpart in the reference's ABI (its adjoint entries take no work buffer): dk_adjoint with a work buffer of
 * dk_adjoint_work_bytes(nw) bytes, in which the worlds are ordered heaviest first (the tape's contacts) before the
 * launch, unless the GPU holds all nw worlds at once (8 per CU: index order, work left unwritten). Same results as
 * dk_adjoint, which is this entry with work = NULL. */
int dk_adjoint_work(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                    const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                    const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work);
long long dk_adjoint_work_bytes(int nw);
/* No counterpart in the reference's ABI: the adjoint's dispatch order on its own, written into work
 * (dk_adjoint_work_bytes(nw) bytes) from the tape; and the adjoint launched with that order already in work, for
 * callers that run several VJPs on one tape (the step Jacobian's 71 one-hot cotangents). d: the diagnostic counters,
 * counted as dk_adjoint_work_diag does, or NULL (no counting, no non-finite bits in info). Results are the same in any
 * order. */
int dk_adjoint_order(hipStream_t st, int nw, int nsub, const float* tape, void* work);
int dk_adjoint_work_ordered(hipStream_t st, int nw, int nsub, const float* tape, const float* fric, const float* com,
                            const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl,
                            int* info, const float* ctrl, float clamp_soft, int clamp_kv, int normal, const void* work,
                            unsigned long long* d);
/* No counterpart in the reference's ABI: ncot VJPs of one tape in one launch (the step Jacobian's 71 one-hot
 * cotangents), each set bitwise what dk_adjoint_work_diag gives for it. gq_out (ncot, nw, 36), gv_out (ncot, nw, 35)
 * -> gq_in (ncot, nw, 36), gv_in (ncot, nw, 35), gctrl (ncot, nw, 29), info (ncot, nw); work as dk_adjoint_work's (one
 * dispatch order for every set); d: the counters (ncot backward calls), or NULL. With ncot >= 2 a workgroup runs a
 * group of one world's sets, the tape-only phases of each substep once for the group, and keeps the sets' running
 * cotangents in their output rows between substeps: the outputs must not overlap the inputs. One launch of at most
 * nw * ncot workgroups of 64 work-items: nw * ncot * 64 < 2^32 (a Jacobian's 71 sets up to 945,195 worlds), else
 * hipErrorInvalidValue. */
int dk_adjoint_many(hipStream_t st, int nw, int ncot, int nsub, const float* tape, const float* fric, const float* com,
                    const float* gq_out, const float* gv_out, float* gq_in, float* gv_in, float* gctrl, int* info,
                    const float* ctrl, float clamp_soft, int clamp_kv, int normal, void* work, unsigned long long* d);

/* The reference's per-variant unit names (jax_ffi.py:180,845-846: dk_kv{0,1,2}_n{0..3}), each the entry above with
 * its (clamp_kv, normal) fixed; _upload, _launch and _sizes as dk_fwd_upload / dk_fwd_launch / dk_fwd_sizes (o[6],
 * o[7] the variant). */
#define DK_VARIANT_DECL(KV, N)                                                                                       \
  int dk_kv##KV##_n##N##_adjoint(hipStream_t st, int nw, int nsub, const float* tape, const float* fric,            \
                                  const float* com, const float* gq_out, const float* gv_out, float* gq_in,          \
                                  float* gv_in, float* gctrl, int* info, const float* ctrl, float clamp_soft);       \
  int dk_kv##KV##_n##N##_upload(const float* consts, hipStream_t st);                                                \
  int dk_kv##KV##_n##N##_launch(int dev, long long* o);                                                              \
  void dk_kv##KV##_n##N##_sizes(long long* o);
DK_VARIANT_DECL(0, 0) DK_VARIANT_DECL(0, 1) DK_VARIANT_DECL(0, 2) DK_VARIANT_DECL(0, 3)
DK_VARIANT_DECL(1, 0) DK_VARIANT_DECL(1, 1) DK_VARIANT_DECL(1, 2) DK_VARIANT_DECL(1, 3)
DK_VARIANT_DECL(2, 0) DK_VARIANT_DECL(2, 1) DK_VARIANT_DECL(2, 2) DK_VARIANT_DECL(2, 3)
#undef DK_VARIANT_DECL

#ifdef __cplusplus
}
#endif
#endif
