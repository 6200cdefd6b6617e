"""TEST INFRASTRUCTURE ONLY: the float64 CPU oracle of the G1 control step (``g1_oracle.cpp``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only
as the checker. The product path (``nablaengine_amd``) never imports it.

Parity status of each function (how it is pinned; the tests that pin it are named):
- ``step``: pinned end to end against MuJoCo C float64 truth (``benchmarks/data/truth/mf_s*.npz`` ``check_out``, 64
  states per corpus, 4 corpora: committed as ``tests/golden/truth_check_*.npz``) in ``tests/test_oracle.py``.
- ``smooth``: M against closed forms (symmetry, positive definiteness, kinetic energy ``0.5 v' M v`` against the sum of
  the bodies' kinetic energies, gravity torque against the finite difference of potential energy) in
  ``tests/test_oracle.py``.
- ``contacts``: pinned by the step truth and by closed forms (sphere-plane depth, segment distance).
- ``integrate_pos``, ``qpos_tangent``: closed forms (quaternion norm, round trip) in ``tests/test_oracle.py``.
- ``kinematics``: the body poses against ``smooth``'s (pinned by the step truth) and the root's pose against qpos; cvel
  against central differences of the poses along qvel (the twist is the poses' time derivative) and the kinetic
  energy of the bodies computed from cvel against ``0.5 v' M v``; subtree_com through the gravity torques of
  ``smooth`` (each joint's torque from the weight of its subtree at its subtree COM) in
  ``tests/test_oracle_kinematics.py``.
- ``kinematics_vjp``: central differences of ``kinematics`` (float64, h = 1e-6), brute force.
- ``vjp``: exact mode by central differences of ``step`` and MuJoCo's ``fd_vjp`` (``tests/test_oracle.py``); clamp_kv 0 / 2
  through lambda measured by central differences in an applied generalized force (the ``qfrc`` hook), normal 1 / 2 / 3
  through the VJP's affine dependence on kappa(nu) (the ``normal_eps`` argument), the near-parallel rule by central
  differences of the forward with frozen segment parameters (the ``freeze`` hook, ``parallel_eps``).
- ``fd_vjp``, ``step_mt``: against ``fd_jacobian`` / ``step`` (the same arithmetic, batched / threaded).
- ``substep_hessian``: H^-1 against central differences of a* in an applied generalized force; ``ltl`` against numpy's
  Cholesky of the order-reversed matrix.
- ``step_f32`` (``g1_oracle_f32.cpp``: the same restatement with float32 storage and mostly float32 arithmetic, a
  yardstick of the error float32 rounding alone gives a step): the float64 ``step`` and its pins carry over, the text
  being the same; it equals ``step`` within float32 accuracy where Newton converges, and differs from it by the
  Hessian's conditioning after one or a few iterations (``tests/test_oracle.py``).
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle_g1.so")
LIB_F32 = os.path.join(HERE, "liboracle_g1_f32.so")
NQ, NV, NU, NB = 36, 35, 29, 31

_lib = None
_lib32 = None


def build():
    """Compile the oracle (g++ on g1_oracle.cpp; the Makefile next to this file)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        dp = ctypes.POINTER(ctypes.c_double)
        ip = ctypes.POINTER(ctypes.c_int)
        L.g1o_step.argtypes = [ctypes.c_int, dp, dp, dp, dp, dp, dp, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                               ctypes.c_double, ctypes.c_int, dp, dp, dp, ip, dp]
        L.g1o_step_ex.argtypes = L.g1o_step.argtypes + [dp, dp, ctypes.c_int]
        L.g1o_step_mt.argtypes = [ctypes.c_int] + L.g1o_step.argtypes[:-1]
        L.g1o_smooth.argtypes = [dp] * 9
        L.g1o_vjp.argtypes = [ctypes.c_int, dp, dp, dp, dp, dp, dp, ctypes.c_int, ctypes.c_double, ctypes.c_int,
                              ctypes.c_double, ctypes.c_int, dp, dp, ctypes.c_int, ctypes.c_int, ctypes.c_double, dp, dp,
                              dp]
        L.g1o_vjp_ex.argtypes = (L.g1o_vjp.argtypes[:17] + [ctypes.c_double, ctypes.c_double]
                                 + L.g1o_vjp.argtypes[17:])
        L.g1o_vjp_count.argtypes = L.g1o_vjp_ex.argtypes + [dp]
        L.g1o_contacts.argtypes = [dp, dp, dp, dp, ctypes.c_double, dp]
        L.g1o_kinematics.argtypes = [ctypes.c_int] + [dp] * 8
        L.g1o_substep_hessian.argtypes = [dp, dp, dp, dp, ctypes.c_double, dp, ctypes.c_int, ctypes.c_double,
                                          ctypes.c_int, ctypes.c_double, dp, dp]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _c(a, shape):
    return np.ascontiguousarray(np.asarray(a, np.float64).reshape(shape))


# the engine's settings (iterations 10, the model's tolerance 1e-8, line search 40 / 1e-7) and MuJoCo C's truth
# settings (benchmarks/data/truth/README.md: 2000 iterations, tolerance 1e-13, 100 line-search steps)
ENGINE = dict(iterations=10, tol=1e-8, ls_max=40, ls_tol=1e-7)
TRUTH = dict(iterations=2000, tol=1e-13, ls_max=100, ls_tol=1e-12)


def step(qpos, qvel, warm, ctrl, friction, com, iterations=10, tol=1e-8, ls_max=40, ls_tol=1e-7, nsub=4,
         flops=False, qfrc=None, freeze=None, freeze_mode=0):
    """One control step of B worlds in float64: (qpos' (B, 36), qvel' (B, 35), warm' (B, 35), info (B, 4) int32),
    and with flops=True the algorithmic flops of each world-step (B,) last.

    The checker's hooks (inert by default): qfrc (B, 35) a generalized force added to qfrc_smooth in every substep;
    freeze (npair, 3) float64 array and freeze_mode 1 / 2: record / replay the segment parameters of the
    capsule-capsule pairs whose both parameters are free (one world per call)."""
    qpos = _c(qpos, (-1, NQ))
    B = qpos.shape[0]
    qvel, warm, ctrl = _c(qvel, (B, NV)), _c(warm, (B, NV)), _c(ctrl, (B, NU))
    friction, com = _c(friction, (B,)), _c(com, (B, 3))
    oq, ov, ow = np.empty((B, NQ)), np.empty((B, NV)), np.empty((B, NV))
    info = np.empty((B, 4), np.int32)
    fl = np.empty(B)
    qf = None if qfrc is None else _c(qfrc, (B, NV))
    if freeze is not None:
        assert B == 1 and freeze.dtype == np.float64 and freeze.flags.c_contiguous
    lib().g1o_step_ex(B, _p(qpos), _p(qvel), _p(warm), _p(ctrl), _p(friction), _p(com), int(iterations), float(tol),
                      int(ls_max), float(ls_tol), int(nsub), _p(oq), _p(ov), _p(ow),
                      info.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), _p(fl), None if qf is None else _p(qf),
                      None if freeze is None else _p(freeze), int(freeze_mode))
    return (oq, ov, ow, info, fl) if flops else (oq, ov, ow, info)


def _f32():
    """The float32 build of the restatement (liboracle_g1_f32.so), its entries' argument types set."""
    global _lib32
    if _lib32 is None:
        if not os.path.exists(LIB_F32):
            build()
        L = ctypes.CDLL(LIB_F32)
        fp, ip, i, f = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_float
        L.g1o_step.argtypes = [i, fp, fp, fp, fp, fp, fp, i, f, i, f, i, fp, fp, fp, ip, fp]
        L.g1o_vjp_ex.argtypes = [i, fp, fp, fp, fp, fp, fp, i, f, i, f, i, fp, fp, i, i, f, f, f, fp, fp, fp]
        _lib32 = L
    return _lib32


def step_f32(qpos, qvel, warm, ctrl, friction, com, iterations=10, tol=1e-8, ls_max=40, ls_tol=1e-7, nsub=4):
    """``step`` evaluated in float32 (the restatement compiled with float storage, g1_oracle_f32.cpp): (qpos' (B, 36),
    qvel' (B, 35), warm' (B, 35), info (B, 4) int32), the outputs float32. A yardstick of float32 rounding, not the
    checker of any output by itself."""
    _f32()
    f = lambda a, shape: np.ascontiguousarray(np.asarray(a, np.float32).reshape(shape))
    qpos = f(qpos, (-1, NQ))
    B = qpos.shape[0]
    qvel, warm, ctrl, friction, com = f(qvel, (B, NV)), f(warm, (B, NV)), f(ctrl, (B, NU)), f(friction, (B,)), f(com, (B, 3))
    oq, ov, ow = np.empty((B, NQ), np.float32), np.empty((B, NV), np.float32), np.empty((B, NV), np.float32)
    info, fl = np.empty((B, 4), np.int32), np.empty(B, np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    _lib32.g1o_step(B, P(qpos), P(qvel), P(warm), P(ctrl), P(friction), P(com), int(iterations), float(tol),
                    int(ls_max), float(ls_tol), int(nsub), P(oq), P(ov), P(ow),
                    info.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), P(fl))
    return oq, ov, ow, info


def vjp_f32(qpos, qvel, warm, ctrl, friction, com, g_qpos, g_qvel, clamp_kv=1, normal=0, clamp_soft=0.2,
            iterations=10, tol=1e-8, ls_max=40, ls_tol=1e-7, nsub=4, normal_eps=1e-3, parallel_eps=1.2e-3):
    """``vjp`` evaluated in float32 (g1_oracle_f32.cpp, as ``step_f32``): the float32 rounding yardstick of a
    gradient, not the checker of any gradient by itself."""
    _f32()
    f = lambda a, shape: np.ascontiguousarray(np.asarray(a, np.float32).reshape(shape))
    qpos = f(qpos, (-1, NQ))
    B = qpos.shape[0]
    args = [qpos, f(qvel, (B, NV)), f(warm, (B, NV)), f(ctrl, (B, NU)), f(friction, (B,)), f(com, (B, 3))]
    gq, gv = f(g_qpos, (B, NQ)), f(g_qvel, (B, NV))
    oq, ov, ou = np.empty((B, NQ), np.float32), np.empty((B, NV), np.float32), np.empty((B, NU), np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    _lib32.g1o_vjp_ex(B, *map(P, args), int(iterations), float(tol), int(ls_max), float(ls_tol), int(nsub), P(gq),
                      P(gv), int(clamp_kv), int(normal), float(clamp_soft), float(normal_eps), float(parallel_eps),
                      P(oq), P(ov), P(ou))
    return oq, ov, ou


def step_mt(threads, qpos, qvel, warm, ctrl, friction, com, iterations=10, tol=1e-8, ls_max=40, ls_tol=1e-7,
            nsub=4):
    """``step`` on ``threads`` host threads (contiguous shares of the worlds; the same results)."""
    qpos = _c(qpos, (-1, NQ))
    B = qpos.shape[0]
    qvel, warm, ctrl = _c(qvel, (B, NV)), _c(warm, (B, NV)), _c(ctrl, (B, NU))
    friction, com = _c(friction, (B,)), _c(com, (B, 3))
    oq, ov, ow = np.empty((B, NQ)), np.empty((B, NV)), np.empty((B, NV))
    info = np.empty((B, 4), np.int32)
    lib().g1o_step_mt(int(threads), B, _p(qpos), _p(qvel), _p(warm), _p(ctrl), _p(friction), _p(com), int(iterations),
                      float(tol), int(ls_max), float(ls_tol), int(nsub), _p(oq), _p(ov), _p(ow),
                      info.ctypes.data_as(ctypes.POINTER(ctypes.c_int)))
    return oq, ov, ow, info


NPAIR = 502  # the model's collision pairs (the freeze hook's table rows)


def vjp(qpos, qvel, warm, ctrl, friction, com, g_qpos, g_qvel, clamp_kv=1, normal=0, clamp_soft=0.2, iterations=10,
        tol=1e-8, ls_max=40, ls_tol=1e-7, nsub=4, normal_eps=1e-3, parallel_eps=1.2e-3, flops=False):
    """Analytic VJP of one control step in float64 (the oracle's adjoint): (g_qpos (B, 36) qpos form, g_qvel (B, 35),
    g_ctrl (B, 29)) from the output cotangents (g_qpos' (B, 36) qpos form, g_qvel' (B, 35)). normal_eps and
    parallel_eps are the eps of the normal options 2 / 3 and the near-parallel rule's sin^2 threshold (the reference's
    compile-time 1e-3 m and 1.2e-3, which the GPU library uses); the checker varies them to pin the options.
    flops=True also returns each world-step VJP's algorithmic flops (B,) last: closed-form phase counts of what the
    adjoint computes from the records (g1_oracle.cpp VJP_FLOPS_*), the forward's step(flops=True) counterpart."""
    qpos = _c(qpos, (-1, NQ))
    B = qpos.shape[0]
    qvel, warm, ctrl = _c(qvel, (B, NV)), _c(warm, (B, NV)), _c(ctrl, (B, NU))
    friction, com = _c(friction, (B,)), _c(com, (B, 3))
    gq, gv = _c(g_qpos, (B, NQ)), _c(g_qvel, (B, NV))
    oq, ov, ou, fl = np.empty((B, NQ)), np.empty((B, NV)), np.empty((B, NU)), np.empty(B)
    lib().g1o_vjp_count(B, _p(qpos), _p(qvel), _p(warm), _p(ctrl), _p(friction), _p(com), int(iterations), float(tol),
                        int(ls_max), float(ls_tol), int(nsub), _p(gq), _p(gv), int(clamp_kv), int(normal),
                        float(clamp_soft), float(normal_eps), float(parallel_eps), _p(oq), _p(ov), _p(ou), _p(fl))
    return (oq, ov, ou, fl) if flops else (oq, ov, ou)


def fd_jacobian(qpos, qvel, warm, ctrl, friction, com, h=1e-6, **kw):
    """Central-difference Jacobian of one state's control step (71 outputs: qpos' 36 | qvel' 35) in the columns
    (qpos tangent 35 | qvel 35 | ctrl 29), qpos perturbed with integrate_pos (benchmarks/bench/truth/fdlib.py fd_job's
    construction)."""
    q0, v0, u0 = (np.asarray(x, np.float64) for x in (qpos, qvel, ctrl))
    Q, V, U = [], [], []
    for j in range(2 * NV + NU):
        for sg in (1.0, -1.0):
            q, v, u = q0.copy(), v0.copy(), u0.copy()
            if j < NV:
                d = np.zeros(NV)
                d[j] = sg * h
                q = integrate_pos(q0, d)
            elif j < 2 * NV:
                v[j - NV] += sg * h
            else:
                u[j - 2 * NV] += sg * h
            Q.append(q); V.append(v); U.append(u)
    n = len(Q)
    oq, ov, _, _ = step(np.array(Q), np.array(V), np.tile(warm, (n, 1)), np.array(U), np.full(n, float(friction)),
                        np.tile(com, (n, 1)), **kw)
    out = np.concatenate([oq, ov], 1).reshape(2 * NV + NU, 2, NQ + NV)
    return (out[:, 0] - out[:, 1]).T / (2 * h)


def fd_vjp(qpos, qvel, warm, ctrl, friction, com, g_qpos, g_qvel, h=1e-6, threads=None, **kw):
    """Central-difference VJPs of B states' control steps, (B, 99) in the columns (qpos tangent 35 | qvel 35 |
    ctrl 29): the cotangents (g_qpos (B, 36) qpos form | g_qvel (B, 35)) times ``fd_jacobian``'s columns, all
    198 B perturbed steps in one ``step_mt`` call on ``threads`` host threads (default: the usable cores, at most 16)."""
    import os
    qpos = _c(qpos, (-1, NQ))
    B = qpos.shape[0]
    qvel, warm, ctrl = _c(qvel, (B, NV)), _c(warm, (B, NV)), _c(ctrl, (B, NU))
    friction, com = _c(friction, (B,)), _c(com, (B, 3))
    n = 2 * NV + NU
    Q = np.repeat(qpos, 2 * n, axis=0).reshape(B, n, 2, NQ)
    V = np.repeat(qvel, 2 * n, axis=0).reshape(B, n, 2, NV)
    U = np.repeat(ctrl, 2 * n, axis=0).reshape(B, n, 2, NU)
    for j in range(NV):
        for s, sg in ((0, 1.0), (1, -1.0)):
            d = np.zeros((B, NV))
            d[:, j] = sg * h
            Q[:, j, s] = integrate_pos(qpos, d)
            V[:, NV + j, s, j] += sg * h
    for j in range(NU):
        U[:, 2 * NV + j, 0, j] += h
        U[:, 2 * NV + j, 1, j] -= h
    if threads is None:
        threads = min(16, len(os.sched_getaffinity(0)))
    rep = lambda a: np.repeat(a, 2 * n, axis=0)
    oq, ov, _, _ = step_mt(threads, Q.reshape(-1, NQ), V.reshape(-1, NV), rep(warm), U.reshape(-1, NU), rep(friction),
                           rep(com), **kw)
    out = np.concatenate([oq, ov], 1).reshape(B, n, 2, NQ + NV)
    J = (out[:, :, 0] - out[:, :, 1]) / (2 * h)  # (B, 99, 71): d output / d input column
    c = np.concatenate([_c(g_qpos, (B, NQ)), _c(g_qvel, (B, NV))], 1)
    return np.einsum("bio,bo->bi", J, c)


def substep_hessian(qpos, qvel, warm, ctrl, friction, com, iterations=2000, tol=1e-13, ls_max=100, ls_tol=1e-12):
    """One substep of one state: (M (35, 35) at the input state, H (35, 35) = M + J'DJ on the rows in the quadratic
    zone at Newton's final a*), float64 (the checker of a tape record's factors)."""
    M, H = np.empty((NV, NV)), np.empty((NV, NV))
    lib().g1o_substep_hessian(_p(_c(qpos, NQ)), _p(_c(qvel, NV)), _p(_c(warm, NV)), _p(_c(ctrl, NU)), float(friction),
                              _p(_c(com, 3)), int(iterations), float(tol), int(ls_max), float(ls_tol), _p(M), _p(H))
    return M, H


def ltl(A):
    """The leaf-first factor A = L' L (L lower triangular, positive diagonal; eliminated from the last row up, as the
    engine and MuJoCo factor M) of a symmetric positive definite A, float64."""
    A = np.array(A, np.float64, copy=True)
    n = len(A)
    L = np.zeros_like(A)
    for k in range(n - 1, -1, -1):
        L[k, k] = np.sqrt(A[k, k])
        L[k, :k] = A[k, :k] / L[k, k]
        A[:k, :k] -= np.outer(L[k, :k], L[k, :k])
    return L


def smooth(qpos, qvel, ctrl, com):
    """Smooth dynamics of one state: M (35, 35), qfrc_smooth, qacc_smooth, xpos (31, 3), xquat (31, 4)."""
    M, qsm, qa = np.empty((NV, NV)), np.empty(NV), np.empty(NV)
    xp, xq = np.empty((NB, 3)), np.empty((NB, 4))
    lib().g1o_smooth(_p(_c(qpos, NQ)), _p(_c(qvel, NV)), _p(_c(ctrl, NU)), _p(_c(com, 3)), _p(M), _p(qsm), _p(qa),
                     _p(xp), _p(xq))
    return M, qsm, qa, xp, xq


def contacts(qpos, qvel, ctrl, com, friction):
    """Contacts of one state at its input pose: (n, 15) rows (pair, slot, dist, pos[3], frame[9])."""
    out = np.empty((64, 15))
    n = lib().g1o_contacts(_p(_c(qpos, NQ)), _p(_c(qvel, NV)), _p(_c(ctrl, NU)), _p(_c(com, 3)), float(friction),
                           _p(out))
    return out[:n].copy()


def quat_mul(a, b):
    w1, x1, y1, z1 = np.moveaxis(a, -1, 0)
    w2, x2, y2, z2 = np.moveaxis(b, -1, 0)
    return np.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2, w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                     w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2, w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2], -1)


def integrate_pos(qpos, dq, scale=1.0):
    """MuJoCo's mj_integratePos for the G1 (free root, then hinges): qpos (.., 36) moved by the tangent dq (.., 35)
    times scale; the root quaternion is rotated by the local rotation vector dq[3:6] scale (reference/jax64.py:686-698,
    the convention of fdlib.py's FD columns)."""
    qpos = np.array(qpos, np.float64, copy=True)
    dq = np.asarray(dq, np.float64) * scale
    qpos[..., :3] += dq[..., :3]
    w = dq[..., 3:6]
    ang = np.linalg.norm(w, axis=-1, keepdims=True)
    safe = np.where(ang > 0, ang, 1.0)
    dqq = np.concatenate([np.cos(0.5 * ang), np.sin(0.5 * ang) * w / safe], -1)
    q = quat_mul(qpos[..., 3:7], dqq)
    qpos[..., 3:7] = q / np.linalg.norm(q, axis=-1, keepdims=True)
    qpos[..., 7:] += dq[..., 6:]
    return qpos


def qpos_tangent(qpos, g_qpos):
    """A qpos-form cotangent (.., 36) as a tangent-space cotangent (.., 35): the transpose of the map dq -> d qpos of
    integrate_pos at dq = 0 (reference/adjoint_groups.py:218-226 qpos_tangent): root position as is, the root
    quaternion's cotangent through d quat / d w = 0.5 quat * (0, w), hinges as is."""
    qpos, g = np.asarray(qpos, np.float64), np.asarray(g_qpos, np.float64)
    out = np.zeros(g.shape[:-1] + (NV,))
    out[..., :3] = g[..., :3]
    out[..., 6:] = g[..., 7:]
    q = qpos[..., 3:7]
    for k in range(3):
        e = np.zeros(4)
        e[1 + k] = 1.0
        dqk = 0.5 * quat_mul(q, np.broadcast_to(e, q.shape))
        out[..., 3 + k] = np.sum(g[..., 3:7] * dqk, -1)
    return out


KIN_SHAPES = ((NQ,), (NB, 3), (NB, 4), (NB, 6), (NB, 3))  # qpos_n, xpos, xquat, cvel, subtree_com per world


def kinematics(qpos, qvel, com):
    """Kinematics outputs of states (B, 36), (B, 35), (B, 3): (qpos_n (B, 36), xpos (B, 31, 3), xquat (B, 31, 4),
    cvel (B, 31, 6), subtree_com (B, 31, 3)), float64 (MJX kinematics + com_pos + com_vel semantics,
    g1_engine/kinematics.py:1-45)."""
    qpos = np.ascontiguousarray(np.asarray(qpos, np.float64).reshape(-1, NQ))
    B = qpos.shape[0]
    qvel, com = _c(qvel, (B, NV)), _c(com, (B, 3))
    out = [np.empty((B,) + s) for s in KIN_SHAPES]
    lib().g1o_kinematics(B, _p(qpos), _p(qvel), _p(com), *map(_p, out))
    return tuple(out)


def kinematics_vjp(qpos, qvel, com, cot, h=1e-6):
    """VJP of ``kinematics`` by central differences (float64): cotangents cot = (g_qpos_n, g_xpos, g_xquat, g_cvel,
    g_subtree_com) of one batch -> (g_qpos (B, 36), g_qvel (B, 35)); qpos's quaternion entries are perturbed
    independently (the map normalizes them), as a VJP through MJX's normalization differentiates."""
    qpos, qvel, com = _c(qpos, (-1, NQ)), _c(qvel, (-1, NV)), _c(com, (-1, 3))
    B = qpos.shape[0]
    cot = [np.asarray(c, np.float64).reshape((B,) + s) for c, s in zip(cot, KIN_SHAPES)]
    gq, gv = np.zeros((B, NQ)), np.zeros((B, NV))
    for which, g, n in ((0, gq, NQ), (1, gv, NV)):
        for j in range(n):
            x = [qpos.copy(), qvel.copy()]
            x[which][:, j] += h
            up = kinematics(x[0], x[1], com)
            x[which][:, j] -= 2 * h
            dn = kinematics(x[0], x[1], com)
            g[:, j] = sum(((a - b) * c).reshape(B, -1).sum(1) for a, b, c in zip(up, dn, cot)) / (2 * h)
    return gq, gv
