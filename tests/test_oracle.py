"""The float64 CPU oracle pinned against the reference's committed MuJoCo data and against closed forms (CPU only)."""
import json
import os

import numpy as np
import pytest

import oracle
from nablaengine_amd import synthetic

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODEL = synthetic.model()


def _golden(cname):
    z = np.load(os.path.join(GOLD, f"truth_{cname}.npz"))
    st = dict(qpos=z["qpos"], qvel=z["qvel"], warm=z["qacc_warmstart"], ctrl=z["ctrl"], friction=z["friction"],
              com=z["com"])
    return {k: v.astype(np.float64) for k, v in st.items()}, z


@pytest.mark.parametrize("cname", ["mf_s0", "mf_s1", "mf_s2", "mf_s3"])
def test_step_matches_mujoco_truth(cname):
    """The control step at MuJoCo C's truth settings against MuJoCo C float64 (check_out, 64 states per corpus): the
    median relative error is at float64 round-off, and >= 90% of the states agree to 1e-10 (the rest are states where
    MuJoCo C's collision conventions differ from MuJoCo Warp's, which the engine follows)."""
    st, z = _golden(cname)
    oq, ov, _, _ = oracle.step(**st, **oracle.TRUTH)
    ref = z["check_out"]
    ev = np.linalg.norm(ov - ref[:, 36:], axis=1) / np.linalg.norm(ref[:, 36:], axis=1)
    eq = np.linalg.norm(oq - ref[:, :36], axis=1) / np.linalg.norm(ref[:, :36], axis=1)
    assert np.median(ev) < 1e-12 and np.median(eq) < 1e-12
    assert (ev < 1e-10).mean() >= 0.9


def test_contacts_match_mujoco_warp():
    """The narrowphase at the input state against MuJoCo Warp 3.17's contacts (pair, dist, pos, normal) on 512 corpus
    states: the same (pair) multiset in >= 99% of the states, and matched contacts agree in dist / pos / normal."""
    z = np.load(os.path.join(GOLD, "mjw_mf_s0.npz"))
    same, n = 0, len(z["con_count"])
    for i in range(n):
        c = oracle.contacts(z["qpos"][i], z["qvel"][i], z["ctrl"][i], z["com"][i], z["friction"][i])
        k = int(z["con_count"][i])
        ref = z["con"][i, :k]
        if sorted(c[:, 0].astype(int).tolist()) != sorted(ref[:, 0].astype(int).tolist()):
            continue
        same += 1
        for row in ref:  # each MuJoCo Warp contact has an oracle contact of its pair at the same point
            cand = c[c[:, 0] == row[0]]
            d = np.min(np.linalg.norm(cand[:, 3:6] - row[2:5], axis=1))
            j = int(np.argmin(np.linalg.norm(cand[:, 3:6] - row[2:5], axis=1)))
            assert d < 1e-4 and abs(cand[j, 2] - row[1]) < 1e-5
            assert np.linalg.norm(cand[j, 6:9] - row[5:8]) < 1e-4
    assert same / n >= 0.99, same / n


def _com_positions(xpos, xquat):
    ip = np.asarray(MODEL["body_ipos"]).reshape(-1, 3)
    out = np.zeros_like(xpos)
    for b in range(len(xpos)):
        out[b] = xpos[b] + oracle.quat_mul(oracle.quat_mul(xquat[b], np.r_[0, ip[b]]), xquat[b] * [1, -1, -1, -1])[1:]
    return out


def test_mass_matrix_closed_forms():
    """M is symmetric positive definite, and 0.5 v' M v equals the bodies' kinetic energy (COM and angular
    velocities from central differences of the poses along v, plus the armature) for random v: a quadratic form that
    pins every entry of M (polarization)."""
    st = synthetic.states(3, config=1, dtype=np.float64)
    mass = np.asarray(MODEL["body_mass"])
    inert = np.asarray(MODEL["body_inertia"]).reshape(-1, 3)
    iquat = np.asarray(MODEL["body_iquat"]).reshape(-1, 4)
    arm = np.asarray(MODEL["dof_armature"])
    rng = np.random.default_rng(0)
    for i in range(3):
        q = st["qpos"][i]
        M, _, _, xp, xq = oracle.smooth(q, st["qvel"][i], st["ctrl"][i], np.zeros(3))
        assert np.allclose(M, M.T, atol=1e-12)
        assert np.linalg.eigvalsh(M).min() > 0
        for _ in range(3):
            v = rng.normal(0, 1, 35)
            h = 1e-6
            _, _, _, xp1, xq1 = oracle.smooth(oracle.integrate_pos(q, v, h), v, st["ctrl"][i], np.zeros(3))
            _, _, _, xp0, xq0 = oracle.smooth(oracle.integrate_pos(q, v, -h), v, st["ctrl"][i], np.zeros(3))
            vc = (_com_positions(xp1, xq1) - _com_positions(xp0, xq0)) / (2 * h)
            T = 0.5 * np.sum(arm * v * v)
            for b in range(1, 31):
                dqq = (xq1[b] - xq0[b]) / (2 * h)
                w = 2 * oracle.quat_mul(dqq, xq[b] * [1, -1, -1, -1])[1:]  # world angular velocity
                R = oracle.quat_mul(xq[b], iquat[b])
                wl = oracle.quat_mul(oracle.quat_mul(R * [1, -1, -1, -1], np.r_[0, w]), R)[1:]  # in the inertia frame
                T += 0.5 * mass[b] * vc[b] @ vc[b] + 0.5 * np.sum(inert[b] * wl * wl)
            assert abs(0.5 * v @ M @ v - T) <= 1e-7 * abs(T), (0.5 * v @ M @ v, T)


def test_gravity_torque_is_potential_gradient():
    """At rest with the PD setpoints at the joint angles (no actuator force), qfrc_smooth = -bias = -dU/dq with
    U = sum_b m_b 9.81 z_com,b: central differences of U along every dof tangent."""
    st = synthetic.states(2, config=1, dtype=np.float64)
    mass = np.asarray(MODEL["body_mass"])
    for i in range(2):
        q = st["qpos"][i]
        _, qsm, _, _, _ = oracle.smooth(q, np.zeros(35), q[7:], np.zeros(3))

        def U(qq):
            _, _, _, xp, xq = oracle.smooth(qq, np.zeros(35), qq[7:], np.zeros(3))
            return float(np.sum(mass * 9.81 * _com_positions(xp, xq)[:, 2]))

        h = 1e-6
        g = np.array([(U(oracle.integrate_pos(q, np.eye(35)[j], h)) - U(oracle.integrate_pos(q, np.eye(35)[j], -h)))
                      / (2 * h) for j in range(35)])
        assert np.allclose(qsm, -g, atol=1e-6 * np.abs(g).max())


def test_integrate_pos_and_tangent():
    """integrate_pos keeps the quaternion unit and is a group action (two steps = one of the sum along a hinge);
    qpos_tangent is the transpose of d integrate_pos / d dq at 0 (central differences of a linear functional)."""
    st = synthetic.states(4, config=1, dtype=np.float64)
    rng = np.random.default_rng(1)
    for q in st["qpos"]:
        dq = rng.normal(0, 0.3, 35)
        q1 = oracle.integrate_pos(q, dq)
        assert abs(np.linalg.norm(q1[3:7]) - 1) < 1e-12
        g = rng.normal(0, 1, 36)
        t = oracle.qpos_tangent(q, g)
        h = 1e-6
        fd = np.array([(g @ oracle.integrate_pos(q, np.eye(35)[j], h) - g @ oracle.integrate_pos(q, np.eye(35)[j], -h))
                       / (2 * h) for j in range(35)])
        assert np.allclose(t, fd, atol=1e-7)


def _vjp_block_errors(an, fd):
    e = {}
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        e[name] = np.linalg.norm(an[..., sl] - fd[..., sl], axis=-1) / np.maximum(np.linalg.norm(fd[..., sl], axis=-1),
                                                                                  1e-12)
    return e


def test_fd_machinery_and_adjoint_vs_mujoco_fd():
    """The oracle's central FD (integrate_pos columns) reproduces MuJoCo C's fd_vjp on G0 states, and the oracle's
    analytic VJP (exact mode) matches both; a gradient perturbed by 3e-3 (relative) fails the 1e-4 gate (the gate
    detects a plausible mistake)."""
    g = np.load(os.path.join(GOLD, "grad_mf_s0.npz"))
    sel = np.nonzero(g["G0"])[0][:4]
    for s in sel:
        q, v, w, u = [g[k][s].astype(np.float64) for k in ("qpos", "qvel", "qacc_warmstart", "ctrl")]
        f, c = float(g["friction"][s]), g["com"][s].astype(np.float64)
        cq, cv = g["cot_qpos"][s].astype(np.float64), g["cot_qvel"][s].astype(np.float64)
        J = oracle.fd_jacobian(q, v, w, u, f, c, **oracle.TRUTH)
        fd = np.concatenate([cq, cv], 1) @ J
        ok = g["bad"][s] == 0
        truth = np.where(ok, g["fd_vjp"][s], 0)
        for name, e in _vjp_block_errors(np.where(ok, fd, 0), truth).items():
            assert np.median(e) < 1e-5, (name, e)
        gq, gv, gu = oracle.vjp(np.tile(q, (3, 1)), np.tile(v, (3, 1)), np.tile(w, (3, 1)), np.tile(u, (3, 1)),
                                np.full(3, f), np.tile(c, (3, 1)), cq, cv, clamp_kv=1, normal=0, **oracle.TRUTH)
        an = np.concatenate([oracle.qpos_tangent(q, gq), gv, gu], 1)
        for name, e in _vjp_block_errors(an, fd).items():
            assert np.median(e) < 1e-5, (name, e)
        rng = np.random.default_rng(int(s))
        bad = an * (1 + 3e-3 * rng.choice([-1.0, 1.0], an.shape))
        assert all(np.median(e) > 1e-4 for e in _vjp_block_errors(bad, fd).values())


def test_gradient_gate_self_test():
    """The reference's gradient gates (tests/gradient_gates.py) pass for the oracle's analytic VJP (exact mode, the
    truth's solver settings) on mf_s0's model_ok G0 states, and fail for the same VJPs moved by 3e-3 relative per
    state, cotangent and block (scripts/gradient_check.py's perturbed_must_fail)."""
    from gradient_gates import block_scores, passes, perturb, truth_states
    z = np.load(os.path.join(GOLD, "grad_mf_s0.npz"))
    sel, st, cq, cv = truth_states(z, "G0")
    sel, cq, cv = sel[:24], cq[:24], cv[:24]
    st = {k: v[:24] for k, v in st.items()}
    n = len(sel)
    g = np.zeros((n, 3, 99))
    for c in range(3):
        gq, gv, gu = oracle.vjp(**st, g_qpos=cq[:, c], g_qvel=cv[:, c], clamp_kv=1, normal=0, **oracle.TRUTH)
        g[:, c] = np.concatenate([oracle.qpos_tangent(st["qpos"], gq), gv, gu], 1)
    valid = z["bad"][sel] == 0
    ok, stats = passes(block_scores(g, z["fd_vjp"][sel], z["fd_vjp_floor"][sel], valid))
    assert ok, stats
    bad, stats_bad = passes(block_scores(perturb(g, 3e-3), z["fd_vjp"][sel], z["fd_vjp_floor"][sel], valid))
    assert not bad, stats_bad


KP, KV, FRCLIM = (np.asarray(MODEL[k]) for k in ("dof_kp", "dof_kv", "dof_frclim"))
ONE_SUBSTEP = dict(oracle.TRUTH, nsub=1)


def _lam_by_fd(s64, cq, cv, h=1e-6):
    """lambda of a one-substep step by central differences: the output loss's derivative with respect to a generalized
    force added to qfrc_smooth (the oracle's qfrc hook). lambda = H^-1 a* bar is that derivative, since qfrc_smooth
    enters the step only through the constrained solve (its IFT gives d a* / d qfrc = H^-1)."""
    B = len(cq)
    rep = {k: np.repeat(v, 2 * oracle.NV, axis=0) for k, v in s64.items()}
    Q = np.zeros((B, oracle.NV, 2, oracle.NV))
    for j in range(oracle.NV):
        Q[:, j, 0, j], Q[:, j, 1, j] = h, -h
    oq, ov, _, _ = oracle.step(**rep, qfrc=Q.reshape(-1, oracle.NV), **ONE_SUBSTEP)
    L = ((oq * np.repeat(cq, 2 * oracle.NV, 0)).sum(1) + (ov * np.repeat(cv, 2 * oracle.NV, 0)).sum(1))
    L = L.reshape(B, oracle.NV, 2)
    return (L[:, :, 0] - L[:, :, 1]) / (2 * h)


@pytest.mark.parametrize("config", [1, 4])
def test_clamp_variants_against_lambda_by_fd(config):
    """The three clamp_kv modes pinned through lambda measured by finite differences (one substep, so one lambda; 64
    states with clamped actuators on about half of them). With the PD force f = kp (u - q) - kv v clamped at +-tau
    (clamped: |f| >= tau, computed here in numpy), the reference's definitions (adjoint.py:43-56,811-846) are:
    clamp_kv=1 (exact): g_ctrl = kp lambda on unclamped dofs and 0 on clamped ones; clamp_kv=0 (MuJoCo Warp's): the
    same except g_qvel gets -kv lambda more on the clamped dofs, nothing else changes; clamp_kv=2 (soft, delta): on a
    clamped dof all three actuator paths take w lambda, w = exp(-max((|f| - tau) / tau, 0) / delta), so
    g_ctrl = w kp lambda and g_qpos / g_qvel differ from clamp_kv=1 by -w kp lambda / -w kv lambda; delta -> 0 gives
    clamp_kv=1. A dropped term, a wrong sign or a weight on the wrong path fails one of these."""
    st = synthetic.states(64, config=config, dtype=np.float64)
    cq, cv = synthetic.cotangents(64, dtype=np.float64)
    lam = _lam_by_fd(st, cq, cv)
    raw = KP[6:] * (st["ctrl"] - st["qpos"][:, 7:]) - KV[6:] * st["qvel"][:, 6:]
    cl = np.abs(raw) >= FRCLIM[6:]
    assert cl.any(1).sum() >= 30
    V = lambda kv, **kw: oracle.vjp(**st, g_qpos=cq, g_qvel=cv, clamp_kv=kv, normal=0, **ONE_SUBSTEP, **kw)
    g1, g0 = V(1), V(0)
    klam = KP[6:] * lam[:, 6:]
    sc = np.abs(klam).max()
    assert np.abs(g1[2] - np.where(cl, 0.0, klam)).max() < 1e-5 * sc
    assert np.array_equal(g0[0], g1[0]) and np.array_equal(g0[2], g1[2])
    d = g0[1] - g1[1]
    assert np.abs(d[:, :6]).max() == 0
    assert np.abs(d[:, 6:] - np.where(cl, -KV[6:] * lam[:, 6:], 0.0)).max() < 1e-5 * sc
    o = np.maximum((np.abs(raw) - FRCLIM[6:]) / FRCLIM[6:], 0.0)
    for delta in (0.05, 0.2, 1.0):
        g2 = V(2, clamp_soft=delta)
        w = np.where(cl, np.exp(-o / delta), 1.0)
        assert np.abs(g2[2] - w * klam).max() < 1e-5 * sc
        assert np.abs(g2[1][:, 6:] - g1[1][:, 6:] - np.where(cl, -w * KV[6:] * lam[:, 6:], 0.0)).max() < 1e-5 * sc
        assert np.abs(g2[0][:, 7:] - g1[0][:, 7:] - np.where(cl, -w * klam, 0.0)).max() < 1e-5 * sc
        assert np.array_equal(g2[1][:, :6], g1[1][:, :6])
    g2 = V(2, clamp_soft=1e-12)
    assert all(np.array_equal(a, b) for a, b in zip(g2, g1))


def _one_self_contact_worlds(st, n):
    """Indices of states with exactly one self contact (a pair of robot geoms) at the input pose, with its pair and
    nu = dist + r1 + r2 (the sphere core's centre distance)."""
    pg1, pg2 = np.asarray(MODEL["pair_g1"]), np.asarray(MODEL["pair_g2"])
    gt, gs = np.asarray(MODEL["geom_type"]), np.asarray(MODEL["geom_size"]).reshape(-1, 3)
    out = []
    for w in range(len(st["qpos"])):
        c = oracle.contacts(st["qpos"][w], st["qvel"][w], st["ctrl"][w], st["com"][w], st["friction"][w])
        sc = [r for r in c if gt[pg1[int(r[0])]] != 0]
        if len(sc) == 1:
            p = int(sc[0][0])
            out.append((w, p, sc[0][2] + gs[pg1[p], 0] + gs[pg2[p], 0]))
        if len(out) == n:
            break
    return out


def test_normal_options_through_kappa():
    """The normal options pinned against the exact mode (normal 0, pinned by FD) on contact-heavy states with exactly
    one self contact (one substep, the near-parallel rule off: parallel_eps 0). The options differ only in kappa(nu),
    the factor of the sphere core's normal derivative kappa (I - n n') (adjoint_contact.py:239-262): 0 exact 1 / nu,
    1 frozen 0, 2 1 / max(nu, eps), 3 nu < eps ? 0 : 1 / nu. The VJP is affine in kappa, g(kappa) = g1 + kappa nu
    (g0 - g1) with g1 normal 1's, so: option 2 and 3 with eps below nu equal option 0 bitwise; option 3 with eps above
    nu equals option 1; option 2 with eps above nu is linear in 1 / eps, and its slope fits nu = dist + r1 + r2 of
    the contact's geometry to 1e-9 (on the states whose self contact has a quadratic row, where g0 != g1)."""
    st = synthetic.states(768, config=4, dtype=np.float64)
    one = _one_self_contact_worlds(st, 32)
    assert len(one) >= 24
    sel = np.array([w for w, _, _ in one])
    nus = np.array([nu for _, _, nu in one])
    sub = {k: v[sel] for k, v in st.items()}
    cq, cv = synthetic.cotangents(len(sel), dtype=np.float64)
    G = lambda n, **kw: np.concatenate(oracle.vjp(**sub, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=n, parallel_eps=0.0,
                                                  **ONE_SUBSTEP, **kw), 1)
    g0, g1 = G(0), G(1)
    assert np.array_equal(G(2, normal_eps=1e-9), g0) and np.array_equal(G(3, normal_eps=1e-9), g0)
    assert np.array_equal(G(3, normal_eps=1.0), g1)
    ga, gb = G(2, normal_eps=1.0), G(2, normal_eps=0.5)
    sc = np.abs(g0).max(1, keepdims=True)
    assert (np.abs((gb - g1) - 2 * (ga - g1)) / sc).max() < 1e-12
    d = g0 - g1
    row = np.abs(d).max(1) > 1e-9 * sc[:, 0]
    assert row.sum() >= 12
    nufit = (d * (ga - g1)).sum(1)[row] / (d * d).sum(1)[row]
    assert np.abs(nufit / nus[row] - 1).max() < 1e-9
    assert np.median(np.abs(d[row]).max(1) / sc[row, 0]) > 1e-2  # the frame's derivative matters


def _fd_vjp(s1, cq, cv, h, **kw):
    J = oracle.fd_jacobian(*(s1[k][0] for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")), h=h, **kw)
    return np.concatenate([cq[0], cv[0]]) @ J


def test_near_parallel_rule_is_the_frozen_parameter_gradient():
    """The near-parallel rule (normal options != 0, adjoint_contact.py:436-448): a capsule-capsule contact whose two
    segment parameters are both free has them held constant in the VJP where sin^2(theta) < 1.2e-3. With the
    threshold raised to 1 (every both-free pair held) and kappa exact (option 2 at eps 1e-9), the VJP must be the
    exact gradient of the forward in which those parameters are frozen at their values (the oracle's freeze hook:
    recorded on the nominal run, replayed in every finite-difference run), and on two states where the held contact
    has a row that matters it must differ from the unfrozen exact VJP. One substep, contact-heavy states with such a
    contact, where the finite differences are smooth (h and h / 10 agree)."""
    st = synthetic.states(256, config=4, dtype=np.float64)
    pg1, gt = np.asarray(MODEL["pair_g1"]), np.asarray(MODEL["geom_type"])
    pg2 = np.asarray(MODEL["pair_g2"])
    done = 0
    for w in range(len(st["qpos"])):
        s1 = {k: v[w:w + 1] for k, v in st.items()}
        c = oracle.contacts(s1["qpos"][0], s1["qvel"][0], s1["ctrl"][0], s1["com"][0], s1["friction"][0])
        fz = np.zeros((oracle.NPAIR, 3))
        oracle.step(**s1, freeze=fz, freeze_mode=1, **ONE_SUBSTEP)
        if not any(fz[int(r[0]), 0] and gt[pg1[int(r[0])]] == 3 and gt[pg2[int(r[0])]] == 3 for r in c):
            continue
        cq, cv = synthetic.cotangents(1, seed=w, dtype=np.float64)
        plain = _fd_vjp(s1, cq, cv, 1e-6, **ONE_SUBSTEP)
        if np.linalg.norm(plain - _fd_vjp(s1, cq, cv, 1e-7, **ONE_SUBSTEP)) > 1e-4 * np.linalg.norm(plain):
            continue  # a row switching on within +-h (the step is not smooth here)
        fd = np.zeros(99)
        J = []
        for j in range(99):
            out = []
            for sg in (1.0, -1.0):
                q, v, u = s1["qpos"].copy(), s1["qvel"].copy(), s1["ctrl"].copy()
                if j < 35:
                    dq = np.zeros(35)
                    dq[j] = sg * 1e-6
                    q = oracle.integrate_pos(q, dq)
                elif j < 70:
                    v[0, j - 35] += sg * 1e-6
                else:
                    u[0, j - 70] += sg * 1e-6
                oq, ov, _, _ = oracle.step(q, v, s1["warm"], u, s1["friction"], s1["com"], freeze=fz, freeze_mode=2,
                                           **ONE_SUBSTEP)
                out.append(np.concatenate([oq[0], ov[0]]))
            J.append((out[0] - out[1]) / 2e-6)
        fd = np.concatenate([cq[0], cv[0]]) @ np.array(J).T
        tang = lambda g: np.concatenate([oracle.qpos_tangent(s1["qpos"][0], g[0][0]), g[1][0], g[2][0]])
        held = tang(oracle.vjp(**s1, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=2, normal_eps=1e-9, parallel_eps=1.0,
                               **ONE_SUBSTEP))
        exact = tang(oracle.vjp(**s1, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=0, **ONE_SUBSTEP))
        assert np.linalg.norm(held - fd) < 1e-6 * np.linalg.norm(fd), w
        if np.linalg.norm(exact - fd) > 1e-3 * np.linalg.norm(fd):  # the held contact has a row that matters
            done += 1
            if done == 2:
                break
    assert done == 2


def test_ten_iteration_tail_is_the_iteration_cap():
    """On 1024 config-1 states the 10-iteration step differs from the converged one (MuJoCo's truth settings: 2000
    iterations, tolerance 1e-13) by p99 > 1e-3 in qvel, while 20 iterations already give the converged result to
    1e-13 on every world: the tail of the engine's default step against converged references is its iteration cap,
    not an error of the solver (an exact Newton method on a piecewise quadratic stops on the minimiser once its
    zones are right)."""
    st = synthetic.states(1024, config=1, dtype=np.float64)
    _, ov, _, _ = oracle.step(**st, **oracle.TRUTH)
    rel = lambda a: np.linalg.norm(a - ov, axis=1) / np.linalg.norm(ov, axis=1)
    e10 = rel(oracle.step(**st, **oracle.ENGINE)[1])
    e20 = rel(oracle.step(**st, **dict(oracle.ENGINE, iterations=20))[1])
    assert np.percentile(e10, 99) > 1e-3 and np.median(e10) < 1e-13
    assert e20.max() < 1e-13


def test_float32_yardstick():
    """oracle.step_f32 (the restatement with float storage) on 256 config-1 states: its outputs are float32 and not
    the float64 ones; where Newton converges (10 iterations) it equals the float64 step to float32 accuracy (qvel
    median <= 2e-6, p99 <= 2e-5); after one iteration its qvel is off by more than 10x that, because the first
    Newton direction solves H p = -g with cond(H) ~ 1e5-1e6 (the contacts' stiffness against M) and only further
    iterations wash the solve's rounding out. That is the float32 error floor a GPU step at a low iteration cap is
    held to."""
    st = synthetic.states(256, config=1, seed=31)
    d = {k: st[k].astype(np.float64) for k in st}
    rel = lambda a, b: np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-12)
    errs = {}
    for it in (1, 10):
        q32, v32, w32, i32 = oracle.step_f32(**st, iterations=it)
        q64, v64, w64, i64 = oracle.step(**d, **dict(oracle.ENGINE, iterations=it))
        assert v32.dtype == np.float32 and not np.array_equal(v32.astype(np.float64), v64)
        errs[it] = rel(v32, v64)
    ev = errs[10]
    assert np.median(ev) <= 2e-6 and np.percentile(ev, 99) <= 2e-5
    assert np.median(errs[1]) > 10 * np.median(ev)
    M, H = oracle.substep_hessian(*(d[k][0] for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")),
                                  iterations=0)
    assert np.linalg.cond(H) > 1e4


def test_ltl_is_the_reversed_cholesky():
    """oracle.ltl (the leaf-first factor A = L' L) against a textbook routine: with J the order reversal, J A J = C C'
    (numpy's Cholesky), so L = J C' J; on random SPD matrices and on M + h kv of a state."""
    rng = np.random.default_rng(3)
    mats = [X @ X.T + 35 * np.eye(35) for X in rng.normal(size=(4, 35, 35))]
    st = synthetic.states(2, config=1, dtype=np.float64)
    M = oracle.smooth(st["qpos"][0], st["qvel"][0], st["ctrl"][0], st["com"][0])[0]
    mats.append(M + MODEL["timestep"] * np.diag(KV))
    for A in mats:
        C = np.linalg.cholesky(A[::-1, ::-1])
        assert np.allclose(oracle.ltl(A), C.T[::-1, ::-1], rtol=1e-12, atol=1e-12 * np.abs(A).max())


def test_substep_hessian_against_fd():
    """oracle.substep_hessian's H (M + J'DJ at Newton's final zones) against finite differences of the step: at one
    substep the step's warm' output is a*, and within the final zones a* moves with a generalized force f added to
    qfrc_smooth as d a* / d f = H^-1 (the optimality condition M a - qfrc_smooth - f - J' f_c(a) = 0 is linear there).
    H^-1 from central differences (oracle qfrc hook) agrees to 1e-6 relative, on 8 config-1 states with active
    constraint rows; H is symmetric."""
    st = synthetic.states(8, config=1, dtype=np.float64)
    fd = 1e-5
    for w in range(8):
        s1 = {k: v[w:w + 1] for k, v in st.items()}
        M, H = oracle.substep_hessian(*(s1[k][0] for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")))
        Q = np.zeros((2 * oracle.NV, oracle.NV))
        for j in range(oracle.NV):
            Q[2 * j, j], Q[2 * j + 1, j] = fd, -fd
        rep = {k: np.repeat(v, 2 * oracle.NV, axis=0) for k, v in s1.items()}
        _, _, ow, _ = oracle.step(**rep, qfrc=Q, **ONE_SUBSTEP)
        Jw = ((ow[0::2] - ow[1::2]) / (2 * fd)).T  # d a* / d f, column j: f_j
        Hi = np.linalg.inv(H)
        assert np.abs(Jw - Hi).max() < 1e-6 * np.abs(Hi).max(), w
        assert np.abs(H - H.T).max() <= 1e-14 * np.abs(H).max()
        assert np.abs(H - M).max() > 1e-3 * np.abs(M).max()  # the states have active constraint rows


def test_flop_count_closed_form():
    """The algorithmic flop count: per world-step 4 x (smooth 2.5e4 + 2 x 3.1e4 factor-solves + 5e3 broadphase) plus
    the contact and Newton terms, so between 4.6e5 (no contacts, no iteration) and 1e7 on config-1 states."""
    st = synthetic.states(32, config=1, dtype=np.float64)
    r = oracle.step(**st, **oracle.ENGINE, flops=True)
    assert (r[4] >= 4 * (2.5e4 + 6.2e4 + 5e3)).all() and (r[4] < 1e7).all()


def test_vjp_flop_count_closed_form():
    """The VJP's algorithmic flop count: per world-step 4 x 3.76e4 for the smooth parts, plus 25 per limit row, 570 per
    contact and 90 per row in the quadratic zone; so at least 1.5e5 and below 1e6 on config-1 and config-4 states,
    larger where there are contacts; and counting leaves the gradients bitwise unchanged."""
    for config in (1, 4):
        st = synthetic.states(24, config=config, dtype=np.float64)
        cq, cv = (x.astype(np.float64) for x in synthetic.cotangents(24))
        r = oracle.vjp(**st, g_qpos=cq, g_qvel=cv, flops=True)
        plain = oracle.vjp(**st, g_qpos=cq, g_qvel=cv)
        assert all(np.array_equal(a, b) for a, b in zip(r[:3], plain))
        fl = r[3]
        assert (fl >= 4 * 3.76e4).all() and (fl < 1e6).all() and (fl > 4 * 3.76e4).any()
        _, _, _, info = oracle.step(**st, **oracle.ENGINE)
        assert np.corrcoef(fl, info[:, 1])[0, 1] > 0.5  # more contacts, more flops


def _jac_state(z, j):
    s = z["jac_index"][j]
    return ([z[k][s].astype(np.float64) for k in ("qpos", "qvel", "qacc_warmstart", "ctrl")]
            + [float(z["friction"][s]), z["com"][s].astype(np.float64)])


def test_fd_vjp_is_the_contracted_fd_jacobian():
    """fd_vjp (all perturbed steps of a batch in one step_mt call) equals the output cotangents times fd_jacobian's
    columns (each state's perturbed steps in one step call) to 1e-12, on config-1 and contact-heavy config-4 states:
    the batched FD the GPU's FD gates use is the textbook central difference."""
    for config, n in ((1, 3), (4, 3)):
        st = {k: v.astype(np.float64) for k, v in synthetic.states(n, config=config, seed=7).items()}
        cq, cv = (x.astype(np.float64) for x in synthetic.cotangents(n, seed=8))
        fd = oracle.fd_vjp(st["qpos"], st["qvel"], st["warm"], st["ctrl"], st["friction"], st["com"], cq, cv,
                           threads=3, **oracle.ENGINE)
        for b in range(n):
            J = oracle.fd_jacobian(*(st[k][b] for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")),
                                   **oracle.ENGINE)
            ref = np.concatenate([cq[b], cv[b]]) @ J
            assert np.linalg.norm(fd[b] - ref) <= 1e-12 * np.linalg.norm(ref), (config, b)


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_step_mt_is_step_bitwise(threads):
    """step_mt (the worlds split in contiguous shares over host threads: the CPU baseline's all-threads leg and
    fd_vjp's engine) gives bitwise step's outputs and info, every world being independent; on 40 config-1 and
    config-4 worlds (more threads than worlds of a share included)."""
    st = {k: np.concatenate([synthetic.states(20, config=c, seed=11)[k] for c in (1, 4)]).astype(np.float64)
          for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")}
    ref = oracle.step(**st, **oracle.ENGINE)
    got = oracle.step_mt(threads, **st, **oracle.ENGINE)
    for a, b in zip(got, ref):
        assert a.dtype == b.dtype and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("cname", ["mf_s0", "mf_s1"])
def test_fd_jacobian_matches_the_mujoco_jacobian(cname):
    """The oracle's central-difference Jacobian (integrate_pos qpos columns, at the truth's solver settings) against
    MuJoCo C's float64 FD Jacobian the truth stores (float32) for all its 64 G0 states, scored as the reference's
    jacobian_errors (benchmarks/bench/accuracy/gradient.py:193-208): per block (qpos tangent, qvel, ctrl) the
    Frobenius relative error over the valid columns. Median <= 2e-7 per block (measured 2.4e-8 to 3.2e-8, the truth's
    float32 storage), every state within max(3e-5, 2 x the truth's floor |J(1e-6) - J(1e-7)|) (measured max 1.5e-5);
    a column permutation (a transposed operand) fails it."""
    z = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
    blocks = {"qpos": slice(0, 35), "qvel": slice(35, 70), "ctrl": slice(70, 99)}
    errs = {name: [] for name in blocks}
    for j in range(len(z["jac_index"])):
        J = oracle.fd_jacobian(*_jac_state(z, j), **oracle.TRUTH)
        Jt = z["jacobian"][j].astype(np.float64)
        valid = z["bad"][z["jac_index"][j]] == 0
        for name, sl in blocks.items():
            v = valid[sl]
            a, b = J[:, sl][:, v], Jt[:, sl][:, v]
            nb = max(np.linalg.norm(b), 1e-9)
            floor = np.linalg.norm(z["jacobian_dcol"][j, sl][v]) / nb
            e = np.linalg.norm(a - b) / nb
            errs[name].append(e)
            assert e <= max(3e-5, 2 * floor), (cname, j, name, e, floor)
            assert np.linalg.norm(a[:, ::-1] - b) / nb > 1e-2
    assert len(z["jac_index"]) == 64
    for name, e in errs.items():
        assert np.median(e) <= 2e-7, (name, np.median(e))
