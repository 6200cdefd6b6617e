"""GPU parity of the adjoint (HIP kernel through the C ABI, via nablaengine_amd.torch_ffi) against float64 central
finite differences (MuJoCo C's fd_vjp golden fixtures, and the float64 oracle's own FD) and the oracle's float64
analytic VJP."""
import os

import numpy as np
import pytest

import oracle
from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4  # gradient median relative error <= 1e-4 against float64 central FD


@pytest.fixture(scope="module")
def ffi():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from nablaengine_amd import torch_ffi
    torch_ffi.init(0)
    return torch_ffi


def _t(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def _vjp_gpu(ffi, st, cq, cv, clamp_kv=1, normal=0, iterations=10, substeps=4):
    import torch
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    r = ffi.forward(*args, tape=True, iterations=iterations, substeps=substeps)
    kw = dict(ctrl=args[3], clamp_soft=None) if clamp_kv == 2 else {}
    gq, gv, gu, info = ffi.backward(r[4], args[4], args[5], _t(cq), _t(cv), clamp_kv=clamp_kv, normal=normal,
                                    substeps=substeps, **kw)
    torch.cuda.synchronize()
    return gq.cpu().numpy().astype(np.float64), gv.cpu().numpy().astype(np.float64), gu.cpu().numpy().astype(
        np.float64), info.cpu().numpy(), r


def _rel_rows(a, b):
    return np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-12)


@pytest.mark.parametrize("cname", ["mf_s0", "mf_s1"])
def test_adjoint_vs_mujoco_fd_truth(ffi, cname):
    """MuJoCo C float64 central FD VJPs (h = 1e-6, 3 cotangents per state) on the truth's G0 states, exact mode
    (clamp_kv=1, normal=0): median relative error per block (qpos tangent / qvel / ctrl) <= 1e-4 (BASELINE gate), on
    the columns the truth marks valid."""
    g = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
    sel = np.nonzero(g["G0"])[0]
    n = len(sel)
    st = {k: np.repeat(g[src][sel], 3, axis=0) for k, src in (("qpos", "qpos"), ("qvel", "qvel"),
                                                              ("warm", "qacc_warmstart"), ("ctrl", "ctrl"),
                                                              ("friction", "friction"), ("com", "com"))}
    cq = g["cot_qpos"][sel].reshape(3 * n, 36)
    cv = g["cot_qvel"][sel].reshape(3 * n, 35)
    gq, gv, gu, info, _ = _vjp_gpu(ffi, st, cq, cv)
    an = np.concatenate([oracle.qpos_tangent(st["qpos"].astype(np.float64), gq), gv, gu], 1)
    fd = g["fd_vjp"][sel].reshape(3 * n, 99)
    bad = np.repeat(g["bad"][sel] != 0, 3, axis=0)
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        a, b = np.where(bad[:, sl], 0, an[:, sl]), np.where(bad[:, sl], 0, fd[:, sl])
        e = _rel_rows(a, b)
        print(f"{cname} {name}: median {np.median(e):.3g} p90 {np.percentile(e, 90):.3g}")
        assert np.median(e) <= TOL, (name, np.median(e))
    assert not (info & (1 << 13)).any(), "a replayed contact was not found"


@pytest.mark.parametrize("cname", ["mf_s0", "mf_s1"])
def test_adjoint_reference_gradient_gates(ffi, cname):
    """The reference's gradient gates (scripts/gradient_check.py: its default 50 iterations, exact mode clamp_kv=1,
    normal=0, groups G0 / G4 / G5 / G6 on the model_ok states, tests/gradient_gates.py's scorer): per group and block
    the floored relative error's p99 <= 2e-3 / 5e-4 / 1e-4 (qpos tangent / qvel / ctrl) and the cosine's 1st percentile
    >= 0.99999; every gradient finite."""
    import torch
    from gradient_gates import block_scores, passes, truth_states
    z = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
    for group in ("G0", "G4", "G5", "G6"):
        sel, st, cq, cv = truth_states(z, group)
        n = len(sel)
        args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
        r = ffi.forward(*args, iterations=50, tape=True)
        g = np.zeros((n, 3, 99))
        for c in range(3):
            gq, gv, gu, info = ffi.backward(r[4], args[4], args[5], _t(cq[:, c]), _t(cv[:, c]), clamp_kv=1, normal=0)
            torch.cuda.synchronize()
            gq, gv, gu = (x.cpu().numpy().astype(np.float64) for x in (gq, gv, gu))
            g[:, c] = np.concatenate([oracle.qpos_tangent(st["qpos"], gq), gv, gu], 1)
        assert np.isfinite(g).all()
        ok, stats = passes(block_scores(g, z["fd_vjp"][sel], z["fd_vjp_floor"][sel], z["bad"][sel] == 0))
        print(f"{cname} {group} ({n} states): " + ", ".join(f"{b} p99 {p:.3g} cos p1 {c:.8f}"
                                                            for b, (p, c) in stats.items()))
        assert ok, (group, stats)


def _blocks(st64, gq, gv, gu):
    return np.concatenate([oracle.qpos_tangent(st64["qpos"], gq), gv, gu], 1)


BLOCKS = (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99)))


def test_adjoint_vs_oracle_config2(ffi):
    """256 config-1 worlds, output cotangents N(0, 1), the GPU's exact-mode VJP (float32, the
    engine's 10 iterations) against the float64 oracle's analytic VJP at the same settings and against the oracle's
    float64 central finite differences (eps 1e-6, MuJoCo's truth settings) on all 256 worlds: per block (qpos tangent
    / qvel / ctrl) median relative error <= 1e-4 (the BASELINE gate); p99 <= 2e-3 against the analytic VJP."""
    st = synthetic.states(256, config=1)
    cq, cv = synthetic.cotangents(256)
    gq, gv, gu, info, _ = _vjp_gpu(ffi, st, cq, cv)
    s64 = {k: st[k].astype(np.float64) for k in st}
    g = _blocks(s64, gq, gv, gu)
    an = _blocks(s64, *oracle.vjp(**s64, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=0, **oracle.ENGINE))
    fd = oracle.fd_vjp(**s64, g_qpos=cq, g_qvel=cv, h=1e-6, **oracle.TRUTH)
    for name, sl in BLOCKS:
        ea, ef = _rel_rows(g[:, sl], an[:, sl]), _rel_rows(g[:, sl], fd[:, sl])
        print(f"config2 {name}: vs analytic median {np.median(ea):.3g} p99 {np.percentile(ea, 99):.3g}; "
              f"vs FD (256 worlds) median {np.median(ef):.3g} p90 {np.percentile(ef, 90):.3g} "
              f"p99 {np.percentile(ef, 99):.3g}")
        assert np.median(ea) <= TOL and np.percentile(ea, 99) <= 2e-3
        assert np.median(ef) <= TOL


@pytest.mark.parametrize("substeps,iterations", [(1, 10), (2, 10), (7, 10), (32, 10), (2, 50)])
def test_adjoint_options_vs_oracle(ffi, substeps, iterations):
    """The VJP of steps of 1, 2, 7 and 32 substeps (the tape holds one record per substep; the adjoint runs them in
    reverse), at the engine's 10 and at 50 Newton iterations, against the float64 oracle's analytic VJP at the same
    settings (exact mode, 256 config-1 worlds, cotangents N(0, 1)): per block (qpos tangent / qvel / ctrl) median
    relative error <= 1e-4 (the BASELINE gate), p99 <= 5x the p99 of the oracle's restatement evaluated in float32
    (oracle.vjp_f32) against the same float64 VJP: the IFT solves with H (cond ~ 1e5-1e6) set the float32 floor, and
    a single 5 ms substep, whose gradient has the least smoothing around them, sits highest (p99 6.7e-4 for the
    float32 restatement's qpos block at 1 substep, 2.9e-4 at 7)."""
    st = synthetic.states(256, config=1, seed=41)
    cq, cv = synthetic.cotangents(256, seed=42)
    gq, gv, gu, info, _ = _vjp_gpu(ffi, st, cq, cv, iterations=iterations, substeps=substeps)
    s64 = {k: st[k].astype(np.float64) for k in st}
    g = _blocks(s64, gq, gv, gu)
    an = _blocks(s64, *oracle.vjp(**s64, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=0,
                                  **dict(oracle.ENGINE, iterations=iterations, nsub=substeps)))
    g32 = _blocks(s64, *(x.astype(np.float64) for x in oracle.vjp_f32(
        **st, g_qpos=cq, g_qvel=cv, clamp_kv=1, normal=0, **dict(oracle.ENGINE, iterations=iterations, nsub=substeps))))
    assert np.isfinite(g).all()
    for name, sl in BLOCKS:
        e, e32 = _rel_rows(g[:, sl], an[:, sl]), _rel_rows(g32[:, sl], an[:, sl])
        print(f"substeps {substeps}, {iterations} iterations, {name}: median {np.median(e):.3g} "
              f"p99 {np.percentile(e, 99):.3g} (float32 restatement: median {np.median(e32):.3g} "
              f"p99 {np.percentile(e32, 99):.3g})")
        assert np.median(e) <= TOL and np.percentile(e, 99) <= 5 * np.percentile(e32, 99)


def test_tape_does_not_change_outputs(ffi):
    """The forward's outputs are bitwise the same with and without the tape, and the tape is bitwise deterministic."""
    import torch
    st = synthetic.states(1024, config=1)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    a = ffi.forward(*args)
    b = ffi.forward(*args, tape=True)
    c = ffi.forward(*args, tape=True)
    torch.cuda.synchronize()
    for x, y in zip(a[:4], b[:4]):
        assert torch.equal(x, y)
    assert torch.equal(b[4].view(torch.int32), c[4].view(torch.int32))  # bitwise (the tape holds bit-cast ints)


def test_autograd_matches_backward(ffi):
    """torch_ffi.step under autograd: the gradients are backward()'s, warm' is not differentiable, grad_decay scales
    the state gradients only (one float32 product); warm, friction and com get no gradient (reference
    torch_ffi.py:751-777); the backward is bitwise deterministic."""
    import torch
    st = synthetic.states(64, config=1)
    cq, cv = synthetic.cotangents(64)
    q, v, w, u, f, c = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    q.requires_grad_(True); v.requires_grad_(True); u.requires_grad_(True)
    q1, v1, w1 = ffi.step(q, v, w, u, f, c)
    assert not w1.requires_grad
    ((q1 * _t(cq)).sum() + (v1 * _t(cv)).sum()).backward()
    r = ffi.forward(q.detach(), v.detach(), w, u.detach(), f, c, tape=True)
    gq, gv, gu, _ = ffi.backward(r[4], f, c, _t(cq), _t(cv))
    gq2, gv2, gu2, _ = ffi.backward(r[4], f, c, _t(cq), _t(cv))
    torch.cuda.synchronize()
    assert torch.equal(q.grad, gq) and torch.equal(v.grad, gv) and torch.equal(u.grad, gu)
    assert torch.equal(gq, gq2) and torch.equal(gv, gv2) and torch.equal(gu, gu2)
    q.grad = v.grad = u.grad = None
    q1, v1, w1 = ffi.step(q, v, w, u, f, c, grad_decay=0.9)
    ((q1 * _t(cq)).sum() + (v1 * _t(cv)).sum()).backward()
    torch.cuda.synchronize()
    assert torch.equal(q.grad, gq * 0.9) and torch.equal(v.grad, gv * 0.9) and torch.equal(u.grad, gu)
    q.grad = v.grad = u.grad = None
    for x in (w, f, c):
        x.requires_grad_(True)
    q1, v1, w1 = ffi.step(q, v, w, u, f, c)
    ((q1 * _t(cq)).sum() + (v1 * _t(cv)).sum()).backward()
    torch.cuda.synchronize()
    assert w.grad is None and f.grad is None and c.grad is None
    assert torch.equal(q.grad, gq) and torch.equal(u.grad, gu)


VARIANTS = [(kv, n) for kv in (0, 1, 2) for n in (0, 1, 2, 3)]


def _variant_case(case):
    """(states, cotangents (cq, cv)) of a variant-parity case: the truth's G4 (clamped actuators) or G6 (self contacts)
    states of both corpora with their first cotangent, or 256 config-1 states."""
    if case == "config1":
        return synthetic.states(256, config=1), synthetic.cotangents(256)
    st, cq, cv = {}, [], []
    for cname in ("mf_s0", "mf_s1"):
        z = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
        sel = np.nonzero(z[case])[0]
        for k, src in (("qpos", "qpos"), ("qvel", "qvel"), ("warm", "qacc_warmstart"), ("ctrl", "ctrl"),
                       ("friction", "friction"), ("com", "com")):
            st.setdefault(k, []).append(z[src][sel])
        cq.append(z["cot_qpos"][sel, 0])
        cv.append(z["cot_qvel"][sel, 0])
    return {k: np.concatenate(v) for k, v in st.items()}, (np.concatenate(cq), np.concatenate(cv))


@pytest.mark.parametrize("case", ["G4", "G6", "config1"])
def test_adjoint_variants_vs_oracle(ffi, case):
    """Every (clamp_kv, normal) variant of the reference (adjoint.py:43-56,811-846, adjoint_contact.py:74-95,239-262;
    clamp_soft 0.2) from one GPU tape against the float64 oracle's analytic VJP of the same variant, both at 50 Newton
    iterations: per block median relative error <= 1e-4 and p99 <= 2e-3. The oracle's variants are pinned in
    tests/test_oracle.py (lambda by finite differences for clamp_kv, the affine dependence on kappa(nu) for normal,
    the frozen-parameter forward for the near-parallel rule)."""
    import torch
    st, (cq, cv) = _variant_case(case)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    r = ffi.forward(*args, iterations=50, tape=True)
    s64 = {k: st[k].astype(np.float64) for k in st}
    for kv, n in VARIANTS:
        kw = dict(ctrl=args[3]) if kv == 2 else {}
        gq, gv, gu, info = ffi.backward(r[4], args[4], args[5], _t(cq), _t(cv), clamp_kv=kv, normal=n, **kw)
        torch.cuda.synchronize()
        g = _blocks(s64, *(x.cpu().numpy().astype(np.float64) for x in (gq, gv, gu)))
        ref = _blocks(s64, *oracle.vjp(**s64, g_qpos=cq, g_qvel=cv, clamp_kv=kv, normal=n, clamp_soft=0.2,
                                       **oracle.TRUTH))
        assert np.isfinite(g).all()
        line = []
        for name, sl in BLOCKS:
            e = _rel_rows(g[:, sl], ref[:, sl])
            line.append(f"{name} {np.median(e):.2g}/{np.percentile(e, 99):.2g}")
            assert np.median(e) <= TOL and np.percentile(e, 99) <= 2e-3, (kv, n, name)
        print(f"{case} ({len(cq)} states) clamp_kv={kv} normal={n}: median/p99 " + ", ".join(line))
    with pytest.raises(ValueError):
        ffi.backward(r[4], args[4], args[5], _t(cq), _t(cv), clamp_kv=2)


def test_soft_clamp_weight_is_at_most_one(ffi):
    """The soft clamp's weight w = exp(-max((|f| - tau) / tau, 0) / delta) is 1 on a dof the tape marks clamped whose
    recomputed PD force lies inside its bound (adjoint.py:822-829), never above 1: with the clamp bit planted in every
    record for every actuated dof that is not clamped, clamp_kv=2 at delta 1e-6 gives bitwise the gradients of the
    untouched tape (where those dofs take the full lambda); without the floor w would overflow to inf."""
    import torch
    st = synthetic.states(128, config=1)
    cq, cv = synthetic.cotangents(128)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    q1, v1, w1, info, tape = ffi.forward(*args, tape=True)
    rw = ffi.rec_words()
    words = tape.view(torch.int32).view(128, 4, rw)
    planted = words.clone()
    planted[:, :, 2] = -64  # bits 6..31: dofs 6..31 (the hinges)
    planted[:, :, 3] = 7    # bits 32..34: dofs 32..34
    assert not torch.equal(planted, words)
    outs = []
    for t in (words, planted):
        g = ffi.backward(t.view(torch.float32).reshape(128, 4 * rw), args[4], args[5], _t(cq), _t(cv), clamp_kv=2,
                         ctrl=args[3], clamp_soft=1e-6)
        torch.cuda.synchronize()
        outs.append(g[:3])
    for a, b in zip(*outs):
        assert torch.isfinite(b).all() and torch.equal(a, b)


def test_variant_entries_bound_as_the_reference(ffi):
    """The 12 reference-named variant units bound exactly as the reference's _bind would (ctypes, argument lists of
    jax_ffi.py:214-258): each dk_kv{0,1,2}_n{0..3}_adjoint returns 0 and gives bitwise dk_adjoint's result with that
    variant; each _sizes reports its variant; each _upload returns 0; each _launch reports the adjoint's LDS bytes
    and a positive number of resident worlds per CU on device 0."""
    import ctypes
    import torch
    lib = ctypes.CDLL(ffi.load_library()._name)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    B = 64
    st = synthetic.states(B, config=4)
    cq, cv = synthetic.cotangents(B)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    r = ffi.forward(*args, tape=True)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    kw = dict(dtype=torch.float32, device="cuda")
    gen = lib.dk_adjoint
    gen.argtypes = [vp, i32, i32] + [vp] * 9 + [vp, f32, i32, i32]
    gen.restype = i32
    for kv, n in VARIANTS:
        f = getattr(lib, f"dk_kv{kv}_n{n}_adjoint")
        f.argtypes = [vp, i32, i32] + [vp] * 9 + [vp, f32]
        f.restype = i32
        sz = np.zeros(9, np.int64)
        getattr(lib, f"dk_kv{kv}_n{n}_sizes")(ctypes.c_void_p(sz.ctypes.data))
        assert tuple(sz[2:9]) == (1472, 36, 35, 64, kv, n, 1)
        up = getattr(lib, f"dk_kv{kv}_n{n}_upload")
        up.argtypes, up.restype = [vp, vp], i32
        assert up(None, stream) == 0
        la = getattr(lib, f"dk_kv{kv}_n{n}_launch")
        la.argtypes, la.restype = [i32, vp], i32
        o = np.zeros(2, np.int64)
        assert la(0, ctypes.c_void_p(o.ctypes.data)) == 0
        assert o[0] == sz[1] and o[1] >= 1
        outs = []
        for call in (lambda *a: f(*a), lambda *a: gen(*a, kv, n)):
            gq, gv, gu = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 29), **kw)
            info = torch.empty((B,), dtype=torch.int32, device="cuda")
            assert call(stream, B, 4, p(r[4]), p(args[4]), p(args[5]), p(_t(cq)), p(_t(cv)), p(gq), p(gv), p(gu),
                        p(info), p(args[3]), f32(0.2)) == 0
            torch.cuda.synchronize()
            outs.append((gq, gv, gu, info))
        for a, b in zip(*outs):
            assert torch.equal(a, b), (kv, n)


# 65 config-4 states (synthetic.states(4096, config=4, seed=1000 + s), world w) with capsule-capsule self contacts at
# the input state whose two segment parameters are both free, found among 163,840 such states: every one of the 39
# contacts at nu < 2 cm with sin^2(theta) < 0.01 (near parallel, above the near-parallel rule's 1.2e-3), and 48
# contacts drawn from those at nu < 1 cm (nu: the segments' distance), as (s, w)
CAPSULE_STATES = [
    (0, 613), (0, 882), (0, 1502), (0, 2914), (0, 3474), (1, 1071), (1, 1723), (1, 1762), (1, 2914),
    (3, 620), (3, 1366), (3, 2392), (4, 3218), (4, 3877), (6, 1623), (6, 1652), (6, 1819), (8, 1064),
    (8, 4000), (9, 1352), (10, 705), (10, 1400), (10, 2408), (11, 1814), (11, 2470), (11, 3345), (15, 1662),
    (15, 2025), (15, 3524), (16, 1636), (16, 2619), (18, 3187), (19, 161), (19, 515), (19, 3009), (20, 28),
    (20, 572), (20, 2034), (20, 2218), (21, 88), (21, 215), (21, 1880), (21, 2554), (23, 1945), (24, 2435),
    (24, 2891), (25, 421), (25, 4056), (26, 235), (27, 1466), (28, 2894), (28, 2935), (29, 4014), (31, 3474),
    (31, 3665), (32, 47), (33, 859), (33, 1660), (33, 1755), (33, 3275), (34, 336), (36, 358), (36, 2004),
    (37, 1200), (38, 3240),
]


def test_capsule_both_free_vjp(ffi):
    """The capsule-capsule contact VJP with both segment parameters free, written without 1 / nu
    (adjoint_contact.py:436-465: the normal n = sg (a1 x a2) / |a1 x a2| of the axes alone; the general chain sums
    terms of order 1 / nu that cancel, losing up to 1e-3 relative in float32 at nu = 5 mm), on the CAPSULE_STATES:
    one substep at 50 iterations against the float64 oracle's analytic VJP of the same variant, exact mode and the
    interface default: per world relative error median <= 1e-4, p90 <= 1e-3, max <= 1e-2 (the general chain's max
    here was 70)."""
    import torch
    cache, st = {}, {k: [] for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")}
    for s_, w in CAPSULE_STATES:
        if s_ not in cache:
            cache[s_] = synthetic.states(4096, config=4, seed=1000 + s_)
        for k in st:
            st[k].append(cache[s_][k][w])
    st = {k: np.array(v) for k, v in st.items()}
    n = len(CAPSULE_STATES)
    cq, cv = synthetic.cotangents(n, seed=7)
    s64 = {k: v.astype(np.float64) for k, v in st.items()}
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    r = ffi.forward(*args, iterations=50, substeps=1, tape=True)
    for kv, nm in ((1, 0), (0, 3)):
        gq, gv, gu, _ = ffi.backward(r[4], args[4], args[5], _t(cq), _t(cv), substeps=1, clamp_kv=kv, normal=nm)
        torch.cuda.synchronize()
        g = _blocks(s64, *(x.cpu().numpy().astype(np.float64) for x in (gq, gv, gu)))
        ref = _blocks(s64, *oracle.vjp(**s64, g_qpos=cq, g_qvel=cv, clamp_kv=kv, normal=nm,
                                       **dict(oracle.TRUTH, nsub=1)))
        e = _rel_rows(g, ref)
        print(f"capsule both-free ({n} states) clamp_kv={kv} normal={nm}: median {np.median(e):.3g} p90 "
              f"{np.percentile(e, 90):.3g} max {e.max():.3g}")
        assert np.median(e) <= 1e-4 and np.percentile(e, 90) <= 1e-3 and e.max() <= 1e-2


def _resident_worlds():
    """worlds resident at once on device 0 (8 per CU in both kernels): batches up to this size run in index order"""
    import torch
    return 8 * torch.cuda.get_device_properties(0).multi_processor_count


def test_dispatch_order_does_not_change_results(ffi):
    """The C entries with a work buffer dispatch the worlds heaviest first; without one (NULL) in index order. The
    outputs, the tape and the gradients are bitwise the same both ways (contact-heavy config-4 states, where the
    order moves the most; more worlds than the GPU holds at once, so that the order is computed)."""
    import ctypes
    import torch
    lib = ffi.load_library()
    B = _resident_worlds() + 512
    st = synthetic.states(B, config=4)
    cq, cv = synthetic.cotangents(B)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for ordered in (False, True):
        kw = dict(dtype=torch.float32, device="cuda")
        q1, v1, w1 = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 35), **kw)
        info = torch.empty((B, 4), dtype=torch.int32, device="cuda")
        tape = torch.empty((B, 4 * ffi.rec_words()), **kw)
        work = torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device="cuda")
        assert lib.dk_fwd_forward(stream, B, *map(p, args), 10, 4, p(q1), p(v1), p(w1), p(info), None, p(tape),
                                  p(work) if ordered else None) == 0
        gq, gv, gu = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 29), **kw)
        binfo = torch.empty((B,), dtype=torch.int32, device="cuda")
        work2 = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device="cuda")
        assert lib.dk_adjoint_work(stream, B, 4, p(tape), p(args[4]), p(args[5]), p(_t(cq)), p(_t(cv)), p(gq), p(gv),
                                   p(gu), p(binfo), None, ctypes.c_float(0.0), 0, 3,
                                   p(work2) if ordered else None) == 0
        torch.cuda.synchronize()
        outs.append((q1, v1, w1, info, tape.view(torch.int32), gq, gv, gu, binfo))
    for x, y in zip(*outs):
        assert torch.equal(x, y)
    perm = work.view(torch.int32)[:B].cpu().numpy()
    assert np.array_equal(np.sort(perm), np.arange(B))  # a permutation of the worlds


def test_resident_batch_runs_in_index_order(ffi):
    """A batch the GPU holds at once starts every world at the launch, so the forward and the one-set adjoint skip the
    dispatch order: the work buffer is left as it was, and the results are bitwise those of an ordered launch of the
    same worlds (dk_fwd_order, then dk_fwd_forward_ordered)."""
    import ctypes
    import torch
    lib = ffi.load_library()
    B = 1000
    assert B <= _resident_worlds()
    st = synthetic.states(B, config=4, seed=7)
    args = [_t(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    kw = dict(dtype=torch.float32, device="cuda")
    outs = []
    for ordered in (False, True):
        q1, v1, w1 = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 35), **kw)
        info = torch.empty((B, 4), dtype=torch.int32, device="cuda")
        work = torch.full((int(lib.dk_fwd_work_bytes(B)),), 0xA5, dtype=torch.uint8, device="cuda")
        if ordered:
            assert lib.dk_fwd_order(stream, B, p(args[0]), p(work)) == 0
            assert lib.dk_fwd_forward_ordered(stream, B, *map(p, args), 10, 4, p(q1), p(v1), p(w1), p(info), None,
                                              None, p(work)) == 0
        else:
            assert lib.dk_fwd_forward(stream, B, *map(p, args), 10, 4, p(q1), p(v1), p(w1), p(info), None, None,
                                      p(work)) == 0
        torch.cuda.synchronize()
        if not ordered:
            assert bool((work == 0xA5).all()), "the forward wrote a dispatch order for a resident batch"
        outs.append((q1, v1, w1, info))
    for x, y in zip(*outs):
        assert torch.equal(x, y)
