"""GPU drivers over the step: the full step Jacobian against MuJoCo C's float64 finite-difference
Jacobian (the truth's `jacobian`, tests/golden/grad_mf_s*.npz) and against the VJP it is built from; the checkpointed
BPTT rollout (config 4) bitwise equal to the plain one."""
import os

import numpy as np
import pytest

from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KEYS = ("qpos", "qvel", "warm", "ctrl", "friction", "com")


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


@pytest.mark.parametrize("cname", ["mf_s0", "mf_s1"])
def test_jacobian_vs_mujoco_fd(ffi, cname):
    """The 71 x 99 step Jacobian of all 64 truth Jacobian states (G0) per corpus against MuJoCo C float64 central
    differences, scored as the reference's jacobian_errors (benchmarks/bench/accuracy/gradient.py:193-208): per block
    (qpos tangent, qvel, ctrl) the Frobenius relative error over the truth's valid columns; median <= 1e-4 per block
    (the gradient gate), and the whole matrix's per-world error median <= 1e-4."""
    import torch
    from nablaengine_amd import rollout
    z = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
    args = [_t(z["jac_" + k]) for k in ("qpos", "qvel", "qacc_warmstart", "ctrl", "friction", "com")]
    J, info = rollout.jacobian(*args)
    torch.cuda.synchronize()
    J = J.cpu().numpy().astype(np.float64)
    ref = z["jacobian"].astype(np.float64)
    assert len(J) == 64 and np.isfinite(J).all()
    valid = z["bad"][z["jac_index"]] == 0
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        e = []
        for w in range(len(J)):
            v = valid[w, sl]
            a, b = J[w][:, sl][:, v], ref[w][:, sl][:, v]
            e.append(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-9))
        print(f"{cname} {name}: Jacobian block relative error median {np.median(e):.3g} p90 "
              f"{np.percentile(e, 90):.3g} max {np.max(e):.3g}")
        assert np.median(e) <= 1e-4, name
    e = np.linalg.norm((J - ref).reshape(len(J), -1), axis=1) / np.linalg.norm(ref.reshape(len(ref), -1), axis=1)
    print(f"{cname}: Jacobian relative error median {np.median(e):.3g} max {e.max():.3g}")
    assert np.median(e) <= 1e-4


def test_jacobian_is_the_vjp(ffi):
    """J^T c equals the step's VJP of c (qpos gradient in tangent form) for random cotangents c, on config-1 states,
    to float32 rounding: the adjoint is linear in its cotangent, but 71 one-hot VJPs summed round differently from
    one VJP of their combination (median relative difference <= 2e-5, max <= 5e-4)."""
    import torch
    from nablaengine_amd import rollout
    B = 128
    st = synthetic.states(B, config=1)
    args = [_t(st[k]) for k in KEYS]
    J, _ = rollout.jacobian(*args)
    cq, cv = synthetic.cotangents(B)
    q1, v1, w1, info, tape = ffi.forward(*args, tape=True)
    gq, gv, gu, _ = ffi.backward(tape, args[4], args[5], _t(cq), _t(cv))
    g = torch.cat([rollout.qpos_tangent(args[0], gq), gv, gu], 1).cpu().numpy().astype(np.float64)
    c = np.c_[cq, cv].astype(np.float64)
    jt = np.einsum("bo,boi->bi", c, J.cpu().numpy().astype(np.float64))
    e = np.linalg.norm(jt - g, axis=1) / np.linalg.norm(g, axis=1)
    print(f"J^T c vs VJP: median {np.median(e):.3g} max {e.max():.3g}")
    assert np.median(e) <= 2e-5 and e.max() <= 5e-4



@pytest.fixture(scope="module")
def heavy(ffi):
    """301 contact-heavy config-4 worlds (a batch size that is a multiple of nothing) and their taped step."""
    B = 301
    st = synthetic.states(B, config=4, seed=85)
    args = [_t(st[k]) for k in KEYS]
    return args, ffi.forward(*args, tape=True)


# every adjoint variant at its default soft-clamp delta, and the soft clamp at an explicit one
JAC_VARIANTS = [(kv, n, None) for kv in (0, 1, 2) for n in (0, 1, 2, 3)] + [(2, 3, 0.05), (2, 0, 1e-6)]


@pytest.mark.parametrize("kv,n,soft", JAC_VARIANTS)
def test_jacobian_rows_are_the_backward_vjps(ffi, heavy, kv, n, soft):
    """The Jacobian driver's 71 VJPs (one dk_adjoint_many launch, one dispatch order): each row is bitwise the VJP
    torch_ffi.backward computes with the same options for that output's one-hot cotangent, in every (clamp_kv, normal)
    variant, the soft clamp at its default delta (clamp_soft None) and at explicit ones; the reference builds its
    Jacobian from its backward (scripts/paper_bench/ours.py:1-13), so its rows are these by construction. The default
    variant also checks that the diagnostics count 71 backward calls."""
    import torch
    from nablaengine_amd import rollout
    args, (q1, v1, w1, info2, tape) = heavy
    B = args[0].shape[0]
    opts = dict(clamp_kv=kv, normal=n, clamp_soft=soft)
    default = (kv, n, soft) == (ffi.CLAMP_KV, ffi.NORMAL, None)
    if default:
        ffi.read_diagnostics(reset=True)
    J, info = rollout.jacobian(*args, **opts)
    if default:
        d = ffi.read_diagnostics()
        assert d["bwd_calls"] == 71 and d["bwd_rows"] == 71 * B and d["fwd_calls"] == 1
    assert torch.equal(info, info2)
    ctrl = args[3] if kv == 2 else None
    for r in (0, 3, 6, 20, 35, 36, 40, 52, 70):
        cq = torch.zeros((B, 36), device="cuda")
        cv = torch.zeros((B, 35), device="cuda")
        (cq if r < 36 else cv)[:, r if r < 36 else r - 36] = 1.0
        gq, gv, gu, _ = ffi.backward(tape, args[4], args[5], cq, cv, ctrl=ctrl, **opts)
        row = torch.cat([rollout.qpos_tangent(args[0], gq), gv, gu], 1)
        assert torch.equal(J[:, r, :].view(torch.int32), row.view(torch.int32)), r


@pytest.mark.parametrize("B,substeps", [(16384, 4), (4096, 2), (1, 4), (301, 1)])
def test_jacobian_rows_at_every_grouping(ffi, B, substeps):
    """The many-cotangent adjoint runs a world's sets in workgroups of a size set by the batch (36 and 35 at 16384
    worlds, 18 at 4096, 2 at 301 with a last group of one, one each for a single world) and keeps each set's running
    cotangent in its output rows between substeps. At each grouping, and with one substep (the seed and the gradients
    in one pass), every checked row is bitwise backward()'s VJP and info is the forward's."""
    import torch
    from nablaengine_amd import rollout
    st = synthetic.states(B, config=1, seed=11 + B)
    args = [_t(st[k]) for k in KEYS]
    J, info = rollout.jacobian(*args, substeps=substeps)
    q1, v1, w1, info2, tape = ffi.forward(*args, substeps=substeps, tape=True)
    assert torch.equal(info, info2)
    for r in (0, 4, 5, 6, 7, 35, 36, 39, 70):
        cq = torch.zeros((B, 36), device="cuda")
        cv = torch.zeros((B, 35), device="cuda")
        (cq if r < 36 else cv)[:, r if r < 36 else r - 36] = 1.0
        gq, gv, gu, binfo = ffi.backward(tape, args[4], args[5], cq, cv, substeps=substeps)
        row = torch.cat([rollout.qpos_tangent(args[0], gq), gv, gu], 1)
        assert torch.equal(J[:, r, :].view(torch.int32), row.view(torch.int32)), r


@pytest.mark.parametrize("B,substeps", [(16384, 4), (4096, 3), (3, 4), (301, 1)])
def test_vjp_sets_are_the_backward_calls(ffi, B, substeps):
    """Nine random cotangent sets in one many-cotangent launch against nine backward() calls, with the counters on:
    the qpos-form, qvel and ctrl gradients and the info words bitwise equal, for a set whose cotangent holds a NaN
    too (its non-finite bits, NONFINITE_COT among them, the same), at groupings of 5 and 4, 3, and 1 set per workgroup and
    at 1, 3 and 4 substeps; the counters count nine backward calls."""
    import torch
    st = synthetic.states(B, config=4, seed=3 + B)
    args = [_t(st[k]) for k in KEYS]
    prev = ffi.set_diagnostics(True)
    try:
        q1, v1, w1, info, tape = ffi.forward(*args, substeps=substeps, tape=True)
        g = torch.Generator(device="cpu").manual_seed(B)
        cq = torch.randn((9, B, 36), generator=g).cuda()
        cv = torch.randn((9, B, 35), generator=g).cuda()
        cq[4, B // 2, 5] = float("nan")
        ffi.read_diagnostics(reset=True)
        many = ffi._vjp_sets(tape, args[4], args[5], cq, cv, substeps=substeps)
        d = ffi.read_diagnostics(reset=True)
        assert d["bwd_calls"] == 9 and d["bwd_rows"] == 9 * B and d["nonfinite_cotangent_rows"] >= 1
        for k in range(9):
            one = ffi.backward(tape, args[4], args[5], cq[k], cv[k], substeps=substeps)
            for a, b in zip(many, one):
                x = a[k]
                assert torch.equal(x.view(torch.int32), b.view(torch.int32)), k
        bits = many[3][4, B // 2].item() >> 16
        assert bits & 8, "NONFINITE_COT"
    finally:
        ffi.set_diagnostics(prev)


def test_empty_batch_everywhere(ffi):
    """B = 0 through every entry: the taped forward's empty tape, backward(), step() under autograd (its backward),
    the many-cotangent VJPs and jacobian() give empty outputs of the right shapes, and nothing is launched on 0
    worlds."""
    import torch
    from nablaengine_amd import rollout
    st = synthetic.states(2, config=1)
    a = [_t(st[k])[:0] for k in KEYS]
    q1, v1, w1, info, tape = ffi.forward(*a, tape=True)
    assert q1.shape == (0, 36) and v1.shape == (0, 35) and info.shape == (0, 4) and tape.shape[0] == 0
    gq, gv, gu, binfo = ffi.backward(tape, a[4], a[5], q1, v1)
    assert gq.shape == (0, 36) and gv.shape == (0, 35) and gu.shape == (0, 29) and binfo.shape == (0,)
    x = [t.clone().requires_grad_(True) for t in a[:2]] + [a[2], a[3].clone().requires_grad_(True)] + a[4:]
    out = ffi.step(*x)
    (out[0].sum() + out[1].sum()).backward()
    assert x[0].grad.shape == (0, 36) and x[1].grad.shape == (0, 35) and x[3].grad.shape == (0, 29)
    many = ffi._vjp_sets(tape, a[4], a[5], torch.zeros((3, 0, 36), device="cuda"), torch.zeros((3, 0, 35), device="cuda"))
    assert [t.shape for t in many] == [(3, 0, 36), (3, 0, 35), (3, 0, 29), (3, 0)]
    J, jinfo = rollout.jacobian(*a)
    assert J.shape == (0, 71, 99) and jinfo.shape == (0, 4)
    torch.cuda.synchronize()


def test_jacobian_options_are_checked(ffi, heavy):
    """The Jacobian driver takes the backward's options with the backward's checks: a delta for clamp_kv 0 / 1, a
    negative or NaN delta are ValueErrors, before any launch."""
    from nablaengine_amd import rollout
    args = heavy[0]
    for kw in (dict(clamp_kv=0, clamp_soft=0.1), dict(clamp_kv=2, clamp_soft=-1.0),
               dict(clamp_kv=2, clamp_soft=float("nan")), dict(clamp_kv=3)):
        with pytest.raises(ValueError):
            rollout.jacobian(*args, **kw)


def test_scale_grad_rollout_is_the_manual_chain(ffi):
    """The reference's rollout check (scripts/torch_ffi_check.py:12-13,187-205): 3 steps, each control requiring
    grad, the state carried with scale_grad((q, v, w), 0.98) at the top of each step, loss = cotangents . final state.
    The gradients of the 3 controls and of the initial state are bitwise a manual chain of backward() calls on the
    steps' tapes, with the state cotangents multiplied by 0.98 (float32) at each step's top; the final state is
    bitwise the chain of forward() calls."""
    import torch
    B = 192
    st = synthetic.states(B, config=1, seed=31)
    tin = [_t(st[k]) for k in KEYS]
    us = [_t(synthetic.states(B, config=1, seed=40 + s)["ctrl"]) for s in range(3)]
    cq, cv = (_t(x) for x in synthetic.cotangents(B, seed=3))
    xs = [tin[0].clone().requires_grad_(), tin[1].clone().requires_grad_()]
    ur = [u.clone().requires_grad_() for u in us]
    q, v, w = xs[0], xs[1], tin[2]
    for u in ur:
        q, v, w = ffi.scale_grad((q, v, w), 0.98)
        q, v, w = ffi.step(q, v, w, u, tin[4], tin[5])
        assert not w.requires_grad
    ((q * cq).sum() + (v * cv).sum()).backward()
    # the manual chain
    tapes, state = [], (tin[0], tin[1], tin[2])
    for u in us:
        q1, v1, w1, _, tp = ffi.forward(*state, u, tin[4], tin[5], tape=True)
        tapes.append(tp)
        state = (q1, v1, w1)
    assert torch.equal(q.detach(), state[0]) and torch.equal(v.detach(), state[1])
    gq, gv = cq, cv
    g_ctrl = [None] * 3
    for s in (2, 1, 0):
        gq, gv, g_ctrl[s], _ = ffi.backward(tapes[s], tin[4], tin[5], gq, gv)
        gq, gv = gq * 0.98, gv * 0.98
    torch.cuda.synchronize()
    for a, b in zip([xs[0].grad, xs[1].grad] + [u.grad for u in ur], [gq, gv] + g_ctrl):
        assert torch.isfinite(b).all() and torch.equal(a, b)


def test_checkpointed_rollout_is_bitwise_the_plain_one(ffi):
    """A 6-step BPTT rollout on contact-heavy config-4 states: the gradients of a loss on every state with segments
    of 2 steps (the first two recomputed in the backward, their first pass writing no tapes; the last keeping its
    tapes) are bitwise those with every tape kept, and so are those of a second backward through the same graph
    (retain_graph: each checkpointed segment recomputed again)."""
    import torch
    from nablaengine_amd import rollout
    B, T = 256, 6
    st = synthetic.states(B, config=4)
    us = _t(synthetic.ctrl_sequence(T, B))
    grads = []
    for k in (0, 2):
        q = _t(st["qpos"]).requires_grad_(True)
        v = _t(st["qvel"]).requires_grad_(True)
        u = us.clone().requires_grad_(True)
        states = rollout.rollout(q, v, _t(st["warm"]), u, _t(st["friction"]), _t(st["com"]), checkpoint_every=k)
        loss = sum((qt[:, 2] ** 2).sum() + 0.01 * (vt ** 2).sum() for qt, vt in states)
        loss.backward(retain_graph=True)
        first = (q.grad.clone(), v.grad.clone(), u.grad.clone())
        q.grad = v.grad = u.grad = None
        loss.backward()
        grads.append(first)
        grads.append((q.grad, v.grad, u.grad))
    torch.cuda.synchronize()
    for g in grads[1:]:
        for a, b in zip(grads[0], g):
            assert torch.isfinite(a).all() and torch.equal(a, b)
