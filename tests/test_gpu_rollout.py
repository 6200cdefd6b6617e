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
    """The 71 x 99 step Jacobian of the truth's Jacobian states against MuJoCo C float64 central differences: per
    world relative Frobenius error median <= 1e-4 (the gradient gate)."""
    import torch
    from nablaengine_amd import rollout
    z = np.load(os.path.join(GOLD, f"grad_{cname}.npz"))
    args = [_t(z["jac_" + k]) for k in ("qpos", "qvel", "qacc_warmstart", "ctrl", "friction", "com")]
    J, info = rollout.jacobian(*args)
    torch.cuda.synchronize()
    J = J.cpu().numpy().astype(np.float64)
    ref = z["jacobian"].astype(np.float64)
    e = np.linalg.norm((J - ref).reshape(len(J), -1), axis=1) / np.linalg.norm(ref.reshape(len(ref), -1), axis=1)
    print(f"{cname}: Jacobian relative error median {np.median(e):.3g} max {e.max():.3g}")
    assert np.isfinite(J).all()
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



def test_jacobian_rows_are_the_backward_vjps(ffi):
    """The Jacobian driver's 71 VJPs share one adjoint dispatch order (dk_adjoint_order, dk_adjoint_work_ordered): each
    row is bitwise the VJP torch_ffi.backward computes for that output's one-hot cotangent, on contact-heavy states at
    a batch size that is not a multiple of anything (the order never changes a result); the diagnostics count 71
    backward calls."""
    import torch
    from nablaengine_amd import rollout
    B = 301
    st = synthetic.states(B, config=4, seed=85)
    args = [_t(st[k]) for k in KEYS]
    ffi.read_diagnostics(reset=True)
    J, info = rollout.jacobian(*args)
    d = ffi.read_diagnostics()
    assert d["bwd_calls"] == 71 and d["bwd_rows"] == 71 * B and d["fwd_calls"] == 1
    q1, v1, w1, info2, tape = ffi.forward(*args, tape=True)
    assert torch.equal(info, info2)
    for r in (0, 3, 6, 35, 36, 40, 70):
        cq = torch.zeros((B, 36), device="cuda")
        cv = torch.zeros((B, 35), device="cuda")
        (cq if r < 36 else cv)[:, r if r < 36 else r - 36] = 1.0
        gq, gv, gu, _ = ffi.backward(tape, args[4], args[5], cq, cv)
        row = torch.cat([rollout.qpos_tangent(args[0], gq), gv, gu], 1)
        assert torch.equal(J[:, r, :].view(torch.int32), row.view(torch.int32)), r

def test_checkpointed_rollout_is_bitwise_the_plain_one(ffi):
    """A 4-step BPTT rollout on contact-heavy config-4 states: the gradients of a loss on every state with segments
    of 2 steps recomputed in the backward are bitwise those with every tape kept."""
    import torch
    from nablaengine_amd import rollout
    B, T = 256, 4
    st = synthetic.states(B, config=4)
    us = _t(synthetic.ctrl_sequence(T, B))
    grads = []
    for k in (0, 2):
        q = _t(st["qpos"]).requires_grad_(True)
        v = _t(st["qvel"]).requires_grad_(True)
        u = us.clone().requires_grad_(True)
        states = rollout.rollout(q, v, _t(st["warm"]), u, _t(st["friction"]), _t(st["com"]), checkpoint_every=k)
        loss = sum((qt[:, 2] ** 2).sum() + 0.01 * (vt ** 2).sum() for qt, vt in states)
        loss.backward()
        grads.append((q.grad, v.grad, u.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.isfinite(a).all() and torch.equal(a, b)
