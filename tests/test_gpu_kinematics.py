"""GPU parity of the kinematics outputs and their VJP (HIP kernels k_kin / k_kin_vjp through the C ABI, via
nablaengine_amd.torch_ffi) against the float64 oracle, with the reference's gates (scripts/kinematics_check.py GATES:
xpos, subtree_com <= 1e-5 m, xquat <= 1e-6, cvel per-world relative error median <= 1e-6 and p99 <= 1e-5, qpos_n's
quaternion <= 1e-6 and its other entries bitwise; VJP per-world relative error median <= 1e-5, p99 <= 1e-4), and the
step's kinematics=True contract (outputs of the step unchanged, kinematics bitwise those of its output state, the
combined backward the composition of the two VJPs)."""
import numpy as np
import pytest

import oracle
from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
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


def _states(B, config=1):
    st = synthetic.states(B, config=config)
    st["com"] = np.random.default_rng(11).uniform(-0.05, 0.05, (B, 3)).astype(np.float32)
    return st


def _rel_rows(a, b):
    a = np.asarray(a, np.float64).reshape(len(a), -1)
    b = np.asarray(b, np.float64).reshape(len(b), -1)
    return np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-9)


@pytest.mark.parametrize("config", [1, 4])
def test_kinematics_vs_oracle(ffi, config):
    """k_kin against the float64 oracle on the same float32 inputs (config 1 standing, config 4 fallen states)."""
    import torch
    B = 512
    st = _states(B, config)
    st["qpos"][:, 3:7] *= 1.1  # an unnormalized root quaternion: qpos_n normalizes it
    out = ffi.kinematics(_t(st["qpos"]), _t(st["qvel"]), _t(st["com"]))
    torch.cuda.synchronize()
    qn, xpos, xquat, cvel, sc = (x.cpu().numpy() for x in out)
    rq, rx, rQ, rc, rs = oracle.kinematics(st["qpos"].astype(np.float64), st["qvel"].astype(np.float64),
                                           st["com"].astype(np.float64))
    ex, eQ, es = np.abs(xpos - rx).max(), np.abs(xquat - rQ).max(), np.abs(sc - rs).max()
    ec = _rel_rows(cvel, rc)
    eqn = np.abs(qn[:, 3:7] - rq[:, 3:7]).max()
    print(f"config {config}: xpos {ex:.3g} xquat {eQ:.3g} subtree_com {es:.3g} cvel median {np.median(ec):.3g} "
          f"p99 {np.percentile(ec, 99):.3g} qpos_n quat {eqn:.3g}")
    assert ex <= 1e-5 and es <= 1e-5 and eQ <= 1e-6 and eqn <= 1e-6
    assert np.median(ec) <= 1e-6 and np.percentile(ec, 99) <= 1e-5
    other = np.r_[0:3, 7:36]
    assert np.array_equal(qn[:, other].view(np.uint32), st["qpos"][:, other].view(np.uint32))


def test_kinematics_vjp_vs_oracle_fd(ffi):
    """k_kin_vjp against central differences of the float64 oracle, N(0, 1) cotangents on each output block alone and
    on all five together: per-world relative error of (g_qpos, g_qvel) median <= 1e-5, p99 <= 1e-4."""
    import torch
    B = 48
    st = _states(B)
    st["qpos"][:, 3:7] *= 0.9
    q, v, c3 = (_t(st[k]) for k in ("qpos", "qvel", "com"))
    rng = np.random.default_rng(2)
    shapes = [(B,) + s for s in oracle.KIN_SHAPES]
    for block in (0, 1, 2, 3, 4, None):
        cot = [rng.normal(0, 1, s).astype(np.float32) if block in (None, k) else np.zeros(s, np.float32)
               for k, s in enumerate(shapes)]
        gq, gv = ffi._ops().kinematics_backward(q, v, c3, *map(_t, cot))
        torch.cuda.synchronize()
        rq, rv = oracle.kinematics_vjp(st["qpos"].astype(np.float64), st["qvel"].astype(np.float64),
                                       st["com"].astype(np.float64), [c.astype(np.float64) for c in cot])
        e = _rel_rows(np.c_[gq.cpu().numpy(), gv.cpu().numpy()], np.c_[rq, rv])
        print(f"cotangent block {block}: median {np.median(e):.3g} p99 {np.percentile(e, 99):.3g} max {e.max():.3g}")
        assert np.median(e) <= 1e-5 and np.percentile(e, 99) <= 1e-4


def test_step_kinematics_contract(ffi):
    """step(..., kinematics=True): (q', v', w') bitwise those of kinematics=False; its kinematics outputs bitwise
    kinematics(q', v', com); the autograd gradient with cotangents on all eight outputs bitwise the composition of the
    kinematics VJP (incoming q', v' cotangents added last) and the step's backward."""
    import torch
    B = 256
    st = _states(B)
    args = [_t(st[k]) for k in KEYS]
    plain = ffi.step(*args)
    withk = ffi.step(*args, kinematics=True)
    assert len(withk) == 8
    for a, b in zip(plain, withk[:3]):
        assert torch.equal(a, b)
    kin = ffi.kinematics(withk[0], withk[1], args[5])
    for a, b in zip(kin, withk[3:]):
        assert torch.equal(a, b)
    rng = np.random.default_rng(4)
    q0 = args[0].clone().requires_grad_(True)
    v0 = args[1].clone().requires_grad_(True)
    u0 = args[3].clone().requires_grad_(True)
    out = ffi.step(q0, v0, args[2], u0, args[4], args[5], kinematics=True)
    cots = [_t(rng.normal(0, 1, tuple(o.shape))) for o in out]
    torch.autograd.backward([out[k] for k in (0, 1, 3, 4, 5, 6, 7)], [cots[k] for k in (0, 1, 3, 4, 5, 6, 7)])
    q1, v1, w1, info, tape = ffi.forward(*args, tape=True)
    gq, gv, gu, _ = ffi.backward(tape, args[4], args[5], cots[0], cots[1],
                                 kinematics=(q1, v1, cots[3], cots[4], cots[5], cots[6], cots[7]))
    torch.cuda.synchronize()
    assert torch.equal(q0.grad, gq) and torch.equal(v0.grad, gv) and torch.equal(u0.grad, gu)
    assert torch.isfinite(gq).all() and torch.isfinite(gv).all()


def test_kinematics_autograd_and_edges(ffi):
    """kinematics() under autograd: the gradient of a linear loss is the VJP of its weights; B = 0 gives empty
    outputs; shape and device errors are TypeError."""
    import torch
    B = 16
    st = _states(B)
    q = _t(st["qpos"]).requires_grad_(True)
    v = _t(st["qvel"]).requires_grad_(True)
    c3 = _t(st["com"])
    out = ffi.kinematics(q, v, c3)
    w = [torch.randn_like(o) for o in out]
    sum((a * b).sum() for a, b in zip(out, w)).backward()
    gq, gv = ffi._ops().kinematics_backward(q.detach(), v.detach(), c3, *w)
    assert torch.equal(q.grad, gq) and torch.equal(v.grad, gv)
    e = ffi.kinematics(_t(st["qpos"][:0]), _t(st["qvel"][:0]), _t(st["com"][:0]))
    assert e[1].shape == (0, 31, 3) and e[3].shape == (0, 31, 6)
    with pytest.raises(TypeError):
        ffi.kinematics(_t(st["qpos"][:, :35]), _t(st["qvel"]), c3)
    with pytest.raises(TypeError):
        ffi.kinematics(torch.from_numpy(st["qpos"]), _t(st["qvel"]), c3)
