"""The torch surface under HIP graph capture and torch.compile (reference docs/api_torch.md "CUDA graphs and
torch.compile"; scripts/torch_ffi_check.py section compile): a captured forward + backward replayed several times,
with eager work between the replays, each replay bitwise the eager result; torch.compile(fullgraph=True) of a loss
through step (and through step(..., kinematics=True)) with no graph break and gradients bitwise eager's."""
import numpy as np
import pytest

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


def _inputs(B, seed=None):
    st = synthetic.states(B, config=1, seed=seed)
    return [_t(st[k]) for k in KEYS]


def test_graph_capture_forward_backward(ffi):
    """forward(tape=True) + backward captured in one graph on static inputs; three replays, each after new inputs were
    copied in and an eager step ran, each bitwise the eager forward and backward of those inputs."""
    import torch
    B = 256
    static = _inputs(B)
    gq0, gv0 = (_t(x) for x in synthetic.cotangents(B))
    ffi.forward(*static, tape=True)  # warm the caching allocator outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        q1, v1, w1, info, tp = ffi.forward(*static, tape=True)
        bq, bv, bu, binfo = ffi.backward(tp, static[4], static[5], gq0, gv0)
    for rep in range(3):
        new = _inputs(B, seed=100 + rep)
        for a, b in zip(static, new):
            a.copy_(b)
        ffi.step(*_inputs(B, seed=200 + rep))  # unrelated eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        e = ffi.forward(*new, tape=True)
        eb = ffi.backward(e[4], new[4], new[5], gq0, gv0)
        torch.cuda.synchronize()
        for a, b in zip((q1, v1, w1, info, bq, bv, bu, binfo), tuple(e[:4]) + tuple(eb)):
            assert torch.equal(a, b), f"replay {rep}"


def _loss_fn(ffi, cq, cv, kin=False, cx=None):
    def f(q, v, w, u, fr, c):
        if kin:
            out = ffi.step(q, v, w, u, fr, c, kinematics=True)
            return (out[0] * cq).sum() + (out[1] * cv).sum() + (out[4] * cx).sum()
        q1, v1, _ = ffi.step(q, v, w, u, fr, c)
        return (q1 * cq).sum() + (v1 * cv).sum()
    return f


@pytest.mark.parametrize("kin,backend", [(False, "aot_eager"), (True, "aot_eager"), (False, "inductor")])
def test_compile_fullgraph(ffi, kin, backend):
    """torch.compile(fullgraph=True) of a loss through step: no graph break; the qpos, qvel, ctrl gradients bitwise
    eager's (the reference's compile check). aot_eager (the graph, the fake implementations and the autograd through
    the custom ops, without a code generator) also gives the loss bitwise; inductor generates its own kernels for the
    loss's products and sums, so its loss agrees to float32 rounding."""
    import torch
    B = 64
    tin = _inputs(B)
    cq, cv = (_t(x) for x in synthetic.cotangents(B))
    cx = _t(np.random.default_rng(5).normal(0, 1, (B, 31, 3)))
    f = _loss_fn(ffi, cq, cv, kin, cx)
    torch._dynamo.reset()
    x = [t.clone().requires_grad_(i in (0, 1, 3)) for i, t in enumerate(tin)]
    ex = torch._dynamo.explain(f)(*x)
    assert ex.graph_break_count == 0, ex.break_reasons
    torch._dynamo.reset()
    cf = torch.compile(f, fullgraph=True, backend=backend)
    x = [t.clone().requires_grad_(i in (0, 1, 3)) for i, t in enumerate(tin)]
    lc = cf(*x)
    lc.backward()
    x2 = [t.clone().requires_grad_(i in (0, 1, 3)) for i, t in enumerate(tin)]
    le = f(*x2)
    le.backward()
    torch.cuda.synchronize()
    assert torch.equal(lc, le) if backend == "aot_eager" else torch.allclose(lc, le, rtol=1e-5, atol=0)
    for i in (0, 1, 3):
        assert torch.equal(x[i].grad, x2[i].grad), i
