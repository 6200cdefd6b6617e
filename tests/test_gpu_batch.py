"""A world's results do not depend on the batch it is in (one world per wavefront; no arithmetic across worlds; the
dispatch order only moves work in time): the forward's outputs, info and tape, and the adjoint's gradients, of any
slice of a batch are bitwise those of the same worlds in the whole batch, at sizes that are not multiples of anything
(1, 3, 63, 65, 1000, 2049), on config-1 and config-4 (contact-heavy) states. GPU."""
import numpy as np
import pytest

from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
SLICES = [(0, 1), (5, 8), (100, 163), (1900, 1965), (7, 1007), (0, 2049)]


@pytest.fixture(scope="module")
def ffi():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from nablaengine_amd import torch_ffi
    torch_ffi.init(0)
    return torch_ffi


def _cat(st, cq, cv):
    import torch
    x = [torch.from_numpy(np.ascontiguousarray(st[k], np.float32)).cuda()
         for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    return x, torch.from_numpy(cq).cuda(), torch.from_numpy(cv).cuda()


def _run(ffi, x, cq, cv):
    q1, v1, w1, info, tape = ffi.forward(*x, tape=True)
    gq, gv, gu, binfo = ffi.backward(tape, x[4], x[5], cq, cv, ctrl=x[3])
    return [t.cpu().numpy() for t in (q1, v1, w1, info, tape, gq, gv, gu, binfo)]


@pytest.mark.parametrize("config", [1, 4])
def test_slices_are_bitwise_the_whole_batch(ffi, config):
    B = 2049
    st = synthetic.states(B, config=config, seed=77)
    cq, cv = synthetic.cotangents(B, seed=78)
    x, tcq, tcv = _cat(st, cq, cv)
    whole = _run(ffi, x, tcq, tcv)
    names = ("qpos'", "qvel'", "warm'", "info", "tape", "g_qpos", "g_qvel", "g_ctrl", "backward info")
    for a, b in SLICES:
        part = _run(ffi, [t[a:b].contiguous() for t in x], tcq[a:b].contiguous(), tcv[a:b].contiguous())
        for name, w, p in zip(names, whole, part):
            assert np.array_equal(w[a:b].view(np.uint32) if w.dtype == np.float32 else w[a:b],
                                  p.view(np.uint32) if p.dtype == np.float32 else p), (config, a, b, name)
