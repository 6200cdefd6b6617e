"""A world's results do not depend on the batch it is in (one world per wavefront; no arithmetic across worlds; the
dispatch order only moves work in time): the forward's outputs, info and tape, and the adjoint's gradients, of any
slice of a batch are bitwise those of the same worlds in the whole batch, at sizes that are not multiples of anything
(1, 3, 63, 65, 1000, 2049), on config-1 and config-4 (contact-heavy) states, and at config 4's full 16384 worlds.
GPU."""
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


def test_nonfinite_worlds_leave_the_others_alone(ffi):
    """Worlds with non-finite inputs (NaN in qvel, inf in ctrl, NaN in the root quaternion, NaN friction) run their
    bounded loops to the end like any other (the Newton iteration cap, the line search's 40 evaluations, contact
    counts from comparisons): every other world's outputs, tape and gradients are bitwise those of the clean batch.
    The NaN state's worlds come out non-finite and the backward flags their gradients in its info (bits << 16); an
    infinite ctrl is a saturated actuator (its force clamped to the limit, the clamp bit set in every record) and
    the world stays finite."""
    import torch
    B = 257
    st = synthetic.states(B, config=1, seed=79)
    cq, cv = synthetic.cotangents(B, seed=80)
    x, tcq, tcv = _cat(st, cq, cv)
    clean = _run(ffi, x, tcq, tcv)
    bad = {3: ("qvel", 0), 100: ("ctrl", 5), 200: ("qpos", 4), 256: ("friction", None)}
    y = [t.clone() for t in x]
    keys = ("qpos", "qvel", "warm", "ctrl", "friction", "com")
    for w, (k, j) in bad.items():
        t = y[keys.index(k)]
        if j is None:
            t[w] = np.nan
        else:
            t[w, j] = np.inf if k == "ctrl" else np.nan
    dirty = _run(ffi, y, tcq, tcv)
    keep = np.setdiff1d(np.arange(B), list(bad))
    names = ("qpos'", "qvel'", "warm'", "info", "tape", "g_qpos", "g_qvel", "g_ctrl", "backward info")
    for name, a, b in zip(names, clean, dirty):
        view = (lambda z: z[keep].view(np.uint32)) if a.dtype == np.float32 else (lambda z: z[keep])
        assert np.array_equal(view(a), view(b)), name
    for w in (3, 200):
        assert not np.isfinite(dirty[1][w]).all(), w
        assert (dirty[8][w] >> 16) & 7, w  # the backward's non-finite gradient bits (qpos 1, qvel 2, ctrl 4)
    assert np.isfinite(dirty[0][100]).all() and np.isfinite(dirty[1][100]).all()
    clamp = dirty[4][100].reshape(4, -1)[:, 2].view(np.uint32)  # each record's clamp mask (bit: dof)
    assert ((clamp >> (6 + 5)) & 1).all()


def test_full_size_batch_is_bitwise_its_slices(ffi):
    """At BASELINE config 4's size (16384 contact-heavy worlds, the largest batch the configs name): the forward's
    outputs, info and tape and the adjoint's gradients of two 256-world slices taken from the whole batch (its start
    and its end) are bitwise those of the same worlds run alone, and every world either stays finite or carries an
    overflow flag."""
    B = 16384
    st = synthetic.states(B, config=4, seed=81)
    cq, cv = synthetic.cotangents(B, seed=82)
    x, tcq, tcv = _cat(st, cq, cv)
    whole = _run(ffi, x, tcq, tcv)
    names = ("qpos'", "qvel'", "warm'", "info", "tape", "g_qpos", "g_qvel", "g_ctrl", "backward info")
    flagged = (whole[3][:, 3] & (4 | 16)) != 0
    finite = np.isfinite(whole[1]).all(1) & np.isfinite(whole[0]).all(1) & np.isfinite(whole[5]).all(1)
    assert (finite | flagged).all(), np.flatnonzero(~(finite | flagged))[:8]
    for a, b in ((0, 256), (B - 256, B)):
        part = _run(ffi, [t[a:b].contiguous() for t in x], tcq[a:b].contiguous(), tcv[a:b].contiguous())
        for name, w, p in zip(names, whole, part):
            assert np.array_equal(w[a:b].view(np.uint32) if w.dtype == np.float32 else w[a:b],
                                  p.view(np.uint32) if p.dtype == np.float32 else p), (a, b, name)
