"""The dispatch order (g1_order.hip): k_order's permutation for the forward and the adjoint launches must be a
bijection of the worlds at every batch size (partial thread batches, fewer worlds than threads, more worlds than one
pass of the workgroup keeps in registers), heaviest first by the cost estimate in the work buffer."""
import ctypes

import numpy as np
import pytest

from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ffi():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from nablaengine_amd import torch_ffi
    torch_ffi.init(0)
    return torch_ffi


def _check(work, nw, cost=None):
    import torch
    w = work.view(torch.int32)[:2 * nw].cpu().numpy()
    perm, cost = w[:nw], (w[nw:] if cost is None else cost)
    assert np.array_equal(np.sort(perm), np.arange(nw)), "not a permutation"
    assert cost.min() >= 0 and cost.max() < 128
    assert np.all(np.diff(cost[perm]) <= 0), "not heaviest first"


@pytest.mark.parametrize("nw", [1, 2, 3, 63, 64, 65, 1000, 1023, 1024, 1025, 4096, 8191, 8192, 8193, 40001])
def test_forward_order_is_a_heaviest_first_bijection(ffi, nw):
    """dk_fwd_order on contact-heavy config-4 states (a wide spread of costs)."""
    import torch
    lib = ffi.load_library()
    st = synthetic.states(nw, config=4, seed=nw)
    qpos = torch.from_numpy(st["qpos"]).cuda()
    work = torch.empty((int(lib.dk_fwd_work_bytes(nw)),), dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.dk_fwd_order(stream, nw, ctypes.c_void_p(qpos.data_ptr()), ctypes.c_void_p(work.data_ptr())) == 0
    _check(work, nw)


@pytest.mark.parametrize("nw", [7, 1000, 4096, 9001])
def test_adjoint_order_is_a_heaviest_first_bijection(ffi, nw):
    """dk_adjoint_order on a taped step's tape, whose last record carries each world's cost (its last word, the
    taped forward's estimate of the adjoint's work)."""
    import torch
    lib = ffi.load_library()
    st = synthetic.states(nw, config=4, seed=nw)
    args = [torch.from_numpy(st[k]).cuda() for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    tape = ffi.forward(*args, tape=True)[4]
    work = torch.empty((int(lib.dk_adjoint_work_bytes(nw)),), dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.dk_adjoint_order(stream, nw, 4, ctypes.c_void_p(tape.data_ptr()),
                                ctypes.c_void_p(work.data_ptr())) == 0
    cost = tape.view(torch.int32).reshape(nw, 4, -1)[:, 3, -1].cpu().numpy()
    _check(work, nw, cost)
