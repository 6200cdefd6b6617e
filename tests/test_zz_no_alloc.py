"""The allocation-free forward (dk_fwd_forward_static, through the C ABI): bitwise dk_fwd_forward's outputs, info
and tape with a caller-provided work buffer, on two calls in a row (the second with fewer worlds, so the shared
static scratch holds the first call's longer order), and the capacity error without a launch."""
import ctypes
import os
import re

import numpy as np
import pytest

from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
KEYS = ("qpos", "qvel", "warm", "ctrl", "friction", "com")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible")
    from nablaengine_amd import torch_ffi
    torch_ffi.init(0)
    L = ctypes.CDLL(torch_ffi.load_library()._name)
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    L.dk_fwd_forward.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 7
    L.dk_fwd_forward_static.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 6
    L.dk_fwd_forward.restype = L.dk_fwd_forward_static.restype = i32
    L.dk_fwd_work_bytes.argtypes, L.dk_fwd_work_bytes.restype = [i32], ctypes.c_longlong
    return L


def _run(lib, st, static):
    import torch
    B = len(st["qpos"])
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [torch.from_numpy(st[k]).cuda() for k in KEYS]
    kw = dict(dtype=torch.float32, device="cuda")
    out = [torch.full((B, 36), np.nan, **kw), torch.full((B, 35), np.nan, **kw), torch.full((B, 35), np.nan, **kw),
           torch.full((B, 4), -1, dtype=torch.int32, device="cuda"), torch.full((B, 64, 8), np.nan, **kw),
           torch.full((B, 4 * 1472), np.nan, **kw)]
    if static:
        rc = lib.dk_fwd_forward_static(stream, B, *map(p, args), 10, 4, *map(p, out))
    else:
        work = torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device="cuda")
        rc = lib.dk_fwd_forward(stream, B, *map(p, args), 10, 4, *map(p, out), p(work))
    torch.cuda.synchronize()
    assert rc == 0
    return out


def test_static_forward_equals_the_work_buffer_forward(lib):
    import torch
    for B in (2048, 600):  # the second call smaller than the first
        print(f"static forward: {B} config-4 worlds", flush=True)
        st = synthetic.states(B, config=4)
        a = _run(lib, st, static=True)
        b = _run(lib, st, static=False)
        for x, y in zip(a, b):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))
        assert torch.isfinite(a[1]).all()


def test_static_forward_at_capacity(lib):
    """At DK_STATIC_MAX_WORLDS worlds the static scratch (a permutation and a cost per world) is exactly full: outputs
    and info bitwise the work-buffer forward's (no tape, no contact output at this size)."""
    import torch
    hdr = open(os.path.join(ROOT, "include", "nablaengine_g1.h")).read()
    B = int(re.search(r"#define DK_STATIC_MAX_WORLDS (\d+)", hdr).group(1))
    print(f"static forward at capacity: {B} config-1 worlds", flush=True)
    st = synthetic.states(B, config=1, seed=5)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [torch.from_numpy(st[k]).cuda() for k in KEYS]
    res = []
    for static in (True, False):
        out = [torch.empty((B, 36), device="cuda"), torch.empty((B, 35), device="cuda"),
               torch.empty((B, 35), device="cuda"), torch.full((B, 4), -1, dtype=torch.int32, device="cuda")]
        if static:
            rc = lib.dk_fwd_forward_static(stream, B, *map(p, args), 10, 4, *map(p, out), None, None)
        else:
            work = torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device="cuda")
            rc = lib.dk_fwd_forward(stream, B, *map(p, args), 10, 4, *map(p, out), None, None, p(work))
        torch.cuda.synchronize()
        assert rc == 0
        res.append(out)
    for x, y in zip(*res):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
    assert torch.isfinite(res[0][1]).all() and (res[0][3][:, 0] >= 1).all()


def test_static_forward_capacity_error(lib):
    import torch
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    hdr = open(os.path.join(ROOT, "include", "nablaengine_g1.h")).read()
    big = int(re.search(r"#define DK_STATIC_MAX_WORLDS (\d+)", hdr).group(1))
    rc = lib.dk_fwd_forward_static(stream, big + 1, *([None] * 6), 10, 4, *([None] * 6))
    assert rc == -2  # DK_ERR_STATIC_CAPACITY: rejected before any launch
    assert lib.dk_fwd_forward_static(stream, 0, *([None] * 6), 10, 4, *([None] * 6)) == 0
