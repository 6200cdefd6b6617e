"""PyTorch interface of the MI355X G1 engine, on torch's current HIP stream (a drop-in for the reference's
``nablaengine.torch_ffi``, ``src/nablaengine/torch_ffi.py``).

  step(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, clamp_kv=0, normal=3, clamp_soft=None,
       grad_decay=1.0, kinematics=False) -> (qpos', qvel', warm')
  forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, tape=False)
       -> (qpos', qvel', warm', info[, tape])
  backward(tape, friction, com, g_qpos, g_qvel, *, substeps=4, clamp_kv=0, normal=3, ctrl=None, clamp_soft=None)
       -> (g_qpos, g_qvel, g_ctrl, info)

Arguments: float32 tensors on one ROCm device, contiguous, leading dimension B (the worlds): qpos (B, 36), qvel (B, 35),
warm (B, 35), ctrl (B, 29), friction (B,), com (B, 3). Other dtypes, devices or shapes raise TypeError; nothing is
cast or copied implicitly (reference torch_ffi.py:419-428 _check). Bad options raise ValueError (torch_ffi.py:824-829),
a failed library call RuntimeError (torch_ffi.py:431-433 _rc). B = 0 returns empty outputs without a launch.

The library is libnablaengine_g1.so next to this file (built in-tree by ``python -m nablaengine_amd.build``), loaded
with ctypes; every call goes to its C entries (include/nablaengine_g1.h) with torch's current stream and the tensors'
device pointers, the inputs' device made current. There is no fallback: without the library, or without a GPU, the
calls raise. After init() the calls only launch kernels and allocate through torch's caching allocator (no host
synchronization), so they can be captured in a HIP graph with fixed shapes.
"""
import ctypes
import math
import os
import threading

ITERATIONS, SUBSTEPS, CLAMP_KV, NORMAL = 10, 4, 0, 3  # reference torch_ffi.py:54
CLAMP_SOFT, GRAD_DECAY = 0.2, 1.0  # reference torch_ffi.py:55
NQ, NV, NU, NBODY = 36, 35, 29, 31
MAXCON = 64
OVERFLOW_CONTACTS, OVERFLOW_ROWS = 4, 16  # forward info[:, 3] bits (reference torch_ffi.py:60)
VARIANTS = tuple((kv, n) for kv in (0, 1, 2) for n in (0, 1, 2, 3))  # adjoint variants (clamp_kv, normal)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnablaengine_g1.so")

_LOCK = threading.Lock()
_STATE = {}
_READY = set()


def _err(msg, exc=TypeError):
    return exc(f"nablaengine_amd.torch_ffi: {msg}")


def load_library(path=None):
    """ctypes handle of the library with the C entries' argument types set; raises RuntimeError when it is missing
    (build it with `python -m nablaengine_amd.build`)."""
    with _LOCK:
        if "lib" in _STATE:
            return _STATE["lib"]
        p = path or os.environ.get("NABLA_G1_LIB", LIB_PATH)
        if not os.path.exists(p):
            raise _err(f"{p} is missing: build it with `python -m nablaengine_amd.build`", RuntimeError)
        lib = ctypes.CDLL(p)
        vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.dk_fwd_forward.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 7
        lib.dk_fwd_forward.restype = i32
        lib.dk_fwd_forward_ordered.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 7
        lib.dk_fwd_forward_ordered.restype = i32
        lib.dk_fwd_order.argtypes, lib.dk_fwd_order.restype = [vp, i32, vp, vp], i32
        lib.dk_fwd_work_bytes.argtypes, lib.dk_fwd_work_bytes.restype = [i32], ctypes.c_longlong
        lib.dk_fwd_upload.argtypes, lib.dk_fwd_upload.restype = [vp, vp], i32
        lib.dk_fwd_sizes.argtypes, lib.dk_fwd_sizes.restype = [vp], None
        lib.dk_adjoint.argtypes = [vp, i32, i32] + [vp] * 10 + [f32, i32, i32]
        lib.dk_adjoint.restype = i32
        lib.dk_adjoint_work.argtypes = [vp, i32, i32] + [vp] * 10 + [f32, i32, i32, vp]
        lib.dk_adjoint_work.restype = i32
        lib.dk_adjoint_work_bytes.argtypes, lib.dk_adjoint_work_bytes.restype = [i32], ctypes.c_longlong
        sizes = (ctypes.c_longlong * 9)()
        lib.dk_fwd_sizes(ctypes.cast(sizes, vp))
        _STATE["sizes"] = [int(x) for x in sizes]
        _STATE["lib"] = lib
        return lib


def rec_words():
    """Tape words per world and substep."""
    load_library()
    return _STATE["sizes"][2]


def init(device=None):
    """Load the library and check that `device` (default: torch's current device) can run it; idempotent per
    device. The model constants are compiled into the library, so nothing is uploaded and nothing synchronizes."""
    import torch
    lib = load_library()
    if not torch.cuda.is_available():
        raise _err("no ROCm GPU visible: the engine runs on the GPU only", RuntimeError)
    dev = torch.cuda.current_device() if device is None else torch.device(device).index
    dev = torch.cuda.current_device() if dev is None else dev
    if dev not in _READY:
        with torch.cuda.device(dev):
            rc = lib.dk_fwd_upload(None, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        if rc:
            raise _err(f"device cuda:{dev} cannot run the kernels (code {rc})", RuntimeError)
        _READY.add(dev)
    return dict(path=LIB_PATH, sizes=list(_STATE["sizes"]))


def tape_bytes(nworld, substeps=SUBSTEPS, steps=1):
    """Bytes of the tapes of `steps` differentiated control steps (reference torch_ffi.py:454-458)."""
    return 4 * rec_words() * substeps * nworld * steps


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check(name, x, shape, dev, dtype=None):
    import torch
    dtype = dtype or torch.float32
    if not isinstance(x, torch.Tensor):
        raise _err(f"{name} must be a torch.Tensor, got {type(x).__name__}")
    if x.dtype != dtype or tuple(x.shape) != tuple(shape) or x.device.type != "cuda" or not x.is_contiguous():
        raise _err(f"{name} must be a contiguous {dtype} GPU tensor {tuple(shape)}, got {x.dtype} {tuple(x.shape)} on "
                   f"{x.device}{'' if x.is_contiguous() else ' (not contiguous)'}")
    if dev is not None and x.device.index != dev:
        raise _err(f"{name} is on {x.device}, the other tensors on cuda:{dev}")


def _rc(rc, what):
    if rc:
        raise _err(f"{what} failed (HIP error {rc})", RuntimeError)


def _soft(clamp_kv, clamp_soft):
    """The soft clamp's delta for clamp_kv 2 (None: CLAMP_SOFT); None for 0 / 1 (reference torch_ffi.py:436-449)."""
    if int(clamp_kv) != 2:
        if clamp_soft is not None:
            raise _err(f"clamp_soft is the soft clamp's (clamp_kv=2), not clamp_kv={clamp_kv}", ValueError)
        return None
    d = float(CLAMP_SOFT if clamp_soft is None else clamp_soft)
    if not (math.isfinite(d) and d >= 0.0):
        raise _err(f"clamp_soft must be finite and >= 0, got {clamp_soft}", ValueError)
    return d


class _OnDevice:
    def __init__(self, dev):
        self.dev = dev

    def __enter__(self):
        import torch
        self.prev = torch.cuda.current_device()
        if self.prev != self.dev:
            torch.cuda.set_device(self.dev)

    def __exit__(self, *a):
        import torch
        if self.prev != self.dev:
            torch.cuda.set_device(self.prev)


def _forward_impl(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape):
    import torch
    if not isinstance(qpos, torch.Tensor):
        raise _err(f"qpos must be a torch.Tensor, got {type(qpos).__name__}")
    if qpos.device.type != "cuda":
        raise _err(f"qpos must be a GPU tensor, got {qpos.device}")
    dev = qpos.device.index
    B = qpos.shape[0] if qpos.dim() == 2 else -1
    for name, x, shape in (("qpos", qpos, (B, NQ)), ("qvel", qvel, (B, NV)), ("warm", warm, (B, NV)),
                           ("ctrl", ctrl, (B, NU)), ("friction", friction, (B,)), ("com", com, (B, 3))):
        _check(name, x, shape, dev)
    if substeps < 1 or substeps > 32 or iterations < 0:
        raise _err("substeps in 1..32 and iterations >= 0", ValueError)
    if dev not in _READY:
        init(dev)
    lib = _STATE["lib"]
    kw = dict(dtype=torch.float32, device=qpos.device)
    q1, v1, w1 = torch.empty((B, NQ), **kw), torch.empty((B, NV), **kw), torch.empty((B, NV), **kw)
    info = torch.empty((B, 4), dtype=torch.int32, device=qpos.device)
    rw = _STATE["sizes"][2]
    tp = torch.empty((B if tape else 0, substeps * rw), **kw)
    if B == 0:
        return [q1, v1, w1, info, tp]
    work = torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device=qpos.device)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _rc(lib.dk_fwd_forward(st, B, *map(_ptr, (qpos, qvel, warm, ctrl, friction, com)), int(iterations),
                               int(substeps), _ptr(q1), _ptr(v1), _ptr(w1), _ptr(info), None,
                               _ptr(tp) if tape else None, _ptr(work) if work.numel() else None),
            "the forward launch")
    return [q1, v1, w1, info, tp]


def _backward_impl(tape, friction, com, g_qpos, g_qvel, ctrl, substeps, clamp_kv, normal, clamp_soft):
    import torch
    if not isinstance(tape, torch.Tensor) or tape.device.type != "cuda":
        raise _err("tape must be a GPU torch.Tensor")
    dev = tape.device.index
    rw = rec_words()
    B = tape.shape[0]
    for name, x, shape in (("tape", tape, (B, substeps * rw)), ("friction", friction, (B,)), ("com", com, (B, 3)),
                           ("g_qpos", g_qpos, (B, NQ)), ("g_qvel", g_qvel, (B, NV))):
        _check(name, x, shape, dev)
    v = (int(clamp_kv), int(normal))
    if v not in VARIANTS:
        raise _err(f"no adjoint variant clamp_kv={clamp_kv} normal={normal}", ValueError)
    if (v[0] == 2) != (ctrl is not None):
        raise _err("clamp_kv=2 (the soft clamp) needs the step's ctrl; 0 and 1 take none", ValueError)
    if ctrl is not None:
        _check("ctrl", ctrl, (B, NU), dev)
    if dev not in _READY:
        init(dev)
    kw = dict(dtype=torch.float32, device=tape.device)
    gq, gv, gu = torch.empty((B, NQ), **kw), torch.empty((B, NV), **kw), torch.empty((B, NU), **kw)
    info = torch.empty((B,), dtype=torch.int32, device=tape.device)
    if B == 0:
        return [gq, gv, gu, info]
    lib = _STATE["lib"]
    work = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device=tape.device)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _rc(lib.dk_adjoint_work(st, B, int(substeps), _ptr(tape), _ptr(friction), _ptr(com), _ptr(g_qpos),
                                _ptr(g_qvel), _ptr(gq), _ptr(gv), _ptr(gu), _ptr(info), _ptr(ctrl),
                                ctypes.c_float(0.0 if clamp_soft is None else clamp_soft), v[0], v[1],
                                _ptr(work) if work.numel() else None),
            "the adjoint launch")
    return [gq, gv, gu, info]


def _make_step_fn():
    import torch

    class _Step(torch.autograd.Function):
        """reference torch_ffi.py:747-779: the tape as the residual; gradients for qpos, qvel and ctrl only."""

        @staticmethod
        def forward(ctx, qpos, qvel, warm, ctrl, friction, com, iterations, substeps, clamp_kv, normal, clamp_soft,
                    grad_decay):
            q1, v1, w1, info, tp = _forward_impl(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, True)
            ctx.save_for_backward(tp, friction, com, ctrl, q1, v1)
            ctx.opts = (substeps, clamp_kv, normal, clamp_soft, grad_decay)
            ctx.mark_non_differentiable(w1)
            return q1, v1, w1

        @staticmethod
        def backward(ctx, g_q1, g_v1, g_w1):
            tp, friction, com, ctrl, q1, v1 = ctx.saved_tensors
            substeps, clamp_kv, normal, clamp_soft, grad_decay = ctx.opts
            g_q1 = torch.zeros_like(q1) if g_q1 is None else g_q1.contiguous()
            g_v1 = torch.zeros_like(v1) if g_v1 is None else g_v1.contiguous()
            gq, gv, gu, _ = _backward_impl(tp, friction, com, g_q1, g_v1, ctrl if clamp_kv == 2 else None, substeps,
                                           clamp_kv, normal, clamp_soft)
            if grad_decay != 1.0:  # the state cotangent through this step times it, ctrl's not (float32 product)
                gq, gv = gq * grad_decay, gv * grad_decay
            return gq, gv, None, gu, None, None, None, None, None, None, None, None

    return _Step


_FNS = {}


def _fn(name, make):
    if name not in _FNS:
        _FNS[name] = make()
    return _FNS[name]


def step(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, clamp_kv=CLAMP_KV,
         normal=NORMAL, clamp_soft=None, grad_decay=GRAD_DECAY, kinematics=False):
    """One control step: (qpos', qvel', warm') (reference torch_ffi.py:817-835). Differentiable in qpos, qvel and ctrl
    when any input requires grad (the forward then also writes the tape); warm' is not differentiable."""
    import torch
    if int(clamp_kv) not in (0, 1, 2) or int(normal) not in (0, 1, 2, 3):
        raise _err("clamp_kv in {0, 1, 2}, normal in 0..3", ValueError)
    if kinematics:
        raise _err("kinematics=True: the kinematics outputs are not in this build", ValueError)
    soft = _soft(clamp_kv, clamp_soft)
    gd = float(grad_decay)
    if not math.isfinite(gd):
        raise _err(f"grad_decay must be finite, got {grad_decay}", ValueError)
    args = (qpos, qvel, warm, ctrl, friction, com)
    if torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in args):
        return _fn("step", _make_step_fn).apply(*args, int(iterations), int(substeps), int(clamp_kv), int(normal),
                                                soft, gd)
    r = _forward_impl(*args, int(iterations), int(substeps), False)
    return tuple(r[:3])


def forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, tape=False):
    """One control step without autograd: (qpos', qvel', warm', info (B, 4) int32[, tape]) (reference
    torch_ffi.py:845-851)."""
    r = _forward_impl(qpos, qvel, warm, ctrl, friction, com, int(iterations), int(substeps), bool(tape))
    return tuple(r[:4]) + ((r[4],) if tape else ())


def backward(tape, friction, com, g_qpos, g_qvel, *, substeps=SUBSTEPS, clamp_kv=CLAMP_KV, normal=NORMAL, ctrl=None,
             clamp_soft=None):
    """The adjoint of one control step from its tape: (g_qpos (B, 36), g_qvel (B, 35), g_ctrl (B, 29), info (B,))
    (reference torch_ffi.py:854-865)."""
    soft = _soft(clamp_kv, clamp_soft)
    if soft is not None and ctrl is None:
        raise _err("clamp_kv=2 (the soft clamp) needs the step's ctrl", ValueError)
    return tuple(_backward_impl(tape, friction, com, g_qpos, g_qvel, ctrl if soft is not None else None, int(substeps),
                                int(clamp_kv), int(normal), soft))


def _make_scale_fn():
    import torch

    class _Scale(torch.autograd.Function):
        @staticmethod
        def forward(ctx, gamma, *xs):
            ctx.gamma = gamma
            return tuple(x.view_as(x) for x in xs)

        @staticmethod
        def backward(ctx, *g):
            return (None,) + tuple(None if x is None else x * ctx.gamma for x in g)

    return _Scale


def scale_grad(tree, gamma):
    """The identity on a pytree of tensors whose cotangent the backward multiplies by gamma (floating tensors only)
    (reference torch_ffi.py:868-899)."""
    import torch
    from torch.utils import _pytree
    g = float(gamma)
    if not math.isfinite(g):
        raise _err(f"scale_grad's gamma must be finite, got {gamma}", ValueError)
    leaves, spec = _pytree.tree_flatten(tree)
    idx = [i for i, x in enumerate(leaves) if isinstance(x, torch.Tensor) and x.is_floating_point()]
    if idx:
        out = _fn("scale", _make_scale_fn).apply(g, *(leaves[i] for i in idx))
        for i, x in zip(idx, out):
            leaves[i] = x
    return _pytree.tree_unflatten(leaves, spec)
