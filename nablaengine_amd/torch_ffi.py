"""PyTorch interface of the MI355X G1 engine, on torch's current HIP stream (a drop-in for the reference's
``nablaengine.torch_ffi``, ``src/nablaengine/torch_ffi.py``).

  step(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, clamp_kv=0, normal=3, clamp_soft=None,
       grad_decay=1.0, kinematics=False) -> (qpos', qvel', warm'[, qpos_n, xpos, xquat, cvel, subtree_com])
  kinematics(qpos, qvel, com) -> (qpos_n, xpos, xquat, cvel, subtree_com)
  forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, tape=False, kinematics=False)
       -> (qpos', qvel', warm', info[, tape][, the kinematics outputs])
  backward(tape, friction, com, g_qpos, g_qvel, *, substeps=4, clamp_kv=0, normal=3, ctrl=None, clamp_soft=None,
           kinematics=None) -> (g_qpos, g_qvel, g_ctrl, info)

The kinematics outputs (reference g1_engine/kinematics.py:1-45, MJX kinematics + com_pos + com_vel) of a state:
qpos_n (B, 36) qpos with the root quaternion normalized, xpos (B, 31, 3), xquat (B, 31, 4) the body frames, cvel
(B, 31, 6) [angular; linear] twists at subtree_com[:, 1], subtree_com (B, 31, 3). step(..., kinematics=True) gives
those of its output state, bitwise kinematics(qpos', qvel', com); their cotangents join the step's in its backward.

Arguments: float32 tensors on one ROCm device, contiguous, leading dimension B (the worlds): qpos (B, 36), qvel (B, 35),
warm (B, 35), ctrl (B, 29), friction (B,), com (B, 3). Other dtypes, devices or shapes raise TypeError; nothing is
cast or copied implicitly (reference torch_ffi.py:419-428 _check). Bad options raise ValueError (torch_ffi.py:824-829),
a failed library call RuntimeError (torch_ffi.py:431-433 _rc). B = 0 returns empty outputs without a launch.

The library is libnablaengine_g1.so next to this file (built in-tree by ``python -m nablaengine_amd.build``), loaded
with ctypes; every call goes to its C entries (include/nablaengine_g1.h) with torch's current stream and the tensors'
device pointers, the inputs' device made current. There is no fallback: without the library, or without a GPU, the
calls raise. After init() the calls only launch kernels and allocate through torch's caching allocator (no host
synchronization), so they can be captured in a HIP graph with fixed shapes. While torch.compile traces, the library
calls are the torch.library custom ops nablaengine::forward, ::backward, ::kinematics and ::kinematics_backward with
fake implementations (opaque nodes, no graph break with fullgraph=True; reference torch_ffi.py:583-655); in eager mode
the same functions are called directly.

Diagnostics (reference torch_ffi.py:56-62, 664-742): per device 18 int64 counters (DIAG) added to on the device by the
forward and adjoint kernels, each world at its end (set_diagnostics(False) skips it; the reference runs a small kernel
after each call, which the library also exports: dk_torch_diag_fwd / _bwd), read with diagnostics() (the tensor)
or read_diagnostics() (a dict; resets). The backward's info then also carries the non-finite bits (NONFINITE_* <<
NONFINITE_SHIFT) besides the union of the records' flags and ADJ_REPLAY_MISMATCH. set_overflow_warnings(True) warns
when worlds exceeded the contact or row capacity.
"""
import atexit
import ctypes
import math
import os
import threading

ITERATIONS, SUBSTEPS, CLAMP_KV, NORMAL = 10, 4, 0, 3  # reference torch_ffi.py:54
CLAMP_SOFT, GRAD_DECAY = 0.2, 1.0  # reference torch_ffi.py:55
NQ, NV, NU, NBODY = 36, 35, 29, 31
MAXCON = 64
OVERFLOW_CONTACTS, OVERFLOW_ROWS = 4, 16  # forward info[:, 3] bits (reference torch_ffi.py:60)
# the diagnostic counters, in the reference's order (torch_ffi.py:56-59); backward info's non-finite bits (61)
DIAG = ("fwd_calls", "fwd_worlds", "fwd_unsupported_worlds", "fwd_iteration_limit_worlds", "tape_records",
        "refact_records", "nonconv_records", "singular_records", "bwd_calls", "bwd_rows", "nonfinite_rows",
        "nonfinite_qpos_rows", "nonfinite_qvel_rows", "nonfinite_ctrl_rows", "nonfinite_cotangent_rows",
        "replay_mismatch_worlds", "fwd_contact_overflow_worlds", "fwd_row_overflow_worlds")
NONFINITE_QPOS, NONFINITE_QVEL, NONFINITE_CTRL, NONFINITE_COT, NONFINITE_SHIFT = 1, 2, 4, 8, 16
ADJ_REPLAY_MISMATCH = 1 << 13  # backward info: a replayed contact was not found
TAPE_REFACT, TAPE_NONCONV, TAPE_SINGULAR = 1 << 8, 1 << 9, 1 << 10  # the records' flags (also in backward info)
VARIANTS = tuple((kv, n) for kv in (0, 1, 2) for n in (0, 1, 2, 3))  # adjoint variants (clamp_kv, normal)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnablaengine_g1.so")
ARCH = "gfx950"  # the one architecture the library is built for

_LOCK = threading.RLock()
_STATE = {}
_READY = set()
_DIAG = {}  # device index -> int64 (len(DIAG),) counters on that device
_DIAG_ON = [True]  # set_diagnostics
_OVERFLOW_WARN = [os.environ.get("DK_OVERFLOW_WARN", "0") not in ("", "0")]  # set_overflow_warnings


def _err(msg, exc=TypeError):
    return exc(f"nablaengine_amd.torch_ffi: {msg}")


def _library_path(artifact):
    """The library an artifact names: a .so path, or a JSON file whose "library" key names it (relative to the JSON
    file), as the reference's artifacts (torch_ffi.py:241-266); None: $DK_TORCH_ARTIFACT, $NABLA_G1_LIB, else the
    in-tree build."""
    a = artifact or os.environ.get("DK_TORCH_ARTIFACT") or os.environ.get("NABLA_G1_LIB") or LIB_PATH
    a = os.fspath(a)
    if a.endswith(".json"):
        import json
        with open(a) as f:
            meta = json.load(f)
        if "library" not in meta:
            raise _err(f"artifact {a} names no library", RuntimeError)
        return os.path.join(os.path.dirname(os.path.abspath(a)), meta["library"])
    return a


def load_library(path=None):
    """ctypes handle of the library with the C entries' argument types set (path: as init's artifact); raises
    RuntimeError when it is missing (build it with `python -m nablaengine_amd.build`), or when another library is
    loaded already (one library per process)."""
    with _LOCK:
        if "lib" in _STATE:
            if path is not None and os.path.realpath(_library_path(path)) != os.path.realpath(_STATE["path"]):
                raise _err(f"{_STATE['path']} is loaded: one library per process", RuntimeError)
            return _STATE["lib"]
        p = _library_path(path)
        if not os.path.exists(p):
            raise _err(f"{p} is missing: build it with `python -m nablaengine_amd.build`", RuntimeError)
        lib = ctypes.CDLL(p)
        vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.dk_fwd_forward.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 7
        lib.dk_fwd_forward.restype = i32
        lib.dk_fwd_forward_diag.argtypes = [vp, i32] + [vp] * 6 + [i32, i32] + [vp] * 8
        lib.dk_fwd_forward_diag.restype = i32
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
        lib.dk_adjoint_work_diag.argtypes = [vp, i32, i32] + [vp] * 10 + [f32, i32, i32, vp, vp]
        lib.dk_adjoint_work_diag.restype = i32
        lib.dk_adjoint_order.argtypes, lib.dk_adjoint_order.restype = [vp, i32, i32, vp, vp], i32
        lib.dk_adjoint_work_ordered.argtypes = [vp, i32, i32] + [vp] * 10 + [f32, i32, i32, vp, vp]
        lib.dk_adjoint_work_ordered.restype = i32
        lib.dk_adjoint_many.argtypes = [vp, i32, i32, i32] + [vp] * 10 + [f32, i32, i32, vp, vp]
        lib.dk_adjoint_many.restype = i32
        lib.dk_adjoint_work_bytes.argtypes, lib.dk_adjoint_work_bytes.restype = [i32], ctypes.c_longlong
        lib.dk_fwd_kinematics.argtypes, lib.dk_fwd_kinematics.restype = [vp, i32] + [vp] * 8, i32
        lib.dk_torch_diag_fwd.argtypes, lib.dk_torch_diag_fwd.restype = [vp, vp, i32, i32, i32, vp, vp], i32
        lib.dk_torch_diag_bwd.argtypes, lib.dk_torch_diag_bwd.restype = [vp, vp, i32] + [vp] * 6, i32
        lib.dk_fwd_kinematics_vjp.argtypes, lib.dk_fwd_kinematics_vjp.restype = [vp, i32] + [vp] * 12, i32
        sizes = (ctypes.c_longlong * 9)()
        lib.dk_fwd_sizes(ctypes.cast(sizes, vp))
        _STATE["sizes"] = [int(x) for x in sizes]
        _STATE["path"] = p
        _STATE["lib"] = lib
        return lib


def rec_words():
    """Tape words per world and substep."""
    load_library()
    return _STATE["sizes"][2]


def init(device=None, artifact=None, model_dir=None, model=None, foot_pairs=None):
    """Load the library and check that `device` (default: torch's current device) can run it; idempotent per device,
    one library per process (reference torch_ffi.py:268-290). artifact: the library (a .so, or a JSON artifact naming
    it); default $DK_TORCH_ARTIFACT, else the in-tree build. The G1 model is compiled into the library, so nothing is
    uploaded and nothing synchronizes; another model (model_dir / model / foot_pairs) is a ValueError. Returns the
    library's path, architecture and sizes."""
    import torch
    if model_dir is not None or model is not None or foot_pairs is not None:
        raise _err("the G1 model is compiled into this library: model_dir / model / foot_pairs are not supported",
                   ValueError)
    with _LOCK:
        lib = load_library(artifact)
        if not torch.cuda.is_available():
            raise _err("no ROCm GPU visible: the engine runs on the GPU only", RuntimeError)
        dev = torch.cuda.current_device() if device is None else torch.device(device).index
        dev = torch.cuda.current_device() if dev is None else dev
        if dev not in _READY:
            arch = getattr(torch.cuda.get_device_properties(dev), "gcnArchName", ARCH).split(":")[0]
            if arch != ARCH:
                raise _err(f"cuda:{dev} is {arch}, the library is built for {ARCH} (one architecture per process)",
                           RuntimeError)
            with torch.cuda.device(dev):
                rc = lib.dk_fwd_upload(None, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
            if rc:
                raise _err(f"device cuda:{dev} cannot run the kernels (code {rc})", RuntimeError)
            _DIAG[dev] = torch.zeros(len(DIAG), dtype=torch.int64, device=f"cuda:{dev}")
            _READY.add(dev)
        _custom_ops()  # defined here, outside any torch.compile trace (a definition inside one is not traceable),
        _fn("step", _make_step_fn)  # as the autograd functions
        _fn("kin", _make_kin_fn)
        return dict(path=_STATE["path"], arch=ARCH, sizes=list(_STATE["sizes"]))


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


def _kin_shapes(B):
    return (B, NQ), (B, NBODY, 3), (B, NBODY, 4), (B, NBODY, 6), (B, NBODY, 3)


def _kin_empty(B, device):
    import torch
    return [torch.empty(s, dtype=torch.float32, device=device) for s in _kin_shapes(B)]


def _forward_impl(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics=False):
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
    kin = _kin_empty(B, qpos.device) if kinematics else []
    if B == 0:
        return [q1, v1, w1, info, tp] + kin
    work = torch.empty((int(lib.dk_fwd_work_bytes(B)),), dtype=torch.uint8, device=qpos.device)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        args = (st, B, *map(_ptr, (qpos, qvel, warm, ctrl, friction, com)), int(iterations), int(substeps),
                _ptr(q1), _ptr(v1), _ptr(w1), _ptr(info), None, _ptr(tp) if tape else None,
                _ptr(work) if work.numel() else None)
        if _DIAG_ON[0]:  # the counters added to by the forward kernel itself (dk_torch_diag_fwd's counts)
            _rc(lib.dk_fwd_forward_diag(*args, _ptr(_DIAG[dev])), "the forward launch")
        else:
            _rc(lib.dk_fwd_forward(*args), "the forward launch")
        if kinematics:  # the output state's kinematics (reference torch_ffi.py:488-489)
            _rc(lib.dk_fwd_kinematics(st, B, _ptr(q1), _ptr(v1), _ptr(com), *map(_ptr, kin)), "the kinematics launch")
    return [q1, v1, w1, info, tp] + kin


def _backward_checks(tape, friction, com, g_qpos, g_qvel, ctrl, substeps, clamp_kv, normal):
    """The backward's argument checks (TypeError / ValueError, reference torch_ffi.py:419-428); returns (device, B)."""
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
    return dev, B


def _backward_impl(tape, friction, com, g_qpos, g_qvel, ctrl, substeps, clamp_kv, normal, clamp_soft, kin_state=(),
                   kin_cot=()):
    import torch
    dev, B = _backward_checks(tape, friction, com, g_qpos, g_qvel, ctrl, substeps, clamp_kv, normal)
    v = (int(clamp_kv), int(normal))
    kw = dict(dtype=torch.float32, device=tape.device)
    gq, gv, gu = torch.empty((B, NQ), **kw), torch.empty((B, NV), **kw), torch.empty((B, NU), **kw)
    info = torch.empty((B,), dtype=torch.int32, device=tape.device)
    if B == 0:
        return [gq, gv, gu, info]
    lib = _STATE["lib"]
    if kin_state:
        q1, v1 = kin_state
        _check("qpos'", q1, (B, NQ), dev)
        _check("qvel'", v1, (B, NV), dev)
        for name, x, shape in zip(("g_qpos_n", "g_xpos", "g_xquat", "g_cvel", "g_subtree_com"), kin_cot,
                                  _kin_shapes(B)):
            _check(name, x, shape, dev)
    work = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device=tape.device)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        if kin_state:  # the kinematics outputs' cotangents pulled back onto (qpos', qvel'), theirs added last
            cq, cv = torch.empty((B, NQ), **kw), torch.empty((B, NV), **kw)
            _rc(lib.dk_fwd_kinematics_vjp(st, B, _ptr(q1), _ptr(v1), _ptr(com), *map(_ptr, kin_cot), _ptr(g_qpos),
                                          _ptr(g_qvel), _ptr(cq), _ptr(cv)), "the kinematics VJP launch")
            g_qpos, g_qvel = cq, cv
        args = (st, B, int(substeps), _ptr(tape), _ptr(friction), _ptr(com), _ptr(g_qpos), _ptr(g_qvel), _ptr(gq),
                _ptr(gv), _ptr(gu), _ptr(info), _ptr(ctrl), ctypes.c_float(0.0 if clamp_soft is None else clamp_soft),
                v[0], v[1], _ptr(work) if work.numel() else None)
        if _DIAG_ON[0]:  # counters, and the non-finite bits into info (reference torch_ffi.py:538-540), by the
            _rc(lib.dk_adjoint_work_diag(*args, _ptr(_DIAG[dev])), "the adjoint launch")  # adjoint kernel itself
        else:
            _rc(lib.dk_adjoint_work(*args), "the adjoint launch")
    return [gq, gv, gu, info]



def _vjps(tape, friction, com, g_qpos, g_qvel, ctrl=None, *, substeps=SUBSTEPS, clamp_kv=CLAMP_KV, normal=NORMAL,
          clamp_soft=None):
    """K VJPs of one taped step in one adjoint launch (dk_adjoint_many): g_qpos (K, B, 36) and g_qvel (K, B, 35)
    output cotangents -> g_qpos_in (K, B, 36), g_qvel_in (K, B, 35), g_ctrl (K, B, 29) and info (K, B). Each k is
    backward(tape, ..., g_qpos[k], g_qvel[k]) bitwise (the diagnostics count K backward calls), the worlds of every set
    in one dispatch order: the step Jacobian's driver."""
    import torch
    K = g_qpos.shape[0] if isinstance(g_qpos, torch.Tensor) and g_qpos.dim() == 3 else 0
    if K < 1 or not isinstance(g_qvel, torch.Tensor) or g_qvel.dim() != 3 or g_qvel.shape[0] != K:
        raise _err("g_qpos (K, B, 36) and g_qvel (K, B, 35), K >= 1")
    dev, B = _backward_checks(tape, friction, com, g_qpos[0], g_qvel[0], ctrl, substeps, clamp_kv, normal)
    _check("g_qpos", g_qpos, (K, B, NQ), dev)
    _check("g_qvel", g_qvel, (K, B, NV), dev)
    kw = dict(dtype=torch.float32, device=tape.device)
    gq, gv, gu = (torch.empty((K, B, n), **kw) for n in (NQ, NV, NU))
    info = torch.empty((K, B), dtype=torch.int32, device=tape.device)
    if B == 0:
        return gq, gv, gu, info
    lib = _STATE["lib"]
    work = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device=tape.device)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _rc(lib.dk_adjoint_many(st, B, K, int(substeps), _ptr(tape), _ptr(friction), _ptr(com), _ptr(g_qpos),
                                _ptr(g_qvel), _ptr(gq), _ptr(gv), _ptr(gu), _ptr(info), _ptr(ctrl),
                                ctypes.c_float(0.0 if clamp_soft is None else clamp_soft), int(clamp_kv), int(normal),
                                _ptr(work), _ptr(_DIAG[dev]) if _DIAG_ON[0] else None), "the adjoint launch")
    return gq, gv, gu, info
    lib = _STATE["lib"]
    work = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device=tape.device)
    soft = ctypes.c_float(0.0 if clamp_soft is None else clamp_soft)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _rc(lib.dk_adjoint_order(st, B, int(substeps), _ptr(tape), _ptr(work)), "the adjoint order launch")
        d = _ptr(_DIAG[dev]) if _DIAG_ON[0] else None
        for k in range(K):
            _check("g_qpos[k]", g_qpos[k], (B, NQ), dev)
            _check("g_qvel[k]", g_qvel[k], (B, NV), dev)
            _rc(lib.dk_adjoint_work_ordered(st, B, int(substeps), _ptr(tape), _ptr(friction), _ptr(com),
                                            _ptr(g_qpos[k]), _ptr(g_qvel[k]), _ptr(gq[k]), _ptr(gv[k]), _ptr(gu[k]),
                                            _ptr(info), _ptr(ctrl), soft, int(clamp_kv), int(normal), _ptr(work), d),
                "the adjoint launch")
    return gq, gv, gu, info
    dev = tape.device.index
    lib = _STATE["lib"]
    work = torch.empty((int(lib.dk_adjoint_work_bytes(B)),), dtype=torch.uint8, device=tape.device)
    soft = ctypes.c_float(0.0 if clamp_soft is None else clamp_soft)
    with _OnDevice(dev):
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _rc(lib.dk_adjoint_order(st, B, int(substeps), _ptr(tape), _ptr(work)), "the adjoint order launch")
        d = _ptr(_DIAG[dev]) if _DIAG_ON[0] else None
        for k in range(1, K):
            _check("g_qpos[k]", g_qpos[k], (B, NQ), dev)
            _check("g_qvel[k]", g_qvel[k], (B, NV), dev)
            _rc(lib.dk_adjoint_work_ordered(st, B, int(substeps), _ptr(tape), _ptr(friction), _ptr(com),
                                            _ptr(g_qpos[k]), _ptr(g_qvel[k]), _ptr(gq[k]), _ptr(gv[k]), _ptr(gu[k]),
                                            _ptr(info), _ptr(ctrl), soft, int(clamp_kv), int(normal), _ptr(work), d),
                "the adjoint launch")
    return gq, gv, gu, info

def _kinematics_impl(qpos, qvel, com):
    import torch
    if not isinstance(qpos, torch.Tensor) or qpos.device.type != "cuda":
        raise _err("qpos must be a GPU torch.Tensor")
    dev = qpos.device.index
    B = qpos.shape[0] if qpos.dim() == 2 else -1
    for name, x, shape in (("qpos", qpos, (B, NQ)), ("qvel", qvel, (B, NV)), ("com", com, (B, 3))):
        _check(name, x, shape, dev)
    if dev not in _READY:
        init(dev)
    out = _kin_empty(B, qpos.device)
    if B:
        with _OnDevice(dev):
            st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            _rc(_STATE["lib"].dk_fwd_kinematics(st, B, _ptr(qpos), _ptr(qvel), _ptr(com), *map(_ptr, out)),
                "the kinematics launch")
    return out


def _kinematics_backward_impl(qpos, qvel, com, *cot):
    import torch
    dev = qpos.device.index
    B = qpos.shape[0]
    for name, x, shape in (("qpos", qpos, (B, NQ)), ("qvel", qvel, (B, NV)), ("com", com, (B, 3))):
        _check(name, x, shape, dev)
    for name, x, shape in zip(("g_qpos_n", "g_xpos", "g_xquat", "g_cvel", "g_subtree_com"), cot, _kin_shapes(B)):
        _check(name, x, shape, dev)
    kw = dict(dtype=torch.float32, device=qpos.device)
    gq, gv = torch.empty((B, NQ), **kw), torch.empty((B, NV), **kw)
    if B:
        with _OnDevice(dev):
            st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            _rc(_STATE["lib"].dk_fwd_kinematics_vjp(st, B, _ptr(qpos), _ptr(qvel), _ptr(com), *map(_ptr, cot), None,
                                                    None, _ptr(gq), _ptr(gv)), "the kinematics VJP launch")
    return [gq, gv]


def _backward_op_impl(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv, normal,
                      clamp_soft):
    """_backward_impl with the custom op's argument order (reference torch_ffi.py:617-622): clamp_soft 0.0 for none."""
    return _backward_impl(tape, friction, com, g_qpos, g_qvel, ctrl, substeps, clamp_kv, normal,
                          None if clamp_kv != 2 else clamp_soft, tuple(kin_state), tuple(kin_cot))


_OPS = {}
_IMPL = dict(forward=_forward_impl, backward=_backward_op_impl, kinematics=_kinematics_impl,
             kinematics_backward=_kinematics_backward_impl)


def _ops():
    """The library calls: the custom ops while torch.compile traces, the same functions called directly in eager
    mode (no custom-op dispatch on the host path); reference torch_ffi.py:583-592."""
    import torch
    if not torch.compiler.is_compiling():
        return _IMPL
    return _custom_ops()


def _custom_ops():
    """nablaengine::forward, ::backward, ::kinematics, ::kinematics_backward (torch.library custom ops, no mutated
    arguments, fresh outputs) with fake implementations giving the outputs' shapes; defined once per process
    (reference torch_ffi.py:595-649)."""
    if _OPS:
        return _OPS
    import torch
    from typing import List, Optional
    from torch import Tensor

    @torch.library.custom_op("nablaengine::forward", mutates_args=())
    def forward_op(qpos: Tensor, qvel: Tensor, warm: Tensor, ctrl: Tensor, friction: Tensor, com: Tensor,
                   iterations: int, substeps: int, tape: bool, kinematics: bool) -> List[Tensor]:
        return _forward_impl(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics)

    @forward_op.register_fake
    def _(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics):
        B = qpos.shape[0]
        out = [qpos.new_empty((B, NQ)), qpos.new_empty((B, NV)), qpos.new_empty((B, NV)),
               qpos.new_empty((B, 4), dtype=torch.int32), qpos.new_empty((B if tape else 0, substeps * rec_words()))]
        return out + ([qpos.new_empty(sh) for sh in _kin_shapes(B)] if kinematics else [])

    @torch.library.custom_op("nablaengine::backward", mutates_args=())
    def backward_op(tape: Tensor, friction: Tensor, com: Tensor, g_qpos: Tensor, g_qvel: Tensor,
                    ctrl: Optional[Tensor], kin_state: List[Tensor], kin_cot: List[Tensor], substeps: int,
                    clamp_kv: int, normal: int, clamp_soft: float) -> List[Tensor]:
        return _backward_op_impl(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv,
                                 normal, clamp_soft)

    @backward_op.register_fake
    def _(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv, normal, clamp_soft):
        B = tape.shape[0]
        return [tape.new_empty((B, NQ)), tape.new_empty((B, NV)), tape.new_empty((B, NU)),
                tape.new_empty((B,), dtype=torch.int32)]

    @torch.library.custom_op("nablaengine::kinematics", mutates_args=())
    def kinematics_op(qpos: Tensor, qvel: Tensor, com: Tensor) -> List[Tensor]:
        return _kinematics_impl(qpos, qvel, com)

    @kinematics_op.register_fake
    def _(qpos, qvel, com):
        return [qpos.new_empty(sh) for sh in _kin_shapes(qpos.shape[0])]

    @torch.library.custom_op("nablaengine::kinematics_backward", mutates_args=())
    def kinematics_backward_op(qpos: Tensor, qvel: Tensor, com: Tensor, g_qpos_n: Tensor, g_xpos: Tensor,
                               g_xquat: Tensor, g_cvel: Tensor, g_subtree_com: Tensor) -> List[Tensor]:
        return _kinematics_backward_impl(qpos, qvel, com, g_qpos_n, g_xpos, g_xquat, g_cvel, g_subtree_com)

    @kinematics_backward_op.register_fake
    def _(qpos, qvel, com, g_qpos_n, g_xpos, g_xquat, g_cvel, g_subtree_com):
        B = qpos.shape[0]
        return [qpos.new_empty((B, NQ)), qpos.new_empty((B, NV))]

    _OPS.update(forward=forward_op, backward=backward_op, kinematics=kinematics_op,
                kinematics_backward=kinematics_backward_op)
    return _OPS


def _make_step_fn():
    import torch

    class _Step(torch.autograd.Function):
        """reference torch_ffi.py:747-779: the tape as the residual; gradients for qpos, qvel and ctrl only; with
        kinematics the output state's kinematics outputs too, their cotangents pulled back onto (qpos', qvel') first."""

        @staticmethod
        def forward(ctx, qpos, qvel, warm, ctrl, friction, com, iterations, substeps, clamp_kv, normal, clamp_soft,
                    grad_decay, kin):
            r = _ops()["forward"](qpos, qvel, warm, ctrl, friction, com, iterations, substeps, True, kin)
            q1, v1, w1, info, tp = r[:5]
            ctx.save_for_backward(tp, friction, com, ctrl, q1, v1)
            ctx.opts = (substeps, clamp_kv, normal, clamp_soft, grad_decay, kin)
            ctx.mark_non_differentiable(w1)
            return (q1, v1, w1) + tuple(r[5:])

        @staticmethod
        def backward(ctx, g_q1, g_v1, g_w1, *g_kin):
            tp, friction, com, ctrl, q1, v1 = ctx.saved_tensors
            substeps, clamp_kv, normal, clamp_soft, grad_decay, kin = ctx.opts
            g_q1 = torch.zeros_like(q1) if g_q1 is None else g_q1.contiguous()
            g_v1 = torch.zeros_like(v1) if g_v1 is None else g_v1.contiguous()
            ks, kc = [], []
            if kin and any(g is not None for g in g_kin):
                ks = [q1, v1]
                kc = [torch.zeros(sh, dtype=torch.float32, device=q1.device) if g is None else g.contiguous()
                      for g, sh in zip(g_kin, _kin_shapes(q1.shape[0]))]
            gq, gv, gu, _ = _ops()["backward"](tp, friction, com, g_q1, g_v1, ctrl if clamp_kv == 2 else None, ks, kc,
                                               substeps, clamp_kv, normal, 0.0 if clamp_soft is None else clamp_soft)
            if grad_decay != 1.0:  # the state cotangent through this step times it, ctrl's not (float32 product)
                gq, gv = gq * grad_decay, gv * grad_decay
            return gq, gv, None, gu, None, None, None, None, None, None, None, None, None

    return _Step


def _make_kin_fn():
    import torch

    class _Kin(torch.autograd.Function):
        """reference torch_ffi.py:787-804: gradients for qpos and qvel, none for com."""

        @staticmethod
        def forward(ctx, qpos, qvel, com):
            out = _ops()["kinematics"](qpos, qvel, com)
            ctx.save_for_backward(qpos, qvel, com)
            return tuple(out)

        @staticmethod
        def backward(ctx, *g):
            qpos, qvel, com = ctx.saved_tensors
            g = [torch.zeros(sh, dtype=torch.float32, device=qpos.device) if x is None else x.contiguous()
                 for x, sh in zip(g, _kin_shapes(qpos.shape[0]))]
            gq, gv = _ops()["kinematics_backward"](qpos, qvel, com, *g)
            return gq, gv, None

    return _Kin


_FNS = {}


def _fn(name, make):
    if name not in _FNS:
        _FNS[name] = make()
    return _FNS[name]


def step(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, clamp_kv=CLAMP_KV,
         normal=NORMAL, clamp_soft=None, grad_decay=GRAD_DECAY, kinematics=False):
    """One control step: (qpos', qvel', warm'); kinematics=True: (qpos', qvel', warm', qpos_n, xpos, xquat, cvel,
    subtree_com), the output state's kinematics (reference torch_ffi.py:817-835). Differentiable in qpos, qvel and ctrl
    when any input requires grad (the forward then also writes the tape); warm' is not differentiable."""
    import torch
    if int(clamp_kv) not in (0, 1, 2) or int(normal) not in (0, 1, 2, 3):
        raise _err("clamp_kv in {0, 1, 2}, normal in 0..3", ValueError)
    soft = _soft(clamp_kv, clamp_soft)
    gd = float(grad_decay)
    if not math.isfinite(gd):
        raise _err(f"grad_decay must be finite, got {grad_decay}", ValueError)
    args = (qpos, qvel, warm, ctrl, friction, com)
    if torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in args):
        return _fn("step", _make_step_fn).apply(*args, int(iterations), int(substeps), int(clamp_kv), int(normal),
                                                soft, gd, bool(kinematics))
    r = _ops()["forward"](*args, int(iterations), int(substeps), False, bool(kinematics))
    return tuple(r[:3]) + tuple(r[5:])


def kinematics(qpos, qvel, com):
    """Differentiable kinematics outputs of states (qpos, qvel, com): (qpos_n, xpos, xquat, cvel, subtree_com)
    (reference torch_ffi.py:838-842); gradients for qpos and qvel, none for com. kinematics(q', v', com) of a step's
    output is bitwise step(..., kinematics=True)'s."""
    import torch
    if torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in (qpos, qvel, com)):
        return _fn("kin", _make_kin_fn).apply(qpos, qvel, com)
    return tuple(_ops()["kinematics"](qpos, qvel, com))


def forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, tape=False,
            kinematics=False):
    """One control step without autograd: (qpos', qvel', warm', info (B, 4) int32[, tape][, the kinematics outputs])
    (reference torch_ffi.py:845-851)."""
    r = _ops()["forward"](qpos, qvel, warm, ctrl, friction, com, int(iterations), int(substeps), bool(tape),
                          bool(kinematics))
    return tuple(r[:4]) + ((r[4],) if tape else ()) + tuple(r[5:])


def backward(tape, friction, com, g_qpos, g_qvel, *, substeps=SUBSTEPS, clamp_kv=CLAMP_KV, normal=NORMAL, ctrl=None,
             clamp_soft=None, kinematics=None):
    """The adjoint of one control step from its tape: (g_qpos (B, 36), g_qvel (B, 35), g_ctrl (B, 29), info (B,))
    (reference torch_ffi.py:854-865); kinematics: None or (qpos', qvel', g_qpos_n, g_xpos, g_xquat, g_cvel,
    g_subtree_com), the cotangents of the output state's kinematics outputs, pulled back and added first."""
    soft = _soft(clamp_kv, clamp_soft)
    if soft is not None and ctrl is None:
        raise _err("clamp_kv=2 (the soft clamp) needs the step's ctrl", ValueError)
    ks, kc = ([], []) if kinematics is None else (list(kinematics[:2]), list(kinematics[2:]))
    if kinematics is not None and len(kc) != 5:
        raise _err("kinematics = (qpos', qvel', g_qpos_n, g_xpos, g_xquat, g_cvel, g_subtree_com)", ValueError)
    return tuple(_ops()["backward"](tape, friction, com, g_qpos, g_qvel, ctrl if soft is not None else None, ks, kc,
                                    int(substeps), int(clamp_kv), int(normal), 0.0 if soft is None else soft))


def set_diagnostics(enabled):
    """Switch the device counters and the backward's non-finite bits on (the default) or off; returns the previous
    setting (reference torch_ffi.py:678-686). When on, the forward and adjoint kernels add each world's counts at its
    end (dk_fwd_forward_diag / dk_adjoint_work_diag); outputs and gradients are the same either way."""
    prev = _DIAG_ON[0]
    _DIAG_ON[0] = bool(enabled)
    return prev


def _device_index(device):
    import torch
    if device is None:
        return torch.cuda.current_device()
    d = torch.device(device)
    return torch.cuda.current_device() if d.index is None else d.index


def diagnostics(device=None):
    """The device's counters: an int64 (len(DIAG),) GPU tensor in DIAG order, added up by every call since init or the
    last reset; not copied or synchronized (reference torch_ffi.py:689-695)."""
    dev = _device_index(device)
    if dev not in _READY:
        init(dev)
    return _DIAG[dev]


def read_diagnostics(device=None, reset=True):
    """The device's counters as {name: int} (synchronizes); reset=True zeroes them afterwards; with
    set_overflow_warnings(True) it warns when worlds exceeded the contact or row capacity (reference
    torch_ffi.py:698-708)."""
    d = diagnostics(device)
    out = dict(zip(DIAG, (int(x) for x in d.cpu())))
    if reset:
        d.zero_()
    if _OVERFLOW_WARN[0]:
        warn_overflow(out)
    return out


def warn_overflow(d, where="nablaengine_amd"):
    """A RuntimeWarning when the counters d count worlds whose contacts (64) or constraint rows (192) exceeded the
    per-world capacity: the extra ones were dropped, so those worlds miss support and friction forces; returns the
    count (reference torch_ffi.py:711-724)."""
    import warnings
    nc, nr = d.get("fwd_contact_overflow_worlds", 0), d.get("fwd_row_overflow_worlds", 0)
    if nc or nr:
        warnings.warn(f"{where}: {nc} world-steps exceeded the contact capacity ({MAXCON} per world) and {nr} the "
                      f"constraint-row capacity (192); their extra contacts / rows were dropped, so those worlds miss "
                      f"support and friction forces (e.g. deep interpenetration)", RuntimeWarning, stacklevel=3)
    return nc + nr


def set_overflow_warnings(enabled):
    """Switch the capacity-overflow warnings on or off (default off, or $DK_OVERFLOW_WARN=1); when on, the counts
    nobody read are reported once more at exit. Returns the previous setting (reference torch_ffi.py:727-735)."""
    prev = _OVERFLOW_WARN[0]
    _OVERFLOW_WARN[0] = bool(enabled)
    return prev


def _exit_report():
    """At exit: the overflow warning for each device's counts since the last read (no reset); never raises."""
    try:
        if not (_DIAG_ON[0] and _OVERFLOW_WARN[0]):
            return
        for dev in sorted(_DIAG):
            warn_overflow(dict(zip(DIAG, (int(x) for x in _DIAG[dev].cpu()))), where=f"nablaengine_amd (cuda:{dev})")
    except Exception:  # noqa: BLE001  (interpreter or the runtime shutting down)
        pass


atexit.register(_exit_report)


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
