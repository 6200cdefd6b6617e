"""PyTorch surface of the MI355X G1 engine: a drop-in for the reference's ``nablaengine.torch_ffi``
(``src/nablaengine/torch_ffi.py``; the entry points, their arguments, defaults and error classes are that module's).

  step(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, clamp_kv=0, normal=3, clamp_soft=None,
       grad_decay=1.0, kinematics=False) -> (qpos', qvel', warm'[, qpos_n, xpos, xquat, cvel, subtree_com])
  kinematics(qpos, qvel, com) -> (qpos_n, xpos, xquat, cvel, subtree_com)
  forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=10, substeps=4, tape=False, kinematics=False)
       -> (qpos', qvel', warm', info[, tape][, the kinematics outputs])
  backward(tape, friction, com, g_qpos, g_qvel, *, substeps=4, clamp_kv=0, normal=3, ctrl=None, clamp_soft=None,
           kinematics=None) -> (g_qpos, g_qvel, g_ctrl, info)
  scale_grad(tree, gamma)

Per-world arrays are float32, contiguous, on one ROCm device, with the worlds B as the leading dimension: qpos (B, 36),
qvel (B, 35), warm (B, 35), ctrl (B, 29), friction (B,), com (B, 3). Anything else is a TypeError: no array is cast,
copied or moved to another device. Bad options are a ValueError, a failed library call a RuntimeError. B = 0 gives
empty outputs and launches nothing.

The kinematics outputs of a state (the reference's g1_engine/kinematics.py:1-45): qpos_n (B, 36), the root
quaternion normalized; xpos (B, 31, 3) and xquat (B, 31, 4), the body frames; cvel (B, 31, 6), [angular; linear]
twists at subtree_com[:, 1]; subtree_com (B, 31, 3). step(..., kinematics=True) returns those of its output state,
bitwise kinematics(qpos', qvel', com), and its backward pulls their cotangents back onto (qpos', qvel') first.

How a call reaches the GPU. The library, libnablaengine_g1.so next to this file (``python -m nablaengine_amd.build``),
is loaded once per process with ctypes; its C entries (include/nablaengine_g1.h) get the tensors' device pointers and
torch's current stream of the inputs' device, made current for the call. Each library call is an operator of the
``nablaengine`` namespace (forward, backward, kinematics, kinematics_backward), defined by schema with the dispatcher
and given a fake (shape-only) implementation, so that torch.compile records it as one opaque node; eager calls go
through the same operators. There is no fallback: without the library or without a GPU every call raises. After
init() a call only launches kernels and takes memory from torch's caching allocator, so it may be captured in a HIP
graph.

Autograd: step is differentiable in qpos, qvel and ctrl when one of the six inputs requires grad; the forward then
also writes the tape (B, substeps x 1472 float32) and keeps it for the backward, the analytic adjoint. warm' is not
differentiable; warm, friction and com get no gradient. grad_decay scales the state's cotangent through the step (a
float32 product), not ctrl's.

Diagnostics: per device an int64 tensor of the 18 counters of DIAG, added to by the forward and adjoint kernels
themselves as each world ends (set_diagnostics(False) stops it); diagnostics() returns the tensor, read_diagnostics()
a dict (synchronizing; by default it zeroes them). With counting on, the backward's info also carries the non-finite
bits (NONFINITE_* << NONFINITE_SHIFT).
"""
import atexit
import ctypes
import math
import os
import threading
import warnings
from typing import NamedTuple, Optional

import torch
from torch import Tensor

# ---- the interface's constants (names and values the reference's, torch_ffi.py:54-61) -------------------------------
ITERATIONS, SUBSTEPS, CLAMP_KV, NORMAL = 10, 4, 0, 3
CLAMP_SOFT, GRAD_DECAY = 0.2, 1.0
NQ, NV, NU, NBODY = 36, 35, 29, 31
MAXCON, MAXROWS = 64, 192
OVERFLOW_CONTACTS, OVERFLOW_ROWS = 4, 16  # forward info[:, 3]: contacts / rows beyond capacity were dropped
DIAG = ("fwd_calls", "fwd_worlds", "fwd_unsupported_worlds", "fwd_iteration_limit_worlds", "tape_records",
        "refact_records", "nonconv_records", "singular_records", "bwd_calls", "bwd_rows", "nonfinite_rows",
        "nonfinite_qpos_rows", "nonfinite_qvel_rows", "nonfinite_ctrl_rows", "nonfinite_cotangent_rows",
        "replay_mismatch_worlds", "fwd_contact_overflow_worlds", "fwd_row_overflow_worlds")
NONFINITE_QPOS, NONFINITE_QVEL, NONFINITE_CTRL, NONFINITE_COT, NONFINITE_SHIFT = 1, 2, 4, 8, 16
ADJ_REPLAY_MISMATCH = 1 << 13  # backward info: a replayed contact was not found among the recomputed ones
TAPE_REFACT, TAPE_NONCONV, TAPE_SINGULAR = 1 << 8, 1 << 9, 1 << 10  # a tape record's flags (also in backward info)
VARIANTS = tuple((kv, n) for kv in (0, 1, 2) for n in (0, 1, 2, 3))  # the adjoint's (clamp_kv, normal) options

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnablaengine_g1.so")
ARCH = "gfx950"  # the library's one target

# the per-world part of each array's shape
_KIN_OUT = (("qpos_n", (NQ,)), ("xpos", (NBODY, 3)), ("xquat", (NBODY, 4)), ("cvel", (NBODY, 6)),
            ("subtree_com", (NBODY, 3)))
_STATE_IN = (("qpos", (NQ,)), ("qvel", (NV,)), ("warm", (NV,)), ("ctrl", (NU,)), ("friction", ()), ("com", (3,)))


def _err(msg, kind=TypeError):
    return kind(f"nablaengine_amd.torch_ffi: {msg}")


# ---- the native library ---------------------------------------------------------------------------------------------
# C prototypes, "result:arguments", one letter a value: p pointer (device array, stream or NULL), i int, f float,
# q long long, - void.
_PROTOTYPES = {
    "dk_fwd_forward": "i:pi" + "p" * 6 + "ii" + "p" * 7,
    "dk_fwd_forward_diag": "i:pi" + "p" * 6 + "ii" + "p" * 8,
    "dk_fwd_forward_ordered": "i:pi" + "p" * 6 + "ii" + "p" * 7,
    "dk_fwd_forward_static": "i:pi" + "p" * 6 + "ii" + "p" * 6,
    "dk_fwd_order": "i:pipp",
    "dk_fwd_work_bytes": "q:i",
    "dk_fwd_upload": "i:pp",
    "dk_fwd_sizes": "-:p",
    "dk_fwd_launch": "i:ip",
    "dk_fwd_kinematics": "i:pi" + "p" * 8,
    "dk_fwd_kinematics_vjp": "i:pi" + "p" * 12,
    "dk_adjoint": "i:pii" + "p" * 10 + "fii",
    "dk_adjoint_work": "i:pii" + "p" * 10 + "fiip",
    "dk_adjoint_work_diag": "i:pii" + "p" * 10 + "fiipp",
    "dk_adjoint_order": "i:piipp",
    "dk_adjoint_work_ordered": "i:pii" + "p" * 10 + "fiipp",
    "dk_adjoint_many": "i:piii" + "p" * 10 + "fiipp",
    "dk_adjoint_work_bytes": "q:i",
    "dk_torch_diag_fwd": "i:ppiiipp",
    "dk_torch_diag_bwd": "i:ppi" + "p" * 6,
    "dk_prof_read": "i:pi",
    "dk_prof_read_adj": "i:pi",
}
_CTYPE = {"p": ctypes.c_void_p, "i": ctypes.c_int, "f": ctypes.c_float, "q": ctypes.c_longlong, "-": None}


class _Native:
    """The loaded library: its path, the ctypes handle with every entry's prototype set, and the sizes it reports
    (dk_fwd_sizes: LDS bytes of the forward and the adjoint, tape words per world and substep, nq, nv, contacts)."""

    def __init__(self, path):
        self.path = path
        self.dll = ctypes.CDLL(path)
        for name, proto in _PROTOTYPES.items():
            result, args = proto.split(":")
            entry = getattr(self.dll, name)
            entry.restype = _CTYPE[result]
            entry.argtypes = [_CTYPE[c] for c in args]
        sizes = (ctypes.c_longlong * 9)()
        self.dll.dk_fwd_sizes(ctypes.cast(sizes, ctypes.c_void_p))
        self.sizes = tuple(int(s) for s in sizes)
        self.rec_words = self.sizes[2]

    def run(self, what, entry, *args):
        """Call a C entry; a nonzero return is a RuntimeError naming `what`."""
        rc = getattr(self.dll, entry)(*args)
        if rc:
            raise _err(f"{what} failed (HIP error {rc})", RuntimeError)


_lock = threading.RLock()
_native: Optional[_Native] = None
_counters = {}  # device index -> int64 (len(DIAG),) tensor; a device is ready once it has one
_settings = {"count": True, "warn": os.environ.get("DK_OVERFLOW_WARN", "0") not in ("", "0")}


def library_path(artifact=None):
    """The library a call of init / load_library loads: artifact (a .so, or a .json file whose "library" names it
    relative to the .json, as the reference's artifacts, torch_ffi.py:241-266), else $DK_TORCH_ARTIFACT, else
    $NABLA_G1_LIB, else the in-tree build."""
    path = os.fspath(artifact or os.environ.get("DK_TORCH_ARTIFACT") or os.environ.get("NABLA_G1_LIB") or LIB_PATH)
    if not path.endswith(".json"):
        return path
    import json
    with open(path) as f:
        lib = json.load(f).get("library")
    if lib is None:
        raise _err(f"artifact {path} names no library", RuntimeError)
    return os.path.join(os.path.dirname(os.path.abspath(path)), lib)


def _load(artifact=None):
    global _native
    with _lock:
        if _native is None:
            path = library_path(artifact)
            if not os.path.exists(path):
                raise _err(f"{path} is missing: build it with `python -m nablaengine_amd.build`", RuntimeError)
            _native = _Native(path)
        elif artifact is not None and os.path.realpath(library_path(artifact)) != os.path.realpath(_native.path):
            raise _err(f"{_native.path} is loaded already: one library per process", RuntimeError)
        return _native


def load_library(path=None):
    """The ctypes handle of the library, every C entry's prototype set (path: as init's artifact). RuntimeError when
    the file is missing or another library is loaded already (one library per process)."""
    return _load(path).dll


def rec_words():
    """Tape words per world and substep."""
    return _load().rec_words


def tape_bytes(nworld, substeps=SUBSTEPS, steps=1):
    """Bytes of the tapes that `steps` differentiated control steps of `nworld` worlds keep."""
    return 4 * rec_words() * substeps * nworld * steps


def init(device=None, artifact=None, model_dir=None, model=None, foot_pairs=None):
    """Load the library (artifact as library_path's) and make `device` (default: torch's current one) ready to run
    it; repeated calls are no-ops (the reference's init, torch_ffi.py:268-290). The G1 model is compiled into the
    library, so nothing is uploaded and nothing synchronizes: naming another model (model_dir, model, foot_pairs) is a
    ValueError. Returns the library's path, architecture and sizes."""
    if (model_dir, model, foot_pairs) != (None, None, None):
        raise _err("this library is built for the G1 model: model_dir / model / foot_pairs cannot change it",
                   ValueError)
    nat = _load(artifact)
    dev = _device_index(device)
    with _lock:
        if dev not in _counters:
            if not torch.cuda.is_available():
                raise _err("no ROCm GPU is visible, and the engine has no CPU path", RuntimeError)
            arch = getattr(torch.cuda.get_device_properties(dev), "gcnArchName", ARCH).split(":")[0]
            if arch != ARCH:
                raise _err(f"cuda:{dev} is {arch}; the library holds {ARCH} code only", RuntimeError)
            with torch.cuda.device(dev):
                nat.run(f"making cuda:{dev} ready", "dk_fwd_upload", None, _stream(dev))
            _counters[dev] = torch.zeros(len(DIAG), dtype=torch.int64, device=f"cuda:{dev}")
        _register_ops()  # outside any torch.compile trace: defining operators inside one is not traceable
    return dict(path=nat.path, arch=ARCH, sizes=list(nat.sizes))


def _device_index(device):
    if device is None:
        return torch.cuda.current_device()
    d = torch.device(device)
    return torch.cuda.current_device() if d.index is None else d.index


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ready(dev):
    if dev not in _counters:
        init(dev)
    return _native


# ---- argument checks ------------------------------------------------------------------------------------------------

class _Worlds:
    """The worlds of one call: the device and the count B come from its first per-world array (B its leading size
    when its rank is 1 + len(per_world), else -1, which no array then matches); every array must be a contiguous
    tensor of the given dtype on that device, shaped (*lead, B, *per_world)."""

    def __init__(self, name, x, per_world):
        if not isinstance(x, Tensor) or x.device.type != "cuda":
            where = x.device if isinstance(x, Tensor) else type(x).__name__
            raise _err(f"{name} must be a torch.Tensor on a ROCm device, got {where}")
        self.device = x.device
        self.dev = x.device.index
        self.B = x.shape[0] if x.dim() == 1 + len(per_world) else -1

    def ptr(self, name, x, per_world, dtype=torch.float32, lead=()):
        """x's device pointer, after the checks (a TypeError naming x when one fails)."""
        want = (*lead, self.B, *per_world)
        if (isinstance(x, Tensor) and x.dtype == dtype and tuple(x.shape) == want and x.device == self.device
                and x.is_contiguous()):
            return ctypes.c_void_p(x.data_ptr())
        got = (f"{x.dtype} {tuple(x.shape)} on {x.device}{'' if x.is_contiguous() else ', not contiguous'}"
               if isinstance(x, Tensor) else type(x).__name__)
        raise _err(f"{name}: expected a contiguous {dtype} tensor {want} on {self.device}, got {got}")

    def empty(self, *per_world, dtype=torch.float32, lead=()):
        return torch.empty((*lead, self.B, *per_world), dtype=dtype, device=self.device)


def _soft_delta(clamp_kv, clamp_soft):
    """The soft clamp's delta: for clamp_kv 2, clamp_soft or CLAMP_SOFT when it is None (finite, >= 0); for 0 and 1
    None, and clamp_soft must be None too."""
    if int(clamp_kv) == 2:
        delta = CLAMP_SOFT if clamp_soft is None else float(clamp_soft)
        if math.isfinite(delta) and delta >= 0.0:
            return delta
        raise _err(f"clamp_soft must be finite and >= 0, got {clamp_soft}", ValueError)
    if clamp_soft is not None:
        raise _err(f"clamp_soft belongs to the soft clamp (clamp_kv=2), not to clamp_kv={clamp_kv}", ValueError)
    return None


def _variant(clamp_kv, normal):
    v = (int(clamp_kv), int(normal))
    if v not in VARIANTS:
        raise _err(f"clamp_kv must be 0, 1 or 2 and normal 0..3, got clamp_kv={clamp_kv} normal={normal}", ValueError)
    return v


# ---- the library calls ----------------------------------------------------------------------------------------------

def _forward_call(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics):
    """One control step: [qpos', qvel', warm', info, tape (B or 0 rows)] + the output state's kinematics outputs."""
    w = _Worlds("qpos", qpos, (NQ,))
    ins = [w.ptr(name, x, shape) for (name, shape), x in zip(_STATE_IN, (qpos, qvel, warm, ctrl, friction, com))]
    if not 1 <= substeps <= 32 or iterations < 0:
        raise _err(f"substeps must be in 1..32 and iterations >= 0, got {substeps} and {iterations}", ValueError)
    nat = _ready(w.dev)
    q1, v1, w1, info = w.empty(NQ), w.empty(NV), w.empty(NV), w.empty(4, dtype=torch.int32)
    tp = torch.empty((w.B if tape else 0, substeps * nat.rec_words), dtype=torch.float32, device=w.device)
    kin = [w.empty(*shape) for _, shape in _KIN_OUT] if kinematics else []
    out = [q1, v1, w1, info, tp] + kin
    if w.B == 0:
        return out
    work = torch.empty((int(nat.dll.dk_fwd_work_bytes(w.B)),), dtype=torch.uint8, device=w.device)
    P = ctypes.c_void_p
    with torch.cuda.device(w.dev):
        st = _stream(w.dev)
        args = [st, w.B, *ins, int(iterations), int(substeps), P(q1.data_ptr()), P(v1.data_ptr()), P(w1.data_ptr()),
                P(info.data_ptr()), None, P(tp.data_ptr()) if tape else None, P(work.data_ptr()) if work.numel() else None]
        if _settings["count"]:  # the kernel adds each world's counts at its end (dk_torch_diag_fwd's counts)
            nat.run("the forward launch", "dk_fwd_forward_diag", *args, P(_counters[w.dev].data_ptr()))
        else:
            nat.run("the forward launch", "dk_fwd_forward", *args)
        if kinematics:
            nat.run("the kinematics launch", "dk_fwd_kinematics", st, w.B, P(q1.data_ptr()), P(v1.data_ptr()),
                    ins[5], *(P(t.data_ptr()) for t in kin))
    return out


def _backward_call(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv, normal,
                   clamp_soft):
    """The adjoint from a tape: [g_qpos (B, 36), g_qvel (B, 35), g_ctrl (B, 29), info (B,)]. kin_state = [qpos',
    qvel'] with kin_cot the five kinematics outputs' cotangents, or both empty. clamp_soft: the delta (read for
    clamp_kv 2 only)."""
    kv, nrm = _variant(clamp_kv, normal)
    if (kv == 2) != (ctrl is not None):
        raise _err("the step's ctrl goes with clamp_kv=2 (the soft clamp) and only with it", ValueError)
    w = _Worlds("tape", tape, (None,))
    nat = _ready(w.dev)
    ptape = w.ptr("tape", tape, (substeps * nat.rec_words,))
    pf, pc = w.ptr("friction", friction, ()), w.ptr("com", com, (3,))
    pgq, pgv = w.ptr("g_qpos", g_qpos, (NQ,)), w.ptr("g_qvel", g_qvel, (NV,))
    pu = w.ptr("ctrl", ctrl, (NU,)) if ctrl is not None else None
    if kin_state or kin_cot:
        if len(kin_state) != 2 or len(kin_cot) != len(_KIN_OUT):
            raise _err("kin_state = [qpos', qvel'] and kin_cot = the five kinematics outputs' cotangents", ValueError)
        pks = [w.ptr(n, x, s) for n, x, s in zip(("qpos'", "qvel'"), kin_state, ((NQ,), (NV,)))]
        pkc = [w.ptr("g_" + n, x, s) for (n, s), x in zip(_KIN_OUT, kin_cot)]
    gq, gv, gu, info = w.empty(NQ), w.empty(NV), w.empty(NU), w.empty(dtype=torch.int32)
    if w.B == 0:
        return [gq, gv, gu, info]
    work = torch.empty((int(nat.dll.dk_adjoint_work_bytes(w.B)),), dtype=torch.uint8, device=w.device)
    P = ctypes.c_void_p
    with torch.cuda.device(w.dev):
        st = _stream(w.dev)
        if kin_state:  # the kinematics cotangents pulled back onto (qpos', qvel'); the step's own added last
            cq, cv = w.empty(NQ), w.empty(NV)
            nat.run("the kinematics VJP launch", "dk_fwd_kinematics_vjp", st, w.B, *pks, pc, *pkc, pgq, pgv,
                    P(cq.data_ptr()), P(cv.data_ptr()))
            pgq, pgv = P(cq.data_ptr()), P(cv.data_ptr())
        args = [st, w.B, int(substeps), ptape, pf, pc, pgq, pgv, P(gq.data_ptr()), P(gv.data_ptr()), P(gu.data_ptr()),
                P(info.data_ptr()), pu, ctypes.c_float(clamp_soft), kv, nrm, P(work.data_ptr()) if work.numel() else None]
        if _settings["count"]:  # counts and the non-finite bits of info, by the adjoint kernel itself
            nat.run("the adjoint launch", "dk_adjoint_work_diag", *args, P(_counters[w.dev].data_ptr()))
        else:
            nat.run("the adjoint launch", "dk_adjoint_work", *args)
    return [gq, gv, gu, info]


def _kinematics_call(qpos, qvel, com):
    w = _Worlds("qpos", qpos, (NQ,))
    ins = [w.ptr("qpos", qpos, (NQ,)), w.ptr("qvel", qvel, (NV,)), w.ptr("com", com, (3,))]
    nat = _ready(w.dev)
    out = [w.empty(*shape) for _, shape in _KIN_OUT]
    if w.B:
        with torch.cuda.device(w.dev):
            nat.run("the kinematics launch", "dk_fwd_kinematics", _stream(w.dev), w.B, *ins,
                    *(ctypes.c_void_p(t.data_ptr()) for t in out))
    return out


def _kinematics_backward_call(qpos, qvel, com, *cot):
    w = _Worlds("qpos", qpos, (NQ,))
    ins = [w.ptr("qpos", qpos, (NQ,)), w.ptr("qvel", qvel, (NV,)), w.ptr("com", com, (3,))]
    ins += [w.ptr("g_" + n, x, s) for (n, s), x in zip(_KIN_OUT, cot)]
    nat = _ready(w.dev)
    gq, gv = w.empty(NQ), w.empty(NV)
    if w.B:
        with torch.cuda.device(w.dev):
            nat.run("the kinematics VJP launch", "dk_fwd_kinematics_vjp", _stream(w.dev), w.B, *ins, None, None,
                    ctypes.c_void_p(gq.data_ptr()), ctypes.c_void_p(gv.data_ptr()))
    return [gq, gv]


def _vjp_sets(tape, friction, com, g_qpos, g_qvel, ctrl=None, *, substeps=SUBSTEPS, clamp_kv=CLAMP_KV,
              normal=NORMAL, clamp_soft=None):
    """K VJPs of one taped step in one adjoint launch (dk_adjoint_many): output cotangents g_qpos (K, B, 36), g_qvel
    (K, B, 35) -> (g_qpos (K, B, 36), g_qvel (K, B, 35), g_ctrl (K, B, 29), info (K, B)). Set k is bitwise
    backward(tape, friction, com, g_qpos[k], g_qvel[k], ...) with the same options (clamp_soft None meaning
    CLAMP_SOFT for clamp_kv 2, as there), and the counters count K backward calls. The step Jacobian's driver."""
    kv, nrm = _variant(clamp_kv, normal)
    delta = _soft_delta(kv, clamp_soft)
    if (kv == 2) != (ctrl is not None):
        raise _err("the step's ctrl goes with clamp_kv=2 (the soft clamp) and only with it", ValueError)
    if not (isinstance(g_qpos, Tensor) and g_qpos.dim() == 3 and g_qpos.shape[0] >= 1):
        raise _err("g_qpos must be a (K, B, 36) tensor with K >= 1")
    K = g_qpos.shape[0]
    w = _Worlds("tape", tape, (None,))
    nat = _ready(w.dev)
    if K * w.B * 64 >= 2 ** 32:
        raise _err(f"{K} cotangent sets of {w.B} worlds exceed one launch's 2^32 work-items", ValueError)
    args = [w.ptr("tape", tape, (substeps * nat.rec_words,)), w.ptr("friction", friction, ()),
            w.ptr("com", com, (3,)), w.ptr("g_qpos", g_qpos, (NQ,), lead=(K,)),
            w.ptr("g_qvel", g_qvel, (NV,), lead=(K,))]
    pu = w.ptr("ctrl", ctrl, (NU,)) if ctrl is not None else None
    outs = [w.empty(n, lead=(K,)) for n in (NQ, NV, NU)] + [w.empty(dtype=torch.int32, lead=(K,))]
    if w.B == 0:
        return tuple(outs)
    work = torch.empty((int(nat.dll.dk_adjoint_work_bytes(w.B)),), dtype=torch.uint8, device=w.device)
    P = ctypes.c_void_p
    with torch.cuda.device(w.dev):
        nat.run("the adjoint launch", "dk_adjoint_many", _stream(w.dev), w.B, K, int(substeps), *args,
                *(P(t.data_ptr()) for t in outs), pu, ctypes.c_float(0.0 if delta is None else delta), kv, nrm,
                P(work.data_ptr()), P(_counters[w.dev].data_ptr()) if _settings["count"] else None)
    return tuple(outs)


# ---- the operators (torch.library) ----------------------------------------------------------------------------------
# Schemas: the reference's custom ops (torch_ffi.py:603-649), so that graphs recorded against either name the same
# operators with the same arguments.
_SCHEMAS = {
    "forward": "forward(Tensor qpos, Tensor qvel, Tensor warm, Tensor ctrl, Tensor friction, Tensor com, "
               "int iterations, int substeps, bool tape, bool kinematics) -> Tensor[]",
    "backward": "backward(Tensor tape, Tensor friction, Tensor com, Tensor g_qpos, Tensor g_qvel, Tensor? ctrl, "
                "Tensor[] kin_state, Tensor[] kin_cot, int substeps, int clamp_kv, int normal, float clamp_soft) "
                "-> Tensor[]",
    "kinematics": "kinematics(Tensor qpos, Tensor qvel, Tensor com) -> Tensor[]",
    "kinematics_backward": "kinematics_backward(Tensor qpos, Tensor qvel, Tensor com, Tensor g_qpos_n, "
                           "Tensor g_xpos, Tensor g_xquat, Tensor g_cvel, Tensor g_subtree_com) -> Tensor[]",
}


def _fake_forward(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics):
    B = qpos.shape[0]
    shapes = [(B, NQ), (B, NV), (B, NV), None, (B if tape else 0, substeps * rec_words())]
    out = [qpos.new_empty(s) if s else qpos.new_empty((B, 4), dtype=torch.int32) for s in shapes]
    return out + ([qpos.new_empty((B, *s)) for _, s in _KIN_OUT] if kinematics else [])


def _fake_backward(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv, normal,
                   clamp_soft):
    B = tape.shape[0]
    return [tape.new_empty((B, n)) for n in (NQ, NV, NU)] + [tape.new_empty((B,), dtype=torch.int32)]


def _fake_kinematics(qpos, qvel, com):
    return [qpos.new_empty((qpos.shape[0], *s)) for _, s in _KIN_OUT]


def _fake_kinematics_backward(qpos, qvel, com, *cot):
    return [qpos.new_empty((qpos.shape[0], NQ)), qpos.new_empty((qpos.shape[0], NV))]


_KERNELS = {"forward": (_forward_call, _fake_forward), "backward": (_backward_call, _fake_backward),
            "kinematics": (_kinematics_call, _fake_kinematics),
            "kinematics_backward": (_kinematics_backward_call, _fake_kinematics_backward)}
_library_defs = []  # the torch.library.Library holding the definitions (kept alive for the process)


def _ops():
    """torch.ops.nablaengine, defined first where it is not yet (no lock taken once it is, so torch.compile traces
    through this)."""
    if not _library_defs:
        _register_ops()
    return torch.ops.nablaengine


def _register_ops():
    """Define the nablaengine operators once per process: the schema, the library call for every backend (a CPU or
    other non-ROCm tensor reaches the checks and raises TypeError) and the fake implementation torch.compile traces
    with. Returns torch.ops.nablaengine."""
    with _lock:
        if not _library_defs:
            lib = torch.library.Library("nablaengine", "DEF")
            for name, schema in _SCHEMAS.items():
                call, fake = _KERNELS[name]
                lib.define(schema)
                lib.impl(name, call, "CompositeExplicitAutograd")
                torch.library.register_fake(f"nablaengine::{name}", fake, lib=lib)
            _library_defs.append(lib)
    return torch.ops.nablaengine


# ---- autograd -------------------------------------------------------------------------------------------------------

class _StepOptions(NamedTuple):
    iterations: int
    substeps: int
    clamp_kv: int
    normal: int
    delta: float  # the soft clamp's delta (clamp_kv 2), else 0
    grad_decay: float
    kinematics: bool


# Set (per thread) while a checkpointed segment's first pass runs (rollout): torch's non-reentrant checkpoint drops
# what that pass saves and recomputes it, tapes included, when the backward reaches the segment.
_tape_unread = threading.local()


class _TapeUnread:
    """The steps inside skip writing their tapes: each saves an unwritten tensor of the tape's shape in its place
    (the checkpoint compares the recomputed saved tensors' shapes with these), which nothing reads."""

    def __enter__(self):
        _tape_unread.depth = getattr(_tape_unread, "depth", 0) + 1

    def __exit__(self, *exc):
        _tape_unread.depth -= 1


class _StepFunction(torch.autograd.Function):
    """step's autograd node: the forward writes the tape and keeps it with the arrays the adjoint reads; the backward
    runs the adjoint (after the kinematics VJP when cotangents reach the kinematics outputs). Inputs (options, qpos,
    qvel, warm, ctrl, friction, com); gradients for qpos, qvel and ctrl only (the reference's _Step,
    torch_ffi.py:747-779)."""

    @staticmethod
    def forward(ctx, opts, qpos, qvel, warm, ctrl, friction, com):
        taped = getattr(_tape_unread, "depth", 0) == 0
        q1, v1, w1, _info, tape, *kin = _ops().forward(qpos, qvel, warm, ctrl, friction, com, opts.iterations,
                                                    opts.substeps, taped, opts.kinematics)
        if not taped:
            tape = torch.empty((qpos.shape[0], opts.substeps * rec_words()), dtype=torch.float32, device=qpos.device)
        ctx.opts = opts
        ctx.save_for_backward(tape, friction, com, ctrl, q1, v1)
        ctx.mark_non_differentiable(w1)
        ctx.set_materialize_grads(False)
        return (q1, v1, w1, *kin)

    @staticmethod
    def backward(ctx, g_q1, g_v1, _g_w1, *g_kin):
        tape, friction, com, ctrl, q1, v1 = ctx.saved_tensors
        o = ctx.opts
        zero_or = lambda g, ref: torch.zeros_like(ref) if g is None else g.contiguous()  # noqa: E731
        kin_state, kin_cot = [], []
        if o.kinematics and any(g is not None for g in g_kin):
            kin_state = [q1, v1]
            kin_cot = [torch.zeros((q1.shape[0], *s), dtype=torch.float32, device=q1.device) if g is None
                       else g.contiguous() for g, (_, s) in zip(g_kin, _KIN_OUT)]
        gq, gv, gu, _ = _ops().backward(tape, friction, com, zero_or(g_q1, q1), zero_or(g_v1, v1),
                                                 ctrl if o.clamp_kv == 2 else None, kin_state, kin_cot, o.substeps,
                                                 o.clamp_kv, o.normal, o.delta)
        if o.grad_decay != 1.0:
            gq, gv = gq * o.grad_decay, gv * o.grad_decay
        return None, gq, gv, None, gu, None, None


class _KinematicsFunction(torch.autograd.Function):
    """kinematics' autograd node: gradients for qpos and qvel, none for com (the reference's _Kin,
    torch_ffi.py:785-804)."""

    @staticmethod
    def forward(ctx, qpos, qvel, com):
        ctx.save_for_backward(qpos, qvel, com)
        ctx.set_materialize_grads(False)
        return tuple(_ops().kinematics(qpos, qvel, com))

    @staticmethod
    def backward(ctx, *g):
        qpos, qvel, com = ctx.saved_tensors
        cot = [torch.zeros((qpos.shape[0], *s), dtype=torch.float32, device=qpos.device) if x is None
               else x.contiguous() for x, (_, s) in zip(g, _KIN_OUT)]
        gq, gv = _ops().kinematics_backward(qpos, qvel, com, *cot)
        return gq, gv, None


def _wants_grad(*xs):
    return torch.is_grad_enabled() and any(isinstance(x, Tensor) and x.requires_grad for x in xs)


# ---- the public calls -----------------------------------------------------------------------------------------------

def step(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, clamp_kv=CLAMP_KV,
         normal=NORMAL, clamp_soft=None, grad_decay=GRAD_DECAY, kinematics=False):
    """One control step -> (qpos', qvel', warm'), with kinematics=True followed by the output state's (qpos_n, xpos,
    xquat, cvel, subtree_com) (the reference's step, torch_ffi.py:817-835). clamp_kv, normal, clamp_soft and
    grad_decay shape the gradient only."""
    kv, nrm = _variant(clamp_kv, normal)
    delta = _soft_delta(kv, clamp_soft)
    decay = float(grad_decay)
    if not math.isfinite(decay):
        raise _err(f"grad_decay must be finite, got {grad_decay}", ValueError)
    ins = (qpos, qvel, warm, ctrl, friction, com)
    if _wants_grad(*ins):
        opts = _StepOptions(int(iterations), int(substeps), kv, nrm, 0.0 if delta is None else delta, decay,
                            bool(kinematics))
        return _StepFunction.apply(opts, *ins)
    q1, v1, w1, _info, _tape, *kin = _ops().forward(*ins, int(iterations), int(substeps), False,
                                                             bool(kinematics))
    return (q1, v1, w1, *kin)


def kinematics(qpos, qvel, com):
    """The kinematics outputs (qpos_n, xpos, xquat, cvel, subtree_com) of the states (qpos, qvel, com), differentiable
    in qpos and qvel (the reference's kinematics, torch_ffi.py:838-842)."""
    if _wants_grad(qpos, qvel, com):
        return _KinematicsFunction.apply(qpos, qvel, com)
    return tuple(_ops().kinematics(qpos, qvel, com))


def forward(qpos, qvel, warm, ctrl, friction, com, *, iterations=ITERATIONS, substeps=SUBSTEPS, tape=False,
            kinematics=False):
    """One control step outside autograd -> (qpos', qvel', warm', info (B, 4) int32[, tape][, kinematics outputs])
    (the reference's forward, torch_ffi.py:845-851). info per world: Newton iterations of the last substep, contacts,
    constraint rows, overflow bits (OVERFLOW_CONTACTS, OVERFLOW_ROWS)."""
    with torch.no_grad():
        q1, v1, w1, info, tp, *kin = _ops().forward(qpos, qvel, warm, ctrl, friction, com, int(iterations),
                                                             int(substeps), bool(tape), bool(kinematics))
    return (q1, v1, w1, info, *((tp,) if tape else ()), *kin)


def backward(tape, friction, com, g_qpos, g_qvel, *, substeps=SUBSTEPS, clamp_kv=CLAMP_KV, normal=NORMAL, ctrl=None,
             clamp_soft=None, kinematics=None):
    """The adjoint of one control step from its tape -> (g_qpos (B, 36) in qpos form, g_qvel (B, 35), g_ctrl (B, 29),
    info (B,) int32) (the reference's backward, torch_ffi.py:854-865). ctrl: the step's controls, for clamp_kv=2 only.
    kinematics: None, or (qpos', qvel', g_qpos_n, g_xpos, g_xquat, g_cvel, g_subtree_com) whose kinematics
    cotangents are pulled back and added to g_qpos, g_qvel first."""
    kv, nrm = _variant(clamp_kv, normal)
    delta = _soft_delta(kv, clamp_soft)
    if kv == 2 and ctrl is None:
        raise _err("clamp_kv=2 (the soft clamp) needs the step's ctrl", ValueError)
    kin_state, kin_cot = [], []
    if kinematics is not None:
        kinematics = list(kinematics)
        if len(kinematics) != 7:
            raise _err("kinematics = (qpos', qvel', g_qpos_n, g_xpos, g_xquat, g_cvel, g_subtree_com)", ValueError)
        kin_state, kin_cot = kinematics[:2], kinematics[2:]
    with torch.no_grad():
        r = _ops().backward(tape, friction, com, g_qpos, g_qvel, ctrl if kv == 2 else None, kin_state,
                                     kin_cot, int(substeps), kv, nrm, 0.0 if delta is None else delta)
    return tuple(r)


# ---- gradient scaling -----------------------------------------------------------------------------------------------

class _ScaledCotangent(torch.autograd.Function):
    """The identity on one tensor whose cotangent comes back multiplied by gamma (a float32 product)."""

    @staticmethod
    def forward(ctx, x, gamma):
        ctx.gamma = gamma
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        return g * ctx.gamma, None


def scale_grad(tree, gamma):
    """The identity on a pytree whose floating-point tensors get their cotangents multiplied by gamma in the backward;
    other leaves pass through (the reference's scale_grad, torch_ffi.py:868-899). Put on a rollout's carried state at
    the top of each step, it makes a gradient through n step boundaries carry gamma^n."""
    from torch.utils import _pytree
    g = float(gamma)
    if not math.isfinite(g):
        raise _err(f"scale_grad's gamma must be finite, got {gamma}", ValueError)
    return _pytree.tree_map(
        lambda x: _ScaledCotangent.apply(x, g) if isinstance(x, Tensor) and x.is_floating_point() else x, tree)


# ---- diagnostics ----------------------------------------------------------------------------------------------------

def set_diagnostics(enabled):
    """Counting on (the default) or off; returns the previous setting (the reference's set_diagnostics,
    torch_ffi.py:678-686). On, the forward and adjoint kernels add each world's counts to the device's counters as it
    ends (dk_fwd_forward_diag, dk_adjoint_work_diag) and the backward's info gets the non-finite bits. Outputs and
    gradients do not depend on it."""
    prev, _settings["count"] = _settings["count"], bool(enabled)
    return prev


def diagnostics(device=None):
    """The device's counters: an int64 (len(DIAG),) GPU tensor in DIAG order, summed over the calls since init or the
    last reset; neither copied nor synchronized (the reference's diagnostics, torch_ffi.py:689-695)."""
    dev = _device_index(device)
    _ready(dev)
    return _counters[dev]


def read_diagnostics(device=None, reset=True):
    """The device's counters as {name: count} (a synchronization); reset zeroes them after the read. With overflow
    warnings on, worlds beyond the contact or row capacity are reported (the reference's read_diagnostics,
    torch_ffi.py:698-708)."""
    t = diagnostics(device)
    counts = {name: int(v) for name, v in zip(DIAG, t.tolist())}
    if reset:
        t.zero_()
    if _settings["warn"]:
        warn_overflow(counts)
    return counts


def warn_overflow(d, where="nablaengine_amd"):
    """Warn (RuntimeWarning) when the counts d hold world-steps that found more than 64 contacts or 192 constraint
    rows: the extra ones were dropped, so those worlds lack some support and friction forces. Returns how many
    world-steps that is (the reference's warn_overflow, torch_ffi.py:711-724)."""
    contacts, rows = d.get("fwd_contact_overflow_worlds", 0), d.get("fwd_row_overflow_worlds", 0)
    if contacts or rows:
        warnings.warn(f"{where}: world-steps over capacity: {contacts} found more than {MAXCON} contacts, {rows} more "
                      f"than {MAXROWS} constraint rows; what did not fit was dropped, so those worlds miss part of "
                      f"their support and friction forces (deep interpenetration?)", RuntimeWarning, stacklevel=3)
    return contacts + rows


def set_overflow_warnings(enabled):
    """Overflow warnings on or off (default off, or $DK_OVERFLOW_WARN=1); on, read_diagnostics warns, and counts no
    read took are reported once more at exit. Returns the previous setting (the reference's set_overflow_warnings,
    torch_ffi.py:727-735)."""
    prev, _settings["warn"] = _settings["warn"], bool(enabled)
    return prev


@atexit.register
def _report_unread_overflow():
    """At exit, with counting and warnings on: warn about each device's counts since the last read. Never raises."""
    if not (_settings["count"] and _settings["warn"]):
        return
    try:
        for dev, t in sorted(_counters.items()):
            warn_overflow(dict(zip(DIAG, t.tolist())), where=f"nablaengine_amd (cuda:{dev})")
    except Exception:  # noqa: BLE001  (the interpreter or the HIP runtime is shutting down)
        pass
