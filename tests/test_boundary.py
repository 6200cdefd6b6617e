"""The drop-in boundary without a GPU: the C ABI library exports every entry include/nablaengine_g1.h declares, the
model constants committed match the model file, the Python surface validates its arguments and fails loudly without a
GPU (no CPU fallback), and bench.py refuses more than one GPU."""
import ctypes
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nablaengine_g1.h")
LIB = os.path.join(ROOT, "nablaengine_amd", "libnablaengine_g1.so")


def _declared():
    txt = open(HEADER).read()
    names = set(re.findall(r"\b(dk_\w+)\s*\(", txt))
    names = {n for n in names if "##" not in n and not n.startswith("dk_kv##")}
    for kv in (0, 1, 2):
        for n in (0, 1, 2, 3):
            names |= {f"dk_kv{kv}_n{n}_adjoint", f"dk_kv{kv}_n{n}_upload", f"dk_kv{kv}_n{n}_sizes",
                      f"dk_kv{kv}_n{n}_launch"}
    return names


def test_library_exports_every_declared_entry():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (python -m nablaengine_amd.build)")
    lib = ctypes.CDLL(LIB)
    names = _declared()
    assert len(names) >= 40
    for n in sorted(names):
        assert hasattr(lib, n), n
    sizes = (ctypes.c_longlong * 9)()
    lib.dk_fwd_sizes(sizes)
    assert list(sizes)[2:6] == [1472, 36, 35, 64]
    lib.dk_kv2_n1_sizes(sizes)
    assert sizes[6] == 2 and sizes[7] == 1
    lib.dk_fwd_work_bytes.restype = lib.dk_adjoint_work_bytes.restype = ctypes.c_longlong
    assert lib.dk_fwd_work_bytes(0) == 0 and lib.dk_adjoint_work_bytes(0) == 0
    # the dispatch order: a permutation and a cost per world (int32)
    assert lib.dk_fwd_work_bytes(4096) >= 8 * 4096 and lib.dk_adjoint_work_bytes(4096) >= 8 * 4096


def test_model_header_matches_json():
    d = json.load(open(os.path.join(ROOT, "nablaengine_amd", "model", "g1_model.json")))
    h = open(os.path.join(ROOT, "nablaengine_amd", "csrc", "g1_model.h")).read()
    assert f"MEANINERTIA = {d['meaninertia']!r}" in h and "NPAIR = 502" in h and f"TORSO_BODY = {d['torso_body']}" in h
    assert d["nq"] == 36 and d["nv"] == 35 and len(d["pair_g1"]) == 502 and d["body_names"][16] == "torso_link"


@pytest.mark.skipif(not os.path.exists("/root/reference/fixtures/mjlab/g1_train.mjb"), reason="no model file here")
def test_model_extraction_reproduces_committed_constants():
    from nablaengine_amd.model import mjb_extract
    f, bn = mjb_extract.extract()
    d = mjb_extract.derive(f, bn)
    committed = json.load(open(os.path.join(ROOT, "nablaengine_amd", "model", "g1_model.json")))
    assert json.loads(json.dumps(d)) == committed


def test_python_surface_errors_without_gpu():
    import torch
    from nablaengine_amd import synthetic, torch_ffi
    st = synthetic.states(2, config=1)
    args = [torch.from_numpy(st[k]) for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    with pytest.raises(TypeError):
        torch_ffi.forward(*args)  # CPU tensors: no implicit copy, no CPU fallback
    with pytest.raises(ValueError):
        torch_ffi.step(*args, clamp_kv=5)
    with pytest.raises(ValueError):
        torch_ffi.backward(None, None, None, None, None, clamp_kv=0, clamp_soft=0.1)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            torch_ffi.init()
    assert torch_ffi.tape_bytes(4096) == 4096 * 4 * 1472 * 4


def test_custom_ops_fake_shapes():
    """The torch.library custom ops torch.compile traces (nablaengine::forward, ::backward, ::kinematics,
    ::kinematics_backward) register without a GPU, and their fake implementations give the library's output shapes
    and dtypes (reference torch_ffi.py:603-649)."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode
    from nablaengine_amd import torch_ffi
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    torch_ffi._register_ops()
    B, rw = 5, torch_ffi.rec_words()
    with FakeTensorMode():
        a = [torch.empty(s) for s in ((B, 36), (B, 35), (B, 35), (B, 29), (B,), (B, 3))]
        r = torch.ops.nablaengine.forward(*a, 10, 4, True, True)
        assert [tuple(t.shape) for t in r] == [(B, 36), (B, 35), (B, 35), (B, 4), (B, 4 * rw), (B, 36), (B, 31, 3),
                                               (B, 31, 4), (B, 31, 6), (B, 31, 3)]
        assert r[3].dtype == torch.int32 and r[0].dtype == torch.float32
        assert tuple(torch.ops.nablaengine.forward(*a, 10, 2, False, False)[4].shape) == (0, 2 * rw)
        b = torch.ops.nablaengine.backward(r[4], a[4], a[5], r[0], r[1], None, [], [], 4, 0, 3, 0.0)
        assert [tuple(t.shape) for t in b] == [(B, 36), (B, 35), (B, 29), (B,)] and b[3].dtype == torch.int32
        k = torch.ops.nablaengine.kinematics(a[0], a[1], a[5])
        assert [tuple(t.shape) for t in k] == [(B, 36), (B, 31, 3), (B, 31, 4), (B, 31, 6), (B, 31, 3)]
        kb = torch.ops.nablaengine.kinematics_backward(a[0], a[1], a[5], *k)
        assert [tuple(t.shape) for t in kb] == [(B, 36), (B, 35)]


def test_init_artifacts_one_library_per_process(tmp_path):
    """init / load_library take the library as a .so path or a JSON artifact naming it (reference torch_ffi.py:241-290);
    a second, different library in the same process is a RuntimeError; another model is a ValueError (the G1 model is
    compiled in)."""
    from nablaengine_amd import torch_ffi
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    lib = torch_ffi.load_library()
    art = tmp_path / "g1.json"
    path = torch_ffi._native.path
    art.write_text(json.dumps({"library": os.path.relpath(path, tmp_path)}))
    assert os.path.realpath(torch_ffi.library_path(str(art))) == os.path.realpath(path)
    assert torch_ffi.load_library(str(art)) is lib
    other = tmp_path / "other.so"
    other.write_bytes(b"")
    with pytest.raises(RuntimeError):
        torch_ffi.load_library(str(other))
    with pytest.raises(ValueError):
        torch_ffi.init(model="g1.xml")


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode != 0 and "one GPU" in r.stderr


def test_diagnostics_names_and_overflow_warning():
    """The counters' names and order are the reference's (torch_ffi.py:56-59); warn_overflow warns only when worlds
    overflowed, and returns their count."""
    import warnings
    from nablaengine_amd import torch_ffi
    assert len(torch_ffi.DIAG) == 18 and torch_ffi.DIAG[0] == "fwd_calls" and torch_ffi.DIAG[-1] == "fwd_row_overflow_worlds"
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        assert torch_ffi.warn_overflow(dict.fromkeys(torch_ffi.DIAG, 0)) == 0 and not w
        assert torch_ffi.warn_overflow({"fwd_contact_overflow_worlds": 2, "fwd_row_overflow_worlds": 1}) == 3
        assert len(w) == 1 and issubclass(w[0].category, RuntimeWarning)
    assert torch_ffi.set_overflow_warnings(True) in (False, True)
    assert torch_ffi.set_overflow_warnings(False) is True


def test_c_abi_rejects_bad_arguments_before_any_launch():
    """The C entries check their arguments on the host and return a hipError_t (hipErrorInvalidValue = 1) or the
    static entry's capacity error (-2) without touching a device, the reference's convention (jax_ffi.py:198-258: an
    int return, 0 on success); an empty batch is a successful no-op. Called here without a GPU: none of these paths
    reaches the HIP runtime."""
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (python -m nablaengine_amd.build)")
    lib = ctypes.CDLL(LIB)
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    fwd = [P, I] + [P] * 6 + [I, I] + [P] * 7
    lib.dk_fwd_forward.argtypes = fwd
    lib.dk_fwd_forward_ordered.argtypes = fwd
    lib.dk_fwd_forward_static.argtypes = fwd[:-1]
    lib.dk_fwd_order.argtypes = [P, I, P, P]
    adj = [P, I, I] + [P] * 10 + [F, I, I, P]
    lib.dk_adjoint_work.argtypes = adj
    lib.dk_adjoint.argtypes = adj[:-1]
    lib.dk_kv2_n3_adjoint.argtypes = adj[:-3]
    lib.dk_fwd_kinematics.argtypes = [P, I] + [P] * 8
    lib.dk_torch_diag_fwd.argtypes = [P, P, I, I, I, P, P]
    n6 = [None] * 6
    f = lambda nw, it=10, nsub=4, work=None: lib.dk_fwd_forward(None, nw, *n6, it, nsub, *[None] * 6, work)
    assert f(0) == 0
    assert f(-1) == 1 and f(3, nsub=0) == 1 and f(3, nsub=33) == 1 and f(3, it=-1) == 1
    assert lib.dk_fwd_forward_ordered(None, 3, *n6, 10, 4, *[None] * 7) == 1  # an order needs its work buffer
    assert lib.dk_fwd_order(None, 3, None, None) == 1 and lib.dk_fwd_order(None, 0, None, None) == 0
    assert lib.dk_fwd_forward_static(None, 131072 + 1, *n6, 10, 4, *[None] * 6) == -2
    a = lambda nw, kv=1, n=0, nsub=4, tape=None, ctrl=None: lib.dk_adjoint_work(
        None, nw, nsub, tape, *[None] * 8, ctrl, 0.2, kv, n, None)
    assert a(0) == 0
    assert a(-1) == 1 and a(3, nsub=0) == 1 and a(3, kv=3) == 1 and a(3, n=4) == 1 and a(3, kv=-1) == 1
    assert a(3, kv=2) == 1  # the soft clamp recomputes the actuator force: ctrl is required
    assert a(3, tape=0x1004) == 1  # the factors are copied 16 bytes at a time: the tape must be 16-byte aligned
    assert lib.dk_kv2_n3_adjoint(None, 3, 4, *[None] * 10, 0.2) == 1
    assert lib.dk_fwd_kinematics(None, -1, *[None] * 8) == 1 and lib.dk_fwd_kinematics(None, 0, *[None] * 8) == 0
    assert lib.dk_torch_diag_fwd(None, None, 3, 4, 10, None, None) == 1
    # the entries with the counters or a precomputed adjoint order
    lib.dk_fwd_forward_diag.argtypes = fwd + [P]
    lib.dk_adjoint_work_diag.argtypes = adj + [P]
    lib.dk_adjoint_work_ordered.argtypes = adj + [P]
    lib.dk_adjoint_order.argtypes = [P, I, I, P, P]
    d = 0x1000  # never dereferenced: every call below returns before a launch
    fd = lambda nw, d=d: lib.dk_fwd_forward_diag(None, nw, *n6, 10, 4, *[None] * 7, d)
    assert fd(0) == 0 and fd(-1) == 1 and fd(3, d=None) == 1  # the counters are required
    ad = lambda nw, d=d: lib.dk_adjoint_work_diag(None, nw, 4, None, *[None] * 9, 0.2, 1, 0, None, d)
    assert ad(0) == 0 and ad(-1) == 1 and ad(3, d=None) == 1
    assert lib.dk_adjoint_order(None, 3, 4, None, None) == 1 and lib.dk_adjoint_order(None, 0, 4, None, None) == 0
    ao = lambda nw, work=None, tape=None, kv=1: lib.dk_adjoint_work_ordered(None, nw, 4, tape, *[None] * 9, 0.2, kv,
                                                                            0, work, None)
    assert ao(0) == 0 and ao(3) == 1  # the order is read from work
    assert ao(3, work=d, kv=2) == 1 and ao(3, work=d, tape=0x1004) == 1
    lib.dk_adjoint_many.argtypes = [P, I, I, I] + [P] * 10 + [F, I, I, P, P]
    am = lambda nw, k, kv=1, tape=None: lib.dk_adjoint_many(None, nw, k, 4, tape, *[None] * 9, 0.2, kv, 0, d, None)
    assert am(0, 71) == 0 and am(-1, 71) == 1 and am(3, 0) == 1 and am(1 << 20, 1 << 12) == 1
    assert am(945196, 71) == 1 and am(1 << 20, 64) == 1  # nw * ncot * 64 work-items < 2^32 in one launch
    assert am(3, 71, kv=2) == 1 and am(3, 71, tape=0x1004) == 1


def test_device_counter_layout_matches_the_python_names():
    """The counters' device layout (csrc/g1_diag.h: the enum the kernels index, the non-finite bits and shift, the
    replay-mismatch bit) is the order and the values torch_ffi reads them with (the reference's, torch_ffi.py:56-61):
    a counter added to the wrong slot would otherwise only show as a wrong name in read_diagnostics()."""
    from nablaengine_amd import torch_ffi
    h = open(os.path.join(ROOT, "nablaengine_amd", "csrc", "g1_diag.h")).read()
    body = re.search(r"enum \{([^}]*)\}", h).group(1)
    names = [n.strip().split("=")[0].strip() for n in body.split(",") if n.strip()]
    assert names[-1] == "NDIAG" and len(names) - 1 == len(torch_ffi.DIAG)
    conv = {"D_FWD_CALLS": "fwd_calls", "D_FWD_WORLDS": "fwd_worlds", "D_FWD_UNSUPPORTED": "fwd_unsupported_worlds",
            "D_FWD_ITER_LIMIT": "fwd_iteration_limit_worlds", "D_TAPE_RECORDS": "tape_records",
            "D_REFACT": "refact_records", "D_NONCONV": "nonconv_records", "D_SINGULAR": "singular_records",
            "D_BWD_CALLS": "bwd_calls", "D_BWD_ROWS": "bwd_rows", "D_NONFINITE": "nonfinite_rows",
            "D_NONFINITE_QPOS": "nonfinite_qpos_rows", "D_NONFINITE_QVEL": "nonfinite_qvel_rows",
            "D_NONFINITE_CTRL": "nonfinite_ctrl_rows", "D_NONFINITE_COT": "nonfinite_cotangent_rows",
            "D_REPLAY_MISMATCH": "replay_mismatch_worlds", "D_CONTACT_OVERFLOW": "fwd_contact_overflow_worlds",
            "D_ROW_OVERFLOW": "fwd_row_overflow_worlds"}
    assert [conv[n] for n in names[:-1]] == list(torch_ffi.DIAG)
    def val(n):  # an integer literal or "a << b"
        a, _, b = re.search(rf"\b{n} = ([^,;]+)[,;]", h).group(1).partition("<<")
        return int(a) << int(b) if b else int(a)
    assert (val("NONFINITE_QPOS"), val("NONFINITE_QVEL"), val("NONFINITE_CTRL"), val("NONFINITE_COT")) == \
        (torch_ffi.NONFINITE_QPOS, torch_ffi.NONFINITE_QVEL, torch_ffi.NONFINITE_CTRL, torch_ffi.NONFINITE_COT)
    assert val("NONFINITE_SHIFT") == torch_ffi.NONFINITE_SHIFT
    assert val("ADJ_REPLAY_MISMATCH") == torch_ffi.ADJ_REPLAY_MISMATCH


# The autograd and operator plumbing of torch_ffi, run on the CPU in a child process whose library calls are replaced
# by stand-ins before the operators are defined (the operators are process-wide, so the stand-ins must not leak into
# other tests). The stand-ins are linear maps with known adjoints and record the options each call received.
_PLUMBING = r'''
import torch
from nablaengine_amd import torch_ffi as F

seen = []

def fwd(qpos, qvel, warm, ctrl, friction, com, iterations, substeps, tape, kinematics):
    B = qpos.shape[0]
    q1 = qpos * 2.0 + friction[:, None]
    v1 = torch.cat([qvel[:, :6] * 3.0, qvel[:, 6:] * 3.0 + ctrl], 1)
    tp = torch.zeros((B if tape else 0, substeps * F.rec_words()))
    kin = [torch.full((B, *s), 0.5) * q1[:, :1].reshape(B, *([1] * len(s))) for _, s in F._KIN_OUT] if kinematics else []
    return [q1, v1, warm + 1.0, torch.full((B, 4), iterations, dtype=torch.int32), tp] + kin

def bwd(tape, friction, com, g_qpos, g_qvel, ctrl, kin_state, kin_cot, substeps, clamp_kv, normal, clamp_soft):
    seen.append((clamp_kv, normal, round(clamp_soft, 6), ctrl is not None, len(kin_state), substeps))
    gq = g_qpos * 2.0
    if kin_state:
        gq = gq + sum(c.reshape(c.shape[0], -1).sum(1, keepdim=True) for c in kin_cot) * 0.5
    w = 1.0 + clamp_soft if clamp_kv == 2 else 1.0
    return [gq, g_qvel * 3.0, g_qvel[:, 6:] * w, torch.zeros(g_qpos.shape[0], dtype=torch.int32)]

F._KERNELS["forward"] = (fwd, F._KERNELS["forward"][1])
F._KERNELS["backward"] = (bwd, F._KERNELS["backward"][1])
B = 5
g = torch.Generator().manual_seed(0)
x = [torch.randn((B, n), generator=g) for n in (36, 35, 35, 29)] + [torch.rand(B, generator=g), torch.randn((B, 3), generator=g)]
cq, cv = torch.randn((B, 36), generator=g), torch.randn((B, 35), generator=g)

def loss(q, v, w, u, fr, c, **kw):
    out = F.step(q, v, w, u, fr, c, **kw)
    assert not out[2].requires_grad  # warm' is not differentiable
    extra = (out[4] * 1.5).sum() if kw.get("kinematics") else 0.0
    return (out[0] * cq).sum() + (out[1] * cv).sum() + extra

def grads(f, **kw):
    xs = [t.clone().requires_grad_(i in (0, 1, 3)) for i, t in enumerate(x)]
    f(*xs, **kw).backward()
    return [xs[i].grad for i in (0, 1, 3)]

# eager: the options reach the backward, grad_decay scales the state's gradients only, the soft clamp's default delta
gq, gv, gu = grads(loss, clamp_kv=2, normal=1, grad_decay=0.98, substeps=3)
assert seen[-1] == (2, 1, 0.2, True, 0, 3), seen[-1]
assert torch.equal(gq, (cq * 2.0) * 0.98) and torch.equal(gv, (cv * 3.0) * 0.98)
assert torch.equal(gu, cv[:, 6:] * 1.2)
grads(loss, clamp_kv=2, clamp_soft=0.05)
assert seen[-1] == (2, 3, 0.05, True, 0, 4), seen[-1]
grads(loss, clamp_kv=1, normal=0)
assert seen[-1] == (1, 0, 0.0, False, 0, 4), seen[-1]
# a loss on the kinematics outputs sends their cotangents (and the state for the kinematics VJP) to the backward
gk = grads(loss, kinematics=True)
assert seen[-1][4] == 2 and not torch.equal(gk[0], grads(loss)[0])
# torch.compile(fullgraph=True): no graph break, the same gradients
for kw in (dict(), dict(clamp_kv=2, grad_decay=0.5), dict(kinematics=True)):
    torch._dynamo.reset()
    f = lambda *a: loss(*a, **kw)
    ex = torch._dynamo.explain(f)(*[t.clone().requires_grad_(i in (0, 1, 3)) for i, t in enumerate(x)])
    assert ex.graph_break_count == 0, ex.break_reasons
    torch._dynamo.reset()
    cf = torch.compile(f, fullgraph=True, backend="aot_eager")
    for a, b in zip(grads(cf), grads(f)):
        assert torch.equal(a, b)
# forward / backward outside autograd: outputs without grad, the options checked
r = F.forward(*[t.requires_grad_(i == 0) for i, t in enumerate(x)], tape=True, kinematics=True)
assert len(r) == 10 and not any(t.requires_grad for t in r)
r = F.backward(r[4], x[4], x[5], cq, cv, clamp_kv=2, ctrl=x[3])
assert seen[-1][:4] == (2, 3, 0.2, True) and len(r) == 4
print("PLUMBING OK")
'''


def test_autograd_and_operator_plumbing_on_cpu():
    """step's autograd node and the nablaengine operators on the CPU, the library calls replaced by linear stand-ins:
    the options (clamp_kv, normal, the soft clamp's default and explicit delta, substeps) reach the backward call, ctrl
    goes with clamp_kv 2 only, grad_decay multiplies the qpos / qvel gradients but not ctrl's, warm' is not
    differentiable, cotangents of the kinematics outputs reach the backward with the output state, and
    torch.compile(fullgraph=True) traces it with no graph break and the eager gradients."""
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    r = subprocess.run([sys.executable, "-c", _PLUMBING], capture_output=True, text=True, cwd=ROOT, timeout=600)
    assert r.returncode == 0 and "PLUMBING OK" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


def test_scale_grad():
    """scale_grad is the identity on a pytree (float tensors bitwise, other leaves the same objects) whose float
    tensors' cotangents are multiplied by gamma in float32; a non-finite gamma is a ValueError (the reference's
    scale_grad, torch_ffi.py:868-899)."""
    import torch
    from nablaengine_amd import torch_ffi
    a = torch.randn(7, 3, requires_grad=True)
    b = torch.randn(4, dtype=torch.float64, requires_grad=True)
    n = torch.arange(5)
    tree = {"a": a, "pair": (b, n), "k": 3}
    out = torch_ffi.scale_grad(tree, 0.98)
    assert set(out) == {"a", "pair", "k"} and out["k"] == 3 and out["pair"][1] is n
    assert torch.equal(out["a"], a) and torch.equal(out["pair"][0], b)
    wa, wb = torch.randn(7, 3), torch.randn(4, dtype=torch.float64)
    ((out["a"] * wa).sum() + (out["pair"][0] * wb).sum()).backward()
    assert torch.equal(a.grad, wa * 0.98) and torch.equal(b.grad, wb * 0.98)
    c = torch.randn(3, requires_grad=True)
    (torch_ffi.scale_grad(torch_ffi.scale_grad(c, 0.5), 0.25) * 2.0).sum().backward()
    assert torch.equal(c.grad, torch.full((3,), 2.0) * 0.25 * 0.5)
    for bad in (float("nan"), float("inf")):
        with pytest.raises(ValueError):
            torch_ffi.scale_grad(tree, bad)
