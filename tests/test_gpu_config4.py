"""GPU parity on BASELINE config 4's contact-heavy states (base z ~ U(0.15, 0.45), tilt N(0, 0.6), joint noise
N(0, 0.4): feet, hands and torso on the floor, self contacts, worlds at the 64-contact / 192-row capacity) against the
float64 oracle: the forward at converged settings, split by the Newton factorization's path, the overflow flags, the
exact-mode VJP against the oracle's analytic VJP and its central finite differences, and an 8-step differentiated
rollout against a manual chain of per-step VJPs (the reference's window check, scripts/jax_ffi_check.py:20-27)."""
import numpy as np
import pytest

import oracle
from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
KEYS = ("qpos", "qvel", "warm", "ctrl", "friction", "com")
MODEL = synthetic.model()
B = 1024


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


def _np(x):
    return x.cpu().numpy().astype(np.float64)


def _rel(a, b):
    return np.linalg.norm(a - b, axis=1) / np.maximum(np.linalg.norm(b, axis=1), 1e-12)


def _fill_class(st):
    """Per state, the Newton factorization path its input-state self contacts call for, by the forward's rule
    (a contact between robot bodies x < y: none when x is y's ancestor; the common fill for a leg against the waist or
    its own arm, or the two legs; else dense): 0 no self contact off the tree's pattern, 1 the common fill, 2 dense.
    A proxy (the forward classifies the active contacts of each Newton iteration of each substep)."""
    parent = np.asarray(MODEL["body_parent"])
    gbody = np.asarray(MODEL["geom_body"])
    pg1, pg2 = np.asarray(MODEL["pair_g1"]), np.asarray(MODEL["pair_g2"])

    def anc(x, y):
        while y > 0:
            if y == x:
                return True
            y = parent[y]
        return False

    out = np.zeros(len(st["qpos"]), int)
    for w in range(len(out)):
        c = oracle.contacts(st["qpos"][w], st["qvel"][w], st["ctrl"][w], st["com"][w], st["friction"][w])
        for r in c:
            b1, b2 = gbody[pg1[int(r[0])]], gbody[pg2[int(r[0])]]
            if b1 == 0:
                continue
            x, y = min(b1, b2), max(b1, b2)
            if x == 1 or anc(x, y):
                continue
            legl, legr = 2 <= x <= 7, 8 <= x <= 13
            common = (legl and 8 <= y <= 23) or (legr and (14 <= y <= 16 or y >= 24))
            out[w] = max(out[w], 1 if common else 2)
    return out


@pytest.fixture(scope="module")
def case4(ffi):
    """1024 config-4 states, the GPU step at 50 iterations (with its tape) and the oracle's at MuJoCo's truth
    settings."""
    import torch
    st = synthetic.states(B, config=4)
    args = [_t(st[k]) for k in KEYS]
    q1, v1, w1, info, tape = ffi.forward(*args, iterations=50, tape=True)
    torch.cuda.synchronize()
    s64 = {k: st[k].astype(np.float64) for k in st}
    oq, ov, ow, oinfo = oracle.step(**s64, **oracle.TRUTH)
    return dict(st=st, s64=s64, args=args, gpu=(_np(q1), _np(v1), info.cpu().numpy()), tape=tape,
                ora=(oq, ov, oinfo), cls=_fill_class(s64))


def test_config4_forward_vs_oracle(case4):
    """The converged step (GPU 50 iterations, float32; oracle 2000, float64) on the worlds neither run flags with a
    capacity overflow (info bits 4 | 16), per factorization path: qvel median relative error <= 2e-6 (the BASELINE
    gate) and p99 <= 5e-5, qpos median <= 5e-7 and p99 <= 5e-6; every world finite."""
    q1, v1, info = case4["gpu"]
    oq, ov, oinfo = case4["ora"]
    assert np.isfinite(q1).all() and np.isfinite(v1).all()
    ok = ((info[:, 3] | oinfo[:, 3]) & 20) == 0
    ev, eq = _rel(v1, ov), _rel(q1, oq)
    for c, name in ((0, "tree pattern"), (1, "common fill"), (2, "dense"), (None, "all")):
        sel = ok & (case4["cls"] == c) if c is not None else ok
        if sel.sum() < 8:
            continue
        print(f"config4 {name} ({sel.sum()} worlds): qvel median {np.median(ev[sel]):.3g} p99 "
              f"{np.percentile(ev[sel], 99):.3g} max {ev[sel].max():.3g}; qpos median {np.median(eq[sel]):.3g} "
              f"p99 {np.percentile(eq[sel], 99):.3g}")
        assert np.median(ev[sel]) <= 2e-6 and np.percentile(ev[sel], 99) <= 5e-5, name
        assert np.median(eq[sel]) <= 5e-7 and np.percentile(eq[sel], 99) <= 5e-6, name
    assert (case4["cls"][ok] == 2).sum() >= 8 and (case4["cls"][ok] == 1).sum() >= 8


def test_config4_overflow_flags_match_oracle(case4):
    """The capacity flags (4: contacts beyond 64 dropped, 16: rows beyond 192 dropped, ORed over the substeps) equal
    the oracle's on >= 99% of the worlds and on >= 90% of the worlds either flags (a contact at zero distance can be
    found by one precision and not the other); some worlds reach the caps."""
    info, oinfo = case4["gpu"][2], case4["ora"][2]
    g, o = info[:, 3] & 20, oinfo[:, 3] & 20
    either = (g | o) != 0
    print(f"config4 overflow: GPU {np.count_nonzero(g)} worlds, oracle {np.count_nonzero(o)}, equal "
          f"{(g == o).mean():.4f}, contacts max {info[:, 1].max()} rows max {info[:, 2].max()}")
    assert either.sum() >= 3
    assert (g == o).mean() >= 0.99 and (g == o)[either].mean() >= 0.9


def test_config4_vjp_vs_oracle(ffi, case4):
    """The exact-mode VJP (clamp_kv=1, normal=0) from the 50-iteration tape against the oracle's analytic VJP on the
    worlds without overflow, per factorization path: per block median relative error <= 1e-4 and p99 <= 2e-3; and
    against the oracle's float64 central finite differences (eps 1e-6) on 64 of them, on the columns where the step is
    smooth: median <= 1e-4."""
    import torch
    args, s64 = case4["args"], case4["s64"]
    cq, cv = synthetic.cotangents(B)
    gq, gv, gu, binfo = ffi.backward(case4["tape"], args[4], args[5], _t(cq), _t(cv), clamp_kv=1, normal=0)
    torch.cuda.synchronize()
    g = np.concatenate([oracle.qpos_tangent(s64["qpos"], _np(gq)), _np(gv), _np(gu)], 1)
    assert np.isfinite(g).all() and not (binfo.cpu().numpy() & (1 << 13)).any()
    info, oinfo = case4["gpu"][2], case4["ora"][2]
    ok = np.nonzero(((info[:, 3] | oinfo[:, 3]) & 20) == 0)[0]
    sub = {k: v[ok] for k, v in s64.items()}
    r = oracle.vjp(**sub, g_qpos=cq[ok], g_qvel=cv[ok], clamp_kv=1, normal=0, **oracle.TRUTH)
    an = np.concatenate([oracle.qpos_tangent(sub["qpos"], r[0]), r[1], r[2]], 1)
    cls = case4["cls"][ok]
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        e = _rel(g[ok, sl], an[:, sl])
        for c in (0, 1, 2):
            ec = e[cls == c]
            print(f"config4 VJP {name} class {c} ({len(ec)}): median {np.median(ec):.3g} p99 "
                  f"{np.percentile(ec, 99):.3g}")
            assert np.median(ec) <= 1e-4 and np.percentile(ec, 99) <= 2e-3, (name, c)
    # central FD columns that are not smooth at these states (a joint clipped to its range sits on its limit, and
    # the limit row switches on within +-h) are marked as the truth's `bad` ones: fd(1e-6) and fd(1e-7) disagree
    pick = ok[:64]
    s_pick = {k: v[pick] for k, v in s64.items()}
    fd6 = oracle.fd_vjp(**s_pick, g_qpos=cq[pick], g_qvel=cv[pick], h=1e-6, **oracle.TRUTH)
    fd7 = oracle.fd_vjp(**s_pick, g_qpos=cq[pick], g_qvel=cv[pick], h=1e-7, **oracle.TRUTH)
    bad = np.abs(fd6 - fd7) > 1e-3 * (np.abs(fd6) + 1e-3 * np.abs(fd6).max(1, keepdims=True))
    print(f"config4 FD: {bad.any(1).sum()} of 64 worlds have non-smooth columns ({bad.sum()} columns)")
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        a, b = np.where(bad[:, sl], 0, g[pick, sl]), np.where(bad[:, sl], 0, fd6[:, sl])
        e = _rel(a, b)
        print(f"config4 VJP vs FD {name} (64 worlds, smooth columns): median {np.median(e):.3g} p90 "
              f"{np.percentile(e, 90):.3g}")
        assert np.median(e) <= 1e-4


@pytest.mark.parametrize("Bw,T,config,every", [(256, 8, 4, 4), (64, 64, 1, 8)])
def test_config4_window_against_chained_vjps(ffi, Bw, T, config, every):
    """A T-step differentiated rollout (rollout(), checkpoints every few steps, interface defaults) with the linear
    loss sum_t <c_t, (qpos_t, qvel_t)> (fixed random c_t, so dL/dx_t is exact): the gradients with respect to (qpos_0,
    qvel_0, ctrl_t) are bitwise a manual chain of per-step forward(tape=True) / backward() VJPs, cotangents summed as
    dL/dx_t + the next step's VJP (the reference's window check; 8 steps of 256 config-4 worlds, and its 64-step
    length on 64 config-1 worlds). The same chain through the float64 oracle's per-step VJPs at the GPU's per-step
    states (8 steps): per world relative error of every gradient median <= 1e-4 and p99 <= 2e-3, on the worlds
    without a capacity overflow in any step."""
    import torch
    from nablaengine_amd import rollout
    st = synthetic.states(Bw, config=config)
    us = synthetic.ctrl_sequence(T, Bw)
    rng = np.random.default_rng(4)
    cqs = rng.normal(0, 1, (T, Bw, 36)).astype(np.float32)
    cvs = rng.normal(0, 1, (T, Bw, 35)).astype(np.float32)
    fr, com, warm = _t(st["friction"]), _t(st["com"]), _t(st["warm"])
    q = _t(st["qpos"]).requires_grad_(True)
    v = _t(st["qvel"]).requires_grad_(True)
    u = _t(us).requires_grad_(True)
    states = rollout.rollout(q, v, warm, u, fr, com, checkpoint_every=every)
    loss = sum((qt * _t(cqs[t])).sum() + (vt * _t(cvs[t])).sum() for t, (qt, vt) in enumerate(states))
    loss.backward()
    # the manual chain
    xs, tapes, flags = [(_t(st["qpos"]), _t(st["qvel"]), warm)], [], np.zeros(Bw, int)
    for t in range(T):
        q1, v1, w1, info, tape = ffi.forward(*xs[-1][:2], xs[-1][2], _t(us[t]), fr, com, tape=True)
        xs.append((q1, v1, w1))
        tapes.append(tape)
        flags |= info[:, 3].cpu().numpy()
    gq, gv = _t(cqs[T - 1]), _t(cvs[T - 1])
    gus = [None] * T
    for t in range(T - 1, -1, -1):
        gq, gv, gus[t], _ = ffi.backward(tapes[t], fr, com, gq, gv)
        if t > 0:
            gq, gv = gq + _t(cqs[t - 1]), gv + _t(cvs[t - 1])
    torch.cuda.synchronize()
    assert torch.equal(q.grad, gq) and torch.equal(v.grad, gv)
    assert torch.equal(u.grad, torch.stack(gus))
    if T > 8:
        return
    # the oracle's chain at the GPU's states (float64 per-step VJPs with the interface defaults)
    x64 = [(_np(a), _np(b), _np(c)) for a, b, c in xs]
    oq, ov = cqs[T - 1].astype(np.float64), cvs[T - 1].astype(np.float64)
    ous = [None] * T
    for t in range(T - 1, -1, -1):
        qs, vs, ws = x64[t]
        oq, ov, ous[t] = oracle.vjp(qs, vs, ws, us[t].astype(np.float64), st["friction"].astype(np.float64),
                                    st["com"].astype(np.float64), oq, ov, clamp_kv=0, normal=3, **oracle.ENGINE)
        if t > 0:
            oq, ov = oq + cqs[t - 1], ov + cvs[t - 1]
    ok = (flags & 20) == 0
    q0 = st["qpos"].astype(np.float64)
    for name, a, b in (("qpos", oracle.qpos_tangent(q0, _np(gq)), oracle.qpos_tangent(q0, oq)), ("qvel", _np(gv), ov),
                       ("ctrl", _np(u.grad).transpose(1, 0, 2).reshape(Bw, -1),
                        np.stack(ous).transpose(1, 0, 2).reshape(Bw, -1))):
        e = _rel(a[ok], b[ok])
        print(f"window vs oracle chain {name} ({ok.sum()} worlds): median {np.median(e):.3g} p99 "
              f"{np.percentile(e, 99):.3g}")
        assert np.median(e) <= 1e-4 and np.percentile(e, 99) <= 2e-3


@pytest.fixture(scope="module")
def case4_default(ffi, case4):
    """The same 1024 states at the interface's defaults (10 Newton iterations, tol 1e-8, 40 line-search steps): the
    GPU step with its tape; the oracle at 10 iterations in float64 and in float32 (step_f32, the float32 rounding
    yardstick) and at 50 iterations with the same tolerance."""
    import torch
    st, s64 = case4["st"], case4["s64"]
    q1, v1, w1, info, tape = ffi.forward(*case4["args"], tape=True)
    torch.cuda.synchronize()
    off = ffi.init(0)["sizes"][8]  # the records' flags word
    flags = tape.view(torch.int32).view(B, 4, -1)[:, :, off].cpu().numpy()
    nonconv = ((flags & ffi.TAPE_NONCONV) != 0).any(1)
    o10 = oracle.step(**s64, **oracle.ENGINE)
    o50 = oracle.step(**s64, **dict(oracle.ENGINE, iterations=50))
    f32 = oracle.step_f32(**st, **oracle.ENGINE)
    # the 10-iteration cap did not bind in float64: 50 iterations at the same tolerance give the same state
    conv = (_rel(o10[1], o50[1]) <= 1e-12) & (_rel(o10[0], o50[0]) <= 1e-12)
    return dict(gpu=(_np(q1), _np(v1), info.cpu().numpy()), nonconv=nonconv, o10=o10, f32=f32, conv=conv, tape=tape)


def _yardstick_gate(name, e, e32, floor_med=2e-6, floor_p90=2e-5):
    """The kernel's errors e against float64 within 5x the float32 restatement's own errors e32 (median and p90),
    with floors at the BASELINE gate's size: where Newton stops at its cap, its iterate carries the rounding of its
    first solves (cond(H) ~ 1e5-1e6), which only further iterations remove."""
    print(f"  {name}: kernel median {np.median(e):.3g} p90 {np.percentile(e, 90):.3g} max {e.max():.3g}; float32 "
          f"restatement median {np.median(e32):.3g} p90 {np.percentile(e32, 90):.3g}")
    assert np.median(e) <= max(floor_med, 5 * np.median(e32)), name
    assert np.percentile(e, 90) <= max(floor_p90, 5 * np.percentile(e32, 90)), name


def test_config4_default_step_vs_oracle(case4_default):
    """The contact-heavy step at the interface's defaults (10 iterations; what every default call and config 4's BPTT
    run; the reference's window check runs at them, scripts/jax_ffi_check.py:20-23) against the oracle at the same
    settings, on the worlds without a capacity overflow. Where both converge (the kernel's tape records no
    non-converged substep, and the float64 oracle's 10 iterations equal its 50): qvel median <= 2e-6 (the BASELINE
    gate), p99 <= 5e-5; qpos median <= 5e-7, p99 <= 5e-6. Where either stops at the cap: within 5x the float32
    restatement's distance from float64, median and p90."""
    q1, v1, info = case4_default["gpu"]
    oq, ov, _, oinfo = case4_default["o10"]
    _, v32, _, _ = case4_default["f32"]
    assert np.isfinite(q1).all() and np.isfinite(v1).all()
    ok = ((info[:, 3] | oinfo[:, 3]) & 20) == 0
    both = ok & case4_default["conv"] & ~case4_default["nonconv"]
    rest = ok & ~both
    ev, eq = _rel(v1, ov), _rel(q1, oq)
    print(f"config4 at 10 iterations: {both.sum()} worlds converged in both, {rest.sum()} at the cap in either, "
          f"{(~ok).sum()} with overflow")
    print(f"  converged: qvel median {np.median(ev[both]):.3g} p99 {np.percentile(ev[both], 99):.3g}; qpos median "
          f"{np.median(eq[both]):.3g} p99 {np.percentile(eq[both], 99):.3g}")
    assert both.sum() >= 256 and rest.sum() >= 16
    assert np.median(ev[both]) <= 2e-6 and np.percentile(ev[both], 99) <= 5e-5
    assert np.median(eq[both]) <= 5e-7 and np.percentile(eq[both], 99) <= 5e-6
    _yardstick_gate("qvel at the cap", ev[rest], _rel(v32[rest].astype(np.float64), ov[rest]))


def test_config4_capped_worlds_vs_oracle(case4_default):
    """Worlds beyond the 64-contact or 192-row capacity, at the defaults: where the kernel's overflow flags equal the
    oracle's, both kept the same contacts and rows (each keeps the first in (pair, slot) order and drops the rest), so
    their outputs are compared with the oracle's like any other world's: within 5x the float32 restatement's distance
    from float64 (median and p90; floors 2e-6 and 2e-5), every output finite (the reference compares its two surfaces'
    capped worlds bitwise, scripts/torch_ffi_check.py:350-388)."""
    q1, v1, info = case4_default["gpu"]
    oq, ov, _, oinfo = case4_default["o10"]
    q32, v32, _, _ = case4_default["f32"]
    g, o = info[:, 3] & 20, oinfo[:, 3] & 20
    cap = (g != 0) & (g == o)
    print(f"config4 capped worlds: {cap.sum()} with flags equal to the oracle's (of {(g != 0).sum()} GPU, "
          f"{(o != 0).sum()} oracle); contacts max {info[cap, 1].max()}, rows max {info[cap, 2].max()}")
    assert cap.sum() >= 5
    assert np.isfinite(q1[cap]).all() and np.isfinite(v1[cap]).all()
    _yardstick_gate("capped qvel", _rel(v1[cap], ov[cap]), _rel(v32[cap].astype(np.float64), ov[cap]))
    _yardstick_gate("capped qpos", _rel(q1[cap], oq[cap]), _rel(q32[cap].astype(np.float64), oq[cap]), 5e-7, 5e-6)


def test_config4_default_vjp_vs_oracle(ffi, case4, case4_default):
    """The VJP config 4's BPTT takes: the interface's default variant (clamp_kv 0, normal 3) from the 10-iteration
    tape, against the oracle's analytic VJP at the same settings, on the worlds without a capacity overflow. Where both
    converge: per block median relative error <= 1e-4 and p99 within 5x the float32 restatement's p99 (vjp_f32, floor
    2e-3); where either stops at the cap: median and p90 within 5x the float32 restatement's (floors 1e-4, 2e-3). Every
    gradient finite, no replay mismatch."""
    import torch
    args, s64, st = case4["args"], case4["s64"], case4["st"]
    cq, cv = synthetic.cotangents(B, seed=77)
    gq, gv, gu, binfo = ffi.backward(case4_default["tape"], args[4], args[5], _t(cq), _t(cv))
    torch.cuda.synchronize()
    g = np.concatenate([oracle.qpos_tangent(s64["qpos"], _np(gq)), _np(gv), _np(gu)], 1)
    assert np.isfinite(g).all() and not (binfo.cpu().numpy() & (1 << 13)).any()
    info, oinfo = case4_default["gpu"][2], case4_default["o10"][3]
    ok = np.nonzero(((info[:, 3] | oinfo[:, 3]) & 20) == 0)[0]
    opts = dict(clamp_kv=ffi.CLAMP_KV, normal=ffi.NORMAL, **oracle.ENGINE)
    sub = {k: v[ok] for k, v in s64.items()}
    r = oracle.vjp(**sub, g_qpos=cq[ok], g_qvel=cv[ok], **opts)
    an = np.concatenate([oracle.qpos_tangent(sub["qpos"], r[0]), r[1], r[2]], 1)
    r32 = oracle.vjp_f32(**{k: v[ok] for k, v in st.items()}, g_qpos=cq[ok], g_qvel=cv[ok], **opts)
    y32 = np.concatenate([oracle.qpos_tangent(sub["qpos"], r32[0].astype(np.float64)), r32[1], r32[2]], 1)
    both = (case4_default["conv"] & ~case4_default["nonconv"])[ok]
    g = g[ok]
    print(f"config4 default VJP: {both.sum()} worlds converged in both, {(~both).sum()} at the cap in either")
    for name, sl in (("qpos", slice(0, 35)), ("qvel", slice(35, 70)), ("ctrl", slice(70, 99))):
        e, e32 = _rel(g[:, sl], an[:, sl]), _rel(y32[:, sl].astype(np.float64), an[:, sl])
        print(f"  {name}: converged median {np.median(e[both]):.3g} p99 {np.percentile(e[both], 99):.3g} (float32 "
              f"restatement p99 {np.percentile(e32[both], 99):.3g}); at the cap median {np.median(e[~both]):.3g} p90 "
              f"{np.percentile(e[~both], 90):.3g} (restatement {np.median(e32[~both]):.3g} / "
              f"{np.percentile(e32[~both], 90):.3g})")
        assert np.median(e[both]) <= 1e-4, name
        assert np.percentile(e[both], 99) <= max(2e-3, 5 * np.percentile(e32[both], 99)), name
        assert np.median(e[~both]) <= max(1e-4, 5 * np.median(e32[~both])), name
        assert np.percentile(e[~both], 90) <= max(2e-3, 5 * np.percentile(e32[~both], 90)), name
