"""The forward's per-substep outputs through the C ABI (reference checks T1-T3, T8 of docs/verification.md:124-137 and
the contact check of scripts/engine_step_check.py): the contacts of a substep (ocon) against MuJoCo Warp 3.17's on the
corpus states; the tape's state chain (record k holds the state after k substeps, bitwise the k-substep forward's
outputs); its contact table against the substep's contacts; and record coverage (a buffer prefilled with 0xA5 bytes
gives bitwise the tape of a zeroed one); the taped factors L_Q and L_H against float64 (T4 / T5)."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from nablaengine_amd import synthetic

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KEYS = ("qpos", "qvel", "warm", "ctrl", "friction", "com")
MAXCON = 64
REC_HDR, REC_CON, REC_QPOS, REC_QVEL, REC_ASTAR = 0, 16, 48, 84, 128


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


def _forward(ffi, args, nsub, tape_fill=None, con=False):
    """dk_fwd_forward with an ocon buffer and (tape_fill not None) a tape prefilled with that 32-bit pattern."""
    import torch
    lib = ffi.load_library()
    B = args[0].shape[0]
    kw = dict(dtype=torch.float32, device="cuda")
    q1, v1, w1 = torch.empty((B, 36), **kw), torch.empty((B, 35), **kw), torch.empty((B, 35), **kw)
    info = torch.empty((B, 4), dtype=torch.int32, device="cuda")
    ocon = torch.empty((B, MAXCON, 8), **kw) if con else None
    tape = None
    if tape_fill is not None:
        tape = torch.full((B, nsub * ffi.rec_words()), tape_fill, dtype=torch.int32, device="cuda").view(torch.float32)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.dk_fwd_forward(st, B, *map(p, args), 10, nsub, p(q1), p(v1), p(w1), p(info), p(ocon), p(tape),
                              None) == 0
    torch.cuda.synchronize()
    return q1, v1, w1, info, ocon, tape


def test_contacts_vs_mujoco_warp(ffi):
    """One substep's contacts (ocon: pair, dist, pos, normal) on 512 corpus states against MuJoCo Warp 3.17's at the
    input state: the same pair multiset in >= 99% of the states; matched contacts (same pair, nearest point) agree in
    position (1e-4 m), distance (2e-5 m) and normal (1e-4), in float32."""
    z = np.load(os.path.join(GOLD, "mjw_mf_s0.npz"))
    st = dict(qpos=z["qpos"], qvel=z["qvel"], warm=z["qacc_warmstart"], ctrl=z["ctrl"], friction=z["friction"],
              com=z["com"])
    q1, v1, w1, info, ocon, _ = _forward(ffi, [_t(st[k]) for k in KEYS], 1, con=True)
    ocon = ocon.cpu().numpy().astype(np.float64)
    n = len(z["con_count"])
    same, worst = 0, [0.0, 0.0, 0.0]
    for i in range(n):
        mine = ocon[i][ocon[i][:, 0] >= 0]
        ref = z["con"][i, :int(z["con_count"][i])]
        assert len(mine) == info[i, 1].item()
        if sorted(mine[:, 0].astype(int).tolist()) != sorted(ref[:, 0].astype(int).tolist()):
            continue
        same += 1
        for row in ref:
            cand = mine[mine[:, 0] == row[0]]
            d = np.linalg.norm(cand[:, 2:5] - row[2:5], axis=1)
            j = int(np.argmin(d))
            worst = [max(worst[0], d[j]), max(worst[1], abs(cand[j, 1] - row[1])),
                     max(worst[2], np.linalg.norm(cand[j, 5:8] - row[5:8]))]
    print(f"same contact set in {same}/{n} states; worst matched pos {worst[0]:.3g} dist {worst[1]:.3g} "
          f"normal {worst[2]:.3g}")
    assert same / n >= 0.99
    assert worst[0] <= 1e-4 and worst[1] <= 2e-5 and worst[2] <= 1e-4


def test_tape_state_chain_and_contact_table(ffi):
    """Record 0 holds the inputs; record k (k >= 1) the state after k substeps, bitwise the outputs of the k-substep
    forward (qpos, qvel), whose warm' is bitwise record k-1's a*. Each record's contact table lists the pairs of that
    substep's contacts (ocon of the (k+1)-substep forward), 0xFFFF past the count, and its header's count is theirs."""
    import torch
    B = 512
    args = [_t(synthetic.states(B, config=4)[k]) for k in KEYS]
    *_, tape = _forward(ffi, args, 4, tape_fill=0)
    rw = ffi.rec_words()
    rec = tape.view(torch.int32).cpu().numpy().reshape(B, 4, rw)
    recf = rec.view(np.float32)
    assert np.array_equal(recf[:, 0, REC_QPOS:REC_QPOS + 36].view(np.uint32),
                          args[0].cpu().numpy().view(np.uint32))
    assert np.array_equal(recf[:, 0, REC_QVEL:REC_QVEL + 35].view(np.uint32),
                          args[1].cpu().numpy().view(np.uint32))
    for k in range(1, 5):
        q, v, w, info, ocon, _ = _forward(ffi, args, k, con=True)
        q, v, w = (x.cpu().numpy() for x in (q, v, w))
        assert np.array_equal(w.view(np.uint32), recf[:, k - 1, REC_ASTAR:REC_ASTAR + 35].view(np.uint32))
        if k < 4:
            assert np.array_equal(q.view(np.uint32), recf[:, k, REC_QPOS:REC_QPOS + 36].view(np.uint32))
            assert np.array_equal(v.view(np.uint32), recf[:, k, REC_QVEL:REC_QVEL + 35].view(np.uint32))
        ocon = ocon.cpu().numpy()
        ncon = rec[:, k - 1, REC_HDR] & 255
        assert np.array_equal(ncon, info[:, 1].cpu().numpy())
        half = rec[:, k - 1, REC_CON:REC_CON + 32].view(np.uint16).reshape(B, 64)  # two 16-bit entries a word
        for i in range(B):
            n = int(ncon[i])
            assert (half[i, n:] == 0xFFFF).all()
            assert sorted((half[i, :n] & 511).tolist()) == sorted(ocon[i, :n, 0].astype(int).tolist())


def test_tape_record_coverage(ffi):
    """A tape buffer prefilled with 0xA5 bytes gives bitwise the tape of a zero-filled one (every word of every record
    is written), with config-4 (contact-heavy) states."""
    import torch
    B = 512
    args = [_t(synthetic.states(B, config=4)[k]) for k in KEYS]
    *_, t0 = _forward(ffi, args, 4, tape_fill=0)
    *_, t1 = _forward(ffi, args, 4, tape_fill=int(np.int32(np.uint32(0xA5A5A5A5))))
    assert torch.equal(t0.view(torch.int32), t1.view(torch.int32))


REC_FLAGS, REC_LH, REC_LQ = 1, 200, 832
NTRI = 35 * 36 // 2


def _unpack(words):
    """A packed lower triangle (row i, column j <= i at i (i + 1) / 2 + j) as a dense (35, 35) float64 matrix."""
    L = np.zeros((35, 35))
    L[np.tril_indices(35)] = words[:NTRI]
    return L


def _tree_pattern():
    """(35, 35) bool: dof j on dof i's chain (j's body is i's or one of its ancestors), j <= i: where M's and L_Q's
    lower triangles can be nonzero."""
    m = synthetic.model()
    db, am = np.asarray(m["dof_body"]), np.asarray(m["body_ancmask"])
    P = np.zeros((35, 35), bool)
    for i in range(35):
        for j in range(i + 1):
            P[i, j] = (int(am[db[i]]) >> int(db[j])) & 1
    return P


@pytest.mark.parametrize("config", [1, 4])
def test_taped_factors_vs_oracle(ffi, config):
    """The reference's tape checks T4 / T5 (docs/verification.md:131-132) at 50 Newton iterations: every record's L_Q
    against the float64 leaf-first factor of M + h diag(kv) at the record's input state (oracle.smooth's M,
    oracle.ltl), relative max-norm error <= 1e-5; and L_H' L_H against the float64 Hessian M + J'DJ at Newton's final
    zones of that substep (oracle.substep_hessian from the record's state and warm start: the previous record's a*),
    median <= 1e-5 and p95 <= 1e-4 over the records without overflow or non-convergence flags (a record whose float32
    and float64 solves end in different zones differs by a row's D J J')."""
    import torch
    B = 128
    st = synthetic.states(B, config=config)
    args = [_t(st[k]) for k in KEYS]
    r = ffi.forward(*args, iterations=50, tape=True)
    torch.cuda.synchronize()
    tape = r[4].cpu().numpy().reshape(B, 4, -1)
    flags = tape[:, :, REC_FLAGS].view(np.uint32)
    m = synthetic.model()
    hkv = m["timestep"] * np.diag(np.asarray(m["dof_kv"]))
    pattern = _tree_pattern()
    eq, eh = [], []
    for w in range(B):
        warm = st["warm"][w].astype(np.float64)
        for k in range(4):
            rec = tape[w, k]  # float32 words; the bit-cast integer fields are never converted
            q, v = rec[REC_QPOS:REC_QPOS + 36].astype(np.float64), rec[REC_QVEL:REC_QVEL + 35].astype(np.float64)
            u, f, c = st["ctrl"][w].astype(np.float64), float(st["friction"][w]), st["com"][w].astype(np.float64)
            M, H = oracle.substep_hessian(q, v, warm, u, f, c)
            LQ, LH = _unpack(rec[REC_LQ:]) * pattern, _unpack(rec[REC_LH:])  # L_Q's other positions: frames
            ref = oracle.ltl(M + hkv)
            eq.append(np.abs(LQ - ref).max() / np.abs(ref).max())
            if not flags[w, k] & (4 | 16 | (1 << 9)):
                eh.append(np.abs(LH.T @ LH - H).max() / np.abs(H).max())
            warm = rec[REC_ASTAR:REC_ASTAR + 35].astype(np.float64)
    eq, eh = np.array(eq), np.array(eh)
    print(f"config {config}: L_Q vs float64 ({len(eq)} records) median {np.median(eq):.3g} max {eq.max():.3g}; "
          f"L_H'L_H vs float64 H ({len(eh)} records) median {np.median(eh):.3g} p95 {np.percentile(eh, 95):.3g} "
          f"max {eh.max():.3g}")
    assert eq.max() <= 1e-5
    assert len(eh) >= 3 * B and np.median(eh) <= 1e-5 and np.percentile(eh, 95) <= 1e-4


def test_taped_frames_vs_oracle(ffi):
    """L_Q is 0 off the tree's pattern, and the record carries the body frames at the substep's qpos in those
    positions (packed order: 31 quaternions, then 31 positions with a fourth word 0; the positions past them 0). On
    contact-heavy states, every record's frames against the float64 oracle's FK of the record's qpos (xquat, xpos of
    oracle.kinematics): max error <= 2e-6 (quaternions) and 2e-6 m (positions); and the adjoint, which takes its
    poses from them, is the VJP (the adjoint tests)."""
    import torch
    B = 64
    st = synthetic.states(B, config=4, seed=5)
    args = [_t(st[k]) for k in KEYS]
    r = ffi.forward(*args, tape=True)
    torch.cuda.synchronize()
    tape = r[4].cpu().numpy().reshape(B, 4, -1)
    pattern = _tree_pattern()
    rows, cols = np.tril_indices(35)
    off = np.flatnonzero(~pattern[rows, cols])  # packed positions off the pattern, in packed order
    nf = 8 * 31
    assert len(off) >= nf
    eq = ep = 0.0
    for k in range(4):
        q = tape[:, k, REC_QPOS:REC_QPOS + 36].astype(np.float64)
        _, xpos, xquat, _, _ = oracle.kinematics(q, np.zeros((B, 35)), st["com"])
        fr = tape[:, k, REC_LQ:REC_LQ + NTRI][:, off[:nf]].astype(np.float64)
        Q, X = fr[:, :124].reshape(B, 31, 4), fr[:, 124:].reshape(B, 31, 4)
        assert np.all(X[:, :, 3] == 0) and np.all(tape[:, k, REC_LQ:REC_LQ + NTRI][:, off[nf:]] == 0)
        eq = max(eq, np.abs(Q - xquat).max())
        ep = max(ep, np.abs(X[:, :, :3] - xpos).max())
    print(f"record frames vs float64 FK: quaternions max {eq:.3g}, positions max {ep:.3g} m")
    assert eq <= 2e-6 and ep <= 2e-6


def test_taped_adjoint_cost(ffi):
    """Each record's last word is the adjoint's dispatch-cost bucket of the substeps up to it (the adjoint's ordering
    reads the last record's): per substep its contacts, plus 4 per distinct robot body they touch and per contact
    between two robot bodies, plus 8 per primitive class present (plane-sphere, sphere-sphere, sphere-capsule,
    capsule-capsule, plane-capsule), summed, in units of 4, at most 127. Restated here from the records' own headers
    and contact tables on contact-heavy states."""
    import torch
    B = 256
    st = synthetic.states(B, config=4, seed=9)
    args = [_t(st[k]) for k in KEYS]
    tape = ffi.forward(*args, tape=True)[4].view(torch.int32).cpu().numpy().reshape(B, 4, -1).astype(np.int64)
    m = synthetic.model()
    g1, g2 = np.asarray(m["pair_g1"]), np.asarray(m["pair_g2"])
    gb, gt = np.asarray(m["geom_body"]), np.asarray(m["geom_type"])
    for w in range(B):
        c = 0
        for k in range(4):
            rec = tape[w, k]
            ncon = int(rec[REC_HDR] & 255)
            half = rec[REC_CON:REC_CON + 32].astype(np.uint32).view(np.uint16).reshape(64)[:ncon]
            prs = (half & 511).astype(int)
            bodies = set(gb[g1[prs]]) | set(gb[g2[prs]])
            bodies.discard(0)
            self_n = int((gb[g1[prs]] != 0).sum())
            classes = {(gt[g1[p]], gt[g2[p]]) for p in prs}
            c += ncon + 4 * (len(bodies) + self_n) + 8 * len(classes)
            assert rec[-1] == min(c >> 2, 127), (w, k, rec[-1], c)
