"""The floor contacts' lane runs (csrc/g1_forward.hip floor_run / run_sum, csrc/g1_device.h wscan_nw / lane_of): the
Hessian's composite stiffness and the Newton gradient take each dof's sum over the floor contacts on the bodies it
moves as P[fhi - 1] - fcl * P[flo - 1] from inclusive prefix sums P over the contact lanes. CPU only:
- the two orders this relies on, restated from the model file: every dof's bodies are one run of body ids
  (depth-first body order), and the floor pairs come first in the pair table, sorted by body (so the contacts,
  compacted in pair order, put the floor contacts in lanes [0, nf) by body);
- a lane emulation of the kernel's steps (the DPP scan as the hardware runs it at 16, 32 and 64 lanes, lanes past
  the scan's width holding their own rows' partial sums, ds_bpermute's lane index modulo 64) against the direct sums
  on random contact sets, and planted mistakes in the emulation that the comparison catches."""
import json
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MODEL = json.load(open(os.path.join(ROOT, "nablaengine_amd", "model", "g1_model.json")))
PARENT, DOF_BODY, NV, NB = MODEL["body_parent"], MODEL["dof_body"], MODEL["nv"], 32
WL = 64


def _subtree(b):  # the bodies a dof of body b moves: b and its descendants
    out = {b}
    for c in range(len(PARENT)):
        k = c
        while k > 0:
            if k == b:
                out.add(c)
                break
            k = PARENT[k]
    return out


DOF_BODIES = [_subtree(DOF_BODY[i]) for i in range(NV)]


def test_dof_bodies_are_one_id_run():
    for i, s in enumerate(DOF_BODIES):
        assert s == set(range(min(s), max(s) + 1)), f"dof {i}"


def test_floor_pairs_first_and_sorted_by_body():
    g1, g2, gb = MODEL["pair_g1"], MODEL["pair_g2"], MODEL["geom_body"]
    floor = [gb[g1[p]] == 0 for p in range(MODEL["npair"])]
    nfloor = sum(floor)
    assert all(floor[:nfloor]) and not any(floor[nfloor:])
    bodies = [gb[g2[p]] for p in range(nfloor)]
    assert bodies == sorted(bodies) and min(bodies) >= 1


def _scan(x, width):  # wscan_nw: row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast 15 / 31 by width
    x = x.copy()
    for s in (1, 2, 4, 8):
        y = np.zeros_like(x)
        for l in range(WL):
            if l % 16 >= s:
                y[l] = x[l - s]
        x = x + y
    if width > 16:
        y = np.zeros_like(x)
        for l in range(16, 32):
            y[l] = x[15]
        for l in range(48, 64):
            y[l] = x[47]
        x = x + y
    if width > 32:
        y = np.zeros_like(x)
        for l in range(32, 64):
            y[l] = x[31]
        x = x + y
    return x


def _runs(b2, floorl, dsub, le_bs=False):  # floor_run: the last lane of each body's run, then lo / hi per dof lane
    nf = int(floorl.sum())
    ends = [l for l in range(WL) if floorl[l] and (l == nf - 1 or b2[(l + 1) % WL] != b2[l])]
    lo, hi = np.zeros(WL, int), np.zeros(WL, int)
    for l in range(WL):
        bs, be = (min(dsub[l]), max(dsub[l]) + 1) if dsub[l] else (NB, NB)
        for e in ends:
            if (b2[e] <= bs) if le_bs else (b2[e] < bs):
                lo[l] = e + 1
            if b2[e] < be:
                hi[l] = e + 1
    return nf, lo, hi


def _run_sum(P, lo, hi, with_cl=True):  # fma(-P[(lo - 1) & 63], cl, P[(hi - 1) & 63])
    cl = ((lo > 0) | (hi == 0)).astype(float) if with_cl else np.ones(WL)
    return P[(hi - 1) % WL] - cl[:, None] * P[(lo - 1) % WL]


def _case(rng, nf, nself):
    """nf floor contacts (bodies drawn from the floor pairs' bodies, sorted), then nself contacts between robot bodies
    (their terms are nonzero but must not enter the floor sums), zero past the contacts."""
    gb, g1, g2 = MODEL["geom_body"], MODEL["pair_g1"], MODEL["pair_g2"]
    floor_bodies = sorted(set(gb[g2[p]] for p in range(MODEL["npair"]) if gb[g1[p]] == 0))
    b2 = np.zeros(WL, int)
    b2[:nf] = np.sort(rng.choice(floor_bodies, size=nf))
    b2[nf:nf + nself] = rng.integers(2, 31, size=nself)
    floorl = np.zeros(WL, bool)
    floorl[:nf] = True
    K = np.zeros((WL, 21))
    K[:nf + nself] = rng.normal(size=(nf + nself, 21))
    K[:nf][rng.random(nf) < 0.3] = 0.0  # inactive floor contacts: exactly zero
    dsub = [DOF_BODIES[l] if l < NV else set() for l in range(WL)]
    want = np.array([K[:nf][np.isin(b2[:nf], list(dsub[l]))].sum(0) if dsub[l] else np.zeros(21) for l in range(WL)])
    return b2, floorl, K, dsub, want


@pytest.mark.parametrize("nf,nself", [(0, 0), (1, 0), (5, 3), (14, 2), (16, 0), (17, 5), (31, 9), (32, 0), (33, 4),
                                      (50, 14), (64, 0)])
def test_runs_give_each_dofs_floor_sum(nf, nself):
    rng = np.random.default_rng(nf * 100 + nself)
    for _ in range(20):
        b2, floorl, K, dsub, want = _case(rng, nf, nself)
        if nf == 0:
            continue  # the kernels skip the sums (R.nf == 0)
        n, lo, hi = _runs(b2, floorl, dsub)
        got = _run_sum(_scan(K, n), lo, hi)
        np.testing.assert_allclose(got[:NV], want[:NV], rtol=1e-12, atol=1e-12)


def test_planted_mistakes_fail():
    rng = np.random.default_rng(7)
    caught = {"lo with <=": 0, "no cl weight": 0, "scan too narrow": 0}
    for _ in range(20):
        b2, floorl, K, dsub, want = _case(rng, 24, 6)
        n, lo, hi = _runs(b2, floorl, dsub, le_bs=True)
        caught["lo with <="] += not np.allclose(_run_sum(_scan(K, n), lo, hi)[:NV], want[:NV])
        n, lo, hi = _runs(b2, floorl, dsub)
        caught["scan too narrow"] += not np.allclose(_run_sum(_scan(K, 16), lo, hi)[:NV], want[:NV])
        # the weight matters where lane 63's prefix is not 0: a scan over all 64 lanes
        b2, floorl, K, dsub, want = _case(rng, 40, 10)
        n, lo, hi = _runs(b2, floorl, dsub)
        caught["no cl weight"] += not np.allclose(_run_sum(_scan(K, n), lo, hi, with_cl=False)[:NV], want[:NV])
    assert all(v > 0 for v in caught.values()), caught
