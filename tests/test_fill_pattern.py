"""The self-contact fill pattern of H's factorization (csrc/g1_device.h fill_bits, csrc/g1_forward.hip hessian()'s
classes), checked with numpy on the G1 tree: the leaf-first L'L factor (A = L'L, as ltl_factor) of random matrices
with the tree's sparsity plus the coupling of a contact between two robot bodies has no entry outside the tree's
pattern united with the fill rows, for every pair of bodies hessian() sends to that variant (a leg against the waist
or its own arm, the two legs, any combination of them); a pair it sends to the dense routine (a leg against the other
side's arm) does leave the pattern, and an ancestor pair stays on the tree's pattern. CPU only."""
import itertools
import json
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MODEL = json.load(open(os.path.join(ROOT, "nablaengine_amd", "model", "g1_model.json")))
PARENT, DOF_BODY, NV = MODEL["body_parent"], MODEL["dof_body"], 35


def _chain(b):
    bodies = set()
    while b > 0:
        bodies.add(b)
        b = PARENT[b]
    return sorted(i for i in range(NV) if DOF_BODY[i] in bodies)


CHAIN = {b: _chain(b) for b in range(1, 31)}
TREE = [set(CHAIN[DOF_BODY[i]]) & set(range(i)) for i in range(NV)]  # row i's tree entries left of the diagonal


def _fill(k):  # the fill rows of the common self-contact pattern
    m = set()
    if 18 <= k <= 27:
        m |= set(range(6, 12))
    if 18 <= k <= 20 or 28 <= k <= 34:
        m |= set(range(12, 18))
    if 12 <= k <= 17:
        m |= set(range(6, 12))
    return m


def _pattern(x, y):  # hessian()'s class of a contact between bodies x < y: 0 tree, 1 common fill, 2 dense
    anc = x in _ancestors(y)
    legl, legr = 2 <= x <= 7, 8 <= x <= 13
    common = (legl and 8 <= y <= 23) or (legr and (14 <= y <= 16 or y >= 24))
    return 0 if anc else 1 if common else 2


def _ancestors(b):
    out = []
    while b > 0:
        out.append(b)
        b = PARENT[b]
    return out


def _factor_outside(pairs, fill, rng):
    A = 0.1 * np.eye(NV)
    for b in range(1, 31):  # a positive definite matrix with the tree's sparsity (bodies' chain Jacobians)
        J = np.zeros((6, NV))
        J[:, CHAIN[b]] = rng.normal(size=(6, len(CHAIN[b])))
        A += J.T @ J
    for x, y in pairs:  # contact rows J_y - J_x on the two chains
        J = np.zeros((4, NV))
        J[:, CHAIN[y]] = rng.normal(size=(4, len(CHAIN[y])))
        J[:, CHAIN[x]] -= rng.normal(size=(4, len(CHAIN[x])))
        A += J.T @ J
    L = np.zeros_like(A)
    for k in range(NV - 1, -1, -1):  # leaf first: A = L' L
        L[k, :k + 1] = A[k, :k + 1] / np.sqrt(A[k, k])
        A[:k, :k] -= np.outer(L[k, :k], L[k, :k])
    allowed = [TREE[k] | (_fill(k) if fill else set()) for k in range(NV)]
    return [(k, m) for k in range(NV) for m in range(k) if abs(L[k, m]) > 1e-9 * abs(L[k, k]) and m not in allowed[k]]


def test_common_fill_covers_its_pairs():
    rng = np.random.default_rng(0)
    common = [(x, y) for x in range(1, 31) for y in range(x + 1, 31) if _pattern(x, y) == 1]
    assert (3, 23) in common and (9, 30) in common and (7, 13) in common and (5, 11) in common
    for x, y in common:
        assert not _factor_outside([(x, y)], True, rng), (x, y)
    for p, q in itertools.combinations([(3, 23), (9, 30), (7, 13), (2, 16), (10, 24)], 2):
        assert not _factor_outside([p, q], True, rng), (p, q)


def test_tree_and_dense_classes():
    rng = np.random.default_rng(1)
    for x, y in [(1, 20), (16, 23), (2, 6), (14, 30)]:
        assert _pattern(x, y) == 0 and not _factor_outside([(x, y)], False, rng), (x, y)
    for x, y in [(3, 30), (9, 23), (20, 27)]:  # a leg against the other side's arm, the two arms
        assert _pattern(x, y) == 2 and _factor_outside([(x, y)], True, rng), (x, y)
