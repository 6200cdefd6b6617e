"""The reference's gradient scorer and gates, restated (scripts/gradient_check.py:52-63 THRESHOLDS / COS_P1,
benchmarks/bench/accuracy/gradient.py:12-18,175-190 block_errors and the floor): per state, cotangent and input block
(qpos tangent 35 / qvel 35 / ctrl 29) on the block's valid columns, e = |g - fd| / max(|fd|, 1e-9) and the cosine;
the truth's floor f = |fd(1e-7) - fd(1e-6)| / max(|fd|, 1e-9); the floored error max(e, f). A group passes when, per
block, the floored error's p99 <= THRESHOLDS[block] and the cosine's 1st percentile >= COS_P1. Test helper only."""
import numpy as np

THRESHOLDS = dict(qpos=2e-3, qvel=5e-4, ctrl=1e-4)
COS_P1 = 0.99999
BLOCKS = dict(qpos=slice(0, 35), qvel=slice(35, 70), ctrl=slice(70, 99))


def block_scores(g, fd, fd_floor, valid):
    """{block: (floored errors, cosines)} over the (state, cotangent) pairs with a valid column in the block.
    g, fd, fd_floor: (N, C, 99) (fd_floor: the truth's VJP at h = 1e-7); valid: (N, 99) bool."""
    out = {}
    for name, sl in BLOCKS.items():
        ef, cs = [], []
        for w in range(len(g)):
            v = valid[w, sl]
            if not v.any():
                continue
            a, b, f = g[w][:, sl][:, v], fd[w][:, sl][:, v], fd_floor[w][:, sl][:, v]
            nb = np.linalg.norm(b, axis=1)
            e = np.linalg.norm(a - b, axis=1) / np.maximum(nb, 1e-9)
            fl = np.linalg.norm(f - b, axis=1) / np.maximum(nb, 1e-9)
            ef.extend(np.fmax(e, fl))
            cs.extend(np.sum(a * b, 1) / np.maximum(np.linalg.norm(a, axis=1) * nb, 1e-30))
        out[name] = (np.asarray(ef), np.asarray(cs))
    return out


def passes(scores):
    """(every block within its gate, {block: (p99 floored error, p1 cosine)})."""
    st = {b: (float(np.percentile(e, 99)), float(np.percentile(c, 1))) for b, (e, c) in scores.items()}
    return all(p99 <= THRESHOLDS[b] and p1 >= COS_P1 for b, (p99, p1) in st.items()), st


def perturb(g, rel, seed=0):
    """g (N, C, 99) moved by rel relative per state, cotangent and block, in a random direction (the reference's
    self-test, scripts/gradient_check.py:72-83)."""
    rng = np.random.default_rng(seed)
    out = np.array(g, np.float64, copy=True)
    for sl in BLOCKS.values():
        b = out[:, :, sl]
        u = rng.standard_normal(b.shape)
        u /= np.maximum(np.linalg.norm(u, axis=-1, keepdims=True), 1e-30)
        out[:, :, sl] = b + rel * np.linalg.norm(b, axis=-1, keepdims=True) * u
    return out


def truth_states(z, group):
    """The group's model_ok states of a gradient fixture: (indices, inputs dict float64, cot_qpos, cot_qvel)."""
    sel = np.nonzero(z[group] & (z["model_flags"] == 0))[0]
    st = {k: z[src][sel].astype(np.float64) for k, src in (("qpos", "qpos"), ("qvel", "qvel"),
                                                             ("warm", "qacc_warmstart"), ("ctrl", "ctrl"),
                                                             ("friction", "friction"), ("com", "com"))}
    return sel, st, z["cot_qpos"][sel], z["cot_qvel"][sel]
