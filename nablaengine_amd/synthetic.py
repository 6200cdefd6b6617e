"""Seeded synthetic G1 states of the benchmark configurations, numpy only.

Config 0/1/2/3 (standing): base xy 0, z ~ U(0.72, 0.80), quaternion = exp(r / 2) of a rotation vector r ~ N(0, 0.05^2
I3), the 29 hinges = the `home` keyframe + N(0, 0.1) clipped to the joint ranges; qvel: base linear N(0, 0.3), base
angular N(0, 0.5), joints N(0, 0.5); ctrl = home + N(0, 0.2) clipped to ctrlrange (the engine does not clamp ctrl,
MuJoCo does: clipping keeps them equal); warm 0; friction ~ U(0.3, 1.2); com ~ U(-0.05, 0.05)^3.
Config 4 (contact-heavy): z ~ U(0.15, 0.45), tilt N(0, 0.6) rad, joint noise N(0, 0.4).
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 20261201  # the committed seed (BASELINE.json gives none): config k uses SEED + k


def model():
    with open(os.path.join(HERE, "model", "g1_model.json")) as f:
        return json.load(f)


def _quat_exp(r):
    ang = np.linalg.norm(r, axis=-1, keepdims=True)
    safe = np.where(ang > 0, ang, 1.0)
    return np.concatenate([np.cos(0.5 * ang), np.sin(0.5 * ang) * r / safe], -1)


def states(n, config=1, seed=None, dtype=np.float32):
    """n synthetic states of `config`: dict qpos (n, 36), qvel (n, 35), warm (n, 35), ctrl (n, 29), friction (n,),
    com (n, 3), as `dtype`."""
    m = model()
    rng = np.random.default_rng(SEED + int(config) if seed is None else seed)
    home_q = np.asarray(m["key_home_qpos"])
    home_u = np.asarray(m["key_home_ctrl"])
    jr = np.asarray(m["jnt_range_full"]).reshape(-1, 2)[1:]
    cr = np.asarray(m["ctrlrange"]).reshape(-1, 2)
    heavy = int(config) == 4
    qpos = np.zeros((n, 36))
    qpos[:, 2] = rng.uniform(0.15, 0.45, n) if heavy else rng.uniform(0.72, 0.80, n)
    qpos[:, 3:7] = _quat_exp(rng.normal(0.0, 0.6 if heavy else 0.05, (n, 3)))
    qpos[:, 7:] = np.clip(home_q[7:] + rng.normal(0.0, 0.4 if heavy else 0.1, (n, 29)), jr[:, 0], jr[:, 1])
    qvel = np.concatenate([rng.normal(0, 0.3, (n, 3)), rng.normal(0, 0.5, (n, 3)), rng.normal(0, 0.5, (n, 29))], 1)
    ctrl = np.clip(home_u + rng.normal(0.0, 0.2, (n, 29)), cr[:, 0], cr[:, 1])
    out = dict(qpos=qpos, qvel=qvel, warm=np.zeros((n, 35)), ctrl=ctrl, friction=rng.uniform(0.3, 1.2, n),
               com=rng.uniform(-0.05, 0.05, (n, 3)))
    return {k: np.ascontiguousarray(v.astype(dtype)) for k, v in out.items()}


def cotangents(n, seed=None, dtype=np.float32):
    """Output cotangents N(0, 1) over (n, 36), (n, 35) (config 2)."""
    rng = np.random.default_rng(SEED + 102 if seed is None else seed)
    return (rng.normal(0, 1, (n, 36)).astype(dtype), rng.normal(0, 1, (n, 35)).astype(dtype))


def ctrl_sequence(T, n, seed=None, dtype=np.float32):
    """A (T, n, 29) control sequence N(0, 0.2) around the home keyframe, clipped to ctrlrange (config 4)."""
    m = model()
    rng = np.random.default_rng(SEED + 104 if seed is None else seed)
    home_u = np.asarray(m["key_home_ctrl"])
    cr = np.asarray(m["ctrlrange"]).reshape(-1, 2)
    return np.ascontiguousarray(np.clip(home_u + rng.normal(0.0, 0.2, (T, n, 29)), cr[:, 0], cr[:, 1]).astype(dtype))
