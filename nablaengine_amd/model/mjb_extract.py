"""Extract the mjlab Unitree G1 model constants from MuJoCo's binary model file, without MuJoCo.

The reference builds its kernels from a live ``mujoco.MjModel`` (``g1_engine/source.py:28-77`` ``constants``,
``g1_engine/step.py:123-152`` ``pair_constants``, ``step.py:2286-2295`` ``extra_constants``). MuJoCo is not available
here, so this script reads ``fixtures/mjlab/g1_train.mjb`` (MuJoCo 3.17.0, sha256 757b0997...) directly and writes
the constants the engine needs as a C header (``g1_model.h``, compiled into the HIP kernels and into the float64 CPU
oracle) and as JSON (``g1_model.json``, read by the Python side).

File layout. ``mj_saveModel`` writes, unaligned and in order: a 5-int header ``{54321, sizeof(mjtNum)=8, nsize=98,
version=3017000, npointer=485}``; 98 int64 sizes; the ``mjOption``, ``mjVisual`` and ``mjStatistic`` structs; then the
485 arrays of ``mjxmacro.h``'s MJMODEL_POINTERS, each ``nrow * ncol`` elements of its C type. The byte offsets below
were found by walking that order array by array and checking every array's contents (tree structure, unit
quaternions, the sole capsules and pair parameters listed in ``fixtures/mjlab/README.md:22-92``); the walk is
re-checked by the assertions in :func:`extract`. The file's sha256 is checked first: the offsets hold for this one
file only.

Run: ``python -m nablaengine_amd.model.mjb_extract [path/to/g1_train.mjb]`` (default: the reference checkout).
"""

import hashlib
import json
import math
import os
import struct
import sys

import numpy as np

MJB_SHA256 = "757b0997d992073b645732a1daaeab92587f00e29691b93aa76094a3f02ef379"
DEFAULT_MJB = "/root/reference/fixtures/mjlab/g1_train.mjb"
HERE = os.path.dirname(os.path.abspath(__file__))

NQ, NV, NU, NBODY, NJNT, NGEOM, NPAIR, NKEY = 36, 35, 29, 31, 30, 34, 502, 2

# (name, C type, count, byte offset) of every array the engine reads
FIELDS = [
    ("opt_timestep", "d", 1, 804), ("opt_impratio", "d", 1, 812), ("opt_tolerance", "d", 1, 820),
    ("opt_gravity", "d", 3, 860), ("stat_meaninertia", "d", 1, 1740),
    ("qpos0", "d", NQ, 1799),
    ("body_parentid", "i", NBODY, 2375), ("body_jntnum", "i", NBODY, 2871), ("body_jntadr", "i", NBODY, 2995),
    ("body_dofnum", "i", NBODY, 3119), ("body_dofadr", "i", NBODY, 3243),
    ("body_pos", "d", NBODY * 3, 3801), ("body_quat", "d", NBODY * 4, 4545), ("body_ipos", "d", NBODY * 3, 5537),
    ("body_iquat", "d", NBODY * 4, 6281), ("body_mass", "d", NBODY, 7273), ("body_subtreemass", "d", NBODY, 7521),
    ("body_inertia", "d", NBODY * 3, 7769), ("body_invweight0", "d", NBODY * 2, 8513),
    ("jnt_type", "i", NJNT, 10189), ("jnt_qposadr", "i", NJNT, 10309), ("jnt_dofadr", "i", NJNT, 10429),
    ("jnt_bodyid", "i", NJNT, 10549), ("jnt_limited", "B", NJNT, 10909), ("jnt_actfrclimited", "B", NJNT, 10939),
    ("jnt_solref", "d", NJNT * 2, 10999), ("jnt_solimp", "d", NJNT * 5, 11479), ("jnt_pos", "d", NJNT * 3, 12679),
    ("jnt_axis", "d", NJNT * 3, 13399), ("jnt_range", "d", NJNT * 2, 14839), ("jnt_actfrcrange", "d", NJNT * 2, 15319),
    ("jnt_margin", "d", NJNT, 15799),
    ("dof_bodyid", "i", NV, 16039), ("dof_jntid", "i", NV, 16179), ("dof_parentid", "i", NV, 16319),
    ("dof_Madr", "i", NV, 16599), ("dof_solref", "d", NV * 2, 16879), ("dof_solimp", "d", NV * 5, 17439),
    ("dof_frictionloss", "d", NV, 18839), ("dof_armature", "d", NV, 19119), ("dof_damping", "d", NV, 19399),
    ("dof_invweight0", "d", NV, 20239), ("dof_M0", "d", NV, 20519),
    ("geom_type", "i", NGEOM, 21099), ("geom_contype", "i", NGEOM, 21235), ("geom_conaffinity", "i", NGEOM, 21371),
    ("geom_condim", "i", NGEOM, 21507), ("geom_bodyid", "i", NGEOM, 21643), ("geom_size", "d", NGEOM * 3, 24669),
    ("geom_rbound", "d", NGEOM, 27117), ("geom_pos", "d", NGEOM * 3, 27389), ("geom_quat", "d", NGEOM * 4, 28205),
    ("geom_friction", "d", NGEOM * 3, 29293), ("geom_margin", "d", NGEOM, 30109), ("geom_gap", "d", NGEOM, 30381),
    ("pair_dim", "i", NPAIR, 37792), ("pair_geom1", "i", NPAIR, 39800), ("pair_geom2", "i", NPAIR, 41808),
    ("pair_solref", "d", NPAIR * 2, 45824), ("pair_solimp", "d", NPAIR * 5, 61888), ("pair_margin", "d", NPAIR, 81968),
    ("pair_gap", "d", NPAIR, 85984), ("pair_friction", "d", NPAIR * 5, 94016),
    ("actuator_trntype", "i", NU, 114096), ("actuator_dyntype", "i", NU, 114212),
    ("actuator_gaintype", "i", NU, 114328), ("actuator_biastype", "i", NU, 114444),
    ("actuator_trnid", "i", NU * 2, 115372), ("actuator_gainprm", "d", NU * 10, 118156),
    ("actuator_biasprm", "d", NU * 10, 120476), ("actuator_ctrlrange", "d", NU * 2, 125580),
    ("key_time", "d", NKEY, 129820), ("key_qpos", "d", NKEY * NQ, 129836), ("key_qvel", "d", NKEY * NV, 130412),
    ("key_ctrl", "d", NKEY * NU, 130972),
]
NAMES_OFFSET = 134074  # the names buffer: bodies, joints, geoms, ... (null separated)

GEOM_PLANE, GEOM_SPHERE, GEOM_CAPSULE = 0, 2, 3  # mjtGeom
JNT_FREE, JNT_HINGE = 0, 3  # mjtJoint
FOOT_PAIRS = [5, 6, 7, 8, 9, 10, 11, 16, 17, 18, 19, 20, 21, 22]  # fixtures/mjlab/g1_meta.json foot_pairs
TORSO_NAME = "torso_link"  # g1_meta.json torso_body


def read_fields(buf):
    out = {}
    for name, t, n, off in FIELDS:
        size = struct.calcsize("<" + t)
        out[name] = np.array(struct.unpack("<%d%s" % (n, t), buf[off:off + n * size]))
    return out


def body_names(buf):
    names = buf[NAMES_OFFSET:NAMES_OFFSET + 4096].split(b"\x00")
    return [n.decode() for n in names[:NBODY]]


def _unit_rows(x, w):
    r = x.reshape(-1, w)
    return np.allclose(np.linalg.norm(r, axis=1), 1.0, atol=1e-6)


def extract(path=DEFAULT_MJB):
    buf = open(path, "rb").read()
    sha = hashlib.sha256(buf).hexdigest()
    assert sha == MJB_SHA256, f"{path}: sha256 {sha}, the offsets are for {MJB_SHA256} only"
    hdr = struct.unpack("<5i", buf[:20])
    assert hdr == (54321, 8, 98, 3017000, 485), hdr
    sizes = struct.unpack("<98q", buf[20:20 + 98 * 8])
    assert sizes[:3] == (NQ, NV, NU) and sizes[6] == NBODY and sizes[11] == NJNT and sizes[17] == NGEOM
    assert sizes[57] == NPAIR and sizes[70] == NKEY and sizes[13] == 341  # nM: the tree's mass-matrix nonzeros
    f = read_fields(buf)
    bn = body_names(buf)
    # landmarks (fixtures/mjlab/README.md, g1_meta.json): every array below was located by these checks
    assert f["opt_timestep"][0] == 0.005 and tuple(f["opt_gravity"]) == (0.0, 0.0, -9.81)
    assert tuple(f["body_parentid"][:8]) == (0, 0, 1, 2, 3, 4, 5, 6)
    assert _unit_rows(f["body_quat"], 4) and _unit_rows(f["body_iquat"], 4) and _unit_rows(f["geom_quat"], 4)
    assert f["jnt_type"][0] == JNT_FREE and (f["jnt_type"][1:] == JNT_HINGE).all()
    assert (f["jnt_limited"][1:] == 1).all() and (f["jnt_actfrclimited"][1:] == 1).all()
    assert (f["geom_type"][[0, 1, 25]] == [GEOM_PLANE, GEOM_SPHERE, GEOM_SPHERE]).all()
    g = f["geom_size"].reshape(-1, 3)
    assert abs(g[6, 1] - 0.025005) < 1e-12 and abs(g[7, 1] - 0.0835) < 1e-12 and (g[6:13, 0] == 0.01).all()
    assert (f["pair_geom1"][:33] == 0).all() and (f["pair_geom2"][:33] == np.arange(1, 34)).all()
    assert (f["pair_margin"] == 0).all() and (f["pair_gap"] == 0).all()
    assert np.allclose(f["pair_solref"].reshape(-1, 2), [0.02, 1.0])
    assert np.allclose(f["pair_solimp"].reshape(-1, 5), [0.9, 0.95, 0.001, 0.5, 2.0])
    pf = f["pair_friction"].reshape(-1, 5)
    assert set(np.unique(pf[:, 0])) == {0.6, 1.0} and (pf[:, 0] == pf[:, 1]).all()
    kp = f["actuator_gainprm"].reshape(-1, 10)[:, 0]
    bp = f["actuator_biasprm"].reshape(-1, 10)
    arm = f["dof_armature"][6:]
    assert np.allclose(kp, arm * (2 * math.pi * 10) ** 2) and np.allclose(-bp[:, 1], kp)
    assert np.allclose(-bp[:, 2], 4 * arm * 2 * math.pi * 10)
    assert (f["actuator_trnid"].reshape(-1, 2)[:, 0] == np.arange(1, 30)).all()
    assert abs(f["key_qpos"][2] - 0.783675) < 1e-9 and bn[16] == TORSO_NAME and bn[0] == "world"
    assert abs(f["body_subtreemass"][0] - 33.3411) < 1e-3
    return f, bn


def derive(f, bn):
    """The engine's view of the model: tree arrays, actuator gains, collision tables (reference semantics:
    source.py:28-77 constants, step.py:123-152 pair_constants, step.py:2286-2295 extra_constants)."""
    par = f["body_parentid"]
    depth = [0] * NBODY
    for b in range(1, NBODY):
        depth[b] = depth[int(par[b])] + 1
    qadr, dadr, axis = [0] * NBODY, [0] * NBODY, [[0.0, 0.0, 0.0] for _ in range(NBODY)]
    jax = f["jnt_axis"].reshape(-1, 3)
    for b in range(2, NBODY):
        j = f["body_jntadr"][b]
        assert f["body_jntnum"][b] == 1 and f["jnt_type"][j] == JNT_HINGE
        assert not f["jnt_pos"].reshape(-1, 3)[j].any()
        qadr[b], dadr[b], axis[b] = int(f["jnt_qposadr"][j]), int(f["jnt_dofadr"][j]), list(jax[j])
    dofbody = [int(x) for x in f["dof_bodyid"]]
    assert dofbody[:6] == [1] * 6 and dofbody[6:] == list(range(2, NBODY))  # dof 6 + k on body 2 + k
    ancmask = []
    for b in range(NBODY):
        m, k = 0, b
        while k > 0:
            m |= 1 << k
            k = int(par[k])
        ancmask.append(m)
    kp = np.zeros(NV)
    kv = np.zeros(NV)
    frclim = np.full(NV, 1e30)
    gp = f["actuator_gainprm"].reshape(-1, 10)
    bp = f["actuator_biasprm"].reshape(-1, 10)
    afr = f["jnt_actfrcrange"].reshape(-1, 2)
    for a in range(NU):
        j = f["actuator_trnid"][2 * a]
        d = f["jnt_dofadr"][j]
        assert d == 6 + a and f["actuator_biastype"][a] == 1
        kp[d], kv[d] = gp[a, 0], -bp[a, 2]
        assert afr[j, 0] == -afr[j, 1]
        frclim[d] = afr[j, 1]
    jrange = np.zeros((NV, 2))
    jr = f["jnt_range"].reshape(-1, 2)
    for j in range(1, NJNT):
        jrange[f["jnt_dofadr"][j]] = jr[j]
    # collision geoms: every geom in some pair, model order; pairs with the lower geom type first (MuJoCo's collision
    # table order, step.py:135-137)
    gt = f["geom_type"]
    order = {GEOM_PLANE: 0, GEOM_SPHERE: 1, GEOM_CAPSULE: 2}
    pg1, pg2, pdim, pmu, pfoot = [], [], [], [], []
    pf = f["pair_friction"].reshape(-1, 5)
    for i in range(NPAIR):
        g1, g2 = int(f["pair_geom1"][i]), int(f["pair_geom2"][i])
        if order[int(gt[g1])] > order[int(gt[g2])]:
            g1, g2 = g2, g1
        pg1.append(g1)
        pg2.append(g2)
        pdim.append(int(f["pair_dim"][i]))
        pmu.append(float(pf[i, 0]))
        pfoot.append(int(i in FOOT_PAIRS))
    torso = bn.index(TORSO_NAME)
    home = 0  # key 0 is "home" (fixtures/mjlab/README.md: keyframes home, knees_bent)
    ctrlrange = f["actuator_ctrlrange"].reshape(-1, 2)
    return dict(
        nq=NQ, nv=NV, nu=NU, nbody=NBODY, ngeom=NGEOM, npair=NPAIR,
        timestep=float(f["opt_timestep"][0]), gravity=[float(x) for x in f["opt_gravity"]],
        impratio=float(f["opt_impratio"][0]), tolerance=float(f["opt_tolerance"][0]),
        meaninertia=float(f["stat_meaninertia"][0]),
        body_parent=[int(x) for x in par], body_depth=depth, body_qadr=qadr, body_dadr=dadr, body_axis=axis,
        body_pos=f["body_pos"].tolist(), body_quat=f["body_quat"].tolist(), body_ipos=f["body_ipos"].tolist(),
        body_iquat=f["body_iquat"].tolist(), body_mass=f["body_mass"].tolist(),
        body_inertia=f["body_inertia"].tolist(), body_invweight0=f["body_invweight0"].reshape(-1, 2)[:, 0].tolist(),
        body_ancmask=ancmask, body_names=bn, torso_body=torso,
        dof_body=dofbody, dof_armature=f["dof_armature"].tolist(), dof_invweight0=f["dof_invweight0"].tolist(),
        dof_frictionloss=f["dof_frictionloss"].tolist(),
        dof_kp=kp.tolist(), dof_kv=kv.tolist(), dof_frclim=frclim.tolist(), dof_range=jrange.ravel().tolist(),
        jnt_solref=f["jnt_solref"].reshape(-1, 2)[1].tolist(), jnt_solimp=f["jnt_solimp"].reshape(-1, 5)[1].tolist(),
        geom_type=[int(x) for x in gt], geom_body=[int(x) for x in f["geom_bodyid"]],
        geom_size=f["geom_size"].tolist(), geom_pos=f["geom_pos"].tolist(), geom_quat=f["geom_quat"].tolist(),
        geom_rbound=f["geom_rbound"].tolist(),
        pair_g1=pg1, pair_g2=pg2, pair_dim=pdim, pair_mu=pmu, pair_foot=pfoot, foot_pairs=FOOT_PAIRS,
        pair_solref=f["pair_solref"].reshape(-1, 2)[0].tolist(), pair_solimp=f["pair_solimp"].reshape(-1, 5)[0].tolist(),
        ctrlrange=ctrlrange.ravel().tolist(), jnt_range_full=f["jnt_range"].tolist(),
        key_home_qpos=f["key_qpos"][home * NQ:(home + 1) * NQ].tolist(),
        key_home_ctrl=f["key_ctrl"][home * NU:(home + 1) * NU].tolist(),
        qpos0=f["qpos0"].tolist(), maxdepth=max(depth),
    )


def _carr(ctype, name, vals):
    if ctype == "double":
        body = ", ".join(repr(float(v)) for v in vals)
    else:
        body = ", ".join(str(int(v)) for v in vals)
    return f"static constexpr {ctype} {name}[{len(vals)}] = {{{body}}};\n"


def write_header(d, path):
    """g1_model.h: the model as constexpr arrays (double; kernels convert to float at compile time)."""
    s = ["// Generated by nablaengine_amd/model/mjb_extract.py from fixtures/mjlab/g1_train.mjb (MuJoCo 3.17.0,\n"
         f"// sha256 {MJB_SHA256}). Do not edit.\n",
         "#pragma once\nnamespace g1 {\n"]
    for k in ("nq", "nv", "nu", "nbody", "ngeom", "npair", "torso_body", "maxdepth"):
        s.append(f"static constexpr int {k.upper()} = {d[k]};\n")
    for k in ("timestep", "impratio", "tolerance", "meaninertia"):
        s.append(f"static constexpr double {k.upper()} = {d[k]!r};\n")
    s.append(_carr("double", "GRAVITY", d["gravity"]))
    ints = ["body_parent", "body_depth", "body_qadr", "body_dadr", "body_ancmask", "dof_body", "geom_type",
            "geom_body", "pair_g1", "pair_g2", "pair_dim", "pair_foot"]
    for k in ints:
        ct = "unsigned" if k == "body_ancmask" else "int"
        s.append(_carr(ct, k.upper(), d[k]))
    dbls = ["body_axis", "body_pos", "body_quat", "body_ipos", "body_iquat", "body_mass", "body_inertia",
            "body_invweight0", "dof_armature", "dof_invweight0", "dof_kp", "dof_kv", "dof_frclim", "dof_range",
            "jnt_solref", "jnt_solimp", "geom_size", "geom_pos", "geom_quat", "geom_rbound", "pair_mu",
            "pair_solref", "pair_solimp", "ctrlrange", "key_home_qpos", "key_home_ctrl"]
    for k in dbls:
        v = np.asarray(d[k], np.float64).ravel()
        s.append(_carr("double", k.upper(), v))
    s.append("}  // namespace g1\n")
    open(path, "w").write("".join(s))


def main(argv):
    path = argv[1] if len(argv) > 1 else DEFAULT_MJB
    f, bn = extract(path)
    d = derive(f, bn)
    with open(os.path.join(HERE, "g1_model.json"), "w") as fh:
        json.dump(d, fh, indent=0)
    write_header(d, os.path.join(HERE, "..", "csrc", "g1_model.h"))
    print("wrote g1_model.json and csrc/g1_model.h")


if __name__ == "__main__":
    main(sys.argv)
