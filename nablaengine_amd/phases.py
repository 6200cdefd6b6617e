"""Per-phase cycle profile of the forward and the adjoint, from the profile build (libnablaengine_g1_prof.so: built
by `python -m nablaengine_amd.build --profile`, phase counters compiled in, never loaded by the product path).

    python -m nablaengine_amd.phases [worlds]

runs `worlds` (default 4096) seeded config-1 worlds through a forward step and a taped forward plus its adjoint, reads
the per-world phase cycles (dk_prof_read / dk_prof_read_adj: s_memtime cycles summed over the substeps, and each
world's start and end on the 100 MHz clock) and prints, per kernel, the mean cycles per world-step of each phase and
its share, for all worlds and for the heaviest 1%.
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NPHASE = 27  # the profile build's counters per world

# forward: phase slots (g1_device.h PH_*) grouped as the cycles they measure
FWD_GROUPS = {
    "smooth dynamics": [0, 23, 24, 25, 26], "collision": [1], "rows": [2], "Newton set-up": [3],
    "Hessian": [4, 17, 18, 19], "factorization of H": [5], "solves": [6], "line search": [7, 15, 16],
    "update": [8], "gradient": [9], "implicitfast": [10], "tape": [11],
}
FWD_COUNTS = {"Newton iterations": 12, "line-search evaluations": 13, "factorizations with self-contact fill": 14}
ADJ_GROUPS = {  # g1_adjoint.hip AP_*
    "record": [0], "poses": [1], "solves": [2], "twists": [3], "contacts": [4], "per-body wrench sums": [5],
    "body forces": [6], "dof terms": [7], "subtree sums": [10],
}


def _report(name, out, groups, counts=None):
    cyc = np.stack([out[:, ix].astype(np.float64).sum(1) for ix in groups.values()], 1)
    tot = cyc.sum(1)
    dur = (out[:, 21 if counts else 9].astype(np.int64) - out[:, 20 if counts else 8].astype(np.int64)) / 100.0
    for label, sel in (("all worlds", np.ones(len(tot), bool)), ("heaviest 1%", tot >= np.percentile(tot, 99))):
        t = tot[sel].mean()
        print(f"{name}, {label} ({sel.sum()}): {t:,.0f} cycles per world-step, duration {dur[sel].mean():.1f} us")
        for (g, _), c in zip(groups.items(), cyc[sel].mean(0)):
            print(f"  {g:40s} {c:12,.0f}  {100 * c / t:5.1f}%")
        for g, ix in (counts or {}).items():
            print(f"  {g:40s} {out[sel, ix].astype(np.float64).mean():12.1f}")


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    B = int(argv[0]) if argv else 4096
    os.environ.setdefault("NABLA_G1_LIB", os.path.join(HERE, "libnablaengine_g1_prof.so"))
    import torch
    from nablaengine_amd import synthetic, torch_ffi
    torch_ffi.init(0)
    lib = torch_ffi.load_library()
    lib.dk_prof_read.argtypes = lib.dk_prof_read_adj.argtypes = [ctypes.c_void_p, ctypes.c_int]
    st = synthetic.states(B, config=1)
    args = [torch.from_numpy(st[k]).cuda() for k in ("qpos", "qvel", "warm", "ctrl", "friction", "com")]
    cq, cv = (torch.from_numpy(x).cuda() for x in synthetic.cotangents(B))
    out = np.zeros((B, NPHASE), np.uint64)
    torch_ffi.forward(*args)
    torch.cuda.synchronize()
    if lib.dk_prof_read(ctypes.c_void_p(out.ctypes.data), B) != 0:
        raise RuntimeError(f"{os.environ['NABLA_G1_LIB']} is not a profile build")
    _report("k_forward", out, FWD_GROUPS, FWD_COUNTS)
    r = torch_ffi.forward(*args, tape=True)
    torch_ffi.backward(r[4], args[4], args[5], cq, cv)
    torch.cuda.synchronize()
    if lib.dk_prof_read_adj(ctypes.c_void_p(out.ctypes.data), B) != 0:
        raise RuntimeError("the adjoint's phase counters could not be read")
    _report("k_adjoint", out, ADJ_GROUPS)


if __name__ == "__main__":
    main()
