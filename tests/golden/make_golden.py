"""Write the golden fixtures under tests/golden/ from the reference's committed data files (run in the build
container, where /root/reference exists; the fixtures are committed, so tests never read the reference).

Every array is data the reference's own checks hold (MuJoCo C float64 truth and the benchmark corpora), subsetted:
- truth_<corpus>.npz (mf_s0..mf_s3): the 64 `check_index` states' inputs (float32 as in the corpus) and MuJoCo C
  float64 outputs `check_out` (qpos' 36 | qvel' 35); model_flags / labels of those states
  (benchmarks/data/truth/README.md, benchmarks/bench/truth/fdlib.py model_job);
- grad_<corpus>.npz (mf_s0, mf_s1): the sampled gradient states: inputs, the 3 stored output cotangents, MuJoCo C
  FD VJPs `fd_vjp` (h = 1e-6) and `fd_vjp_floor` (h = 1e-7), validity bits `bad`, groups G0/G4/G5/G6, outputs `out`;
  all 64 G0 states' full 71 x 99 step Jacobian `jacobian` (float32) with `jac_index` and `jacobian_dcol`;
- mjw_<corpus>.npz (mf_s0): MuJoCo Warp 3.17 float32 contacts at the input state (`con`: pair, dist, pos[3],
  normal[3]) and per-substep counts for the first 512 states (fixtures/mjlab/mjw317_mf_s0.npz);
- corpus_mf_s0.npz: the inputs of all 4096 states of the benchmark corpus mf_s0 (benchmarks/data/mf_s0.npz), the
  states the reference's published timings are measured on (docs/results/paper_rtx6000/paper_bench.md:91-92), for
  bench.py's corpus line.
"""
import os
import sys

import numpy as np

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.dirname(os.path.abspath(__file__))
INPUTS = ("qpos", "qvel", "qacc_warmstart", "ctrl", "friction", "com")


def main():
    data = os.path.join(REF, "benchmarks", "data")
    for cname in ("mf_s0", "mf_s1", "mf_s2", "mf_s3"):
        c = np.load(os.path.join(data, cname + ".npz"))
        t = np.load(os.path.join(data, "truth", cname + ".npz"))
        ix = t["check_index"]
        np.savez_compressed(os.path.join(OUT, f"truth_{cname}.npz"), index=ix, check_out=t["check_out"],
                            model_flags=t["model_flags"][ix], labels=t["labels"][ix],
                            **{k: c[k][ix] for k in INPUTS})
        if cname in ("mf_s0", "mf_s1"):
            gi = t["index"]
            ji = t["jac_index"]  # every Jacobian the truth holds (64 G0 states)
            extra = dict(jac_index=ji, jacobian=t["jacobian"], jacobian_dcol=t["jacobian_dcol"])
            np.savez_compressed(os.path.join(OUT, f"grad_{cname}.npz"), index=gi, out=t["out"], fd_vjp=t["fd_vjp"],
                                fd_vjp_floor=t["fd_vjp_floor"], bad=t["bad"], model_flags=t["model_flags"][gi],
                                cot_qpos=c["cot_qpos"][gi], cot_qvel=c["cot_qvel"][gi],
                                **{g: t["group_" + g] for g in ("G0", "G4", "G5", "G6")},
                                **{k: c[k][gi] for k in INPUTS}, **extra,
                                **{"jac_" + k: c[k][gi[ji]] for k in INPUTS})  # jac_index: positions into index
    c = np.load(os.path.join(data, "mf_s0.npz"))
    np.savez_compressed(os.path.join(OUT, "corpus_mf_s0.npz"), **{k: c[k] for k in INPUTS})
    m = np.load(os.path.join(REF, "fixtures", "mjlab", "mjw317_mf_s0.npz"))
    c = np.load(os.path.join(data, "mf_s0.npz"))
    n = 512
    np.savez_compressed(os.path.join(OUT, "mjw_mf_s0.npz"), con=m["con"][:n], con_count=m["con_count"][:n],
                        ncon=m["ncon"][:n], nefc=m["nefc"][:n], out_qpos=m["out_qpos"][:n],
                        out_qvel=m["out_qvel"][:n], **{k: c[k][:n] for k in INPUTS})


if __name__ == "__main__":
    main()
