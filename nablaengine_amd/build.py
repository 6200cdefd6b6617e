"""Build the HIP library libnablaengine_g1.so in-tree for gfx950 (hipcc; one shared library, the C ABI of
include/nablaengine_g1.h). `python -m nablaengine_amd.build`."""
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libnablaengine_g1.so")
PROF_LIB = os.path.join(HERE, "libnablaengine_g1_prof.so")
SOURCES = ["g1_forward.hip", "g1_adjoint.hip", "g1_order.hip", "g1_kinematics.hip", "g1_diag.hip", "g1_capi.hip"]
ARCH = os.environ.get("NABLA_OFFLOAD_ARCH", "gfx950")
# packed FP32 instructions off (-packed-fp32-ops): the kernels are written for scalar FP32. Warnings that mark
# undefined behaviour the optimizer exploits (a non-void function falling off its end becomes unreachable code, and a
# kernel then runs into whatever follows) are errors. Machine LICM off: the kernels hold one world per wave at the
# 256-VGPR limit, and values it hoists out of the substep and Newton loops are spilled to scratch inside them.
FLAGS = ["-O3", f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-shared", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-ffp-contract=fast", "-mllvm", "-disable-machine-licm",
         "-Wno-unused-command-line-argument", "-Werror=return-type",
         "-Werror=uninitialized", "-Werror=sometimes-uninitialized", "-Werror=array-bounds"]


def build(verbose=False, profile=False):
    """Compile every HIP source into the library (a temporary file renamed into place: a running process that
    has the old library loaded keeps it). profile=True builds libnablaengine_g1_prof.so with the phase counters
    (-DG1_PROFILE), a measurement build."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    target = PROF_LIB if profile else LIB
    fd, tmp = tempfile.mkstemp(prefix="libnablaengine_g1.", suffix=".so.tmp", dir=HERE)
    os.close(fd)
    cmd = [hipcc] + FLAGS + (["-DG1_PROFILE"] if profile else []) + ["-o", tmp] + [os.path.join(CSRC, s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd))
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        os.unlink(tmp)
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode})")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    print(build(verbose=True, profile="--profile" in sys.argv))
