"""Build ``libhi2x.so`` (the gfx950 HIP library behind the C ABI in include/hi2x.h).

    python -m hi2_amd.build          # or hi2_amd.build.build()

Flags: -O3, no FP contraction (the reference rounds every product and sum
separately), IEEE-correct fp32 division and square root, no packed-fp32 code
generation, gfx950 only.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libhi2x.so")
SOURCES = ["api.hip", "gptq.hip", "ladder.hip", "format.hip", "hessian.hip", "chol.hip",
           "refine.hip", "stats.hip", "qad.hip"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into ``hi2_amd/libhi2x.so`` (always recompiles)."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
