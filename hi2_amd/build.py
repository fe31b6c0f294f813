"""Build ``libhi2x.so`` (the gfx950 HIP library behind the C ABI in include/hi2x.h).

    python -m hi2_amd.build          # or hi2_amd.build.build()

Flags: -O3, no FP contraction (the reference rounds every product and sum
separately), IEEE-correct fp32 division and square root, no packed-fp32 code
generation, gfx950 only.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libhi2x.so")
SOURCES = ["api.hip", "gptq.hip", "ladder.hip", "format.hip", "hessian.hip", "chol.hip",
           "refine.hip", "stats.hip", "qad.hip"]
ARCH = "gfx950"

OBJDIR = os.path.join(os.path.dirname(HERE), "_build")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd: list[str]) -> tuple[int, str]:
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    return r.returncode, out


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every HIP source into ``hi2_amd/libhi2x.so`` (always recompiles): one
    object per source, compiled in parallel under ``_build/``, then one link."""
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[hipcc(), *FLAGS, "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, min(os.cpu_count() or 1, 16)))
    with ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(_run, cmds))
    for cmd, (rc, out) in zip(cmds, results):
        if verbose:
            print(" ".join(cmd), flush=True)
            if out.strip():
                print(out)
        if rc != 0:
            raise RuntimeError(f"hipcc failed ({rc}) on {cmd[-3]}:\n{out}")
    tmp = LIB + ".tmp"
    rc, out = _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{out}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
