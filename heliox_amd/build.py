"""Build the HIP library ``heliox_amd/libheliox_amd.so`` for gfx950.

Every source is compiled with hipcc; device code targets gfx950 only, with
fp contraction off (the reference host path is built with -ffp-contract=off)
and packed fp32 instructions disabled.  Objects go to ``heliox_amd/_build``.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libheliox_amd.so")
ARCH = os.environ.get("HELIOX_OFFLOAD_ARCH", "gfx950")

SOURCES = ["kernels.hip", "adjoint.hip", "learn.hip", "learn_runtime.cpp", "runtime.cpp", "schedule.cpp",
           "coredat.cpp", "h5out.cpp"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]
DEVICE = [f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if p and (os.path.isabs(p) and os.path.exists(p) or not os.path.isabs(p)):
            return p
    return "hipcc"


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    # hipcc treats every source as HIP; give all of them the gfx950 target
    cmd = [_hipcc()] + COMMON + DEVICE + ["-x", "hip"]
    cmd += ["-I", os.path.join(HERE, "..", "include"), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name; that warning is expected
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def sources() -> list:
    """The library's sources, with every mechanism plugin under csrc/mechs/."""
    plugins = sorted(os.path.join("mechs", f) for f in os.listdir(os.path.join(CSRC, "mechs")) if f.endswith(".hip"))
    return SOURCES + plugins


def build(verbose: bool = True) -> str:
    os.makedirs(os.path.join(BUILD, "mechs"), exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp] + objs + ["-ldl"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
