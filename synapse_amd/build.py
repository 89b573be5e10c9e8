"""Build libsynapse_hip.so for gfx950 in-tree (hipcc; no JIT cache).

Every .hip file under csrc/ is compiled to an object in parallel, then linked
into ``synapse_amd/libsynapse_hip.so``.  The floating-point flags are part of
the parity contract: no FMA contraction (the reference rounds a*b and +c
separately unless it says @mulAdd), no fast-math, IEEE denormals, and packed
FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libsynapse_hip.so")
PT_LIB_PATH = os.path.join(HERE, "libsynapse_hip_pt.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, verbose: bool, bdir: str = BUILD_DIR, flags=None) -> str:
    obj = os.path.join(bdir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *(FLAGS if flags is None else flags), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, phase_timing: bool = False) -> str:
    """phase_timing: the instrumented profiling build (-DSYN_PHASE_TIMING:
    s_memtime / s_memrealtime stamps of the decode-step kernels, read back by
    the syn_hip_debug_* exports) into libsynapse_hip_pt.so, loaded only when
    SYN_HIP_LIBRARY names it."""
    bdir = BUILD_DIR + ("_pt" if phase_timing else "")
    out = PT_LIB_PATH if phase_timing else LIB_PATH
    flags = FLAGS + (["-DSYN_PHASE_TIMING"] if phase_timing else [])
    os.makedirs(bdir, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, bdir, flags), srcs))
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, phase_timing="--phase-timing" in sys.argv))
