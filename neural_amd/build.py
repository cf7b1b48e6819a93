"""Compile the HIP sources of neural_amd/csrc into one C-ABI shared library for gfx950 (MI355X).

    python -m neural_amd.build            # -> neural_amd/_lib/libneural_amd.so

The library is built in-tree so that it travels with the repository snapshot; nothing is JIT-compiled at import time.
Every .hip file is compiled as its own object (parallel), then linked.  All device code is built with packed-fp32
instructions disabled (-target-feature -packed-fp32-ops): hipcc would otherwise form v_pk_{add,mul,fma}_f32 from
ordinary float code.  The first kernel arguments (up to 14 dwords) are preloaded into scalar registers at wave launch
(-amdgpu-kernarg-preload-count), so that a kernel's first dependent read is issued without a round trip for its
pointer; each kernel keeps the compiler's fallback prologue that loads them where the firmware does not preload.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libneural_amd.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16", "-Wno-unused-result",
         f"-I{os.path.join(os.path.dirname(HERE), 'include')}"]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _compile(src: str, obj: str) -> None:
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{r.stderr[-6000:]}")


def build(verbose: bool = True) -> str:
    """Compile every csrc/*.hip and link LIB_PATH.  Always recompiles (the build check is meant to compile)."""
    os.makedirs(OUT_DIR, exist_ok=True)
    objs = []
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        futs = []
        for s in srcs:
            o = os.path.join(OUT_DIR, os.path.basename(s) + ".o")
            objs.append(o)
            futs.append(ex.submit(_compile, s, o))
        for f in futs:
            f.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)
    for o in objs:
        os.remove(o)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
