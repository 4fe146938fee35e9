"""Builds the HIP sampler library in-tree for gfx950 (no JIT cache, no pip install).

The kernels live in several translation units (the C ABI and small kernels in
sampler.hip; k_scan, k_finish per dtype and k_lmhead in their own files), compiled
to objects in parallel and linked into one shared library."""

from __future__ import annotations

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG_ROOT = os.path.dirname(_HERE)                       # full-inference-engine_amd/
_REPO = os.path.dirname(_PKG_ROOT)
CSRC = os.path.join(_PKG_ROOT, "csrc")
INCLUDE = os.path.join(_REPO, "include")
OUT = os.path.join(_HERE, "_native", "libfie_sampler.so")
OBJ_DIR = os.path.join(_HERE, "_native", "obj")

SOURCES = ("sampler.hip", "k_scan.hip", "k_finish_f32.hip", "k_finish_f16.hip", "k_finish_bf16.hip",
           "k_lmhead.hip")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # No compiler-introduced fusions: the canonical arithmetic is op-by-op IEEE.
    "-ffp-contract=off",
    # Packed fp32 VALU ops are disabled on this hardware pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

    def compile_one(src: str) -> str:
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", f"-I{INCLUDE}", f"-I{CSRC}", "-o", obj + ".tmp",
               os.path.join(CSRC, src)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(obj + ".tmp", obj)
        return obj

    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", OUT + ".tmp", *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
