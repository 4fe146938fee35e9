"""Builds the HIP sampler library in-tree for gfx950 (no JIT cache, no pip install)."""

from __future__ import annotations

import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG_ROOT = os.path.dirname(_HERE)                       # full-inference-engine_amd/
_REPO = os.path.dirname(_PKG_ROOT)
CSRC = os.path.join(_PKG_ROOT, "csrc")
INCLUDE = os.path.join(_REPO, "include")
OUT = os.path.join(_HERE, "_native", "libfie_sampler.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # No compiler-introduced fusions: the canonical arithmetic is op-by-op IEEE.
    "-ffp-contract=off",
    # Packed fp32 VALU ops are disabled on this hardware pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    cmd = [hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-o", OUT + ".tmp",
           os.path.join(CSRC, "sampler.hip")]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
