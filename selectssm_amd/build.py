"""Build recipe for the in-tree HIP library ``selectssm_amd/libselectssm.so``.

The scan (csrc/selectssm.hip) and the causal conv (csrc/conv.hip), compiled
for gfx950 with hipcc into one shared library.  Packed-FP32 VALU
instructions are disabled for all device code (``-packed-fp32-ops``).
Run ``python -m selectssm_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SRCS = [os.path.join(PKG_DIR, "csrc", f) for f in ("selectssm.hip", "conv.hip")]
LIB = os.path.join(PKG_DIR, "libselectssm.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_DIR, "include"),
    "-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx",  # roctx ranges over the C-ABI calls
]


def hipcc_path() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def build(verbose: bool = False) -> str:
    """Compile ``libselectssm.so`` (always recompiles).  Returns its path."""
    tmp = LIB + ".tmp"
    cmd = [hipcc_path(), *HIPCC_FLAGS, "-o", tmp, *SRCS]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
