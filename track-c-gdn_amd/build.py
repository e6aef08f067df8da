"""Build recipe for libgdn_hip.so (all HIP sources under csrc/, gfx950 only).

Run as ``python -m`` or through ``__graft_entry__.build()``.  The library is
written in-tree next to this file so that it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libgdn_hip.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for every HIP translation unit.  MFMA
# accumulators stay in VGPRs (amdgpu-mfma-vgpr-form): kernels that run one
# wave per SIMD would otherwise get AGPR accumulators and a copy to VGPRs for
# every VALU touch of them.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def sources():
    return sorted(CSRC.glob("*.hip"))


def build_library(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip into ``libgdn_hip.so`` next to this file."""
    out = PKG_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC),
           *[str(s) for s in sources()], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    p = build_library(verbose="-v" in sys.argv)
    print(p)
