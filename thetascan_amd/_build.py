"""Build the in-tree HIP library ``libthetascan_hip.so`` for gfx950.

The library is a plain C-ABI shared object (see ``include/thetascan_hip.h``)
compiled directly with ``hipcc``; no torch extension machinery is involved, so
the same artifact can be loaded from Python (ctypes) or linked from C/C++.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libthetascan_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = ("ts_scan.hip", "ts_features.hip", "ts_elementwise.hip")

HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Never let the compiler form packed-fp32 VALU ops on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build thetascan_amd")
    return found


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into ``thetascan_amd/libthetascan_hip.so``."""
    sources = [str(CSRC / name) for name in SOURCES if (CSRC / name).exists()]
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *sources, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errors = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{errors}")
    if verbose and errors.strip():
        print(errors, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
