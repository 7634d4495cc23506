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
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libthetascan_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
ARCH = "gfx950"

SOURCES = ("ts_scan.hip", "ts_scan_views.hip", "ts_features.hip", "ts_elementwise.hip", "ts_maps.hip", "ts_gn.hip", "ts_memory.hip",
           "ts_retention.hip",
           "ts_contract.hip", "ts_readout.hip", "ts_anchor.hip", "ts_kmap.hip", "ts_gnact.hip", "ts_absmass.hip",
           "ts_rownorm.hip", "ts_rowglue.hip")

HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Never let the compiler form packed-fp32 VALU ops on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)
NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build thetascan_amd")
    return found


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    messages = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if NOISE not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{messages}")
    if verbose and messages.strip():
        print(messages, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source (in parallel) and link ``thetascan_amd/libthetascan_hip.so``."""
    sources = [CSRC / name for name in SOURCES if (CSRC / name).exists()]
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="thetascan_build_") as tmpdir:
        objects = [Path(tmpdir) / (src.stem + ".o") for src in sources]
        cmds = [[cc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
                for src, obj in zip(sources, objects)]
        with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
            for fut in [pool.submit(_run, cmd, verbose) for cmd in cmds]:
                fut.result()
        tmp = LIB_PATH.with_suffix(".so.tmp")
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
