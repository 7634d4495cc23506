"""The C-ABI library loads and exports every entry point the header declares
(CPU test: no compute call is made)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


def declared_functions():
    names = []
    for header in sorted((REPO / "include").glob("*.h")):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(ts_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_scan_boundary():
    names = declared_functions()
    for required in ("ts_abi_version", "ts_last_error", "ts_scan_fwd", "ts_scan_workspace_bytes"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (bind to torch's HIP runtime first)

    from thetascan_amd import _lib

    if not _lib.library_path().exists():
        pytest.fail("libthetascan_hip.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.library_path()))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing
    lib.ts_abi_version.restype = ctypes.c_int
    assert lib.ts_abi_version() == 4
