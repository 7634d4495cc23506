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
    assert lib.ts_abi_version() == 17


def test_views_descriptor_validation_on_the_host():
    """ts_scan_views_workspace_bytes checks the descriptor without touching a
    GPU: unsupported view counts, dtypes and widths are refused with the
    reference's error kinds, and the workspace holds one set of segment
    summaries per view."""
    import torch  # noqa: F401

    from thetascan_amd import _lib

    if not _lib.library_path().exists():
        pytest.fail("libthetascan_hip.so is not built: run __graft_entry__.build()")
    lib = _lib.load()

    def ws(**kw):
        fields = dict(B=2, H=8, T=32768, dk=128, dv=64, dtype=_lib.dtype_code(torch.bfloat16), n_views=3, mass=1,
                      seg_chunks=0)
        fields.update(kw)
        desc = _lib.ScanViewsDesc(*fields.values())
        out = ctypes.c_size_t()
        return lib.ts_scan_views_workspace_bytes(ctypes.byref(desc), ctypes.byref(out)), out.value

    rc, nbytes = ws()
    assert rc == _lib.TS_OK
    # 16 (batch, head) lanes, 512 tiles -> 32 segments of 16 tiles, 31 summaries kept;
    # per segment: S [128][64] + u [64] + D [128] floats, plus one decay per segment
    nseg, nelem = 32, 128 * 64 + 64 + 128
    assert nbytes == 3 * (16 * nseg * nelem + 16 * nseg) * 4 + 256
    assert ws(n_views=4)[0] == _lib.TS_ERR_NOT_IMPLEMENTED
    assert ws(n_views=1)[0] == _lib.TS_ERR_NOT_IMPLEMENTED
    assert ws(dtype=_lib.dtype_code(torch.float32))[0] == _lib.TS_ERR_NOT_IMPLEMENTED
    assert ws(dv=72)[0] == _lib.TS_ERR_NOT_IMPLEMENTED
    assert ws(dk=136)[0] == _lib.TS_ERR_NOT_IMPLEMENTED
    assert ws(T=-1)[0] == _lib.TS_ERR_VALUE
    assert ws(T=64) == (_lib.TS_OK, 0)  # one segment: no summaries


def test_initial_state_rules_on_the_host():
    """An initial state needs a workspace even for one segment, and is refused
    together with kept segment states."""
    import torch  # noqa: F401

    from thetascan_amd import _lib

    lib = _lib.load()

    def ws(**kw):
        f = dict(B=1, H=2, T=50, dk=64, dv=64, dtype=0, retention=0, reverse=0, q_ext=0, k_ext=0, v_ext=0,
                 out_mode=0, out_scale=1.0, seg_chunks=0, want_final=0, value_split=0, states_in=0, init_state=0)
        f.update(kw)
        desc = _lib.ScanDesc(*f.values())
        out = ctypes.c_size_t()
        return lib.ts_scan_workspace_bytes(ctypes.byref(desc), ctypes.byref(out)), out.value

    assert ws() == (_lib.TS_OK, 0)  # one segment, nothing carried
    rc, nbytes = ws(init_state=1)
    assert rc == _lib.TS_OK and nbytes >= 2 * (64 * 64 + 64 + 64) * 4
    assert ws(init_state=1, states_in=1)[0] == _lib.TS_ERR_NOT_IMPLEMENTED


def test_retention_grad_refuses_slices_beyond_2_gib_on_the_host():
    """ts_retention_grad computes its tile offsets in 32-bit integers, so a
    (batch, head) slice that reaches 2 GiB or more is refused before any
    launch or workspace check (no device memory is touched: the pointers here
    are never dereferenced)."""
    import torch  # noqa: F401

    from thetascan_amd import _lib

    lib = _lib.load()
    desc = _lib.RetentionDesc(B=1, H=2, T=4096, dk=64, dv=64, dtype=_lib.dtype_code(torch.bfloat16), has_mass=0,
                              seg_tiles=0)

    def call(q_stride):
        fake = 1 << 20  # 16-byte aligned, never dereferenced on this path
        s = lambda st: _lib.Strided(fake, 0, 0, st)  # noqa: E731
        io = _lib.RetentionIO(s(q_stride), s(64), s(64), s(64), _lib.Strided(None, 0, 0, 0), fake)
        out = ctypes.c_void_p(fake)
        return lib.ts_retention_grad(ctypes.byref(desc), ctypes.byref(io), out, None, 0, None)

    # 4096 + 64 + 64 rows of 262144 bf16 elements: 2.2 GB of reach
    assert call(262144) == _lib.TS_ERR_NOT_IMPLEMENTED
    assert b"2 GiB" in lib.ts_last_error()
    # an in-range slice passes the span check and stops at the missing workspace
    assert call(64) == _lib.TS_ERR_VALUE
    assert b"workspace" in lib.ts_last_error()
