"""ts_scan_fwd_noalloc: the scan entry point that allocates nothing (GPU tests).

It runs the kernels of ts_scan_fwd with the segment summaries in the
library's own per-GPU scratch buffer.  Called through the C ABI, two calls in a
row (the second smaller, so it reuses the buffer the first one filled) must
give exactly ts_scan_fwd's outputs and final states; scans whose workspace
exceeds the buffer, and kept segment states, are refused on the host.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from tests.conftest import rel_err
from oracle import scans as oracle

pytestmark = pytest.mark.gpu


def _desc(B, H, T, dk, dv, dtype, **kw):
    from thetascan_amd import _lib

    f = dict(B=B, H=H, T=T, dk=dk, dv=dv, dtype=_lib.dtype_code(dtype), retention=_lib.RET_NONE, reverse=0,
             q_ext=_lib.EXT_NONE, k_ext=_lib.EXT_NONE, v_ext=_lib.EXT_NONE, out_mode=_lib.OUT_STORE, out_scale=1.0,
             seg_chunks=0, want_final=0, value_split=0, states_in=0, init_state=0)
    f.update(kw)
    return _lib.ScanDesc(*f.values())


def _case(cuda, B, H, T, D, dtype, kind, seed):
    """Inputs and one scan's io (outputs freshly allocated and poisoned)."""
    from thetascan_amd import _lib

    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, T, D, generator=g).to(cuda, dtype) for _ in range(3))
    la = torch.log(torch.rand(H, generator=g) * 0.099 + 0.9).to(cuda)
    dec = (-torch.rand(B, H, T, generator=g) * 0.1).to(cuda)
    ret = {"none": _lib.RET_NONE, "static": _lib.RET_STATIC, "stream": _lib.RET_STREAM}[kind]
    desc = _desc(B, H, T, D, D, dtype, retention=ret, v_ext=_lib.EXT_ONES, want_final=1)
    return q, k, v, la, dec, desc


def _run(lib, cuda, desc, q, k, v, la, dec, noalloc):
    from thetascan_amd import _lib

    B, H, T, D = q.shape
    out = torch.full((B, H, T, D), float("nan"), dtype=q.dtype, device=cuda)
    mass = torch.full((B, H, T), float("nan"), dtype=torch.float32, device=cuda)
    dk_pad, dv_pad = ctypes.c_int32(), ctypes.c_int32()
    assert lib.ts_scan_layout(ctypes.byref(desc), ctypes.byref(dk_pad), ctypes.byref(dv_pad), None) == 0
    final = torch.full((B * H, dk_pad.value, dv_pad.value), float("nan"), dtype=torch.float32, device=cuda)
    io = _lib.ScanIO(_lib.strided(q), _lib.strided(k), _lib.strided(v), _lib.strided(None), _lib.strided(None),
                     _lib.strided(None), la.data_ptr() if desc.retention == _lib.RET_STATIC else None,
                     _lib.strided(dec) if desc.retention == _lib.RET_STREAM else _lib.strided(None),
                     _lib.strided(out), _lib.strided(mass), final.data_ptr(), None)
    stream = _lib.stream_handle(cuda)
    if noalloc:
        rc = lib.ts_scan_fwd_noalloc(ctypes.byref(desc), ctypes.byref(io), stream)
    else:
        nbytes = ctypes.c_size_t()
        assert lib.ts_scan_workspace_bytes(ctypes.byref(desc), ctypes.byref(nbytes)) == 0
        ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=cuda)
        rc = lib.ts_scan_fwd(ctypes.byref(desc), ctypes.byref(io), ws.data_ptr(), nbytes.value, stream)
    assert rc == 0, lib.ts_last_error().decode()
    torch.cuda.synchronize()
    return out, mass, final


def test_noalloc_scan_equals_the_workspace_scan(cuda):
    """Two calls in a row, the second smaller: outputs, key masses and final
    states equal ts_scan_fwd's bit for bit, and match the float64 recurrence."""
    from thetascan_amd import _lib

    lib = _lib.load()
    cases = [
        (cuda, 8, 8, 4096, 64, torch.bfloat16, "none", 1),    # the benchmarked scan: 8 segments per (b, h)
        (cuda, 1, 3, 700, 64, torch.float32, "stream", 2),    # smaller, per-token retention
    ]
    for case in cases:
        print(f"noalloc case {case[1:]}", flush=True)
        q, k, v, la, dec, desc = _case(*case)
        got = _run(lib, cuda, desc, q, k, v, la, dec, noalloc=True)
        ref = _run(lib, cuda, desc, q, k, v, la, dec, noalloc=False)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), case[1:]
        if q.dtype == torch.float32:
            # and the result is the scan: outputs and key masses of one head against the recurrence
            unit = torch.cat([v[:1, :1], torch.ones_like(v[:1, :1, :, :1])], dim=-1).double().cpu()
            decay = None
            if desc.retention == _lib.RET_STREAM:
                decay = dec[:1, :1].double().cpu().unsqueeze(-1)
            ref64 = oracle.linattn_chunk(q[:1, :1].double().cpu(), k[:1, :1].double().cpu(), unit, decay)
            assert rel_err(got[0][:1, :1], ref64[..., :-1]) < 1e-3
            assert rel_err(got[1][:1, :1], ref64[..., -1]) < 1e-3


def test_noalloc_scan_refuses_what_it_cannot_hold(cuda):
    """A workspace above the scratch maximum and kept segment states are
    refused on the host (no kernel is launched)."""
    from thetascan_amd import _lib

    lib = _lib.load()
    big = _desc(64, 16, 32768, 128, 128, torch.bfloat16, want_final=1)
    nbytes = ctypes.c_size_t()
    assert lib.ts_scan_workspace_bytes(ctypes.byref(big), ctypes.byref(nbytes)) == 0
    assert nbytes.value > 32 * 1024 * 1024
    io = _lib.ScanIO()
    assert lib.ts_scan_fwd_noalloc(ctypes.byref(big), ctypes.byref(io), _lib.stream_handle(cuda)) == _lib.TS_ERR_VALUE
    assert b"scratch" in lib.ts_last_error()
    kept = _desc(2, 2, 1000, 64, 64, torch.bfloat16, states_in=1)
    assert lib.ts_scan_fwd_noalloc(ctypes.byref(kept), ctypes.byref(io),
                                   _lib.stream_handle(cuda)) == _lib.TS_ERR_NOT_IMPLEMENTED


def test_noalloc_scan_replays_inside_a_graph(cuda):
    """After one eager call on the device (which looks up the scratch address
    and sets the kernels' LDS limits), a ts_scan_fwd_noalloc call captured in
    a graph replays, twice, to exactly ts_scan_fwd's outputs and final states;
    the inputs change between the replays, with eager work and a
    synchronization in between."""
    from thetascan_amd import _lib

    lib = _lib.load()
    B, H, T, D = 2, 4, 1300, 64
    q, k, v, la, dec, desc = _case(cuda, B, H, T, D, torch.bfloat16, "static", 3)
    _run(lib, cuda, desc, q, k, v, la, dec, noalloc=True)
    out = torch.empty(B, H, T, D, dtype=q.dtype, device=cuda)
    mass = torch.empty(B, H, T, dtype=torch.float32, device=cuda)
    dk_pad, dv_pad = ctypes.c_int32(), ctypes.c_int32()
    assert lib.ts_scan_layout(ctypes.byref(desc), ctypes.byref(dk_pad), ctypes.byref(dv_pad), None) == 0
    final = torch.empty(B * H, dk_pad.value, dv_pad.value, dtype=torch.float32, device=cuda)
    io = _lib.ScanIO(_lib.strided(q), _lib.strided(k), _lib.strided(v), _lib.strided(None), _lib.strided(None),
                     _lib.strided(None), la.data_ptr(), _lib.strided(None),
                     _lib.strided(out), _lib.strided(mass), final.data_ptr(), None)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.ts_scan_fwd_noalloc(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(cuda))
    assert rc == 0, lib.ts_last_error().decode()
    g = torch.Generator().manual_seed(4)
    for replay in range(2):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g).to(cuda, t.dtype))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _run(lib, cuda, desc, q, k, v, la, dec, noalloc=False)
        print(f"noalloc graph replay {replay}", flush=True)
        for a, b in zip((out, mass, final), ref):
            assert torch.equal(a, b), replay
