"""Parity of the HIP scan kernels with the CPU oracle (GPU tests).

Mirrors the reference's scan tests (tests/test_scan_chunk.py:55-138, 236-301,
484-548): every retention form against the sequential oracle, ragged tiles,
multi-segment decomposition, exact causality by perturbation, gradients
(q, k, v and the retention) against float64 autograd through the oracle, and
the multi-view / key-mass variants.  Tolerances: rel 1e-3 for fp32 and rel
2e-2 for bf16 (max-abs error / max-abs oracle).
"""
from __future__ import annotations

import pytest
import torch

from oracle import scans as oracle
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2}


def _streams(B, H, T, Dk, Dv, seed=20260725, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, Dk, generator=g, dtype=dtype)
    k = torch.randn(B, H, T, Dk, generator=g, dtype=dtype)
    v = torch.randn(B, H, T, Dv, generator=g, dtype=dtype)
    return q, k, v


def _rounded(x, dtype):
    """Round to the kernel dtype and back, so the oracle sees the same inputs."""
    return x.to(dtype).to(torch.float64)


def _retention(kind, B, H, T, seed=11):
    g = torch.Generator().manual_seed(seed)
    if kind == "none":
        return None
    if kind == "static":
        return torch.log(torch.rand(H, generator=g, dtype=torch.float64) * 0.099 + 0.9)
    return -torch.rand(B, H, T, 1, generator=g, dtype=torch.float64) * 0.2


def _oracle_decay(ret, like):
    if ret is None:
        return None
    return oracle.as_stream(ret, like) if ret.ndim == 1 else ret


SHAPES = [
    (2, 3, 37, 5, 4),      # the reference's _streams fixture shape
    (1, 2, 64, 64, 64),    # exactly one tile
    (2, 2, 300, 64, 64),   # ragged, several tiles
    (1, 2, 260, 128, 64),  # wide keys
    (1, 1, 130, 64, 128),  # wide values
    (1, 2, 200, 72, 64),   # keys padded to 80: a 16-wide contraction tail
    (1, 1, 150, 136, 48),  # keys padded to 144, values narrower than a tile
    (1, 1, 1, 8, 8),       # a single token
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_matches_naive(cuda, dtype, kind, shape):
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = shape
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, Dk, Dv))
    ret = _retention(kind, B, H, T)
    expected = oracle.linattn_naive(q, k, v, _oracle_decay(ret, q))
    r_dev = None if ret is None else ret.to(cuda, torch.float32)
    actual = scan_hip.linattn_views(q.to(cuda, dtype), k.to(cuda, dtype), v.to(cuda, dtype), (r_dev,), 64)[0]
    assert actual.dtype == dtype and actual.shape == expected.shape
    assert rel_err(actual, expected) < TOL[dtype], (shape, kind, dtype)


@pytest.mark.parametrize("seg_chunks", [1, 2, 3, 7])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_segmented_decomposition_is_exact(cuda, seg_chunks, kind):
    """Any segmentation of the tile axis gives the same scan (fp32)."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T, Dk, Dv = 2, 2, 450, 64, 64
    q, k, v = _streams(B, H, T, Dk, Dv, dtype=torch.float32)
    ret = _retention(kind, B, H, T)
    expected = oracle.linattn_naive(q.double(), k.double(), v.double(), _oracle_decay(ret, q.double()))
    kw = {"retention": {"none": _lib.RET_NONE, "static": _lib.RET_STATIC, "stream": _lib.RET_STREAM}[kind]}
    if kind == "static":
        kw["log_alpha"] = ret.to(cuda, torch.float32)
    if kind == "stream":
        kw["decay"] = ret.to(cuda, torch.float32)
    out, _, _ = scan_hip.scan_launch(q.to(cuda), k.to(cuda), v.to(cuda), seg_chunks=seg_chunks, **kw)
    assert rel_err(out, expected) < 1e-4


@pytest.mark.parametrize("split,Dv", [(16, 64), (32, 64), (64, 64), (16, 40), (0, 72)])
@pytest.mark.parametrize("seg_chunks", [0, 1, 3])
@pytest.mark.parametrize("kind", ["none", "stream"])
def test_value_slices_are_exact(cuda, split, Dv, seg_chunks, kind):
    """Workgroups that carry only a slice of the value columns (and, with
    segments, their slice of the segment summaries) give the same scan, the
    key-mass column of slice 0 included; the last slice may be ragged."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T, Dk = 2, 3, 333, 64
    q, k, v = _streams(B, H, T, Dk, Dv, dtype=torch.float32, seed=11)
    ret = _retention(kind, B, H, T)
    vc = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1)
    expected = oracle.linattn_naive(q.double(), k.double(), vc.double(), _oracle_decay(ret, q.double()))
    kw = {"retention": _lib.RET_STREAM if kind == "stream" else _lib.RET_NONE}
    if kind == "stream":
        kw["decay"] = ret.to(cuda, torch.float32)
    out, mass, _ = scan_hip.scan_launch(q.to(cuda), k.to(cuda), v.to(cuda), v_ext="ones", want_ext_out=True,
                                        seg_chunks=seg_chunks, value_split=split, **kw)
    assert rel_err(out, expected[..., :Dv]) < 1e-4, (split, Dv, seg_chunks, kind)
    assert rel_err(mass, expected[..., Dv]) < 1e-4, (split, Dv, seg_chunks, kind)


@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
def test_kept_segment_states_are_exact(cuda, kind, reverse, dtype, D):
    """A scan that reads the segment states an earlier scan left in its
    workspace (states_in=1), or those of the swapped scan read transposed
    (states_in=2: keys and values exchanged), equals the scan computed from
    scratch.  This is how the backward's dq (dv) scan reuses the forward's
    (dk's) states.  At D = 128 both scans run in two 64-column value slices."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T = 2, 3, 700
    q, k, v, w = (x.to(cuda, dtype) for x in _streams(B, H, T, D, D, seed=21) + (_streams(B, H, T, D, D, seed=22)[0],))
    ret = _retention(kind, B, H, T)
    kw = {"retention": {"none": _lib.RET_NONE, "static": _lib.RET_STATIC, "stream": _lib.RET_STREAM}[kind],
          "reverse": reverse, "seg_chunks": 3}
    if kind == "static":
        kw["log_alpha"] = ret.to(cuda, torch.float32)
    if kind == "stream":
        kw["decay"] = ret.to(cuda, torch.float32)
    # forward-like scan scan(q, k, v) keeps its states
    ws = scan_hip.workspace_for(q, k, v, seg_chunks=3, retention=kw["retention"], reverse=reverse)
    assert ws is not None
    out, _, _ = scan_hip.scan_launch(q, k, v, workspace=ws, **kw)
    again, _, _ = scan_hip.scan_launch(q, k, v, workspace=ws, states_in=1, **kw)
    assert torch.equal(again, out)
    # swapped scan scan(w, v, k): keys v, values k -- its states are the transpose
    ref, _, _ = scan_hip.scan_launch(w, v, k, **kw)
    got, _, _ = scan_hip.scan_launch(w, v, k, workspace=ws, states_in=2, **kw)
    assert rel_err(got, ref) < (1e-5 if dtype == torch.float32 else 1e-2), (kind, reverse)


@pytest.mark.parametrize("reverse", [False, True])
def test_kept_segment_states_with_mass_columns(cuda, reverse):
    """The normalized read's pair: scan(q, k, v | ones) keeps its states, and
    the swapped scan(w, v, k) with a q ext array and unit k ext column reads
    them transposed, its key-side row u being the first scan's value-side
    sum of keys."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 3, 650, 64
    q, k, v = (x.to(cuda, torch.float32) for x in _streams(B, H, T, D, D, seed=31))
    w = _streams(B, H, T, D, D, seed=32)[0].to(cuda, torch.float32)
    we = torch.randn(B, H, T, generator=torch.Generator().manual_seed(4)).to(cuda)
    ws = scan_hip.workspace_for(q, k, v, seg_chunks=3, reverse=reverse, v_ext=True)
    scan_hip.scan_launch(q, k, v, v_ext="ones", want_ext_out=True, seg_chunks=3, reverse=reverse, workspace=ws)
    ref, _, _ = scan_hip.scan_launch(w, v, k, q_ext=we, k_ext="ones", seg_chunks=3, reverse=reverse)
    got, _, _ = scan_hip.scan_launch(w, v, k, q_ext=we, k_ext="ones", seg_chunks=3, reverse=reverse, workspace=ws,
                                     states_in=2)
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_reverse_scan_is_the_time_reversed_scan(cuda, kind):
    """The anti-causal mode used by the backward equals flipping time."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T, D = 1, 2, 200, 32
    q, k, v = _streams(B, H, T, D, D, dtype=torch.float32)
    ret = _retention(kind, B, H, T)
    # out_i = sum_{t>=i} w(t,i) <q_i, k_t> v_t  with w(t,i) = prod_{i<j<=t} a_j
    decay = _oracle_decay(ret, q.double())
    if decay is None:
        rdecay = None
    else:
        # reversed logical position s uses the decay of physical T - s (0 at s = 0)
        flipped = decay.flip(2)
        rdecay = torch.cat([torch.zeros_like(flipped[:, :, :1]), flipped[:, :, :-1]], dim=2)
    expected = oracle.linattn_naive(q.double().flip(2), k.double().flip(2), v.double().flip(2), rdecay).flip(2)
    kw = {"retention": {"none": _lib.RET_NONE, "static": _lib.RET_STATIC, "stream": _lib.RET_STREAM}[kind]}
    if kind == "static":
        kw["log_alpha"] = ret.to(cuda, torch.float32)
    if kind == "stream":
        kw["decay"] = ret.to(cuda, torch.float32)
    out, _, _ = scan_hip.scan_launch(q.to(cuda), k.to(cuda), v.to(cuda), reverse=True, seg_chunks=1, **kw)
    assert rel_err(out, expected) < 1e-4


def test_exact_causality_by_perturbation(cuda):
    """Adding to k, v at t >= cut leaves every output before cut bitwise unchanged
    (tests/test_scan_chunk.py:236-268)."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 2, 333, 64
    q, k, v = (x.to(cuda, torch.bfloat16) for x in _streams(B, H, T, D, D, dtype=torch.float32))
    la = torch.log(torch.tensor([0.9, 0.99], device=cuda))
    for cut in (1, 63, 64, 65, 200):
        k2, v2 = k.clone(), v.clone()
        k2[:, :, cut:] += 2.0
        v2[:, :, cut:] += 2.0
        for ret in (None, la):
            a = scan_hip.linattn_views(q, k, v, (ret,), 64)[0]
            b = scan_hip.linattn_views(q, k2, v2, (ret,), 64)[0]
            assert torch.equal(a[:, :, :cut], b[:, :, :cut]), cut


def test_deterministic_replay(cuda):
    from thetascan_amd._core.ops import scan_hip

    q, k, v = (x.to(cuda, torch.bfloat16) for x in _streams(2, 4, 1000, 64, 64, dtype=torch.float32))
    a = scan_hip.linattn_views(q, k, v, (None,), 64)[0]
    b = scan_hip.linattn_views(q, k, v, (None,), 64)[0]
    assert torch.equal(a, b)


def test_multi_view_matches_separate_views(cuda):
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 3, 150, 32
    q, k, v = (_rounded(x, torch.float32) for x in _streams(B, H, T, D, D))
    la = torch.log(torch.tensor([0.9, 0.5, 0.99], dtype=torch.float64))
    stream = _retention("stream", B, H, T)
    rets = (None, la, stream)
    outs = scan_hip.linattn_views(q.to(cuda, torch.float32), k.to(cuda, torch.float32),
                                  v.to(cuda, torch.float32), tuple(None if r is None else r.to(cuda, torch.float32) for r in rets))
    for out, ret in zip(outs, rets):
        assert rel_err(out, oracle.linattn_naive(q, k, v, _oracle_decay(ret, q))) < 1e-3


VIEW_SHAPES = [
    (2, 3, 700, 128, 64),  # the B-spline bank's widths, several segments, ragged last tile
    (1, 2, 1100, 64, 64),  # 64-wide keys
    (2, 2, 333, 40, 24),   # keys and values padded inside the tile
    (1, 1, 64, 128, 64),   # exactly one tile
    (1, 2, 5, 16, 8),      # a few tokens
]


@pytest.mark.parametrize("seg_chunks", [0, 3])
@pytest.mark.parametrize("mass", [False, True])
@pytest.mark.parametrize("n_views", [2, 3])
@pytest.mark.parametrize("shape", VIEW_SHAPES)
def test_views_scan_equals_one_view_scans(cuda, shape, n_views, mass, seg_chunks):
    """ts_scan_views_fwd (one pass, the score tile shared by every retention)
    gives each view exactly what ts_scan_fwd gives for that retention alone:
    bit for bit, for the plain sum and static retentions, with and without
    the key-mass column; and both match the float64 recurrence."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T, Dk, Dv = shape
    q, k, v = (_rounded(x, torch.bfloat16) for x in _streams(B, H, T, Dk, Dv, seed=41))
    if mass:
        q, k = q.abs(), k.abs()
    g = torch.Generator().manual_seed(5)
    rets = [None] + [torch.log(torch.rand(H, generator=g, dtype=torch.float64) * 0.099 + 0.9)
                     for _ in range(n_views - 1)]
    rets_dev = [None if r is None else r.to(cuda, torch.float32) for r in rets]
    qd, kd, vd = (x.to(cuda, torch.bfloat16) for x in (q, k, v))
    outs, masses = scan_hip.scan_views_launch(qd, kd, vd, rets_dev, mass=mass, seg_chunks=seg_chunks)
    assert (masses is not None) == mass
    for j, (r, r_dev) in enumerate(zip(rets, rets_dev)):
        kw = {"retention": _lib.RET_NONE} if r is None else {"retention": _lib.RET_STATIC, "log_alpha": r_dev}
        one, one_mass, _ = scan_hip.scan_launch(qd, kd, vd, v_ext="ones" if mass else None, want_ext_out=mass,
                                                seg_chunks=seg_chunks, **kw)
        assert torch.equal(outs[j], one), (shape, n_views, j)
        if mass:
            assert torch.equal(masses[j], one_mass), (shape, n_views, j)
        unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1) if mass else v
        expected = oracle.linattn_naive(q, k, unit, _oracle_decay(r, q))
        assert rel_err(outs[j], expected[..., :Dv]) < TOL[torch.bfloat16], (shape, j)
        if mass:
            assert rel_err(masses[j], expected[..., Dv]) < TOL[torch.bfloat16], (shape, j)


def test_views_scan_serves_the_bank_views(cuda):
    """linattn_views_mass with a plain and two static retentions (a two-rate
    recency bank) takes the one-pass kernel and matches separate views."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = 1, 2, 300, 128, 64
    q, k, v = (_rounded(x, torch.bfloat16).abs() for x in _streams(B, H, T, Dk, Dv, seed=43))
    rets = (None, torch.log(torch.tensor([0.9, 0.95], dtype=torch.float64)),
            torch.log(torch.tensor([0.999, 0.99], dtype=torch.float64)))
    rets_dev = tuple(None if r is None else r.to(cuda, torch.float32) for r in rets)
    qd, kd, vd = (x.to(cuda, torch.bfloat16) for x in (q, k, v))
    calls = []
    real = scan_hip.scan_views_launch

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    scan_hip.scan_views_launch = spy
    try:
        pairs = scan_hip.linattn_views_mass(qd, kd, vd, rets_dev)
    finally:
        scan_hip.scan_views_launch = real
    assert calls == [1]
    unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1)
    for (num, mass), r in zip(pairs, rets):
        expected = oracle.linattn_naive(q, k, unit, _oracle_decay(r, q))
        assert rel_err(num, expected[..., :Dv]) < TOL[torch.bfloat16]
        assert rel_err(mass, expected[..., Dv]) < TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mass_column_matches_unit_value_column(cuda, dtype):
    """linattn_views_mass == scan against cat([v, 1]) (engine.py:430-442)."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = 2, 2, 200, 64, 64
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, Dk, Dv))
    q, k = q.abs(), k.abs()
    la = torch.log(torch.tensor([0.9, 0.99], dtype=torch.float64))
    unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1)
    for ret in (None, la):
        expected = oracle.linattn_naive(q, k, unit, _oracle_decay(ret, q))
        r_dev = None if ret is None else ret.to(cuda, torch.float32)
        (num, mass), = scan_hip.linattn_views_mass(q.to(cuda, dtype), k.to(cuda, dtype), v.to(cuda, dtype), (r_dev,))
        assert rel_err(num, expected[..., :-1]) < TOL[dtype]
        assert rel_err(mass, expected[..., -1]) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dk", [32, 64])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("kind", ["none", "static"])
def test_ext_columns_match_concatenated_features(cuda, dtype, dk, reverse, kind):
    """A q ext column (array) and a k ext column (ones) equal one more feature
    of q and k; used by the key-mass backward (engine.py:430-442)."""
    from thetascan_amd._core.ops import scan_hip
    from thetascan_amd import _lib

    B, H, T, Dv = 2, 2, 170, 64
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, dk, Dv, seed=3))
    g = torch.Generator().manual_seed(8)
    qe = torch.randn(B, H, T, generator=g, dtype=torch.float64)
    qe = qe.to(torch.float32).double()
    ret = _retention(kind, B, H, T)
    qc = torch.cat([q, qe[..., None]], dim=-1)
    kc = torch.cat([k, torch.ones_like(k[..., :1])], dim=-1)
    decay = _oracle_decay(ret, q)
    if reverse:
        rdecay = None
        if decay is not None:
            flipped = decay.flip(2)
            rdecay = torch.cat([torch.zeros_like(flipped[:, :, :1]), flipped[:, :, :-1]], dim=2)
        expected = oracle.linattn_naive(qc.flip(2), kc.flip(2), v.flip(2), rdecay).flip(2)
    else:
        expected = oracle.linattn_naive(qc, kc, v, decay)
    kw = {"retention": _lib.RET_STATIC if kind == "static" else _lib.RET_NONE}
    if kind == "static":
        kw["log_alpha"] = ret.to(cuda, torch.float32)
    out, _, _ = scan_hip.scan_launch(q.to(cuda, dtype), k.to(cuda, dtype), v.to(cuda, dtype), reverse=reverse,
                                     q_ext=qe.to(cuda, torch.float32), k_ext="ones", seg_chunks=2, **kw)
    assert rel_err(out, expected) < TOL[dtype], (dk, reverse, kind)
    # the same columns the other way round (k ext array, q ext ones)
    out2, _, _ = scan_hip.scan_launch(k.to(cuda, dtype), q.to(cuda, dtype), v.to(cuda, dtype), reverse=reverse,
                                      q_ext="ones", k_ext=qe.to(cuda, torch.float32), seg_chunks=2, **kw)
    if reverse:
        expected2 = oracle.linattn_naive(kc.flip(2), qc.flip(2), v.flip(2), rdecay).flip(2)
    else:
        expected2 = oracle.linattn_naive(kc, qc, v, decay)
    assert rel_err(out2, expected2) < TOL[dtype], (dk, reverse, kind, "swapped")


@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_final_state_matches_recurrence(cuda, kind):
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = 2, 2, 299, 64, 64
    q, k, v = _streams(B, H, T, Dk, Dv, dtype=torch.float32)
    ret = _retention(kind, B, H, T)
    expected = oracle.final_state_naive(k.double(), v.double(), _oracle_decay(ret, q.double()))
    r_dev = None if ret is None else ret.to(cuda, torch.float32)
    state = scan_hip.final_state(q.to(cuda), k.to(cuda), v.to(cuda), r_dev, with_mass=True)
    assert rel_err(state[..., :Dv], expected) < 1e-4
    mass = oracle.final_state_naive(k.double(), torch.ones_like(v[..., :1]).double(), _oracle_decay(ret, q.double()))
    assert rel_err(state[..., Dv:], mass) < 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("with_mass", [False, True])
@pytest.mark.parametrize("width", [32, 64])
def test_gradients_match_float64_autograd(cuda, dtype, kind, with_mass, width):
    """q, k, v and retention gradients (tests/test_scan_chunk.py:271-301)."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = 2, 2, 150, width, width
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, Dk, Dv))
    ret = _retention(kind, B, H, T)
    g = torch.Generator().manual_seed(5)
    dO = _rounded(torch.randn(B, H, T, Dv, generator=g, dtype=torch.float64), dtype)
    dm = torch.randn(B, H, T, generator=g, dtype=torch.float64) * 0.1

    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    r_ref = None if ret is None else ret.clone().requires_grad_(True)
    if with_mass:
        unit = torch.cat([leaves[2], torch.ones_like(v[..., :1])], dim=-1)
        full = oracle.linattn_quad(leaves[0], leaves[1], unit, _oracle_decay(r_ref, q))
        loss = (full[..., :-1] * dO).sum() + (full[..., -1] * dm).sum()
    else:
        full = oracle.linattn_quad(leaves[0], leaves[1], leaves[2], _oracle_decay(r_ref, q))
        loss = (full * dO).sum()
    loss.backward()

    dev = [t.to(cuda, dtype).requires_grad_(True) for t in (q, k, v)]
    r_dev = None if ret is None else ret.to(cuda, torch.float32).requires_grad_(True)
    if with_mass:
        (num, mass), = scan_hip.linattn_views_mass(*dev, (r_dev,))
        loss_dev = (num.float() * dO.to(cuda, torch.float32)).sum() + (mass * dm.to(cuda, torch.float32)).sum()
    else:
        out = scan_hip.linattn_views(*dev, (r_dev,))[0]
        loss_dev = (out.float() * dO.to(cuda, torch.float32)).sum()
    loss_dev.backward()
    tol = TOL[dtype]
    for a, e, name in zip(dev, leaves, "qkv"):
        assert rel_err(a.grad, e.grad) < tol, name
    if ret is not None:
        assert rel_err(r_dev.grad, r_ref.grad) < (1e-3 if dtype == torch.float32 else 2e-2), "retention"


def test_errors_match_the_reference(cuda):
    from thetascan_amd._core.ops import scan_hip

    q, k, v = (x.to(cuda) for x in _streams(1, 2, 10, 8, 8, dtype=torch.float32))
    with pytest.raises(ValueError, match="chunk must be >= 1"):
        scan_hip.linattn(q, k, v, chunk=0)
    with pytest.raises(NotImplementedError, match="scalar decay only"):
        scan_hip.linattn(q, k, v, decay=torch.zeros(1, 2, 10, 8, device=cuda))
    with pytest.raises(ValueError, match="one entry per head"):
        scan_hip.linattn(q, k, v, log_alpha=torch.zeros(3, device=cuda))
    with pytest.raises(RuntimeError, match="GPU"):
        scan_hip.linattn(q.cpu(), k.cpu(), v.cpu())


def _ret_for(kind, r, lo, hi, cuda):
    """The retention of tokens lo:hi (static: all of it) on the GPU."""
    if r is None:
        return None
    if r.ndim == 1:
        return r.to(cuda, torch.float32)
    return r[:, :, lo:hi].to(cuda, torch.float32).contiguous()


@pytest.mark.parametrize("mass", [False, True])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_continues_from_a_carried_state(cuda, dtype, kind, mass):
    """Streaming: scanning the pieces of a sequence in order, each from the
    state the previous piece ended in (ragged pieces, a piece shorter than a
    tile, single-token decode steps), gives the scan of the whole sequence
    and its final state (the recurrence S_t = a_t S_{t-1} + k_t v_t^T).  An
    empty piece passes the carried state through unchanged."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dk, Dv = 2, 3, 1000, 64, 48
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, Dk, Dv, seed=51))
    if mass:
        q, k = q.abs(), k.abs()
    ret = _retention(kind, B, H, T, seed=52)
    cuts = [0, 517, 517, 560, 995, 996, 997, 998, 999, 1000, 1000]
    outs, masses, state = [], [], None
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        out, m, state = scan_hip.linattn_state(q[:, :, lo:hi].to(cuda, dtype), k[:, :, lo:hi].to(cuda, dtype),
                                               v[:, :, lo:hi].to(cuda, dtype), _ret_for(kind, ret, lo, hi, cuda),
                                               state, mass=mass)
        outs.append(out)
        if mass:
            masses.append(m)
    got = torch.cat(outs, dim=2)
    unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1) if mass else v
    expected = oracle.linattn_naive(q, k, unit, _oracle_decay(ret, q))
    assert rel_err(got, expected[..., :Dv]) < TOL[dtype], (kind, dtype)
    if mass:
        assert rel_err(torch.cat(masses, dim=2), expected[..., Dv]) < TOL[dtype], (kind, dtype)
    # the final state: S_T = sum_i w(T-1, i) k_i v_i^T (+ the key-mass column sum_i w k_i)
    decay = _oracle_decay(ret, q)
    w = torch.ones(B, H, T, dtype=torch.float64) if decay is None else \
        torch.exp(decay[..., 0].flip(-1).cumsum(-1).flip(-1) - decay[..., 0])
    S = torch.einsum("bht,bhtk,bhtv->bhkv", w, k, unit)
    assert state.shape == (B, H, Dk, Dv + (1 if mass else 0))
    assert rel_err(state, S) < (1e-4 if dtype == torch.float32 else 1e-2), (kind, dtype)


@pytest.mark.parametrize("mass", [False, True])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Dk,Dv", [(5, 4), (16, 16), (32, 64), (48, 40), (64, 64), (128, 128), (100, 24)])
def test_short_continuations_walk_the_recurrence(cuda, dtype, kind, mass, Dk, Dv):
    """Continuations of at most eight tokens (decode steps) take a
    token-by-token launch over the register-resident state; a fresh sequence
    that short, then pieces of 1..8 tokens after a long one, give the whole
    sequence's scan and final state (S_t = a_t S_{t-1} + k_t v_t^T, with the
    key-mass column D_t = a_t D_{t-1} + k_t when ``mass``)."""
    from thetascan_amd._core.ops import scan_hip

    B, H = 2, 3
    cuts = [0, 3, 70, 71, 73, 76, 80, 85, 91, 98, 106, 107]
    T = cuts[-1]
    q, k, v = (_rounded(x, dtype) for x in _streams(B, H, T, Dk, Dv, seed=53 + Dk))
    if mass:
        q, k = q.abs(), k.abs()
    ret = _retention(kind, B, H, T, seed=54)
    outs, masses, state = [], [], None
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        out, m, state = scan_hip.linattn_state(q[:, :, lo:hi].to(cuda, dtype), k[:, :, lo:hi].to(cuda, dtype),
                                               v[:, :, lo:hi].to(cuda, dtype), _ret_for(kind, ret, lo, hi, cuda),
                                               state, mass=mass)
        assert out.dtype == dtype and out.shape == (B, H, hi - lo, Dv)
        outs.append(out)
        if mass:
            masses.append(m)
    unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1) if mass else v
    decay = _oracle_decay(ret, q)
    expected = oracle.linattn_naive(q, k, unit, decay)
    got = torch.cat(outs, dim=2)
    errs = {"out": rel_err(got, expected[..., :Dv])}
    if mass:
        errs["mass"] = rel_err(torch.cat(masses, dim=2), expected[..., Dv])
    w = torch.ones(B, H, T, dtype=torch.float64) if decay is None else \
        torch.exp(decay[..., 0].flip(-1).cumsum(-1).flip(-1) - decay[..., 0])
    S = torch.einsum("bht,bhtk,bhtv->bhkv", w, k, unit)
    # widths round up to whole 16-byte vectors; the padding rows and columns stay zero
    vec = 8 if dtype == torch.bfloat16 else 4
    dkw, dvw = -(-Dk // vec) * vec, -(-Dv // vec) * vec
    assert state.shape == (B, H, dkw, dvw + (1 if mass else 0))
    cols = list(range(Dv)) + ([dvw] if mass else [])
    kept = state[:, :, :Dk][..., cols]
    rest = state.clone()
    rest[:, :, :Dk, cols] = 0
    assert not rest.any()
    errs["state"] = rel_err(kept, S)
    print(f"short continuations {Dk}x{Dv} {kind} {dtype} mass={mass}: {errs}", flush=True)
    for name, e in errs.items():
        assert e < (TOL[dtype] if name != "state" else (1e-4 if dtype == torch.float32 else 1e-2)), (name, e)


@pytest.mark.parametrize("T", [1, 8, 200])
@pytest.mark.parametrize("mass", [False, True])
def test_final_state_written_in_place(cuda, T, mass):
    """A continuation may write its final state over the state it starts
    from (the captured decode step does): the result equals the out-of-place
    call bit for bit, for the token-by-token launch and the tiled passes."""
    from thetascan_amd._core.ops import scan_hip

    q, k, v = (x.to(cuda, torch.bfloat16) for x in _streams(2, 3, T, 64, 64, seed=57, dtype=torch.float32))
    if mass:
        q, k = q.abs(), k.abs()
    la = torch.log(torch.rand(3, generator=torch.Generator().manual_seed(58)) * 0.09 + 0.9).to(cuda)
    _, _, st = scan_hip.linattn_state(q[:, :, :5], k[:, :, :5], v[:, :, :5], la, mass=mass)
    ref_out, ref_mass, ref_fin = scan_hip.linattn_state(q, k, v, la, st, mass=mass)
    buf = st.clone()
    kind = scan_hip._classify(la, q)
    out, m, fin = scan_hip.scan_launch(q, k, v, **scan_hip._ret_kwargs(kind, la), v_ext="ones" if mass else None,
                                       want_ext_out=mass, want_final=True, init_state=buf, final_out=buf)
    assert fin.data_ptr() == buf.data_ptr()
    assert torch.equal(out, ref_out) and torch.equal(buf, ref_fin)
    if mass:
        assert torch.equal(m, ref_mass)


def test_short_continuation_equals_the_tiled_path(cuda):
    """A one-token step gives what the tiled passes give for the same token
    appended to a tile-aligned prefix, to fp32 rounding."""
    from thetascan_amd._core.ops import scan_hip

    q, k, v = (x.float() for x in _streams(1, 4, 73, 64, 64, seed=55))
    ret = -torch.rand(1, 4, 73, 1, generator=torch.Generator().manual_seed(56)) * 0.1
    dev = [x.to(cuda) for x in (q, k, v, ret)]
    whole, _, fin_whole = scan_hip.linattn_state(*dev)
    _, _, st = scan_hip.linattn_state(*(x[:, :, :72] for x in dev))
    step, _, fin_step = scan_hip.linattn_state(*(x[:, :, 72:] for x in dev), st)
    assert rel_err(step, whole[:, :, 72:]) < 1e-5
    assert rel_err(fin_step, fin_whole) < 1e-5


@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_sequence_sharded_scan_equals_the_whole_scan(cuda, kind):
    """The sequence-sharding design on one GPU: P shards scan their slices
    from zero and report their final states; an exclusive combine of those
    carries (each decayed by the later shards' retention) gives each shard its
    incoming state; re-scanning every shard from it reproduces the whole
    scan.  This is the step an all-gather of carries across GPUs would feed."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 1, 2, 1200, 64
    q, k, v = _streams(B, H, T, D, D, seed=61, dtype=torch.float32)
    ret = _retention(kind, B, H, T, seed=62)
    bounds = [0, 300, 650, 900, 1200]
    # 1. every shard from zero: its carry U_p and its total log-decay
    carries, logs = [], []
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        _, _, fin = scan_hip.linattn_state(q[:, :, lo:hi].to(cuda), k[:, :, lo:hi].to(cuda), v[:, :, lo:hi].to(cuda),
                                           _ret_for(kind, ret, lo, hi, cuda), None)
        carries.append(fin)
        if ret is None:
            logs.append(torch.zeros(B, H, device=cuda))
        elif ret.ndim == 1:
            logs.append((ret.to(cuda, torch.float32) * (hi - lo)).view(1, H).expand(B, H))
        else:
            logs.append(ret[:, :, lo:hi, 0].sum(-1).to(cuda, torch.float32))
    # 2. exclusive combine: S_in(p) = exp(L_{p-1}) S_in(p-1) + U_{p-1}
    s_in = [None]
    for p in range(1, len(carries)):
        prev = torch.zeros_like(carries[0]) if s_in[-1] is None else s_in[-1]
        s_in.append(torch.exp(logs[p - 1]).view(B, H, 1, 1) * prev + carries[p - 1])
    # 3. every shard from its incoming state
    outs = []
    for p, (lo, hi) in enumerate(zip(bounds[:-1], bounds[1:])):
        out, _, _ = scan_hip.linattn_state(q[:, :, lo:hi].to(cuda), k[:, :, lo:hi].to(cuda), v[:, :, lo:hi].to(cuda),
                                           _ret_for(kind, ret, lo, hi, cuda), s_in[p])
        outs.append(out)
    expected = oracle.linattn_naive(q.double(), k.double(), v.double(), _oracle_decay(ret, q.double()))
    assert rel_err(torch.cat(outs, dim=2), expected) < 1e-4, kind


@pytest.mark.parametrize("reverse", [True, False])
@pytest.mark.parametrize("seg_chunks", [0, 1, 3])
@pytest.mark.parametrize("T", [700, 64, 5, 4096])
def test_pair_scan_equals_its_two_scans(cuda, T, seg_chunks, reverse):
    """ts_scan_pair_fwd (the backward's dk and dv scans in one pass: K and V
    read once, one state) gives scan(qa, k, v) and scan(qb, v, k) bit for bit
    as two ts_scan_fwd calls do, and both match the float64 recurrence."""
    from thetascan_amd._core.ops import scan_hip

    B, H, D = 2, 3, 64
    g = torch.Generator().manual_seed(71 + T)
    qa, k, v, qb = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).to(torch.float64)
                    for _ in range(4))
    dev = [x.to(cuda, torch.bfloat16) for x in (qa, k, v, qb)]
    a, b = scan_hip.scan_pair_launch(*dev, reverse=reverse, seg_chunks=seg_chunks)
    ref_a, _, _ = scan_hip.scan_launch(dev[0], dev[1], dev[2], reverse=reverse, seg_chunks=seg_chunks)
    ref_b, _, _ = scan_hip.scan_launch(dev[3], dev[2], dev[1], reverse=reverse, seg_chunks=seg_chunks)
    assert torch.equal(a, ref_a) and torch.equal(b, ref_b), (T, seg_chunks, reverse)

    def naive(q, kk, vv):
        # the tiled float64 oracle (equal to the recurrence at 1e-12) reaches T = 4096
        if reverse:
            return oracle.linattn_chunk(q.flip(2), kk.flip(2), vv.flip(2)).flip(2)
        return oracle.linattn_chunk(q, kk, vv)

    assert rel_err(a, naive(qa, k, v)) < TOL[torch.bfloat16]
    assert rel_err(b, naive(qb, v, k)) < TOL[torch.bfloat16]


def test_pair_scan_writes_strided_outputs(cuda):
    """The dv output goes straight into a strided view of the qkv gradient."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 4, 300, 64
    g = torch.Generator().manual_seed(77)
    qa, k, v, qb = (torch.randn(B, H, T, D, generator=g).to(cuda, torch.bfloat16) for _ in range(4))
    big = torch.zeros(B, T, 3, H, D, dtype=torch.bfloat16, device=cuda)
    view = big[:, :, 2].transpose(1, 2)
    _, b = scan_hip.scan_pair_launch(qa, k, v, qb, reverse=True, out_b=view)
    ref_b, _, _ = scan_hip.scan_launch(qb, v, k, reverse=True)
    assert b.data_ptr() == view.data_ptr()
    assert torch.equal(view, ref_b)
    assert not big[:, :, :2].any()


@pytest.mark.parametrize("T,seg_chunks,reverse", [(1, 0, True), (200, 1, False), (700, 2, True), (4096, 0, True)])
def test_pair_scan_with_key_ext_equals_its_two_scans(cuda, T, seg_chunks, reverse):
    """With scan A's key-side ext pair (the key-mass read's backward: queries
    carry a ones column, keys the fp32 dmass), ts_scan_pair_fwd gives
    scan(qa, k, v; ones x dmass) and scan(qb, v, k) bit for bit as two
    ts_scan_fwd calls do, and scan A matches the float64 recurrence with the
    ext column appended."""
    from thetascan_amd._core.ops import scan_hip

    B, H, D = 2, 3, 64
    g = torch.Generator().manual_seed(97 + T)
    qa, k, v, qb = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).to(torch.float64)
                    for _ in range(4))
    ke = torch.randn(B, H, T, generator=g, dtype=torch.float64).to(torch.float32).to(torch.float64)
    dev = [x.to(cuda, torch.bfloat16) for x in (qa, k, v, qb)]
    ke_d = ke.to(cuda, torch.float32)
    a, b = scan_hip.scan_pair_launch(*dev, reverse=reverse, seg_chunks=seg_chunks, k_ext=ke_d)
    ref_a, _, _ = scan_hip.scan_launch(dev[0], dev[1], dev[2], reverse=reverse, seg_chunks=seg_chunks,
                                       q_ext="ones", k_ext=ke_d)
    ref_b, _, _ = scan_hip.scan_launch(dev[3], dev[2], dev[1], reverse=reverse, seg_chunks=seg_chunks)
    assert torch.equal(a, ref_a) and torch.equal(b, ref_b), (T, seg_chunks, reverse)
    ones = torch.ones(B, H, T, 1, dtype=torch.float64)
    qx, kx = torch.cat([qa, ones], -1), torch.cat([k, ke.unsqueeze(-1)], -1)
    if reverse:
        want = oracle.linattn_chunk(qx.flip(2), kx.flip(2), v.flip(2)).flip(2)
    else:
        want = oracle.linattn_chunk(qx, kx, v)
    assert rel_err(a, want) < TOL[torch.bfloat16]


@pytest.mark.parametrize("T,seg_chunks,reverse,kx,static,out_mode", [
    (700, 0, True, False, True, "store"),
    (5, 0, False, False, True, "store"),
    (4096, 3, True, True, True, "accum"),
    (300, 1, False, True, True, "store_f32"),
    (1, 0, True, True, True, "accum"),
    (700, 2, True, False, False, "accum"),
    (200, 0, False, True, False, "store_f32"),
])
def test_pair_scan_retention_and_fp32_outputs_equal_its_two_scans(cuda, T, seg_chunks, reverse, kx, static, out_mode):
    """With a static per-head retention shared by both scans and fp32
    outputs (stored, or accumulated with a scale into existing values),
    ts_scan_pair_fwd gives scan A with the same bits as its ts_scan_fwd call
    and scan B within bf16 rounding of its own (plain scans: the same bits).
    The pair keeps one state, sum_i alpha^(t-i) v_i k_i^T, whose decay
    weights round with v as scan A's own call rounds them; scan B's own call
    weights (and rounds) k instead.  Retained scans match the float64
    decayed recurrence."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import scan_hip

    B, H, D = 2, 3, 64
    g = torch.Generator().manual_seed(131 + T)
    qa, k, v, qb = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).to(torch.float64)
                    for _ in range(4))
    dev = [x.to(cuda, torch.bfloat16) for x in (qa, k, v, qb)]
    la = torch.log(torch.tensor([0.9, 0.97, 0.995])) if static else None
    ke = torch.randn(B, H, T, generator=g).to(cuda) if kx else None
    mode = {"store": _lib.OUT_STORE, "store_f32": _lib.OUT_STORE_F32, "accum": _lib.OUT_ACCUM_F32}[out_mode]
    scale = 0.75 if mode == _lib.OUT_ACCUM_F32 else 1.0
    rk = dict(retention=_lib.RET_STATIC, log_alpha=la) if static else {}
    base_a = torch.randn(B, H, T, D, generator=g).to(cuda)
    base_b = torch.randn(B, H, T, D, generator=g).to(cuda)
    pa = pb = ra = rb = None
    if mode == _lib.OUT_ACCUM_F32:
        pa, pb, ra, rb = base_a.clone(), base_b.clone(), base_a.clone(), base_b.clone()
    a, b = scan_hip.scan_pair_launch(*dev, reverse=reverse, seg_chunks=seg_chunks, k_ext=ke, log_alpha=la,
                                     out_mode=mode, out_scale=scale, out_a=pa, out_b=pb)
    ref_a, _, _ = scan_hip.scan_launch(dev[0], dev[1], dev[2], **rk, reverse=reverse, seg_chunks=seg_chunks,
                                       q_ext="ones" if kx else None, k_ext=ke, out=ra, out_mode=mode,
                                       out_scale=scale)
    ref_b, _, _ = scan_hip.scan_launch(dev[3], dev[2], dev[1], **rk, reverse=reverse, seg_chunks=seg_chunks,
                                       out=rb, out_mode=mode, out_scale=scale)
    assert torch.equal(a, ref_a[..., :D]), (T, seg_chunks, reverse, kx, out_mode)
    if static:
        acc = base_b if mode == _lib.OUT_ACCUM_F32 else 0
        assert rel_err(b - acc, ref_b[..., :D] - acc) < 1e-2
    else:
        assert torch.equal(b, ref_b[..., :D]), (T, seg_chunks, reverse, kx, out_mode)
    if static and not kx and mode != _lib.OUT_ACCUM_F32:
        idx = torch.arange(T, dtype=torch.float64)
        dist = (idx[:, None] - idx[None, :]) if not reverse else (idx[None, :] - idx[:, None])
        w = torch.where(dist >= 0, torch.exp(la.double().view(H, 1, 1) * dist.clamp(min=0)), torch.zeros(()))
        want_a = torch.einsum("bhts,bhsd->bhtd", torch.einsum("bhtd,bhsd->bhts", qa, k) * w, v)
        want_b = torch.einsum("bhts,bhsd->bhtd", torch.einsum("bhtd,bhsd->bhts", qb, v) * w, k)
        assert rel_err(a, want_a) < TOL[torch.bfloat16]
        assert rel_err(b, want_b) < TOL[torch.bfloat16]


@pytest.mark.parametrize("Dk,with_mass,used", [(64, True, (1, 2)), (64, False, (0, 1, 2)), (192, True, (0, 2)),
                                               (64, True, (2,))])
def test_bank_view_gradients_match_float64_autograd(cuda, Dk, with_mass, used):
    """q, k, v and retention gradients of a bank's views (plain and two static
    retentions), some views left out of the loss: the first scan into each
    fp32 gradient stores, later ones accumulate (64-wide: the paired dk/dv
    scan; 192-wide keys: key chunks), and a view with no upstream gradient
    adds nothing."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, Dv = 2, 2, 330, 64
    q, k, v = (_rounded(x, torch.bfloat16) for x in _streams(B, H, T, Dk, Dv, seed=61))
    rets = (None, torch.log(torch.tensor([0.9, 0.95], dtype=torch.float64)),
            torch.log(torch.tensor([0.99, 0.97], dtype=torch.float64)))
    g = torch.Generator().manual_seed(9)
    dOs = [_rounded(torch.randn(B, H, T, Dv, generator=g, dtype=torch.float64), torch.bfloat16) for _ in rets]
    dms = [torch.randn(B, H, T, generator=g, dtype=torch.float64) * 0.1 for _ in rets]

    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    r_ref = [None if r is None else r.clone().requires_grad_(True) for r in rets]
    loss = 0
    for j in used:
        unit = torch.cat([leaves[2], torch.ones_like(v[..., :1])], dim=-1) if with_mass else leaves[2]
        full = oracle.linattn_quad(leaves[0], leaves[1], unit, _oracle_decay(r_ref[j], q))
        loss = loss + (full[..., :Dv] * dOs[j]).sum() + ((full[..., -1] * dms[j]).sum() if with_mass else 0)
    loss.backward()

    dev = [t.to(cuda, torch.bfloat16).requires_grad_(True) for t in (q, k, v)]
    r_dev = [None if r is None else r.to(cuda, torch.float32).requires_grad_(True) for r in rets]
    if with_mass:
        outs = scan_hip.linattn_views_mass(*dev, tuple(r_dev))
    else:
        outs = [(o, None) for o in scan_hip.linattn_views(*dev, tuple(r_dev))]
    loss_dev = 0
    for j in used:
        num, mass = outs[j]
        loss_dev = loss_dev + (num.float() * dOs[j].to(cuda, torch.float32)).sum()
        if with_mass:
            loss_dev = loss_dev + (mass * dms[j].to(cuda, torch.float32)).sum()
    loss_dev.backward()
    for a, e, name in zip(dev, leaves, "qkv"):
        assert rel_err(a.grad, e.grad) < 2 * TOL[torch.bfloat16], name
    for j in (1, 2):
        if j in used:
            assert rel_err(r_dev[j].grad, r_ref[j].grad) < 5e-2, j
        else:
            assert r_dev[j].grad is None or not r_dev[j].grad.any(), j


@pytest.mark.parametrize("out_mode", ["store", "store_f32", "accum"])
@pytest.mark.parametrize("Dk,Dv", [(192, 64), (64, 200), (300, 136)])
def test_wide_scans_in_every_output_mode(cuda, Dk, Dv, out_mode):
    """Keys wider than one launch (fp32 partial scans over key chunks, the
    first stored) and values wider than one launch (value chunks written into
    one output, the last padded to the vector width), in the bf16 store, fp32
    store and fp32 accumulate modes, against the float64 recurrence, with a
    static retention and the key-mass column."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import scan_hip

    B, H, T = 1, 2, 333
    q, k, v = (_rounded(x, torch.bfloat16) for x in _streams(B, H, T, Dk, Dv, seed=83))
    q, k = q.abs() / Dk ** 0.5, k.abs()
    la = torch.log(torch.tensor([0.9, 0.99], dtype=torch.float64))
    qd, kd, vd = (x.to(cuda, torch.bfloat16) for x in (q, k, v))
    mode = {"store": _lib.OUT_STORE, "store_f32": _lib.OUT_STORE_F32, "accum": _lib.OUT_ACCUM_F32}[out_mode]
    vec = 8
    width = -(-Dv // vec) * vec
    base = torch.randn(B, H, T, width, generator=torch.Generator().manual_seed(3)).to(cuda)
    base_m = torch.randn(B, H, T, generator=torch.Generator().manual_seed(4)).to(cuda)
    out = base.clone() if mode == _lib.OUT_ACCUM_F32 else None
    ext = base_m.clone() if mode == _lib.OUT_ACCUM_F32 else None
    scale = 0.5 if mode != _lib.OUT_STORE else 1.0
    res, mass, _ = scan_hip.scan_launch(qd, kd, vd, retention=_lib.RET_STATIC, log_alpha=la.to(cuda, torch.float32),
                                        v_ext="ones", want_ext_out=True, out=out, ext_out=ext, out_mode=mode,
                                        out_scale=scale)
    unit = torch.cat([v, torch.ones_like(v[..., :1])], dim=-1)
    want = oracle.linattn_naive(q, k, unit, _oracle_decay(la, q)) * scale
    got, got_m = res[..., :Dv].double().cpu(), mass.double().cpu()
    if mode == _lib.OUT_ACCUM_F32:
        got, got_m = got - base[..., :Dv].double().cpu(), got_m - base_m.double().cpu()
    assert res.dtype == (torch.bfloat16 if mode == _lib.OUT_STORE else torch.float32)
    assert rel_err(got, want[..., :Dv]) < TOL[torch.bfloat16], (Dk, Dv, out_mode)
    assert rel_err(got_m, want[..., Dv]) < TOL[torch.bfloat16], (Dk, Dv, out_mode)
