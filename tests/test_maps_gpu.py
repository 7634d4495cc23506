"""HIP B-spline feature map and bank blend against the oracle (fp64, CPU).

The B-spline kernel (ts_bspline_fwd/bwd) is checked against the reference's
own basis vectors (tests/golden/features.npz) and against the oracle's
differentiable restatement of kernel_features.py:138-230, gradients
included, over bases of several sizes and degrees, coordinates on both sides
of the clamp and exactly on knots.  The blend (ts_blend_fwd/bwd) is checked
against the fast and stale blends of block.py:667-718 written out in fp64.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import mixer
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _cfg(n_basis, degree, bound):
    return {"bspline_basis_count": n_basis, "bspline_degree": degree, "bspline_bound": bound}


def test_bspline_matches_reference_vectors(cuda):
    from thetascan_amd._core.ops import maps

    d = np.load(GOLDEN / "features.npz")
    coords = torch.from_numpy(d["bspline_coords"])  # [1,1,97,1] spanning [-4, 4]
    got = maps.bspline_features(coords.to(cuda, torch.float32), n_basis=8, degree=3, bound=3.0, scale=1.0)
    # one coordinate per row: the map is basis / P with P = 1
    assert rel_err(got, torch.from_numpy(d["bspline_basis"]).view(1, 1, 97, 8)) < 1e-5
    pre = torch.from_numpy(d["pre"])[..., :4]
    got = maps.bspline_features(pre.to(cuda, torch.float32), n_basis=8, degree=3, bound=3.0, scale=1.0)
    assert rel_err(got, torch.from_numpy(d["bspline_features"])) < 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_basis,degree,bound,P,per_head", [
    (8, 3, 3.0, 8, False),
    (8, 3, 3.0, 16, True),
    (5, 2, 2.0, 4, True),
    (12, 3, 3.0, 6, False),
    (16, 5, 2.5, 8, True),
    (4, 0, 1.0, 8, False),
    (32, 3, 3.0, 4, True),
])
def test_bspline_forward_and_gradients(cuda, dtype, n_basis, degree, bound, P, per_head):
    from thetascan_amd._core.ops import maps

    g = torch.Generator().manual_seed(1000 * n_basis + 10 * degree + P)
    B, H, T = 2, 3, 37
    pre = torch.randn(B, H, T, P, generator=g, dtype=torch.float64) * 1.7
    # exact knots, the clamp ends and points beyond them
    pre[0, 0, 0, :4] = torch.tensor([0.0, bound, -bound, 2 * bound], dtype=torch.float64)
    pre = pre.to(dtype).to(torch.float64)  # representable in the kernel dtype
    scale = (torch.rand(H, generator=g, dtype=torch.float64) + 0.5) if per_head else 1.3
    dout = torch.randn(B, H, T, P * n_basis, generator=g, dtype=torch.float64)

    ref_pre = pre.clone().requires_grad_(True)
    ref_scale = scale.clone().requires_grad_(True) if per_head else scale
    ref = mixer.bspline_features(ref_pre, ref_scale, _cfg(n_basis, degree, bound))
    if ref.requires_grad:
        ref.backward(dout)
        ref_dpre = ref_pre.grad
        ref_dscale = ref_scale.grad if per_head else None
    else:  # degree 0: piecewise constant, zero gradient almost everywhere
        ref_dpre = torch.zeros_like(pre)
        ref_dscale = torch.zeros_like(scale) if per_head else None

    x = pre.to(cuda, dtype).requires_grad_(True)
    s = scale.to(cuda, torch.float32).requires_grad_(True) if per_head else scale
    out = maps.bspline_features(x, n_basis=n_basis, degree=degree, bound=bound, scale=s)
    assert out.shape == ref.shape and out.dtype == dtype
    out.backward(dout.to(cuda, dtype))
    tol = TOL[dtype]
    assert rel_err(out, ref) < tol
    if degree == 0:
        assert float(x.grad.abs().max()) == 0.0
        return
    assert rel_err(x.grad, ref_dpre) < (1e-4 if dtype == torch.float32 else 3e-2)
    if per_head:
        assert rel_err(s.grad, ref_dscale) < (1e-4 if dtype == torch.float32 else 3e-2)


def test_bspline_rejects_what_the_reference_rejects(cuda):
    from thetascan_amd._core.ops import maps

    x = torch.zeros(1, 1, 4, 4, device=cuda)
    with pytest.raises(ValueError):
        maps.bspline_features(x, n_basis=3, degree=3, bound=3.0, scale=1.0)
    with pytest.raises(ValueError):
        maps.bspline_features(x, n_basis=8, degree=3, bound=0.0, scale=1.0)
    with pytest.raises(ValueError):
        maps.bspline_features(x, n_basis=8, degree=-1, bound=1.0, scale=1.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode,J,d,T", [("fast", 2, 64, 77), ("fast", 4, 64, 300), ("stale", 2, 32, 41),
                                        ("stale", 4, 24, 50), ("fast", 1, 12, 9)])
def test_bank_blend_matches_the_fade_blends(cuda, dtype, mode, J, d, T):
    from thetascan_amd._core.ops import maps

    g = torch.Generator().manual_seed(J * 100 + d + T)
    B, H = 2, 3
    n_in = J + 1 if mode == "fast" else J + 2
    reads = [torch.randn(B, H, T, d, generator=g, dtype=torch.float64).to(dtype).to(torch.float64)
             for _ in range(n_in)]
    etas = [torch.randn(H, generator=g, dtype=torch.float64) * 0.3 for _ in range(J)]
    dy = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)

    ref_reads = [r.clone().requires_grad_(True) for r in reads]
    ref_etas = [e.clone().requires_grad_(True) for e in etas]
    y = ref_reads[0]
    if mode == "fast":  # block.py:683-695
        for out_fast, eta in zip(ref_reads[1:], ref_etas):
            y = y + eta.view(1, -1, 1, 1) * (out_fast - ref_reads[0])
    else:  # block.py:697-717
        for out_stale, eta in zip(ref_reads[1:-1], ref_etas):
            y = y - eta.view(1, -1, 1, 1) * (out_stale - ref_reads[-1])
    y.backward(dy)

    xs = [r.to(cuda, dtype).requires_grad_(True) for r in reads]
    es = [e.to(cuda, torch.float32).requires_grad_(True) for e in etas]
    coef = maps.fast_coefficients(es) if mode == "fast" else maps.stale_coefficients(es)
    out = maps.bank_blend(xs, coef)
    out.backward(dy.to(cuda, dtype))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(out, y) < tol
    for a, b in zip(xs, ref_reads):
        assert rel_err(a.grad, b.grad) < tol
    for a, b in zip(es, ref_etas):
        assert rel_err(a.grad, b.grad) < (1e-4 if dtype == torch.float32 else 2e-2)


def test_bank_blend_strided_views(cuda):
    """Non-contiguous head-major views (the transposed read layout) take the
    strided path and give the same result."""
    from thetascan_amd._core.ops import maps

    g = torch.Generator().manual_seed(7)
    B, H, T, d = 2, 4, 33, 16
    base = [torch.randn(B, T, H, d, generator=g) for _ in range(3)]
    views = [t.to(cuda).transpose(1, 2) for t in base]
    coef = torch.randn(3, H, generator=g).to(cuda)
    out = maps.bank_blend(views, coef)
    ref = sum(coef[i].view(1, -1, 1, 1).cpu().double() * base[i].transpose(1, 2).double() for i in range(3))
    assert rel_err(out, ref) < 1e-5


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("P,n_basis,learned,shifted", [(16, 8, False, False), (16, 8, True, True), (4, 8, True, False),
                                                       (2, 5, False, True), (64, 8, False, False)])
def test_bspline_of_rmsnormed_inputs_matches_the_oracle(cuda, dtype, tol, P, n_basis, learned, shifted):
    """ts_bspline_norm_fwd / _bwd: basis((rmsnorm(a) + shift) * scale) / P of the
    raw W1 products against the float64 oracle (rmsnorm, bspline_features),
    with the gradients of a, the per-head scale and the shift; ragged T."""
    from oracle import mixer as om
    from thetascan_amd._core.ops import maps

    B, H, T = 2, 3, 301
    g0 = torch.Generator().manual_seed(P * 7 + n_basis)
    a = (torch.randn(B, H, T, P, generator=g0) * 1.5).to(dtype).double()
    scale = torch.rand(H, generator=g0) + 0.5 if learned else 1.3
    shift = torch.randn(H, P, generator=g0) * 0.4 if shifted else None
    dout = torch.randn(B, H, T, P * n_basis, generator=g0)
    c = {"bspline_basis_count": n_basis, "bspline_degree": 3, "bspline_bound": 3.0}

    a64 = a.clone().requires_grad_(True)
    s64 = scale.double().requires_grad_(True) if learned else scale
    h64 = None if shift is None else shift.double().requires_grad_(True)
    z, _ = om.rmsnorm(a64)
    if h64 is not None:
        z = z + h64.view(1, H, 1, P)
    ref = om.bspline_features(z, s64, c)
    ref.backward(dout.to(dtype).double())

    ad = a.to(dtype).to(cuda).requires_grad_(True)
    sd = scale.to(cuda).requires_grad_(True) if learned else scale
    hd = None if shift is None else shift.to(cuda).requires_grad_(True)
    out = maps.bspline_norm_features(ad, shift=hd, eps=1e-6, n_basis=n_basis, degree=3, bound=3.0, scale=sd)
    out.backward(dout.to(dtype).to(cuda))
    torch.cuda.synchronize()
    assert out.shape == (B, H, T, P * n_basis) and out.dtype == dtype
    assert rel_err(out.float(), ref) < tol
    assert rel_err(ad.grad.float(), a64.grad) < tol
    if learned:
        assert rel_err(sd.grad, s64.grad) < tol
    if shifted:
        assert rel_err(hd.grad, h64.grad) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 1e-2)])
def test_gated_blend_matches_blend_then_gate(cuda, dtype, tol):
    """ts_blend_gated_fwd (inference) against float64 (sum_i coef_i in_i) *
    silu(gate + bias) on views of token-major memory (fp32 1e-6, bf16 one
    rounding)."""
    from thetascan_amd._core.ops import maps

    g = torch.Generator().manual_seed(21)
    B, H, T, d, n = 2, 3, 130, 64, 4
    ins = [torch.randn(B, H, T, d, generator=g).to(dtype) for _ in range(n)]
    coef = torch.randn(n, H, generator=g)
    gate = torch.randn(B, T, H, d, generator=g).to(dtype).transpose(1, 2)
    bias = torch.randn(H * d, generator=g)
    ref = sum(coef[i].double().view(1, H, 1, 1) * ins[i].double() for i in range(n))
    ref = ref * torch.nn.functional.silu(gate.double() + bias.double().view(H, 1, d))
    with torch.no_grad():
        y = maps.bank_blend_gated([t.to(cuda) for t in ins], coef.to(cuda), gate.to(cuda), bias.to(cuda))
    torch.cuda.synchronize()
    assert y.shape == (B, H, T, d) and y.transpose(1, 2).is_contiguous()
    err = rel_err(y.double().cpu(), ref)
    print(f"gated blend {dtype}: {err:.3g}", flush=True)
    assert err < tol
    with pytest.raises(RuntimeError, match="forward-only"):
        maps.bank_blend_gated([t.to(cuda) for t in ins], coef.to(cuda), gate.to(cuda), bias.to(cuda))
