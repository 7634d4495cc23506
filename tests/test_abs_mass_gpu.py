"""Mass of absolute features (ts_abs_mass_fwd / ts_abs_mass_bwd) against float64.

mass_t = sum_j |q_tj| C_tj with C the view's decayed prefix of |k| (plain,
static per-head, per-token retention) is the normalizer of the tanh GN read.
The float64 reference is the oracle's prefix (oracle/scans.py:
causal_prefix_sum, ema_cumsum, and the per-token recurrence written out),
times |q|, summed over features; its autograd gives dq and dk (torch's abs
backward, sign(x) with sign(0) = 0).  Tolerances: rel 1e-3 (fp32) and 2e-2
(bf16) on mass and on both gradients (max-abs error over max-abs reference).
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def prefix64(x, kind, la, dec):
    from oracle import scans

    if kind == "none":
        return scans.causal_prefix_sum(x)
    if kind == "static":
        return scans.ema_cumsum(x, la)
    z = torch.zeros_like(x[:, :, 0])
    rows = []
    for t in range(x.shape[2]):
        z = z * dec[:, :, t].exp().unsqueeze(-1) + x[:, :, t]
        rows.append(z)
    return torch.stack(rows, dim=2)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("F", [16, 64, 128, 256])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_abs_mass_matches_float64(cuda, dtype, tol, F, kind):
    from thetascan_amd._core.ops import fused

    B, H, T = 2, 3, 777
    g = torch.Generator().manual_seed(F + len(kind))
    q = torch.randn(B, H, T, F, generator=g).to(dtype).double()
    k = torch.randn(B, H, T, F, generator=g).to(dtype).double()
    q[0, 0, 5, :4] = 0.0  # sign(0) = 0 in the backward
    la = torch.log(torch.rand(H, generator=g) * 0.2 + 0.79).double()
    dec = torch.log(torch.rand(B, H, T, 1, generator=g) * 0.3 + 0.69).double()
    dmass = torch.randn(B, H, T, generator=g).double()

    rq, rk = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    ref = (rq.abs() * prefix64(rk.abs(), kind, la, dec[..., 0] if kind == "stream" else None)).sum(-1)
    ref.backward(dmass)

    qd = q.to(dtype).to(cuda).requires_grad_(True)
    kd = k.to(dtype).to(cuda).requires_grad_(True)
    ret = None if kind == "none" else (la.float().to(cuda) if kind == "static" else dec.float().to(cuda))
    assert fused.abs_mass_eligible(qd, kd, ret)
    mass = fused.abs_mass(qd, kd, ret)
    mass.backward(dmass.float().to(cuda))
    torch.cuda.synchronize()
    assert mass.dtype == torch.float32 and mass.shape == (B, H, T)
    assert rel_err(mass, ref) < tol
    assert rel_err(qd.grad.float(), rq.grad) < tol
    assert rel_err(kd.grad.float(), rk.grad) < tol


def test_abs_mass_of_nonnegative_features_is_the_unit_column(cuda):
    """For features >= 0 the mass is the scan's key-mass column (the
    reference's normalizer, engine.py:440-442)."""
    from thetascan_amd._core.ops import fused, scan_hip

    g = torch.Generator().manual_seed(3)
    q = torch.rand(1, 2, 300, 64, generator=g).to(cuda)
    k = torch.rand(1, 2, 300, 64, generator=g).to(cuda)
    v = torch.randn(1, 2, 300, 64, generator=g).to(cuda)
    (num, unit), = scan_hip.linattn_views_mass(q, k, v, (None,))
    assert rel_err(fused.abs_mass(q, k), unit.double()) < 1e-5


def test_abs_mass_rejects_unsupported_widths(cuda):
    from thetascan_amd._core.ops import fused

    q = torch.zeros(1, 1, 8, 48, device=cuda)
    assert not fused.abs_mass_eligible(q, q)
    with pytest.raises(NotImplementedError):
        fused.abs_mass(q, q)
