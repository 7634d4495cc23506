"""Per-row GN hidden activation with its Jacobian scales (ts_gn_act_fwd /
ts_gn_act_bwd) against the float64 oracle.

The reference evaluates a GN block's hidden layer and the per-feature scales
that multiply W2 in its Jacobian payload and Gauss-Newton diagonal in torch
(engine.py:117-158, 180-255).  The oracle restates those formulas
(oracle/mixer.py: rmsnorm, the ACT table and dsilu, pinned through the GN
golden mixer vectors); float64 autograd of them gives every gradient: da, db
and the threshold's.  Every nonlinearity (relu2, silu, tanh and SwiGLU), with
and without a threshold, bf16 and fp32, widths 16 to 256, ragged T.
Tolerances: rel 1e-3 (fp32) and 2e-2 (bf16) on the values and the gradients
(measured at most 6.7e-7 and 3.7e-3); max-abs error over max-abs reference.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def oracle_rows(a, b, tau, nonlin):
    from oracle import mixer as om

    za, ra = om.rmsnorm(a)
    if nonlin == "swiglu":
        zb, rb = om.rmsnorm(b)
        return F.silu(zb) * za, F.silu(zb) * ra, za * om.dsilu(zb) * rb
    z = za if tau is None else za - tau.view(1, tau.shape[0], 1, tau.shape[1])
    act, dact = om.ACT[nonlin]
    return act(z), dact(z) * ra, None


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("m", [16, 48, 64, 128, 256])
@pytest.mark.parametrize("nonlin,has_tau", [("relu2", False), ("relu2", True), ("silu", False), ("silu", True),
                                            ("tanh", True), ("swiglu", False)])
def test_gn_act_matches_the_oracle(cuda, dtype, tol, m, nonlin, has_tau):
    from thetascan_amd._core.ops import gn

    B, H, T = 2, 3, 300
    g0 = torch.Generator().manual_seed(m * 7 + len(nonlin) + (3 if has_tau else 0))
    glu = nonlin == "swiglu"
    a = (torch.randn(B, H, T, m, generator=g0) * 2).to(dtype).double()
    b = (torch.randn(B, H, T, m, generator=g0) * 2).to(dtype).double() if glu else None
    tau = torch.randn(H, m, generator=g0) * 0.3 if has_tau else None
    dh = torch.randn(B, H, T, m, generator=g0)
    dsa = torch.randn(B, H, T, m, generator=g0)
    dsb = torch.randn(B, H, T, m, generator=g0) if glu else None

    ra_ = a.clone().requires_grad_(True)
    rb_ = b.clone().requires_grad_(True) if glu else None
    rt_ = tau.double().requires_grad_(True) if has_tau else None
    h_ref, sa_ref, sb_ref = oracle_rows(ra_, rb_, rt_, nonlin)
    outs, grads = [h_ref, sa_ref], [dh.to(dtype).double(), dsa.to(dtype).double()]
    if glu:
        outs.append(sb_ref)
        grads.append(dsb.to(dtype).double())
    torch.autograd.backward(outs, grads)

    ad = a.to(dtype).to(cuda).requires_grad_(True)
    bd = b.to(dtype).to(cuda).requires_grad_(True) if glu else None
    td = tau.to(cuda).requires_grad_(True) if has_tau else None
    h, sa, sb = gn.act_rows(ad, bd, td, nonlin=nonlin)
    douts = [h, sa] + ([sb] if glu else [])
    torch.autograd.backward(douts, [t.to(dtype).to(cuda) for t in ([dh, dsa] + ([dsb] if glu else []))])
    torch.cuda.synchronize()
    assert h.dtype == dtype and sa.dtype == dtype
    assert rel_err(h.float(), h_ref) < tol
    assert rel_err(sa.float(), sa_ref) < tol
    if glu:
        assert rel_err(sb.float(), sb_ref) < tol
        assert rel_err(bd.grad.float(), rb_.grad) < tol
    assert rel_err(ad.grad.float(), ra_.grad) < tol
    if has_tau:
        assert rel_err(td.grad, rt_.grad) < tol


@pytest.mark.parametrize("nonlin", ["silu", "swiglu"])
def test_gn_act_features_only(cuda, nonlin):
    """The read side asks for h only: no scales are written, and the gradient
    of h alone matches."""
    from thetascan_amd._core.ops import gn

    g0 = torch.Generator().manual_seed(11)
    glu = nonlin == "swiglu"
    a = torch.randn(1, 2, 77, 64, generator=g0, dtype=torch.float64)
    b = torch.randn(1, 2, 77, 64, generator=g0, dtype=torch.float64) if glu else None
    dh = torch.randn(1, 2, 77, 64, generator=g0, dtype=torch.float64)
    ra_ = a.clone().requires_grad_(True)
    rb_ = b.clone().requires_grad_(True) if glu else None
    h_ref = oracle_rows(ra_, rb_, None, nonlin)[0]
    h_ref.backward(dh)
    ad = a.float().to(cuda).requires_grad_(True)
    bd = b.float().to(cuda).requires_grad_(True) if glu else None
    h, sa, sb = gn.act_rows(ad, bd, nonlin=nonlin, want_scales=False)
    assert sa is None and sb is None
    h.backward(dh.float().to(cuda))
    assert rel_err(h, h_ref) < 1e-3
    assert rel_err(ad.grad, ra_.grad) < 1e-3
    if glu:
        assert rel_err(bd.grad, rb_.grad) < 1e-3


def test_gn_act_rejects_bad_calls(cuda):
    from thetascan_amd._core.ops import gn

    a = torch.zeros(1, 1, 8, 12, device=cuda, dtype=torch.bfloat16)  # 12 is not a multiple of 8
    with pytest.raises(NotImplementedError):
        gn.act_rows(a, nonlin="relu2")
    a = torch.zeros(1, 1, 8, 16, device=cuda)
    with pytest.raises(ValueError):
        gn.act_rows(a, nonlin="swiglu")
    with pytest.raises(ValueError):
        gn.act_rows(a, a, nonlin="silu")
