"""Value-anchor deposit (ts_anchor_fwd / ts_anchor_bwd) against float64 autograd.

r = softmax(gain * C (v / max(||v||, eps))) over a codebook C [1|H, V, d]
(engine.py:284-296).  Checked: the code r, dL/dv and dL/dC (a shared
codebook's gradient summed over heads) for bf16 and fp32, value widths 16-128,
5-64 anchors, ragged T, values as a strided view of a projection, and a value
row of zeros (the eps floor of the norm).  Tolerances: rel 1e-3 (fp32),
2e-2 (bf16); max-abs error over max-abs reference.
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def reference(v, c, gain, eps, dr):
    v = v.double().cpu().requires_grad_(True)
    c = c.double().cpu().requires_grad_(True)
    ce = c if c.shape[0] == v.shape[1] else c.expand(v.shape[1], -1, -1)
    vn = v / v.norm(dim=-1, keepdim=True).clamp_min(eps)
    r = torch.softmax(gain * torch.einsum("hvd,bhtd->bhtv", ce, vn), -1)
    r.backward(dr.double().cpu())
    return r.detach(), v.grad, c.grad


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("B,H,T,d,V,shared", [(2, 2, 37, 16, 5, True), (1, 4, 300, 64, 8, False),
                                              (1, 2, 100, 128, 64, True), (2, 1, 257, 32, 17, True)])
def test_anchor_code_matches_autograd(cuda, dtype, tol, B, H, T, d, V, shared):
    from thetascan_amd._core.ops import maps

    g0 = torch.Generator().manual_seed(B * 100 + T + d + V)
    # values as the v slot of a [B, T, 3, H, d] projection
    proj = torch.randn(B, T, 3, H, d, generator=g0)
    proj[0, 3, 2, 0] = 0.0  # a zero value row: the norm's eps floor
    c = torch.randn(1 if shared else H, V, d, generator=g0) / d ** 0.5
    dr = torch.randn(B, H, T, V, generator=g0)
    gain = 8.0
    v_in = proj.to(dtype).float()[:, :, 2].transpose(1, 2)
    r64, dv64, dc64 = reference(v_in, c, gain, 1e-6, dr.to(dtype).float())

    pd = proj.to(dtype).to(cuda).requires_grad_(True)
    v = pd[:, :, 2].transpose(1, 2)
    cd = c.to(cuda).requires_grad_(True)
    r = maps.anchor_code(v, cd, gain=gain, eps=1e-6)
    assert r.dtype == dtype and r.shape == (B, H, T, V)
    r.backward(dr.to(dtype).to(cuda))
    torch.cuda.synchronize()
    assert rel_err(r.float(), r64) < tol
    dv = pd.grad[:, :, 2].transpose(1, 2)
    assert rel_err(dv.float(), dv64) < tol
    assert rel_err(cd.grad, dc64) < tol
    assert torch.all(pd.grad[:, :, :2] == 0)
