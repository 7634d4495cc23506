"""Read epilogue kernels (ts_read_fwd / ts_read_bwd) against float64 autograd.

y = (resid + s * num / (mass + eps)) * silu(g + g_bias)   (engine.py:440-442,
526-528; gates.py:34-40).  Covered: ragged T, head widths whose 16-byte chunk
count is not a power of two, strided gate / output views, with and without
the gate, the key-mass normalization and the gate bias, and the gate-bias
gradient the backward forms from per-workgroup column sums.  Tolerances: rel
1e-3 (fp32), 2e-2 (bf16), max-abs error over max-abs reference.
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def reference(num, mass, resid, g, gbias, dy, s, eps):
    num, resid, dy = (t.double().cpu().requires_grad_(True) for t in (num, resid, dy))
    mass_ = None if mass is None else mass.double().cpu().requires_grad_(True)
    g_ = None if g is None else g.double().cpu().requires_grad_(True)
    gb_ = None if gbias is None else gbias.double().cpu().requires_grad_(True)
    mem = num if mass_ is None else num / (mass_.unsqueeze(-1) + eps)
    y = resid + s * mem
    if g_ is not None:
        H, d = g_.shape[1], g_.shape[-1]
        pre = g_ if gb_ is None else g_ + gb_.view(1, H, 1, d)
        y = y * torch.nn.functional.silu(pre)
    y.backward(dy)
    return y.detach(), num.grad, None if mass_ is None else mass_.grad, resid.grad, \
        None if g_ is None else g_.grad, None if gb_ is None else gb_.grad.view(-1)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("B,H,T,d", [(2, 3, 37, 64), (1, 2, 1, 16), (2, 2, 300, 48), (1, 1, 513, 128),
                                     (1, 2, 130, 24)])
@pytest.mark.parametrize("normalize,gate,bias", [(False, True, True), (True, True, False), (True, False, False),
                                                 (False, False, False)])
def test_read_kernels_match_autograd(cuda, dtype, tol, B, H, T, d, normalize, gate, bias):
    from thetascan_amd._core.ops import fused

    vec = 16 // torch.tensor([], dtype=dtype).element_size()
    if d % vec:
        pytest.skip("width must be a multiple of 16 bytes")
    g0 = torch.Generator().manual_seed(B * 1000 + T + d)
    num = torch.randn(B, H, T, d, generator=g0)
    resid = torch.randn(B, H, T, d, generator=g0)
    mass = torch.rand(B, H, T, generator=g0) * 3 + 0.1 if normalize else None
    # gate and output as strided views of token-major [B, T, H * d] buffers
    gbuf = torch.randn(B, T, 2 * H * d, generator=g0) * 2 if gate else None
    gbias = torch.randn(H * d, generator=g0) * 0.5 if bias else None
    dy = torch.randn(B, H, T, d, generator=g0)
    s, eps = 0.7, 1e-6
    q = lambda t: None if t is None else t.to(dtype).float()  # noqa: E731  (inputs as the kernel sees them)
    g_view = None if gbuf is None else gbuf[..., H * d:].reshape(B, T, H, d).transpose(1, 2)
    ref = reference(q(num), mass, q(resid), q(g_view), gbias, q(dy), s, eps)

    dev = lambda t: None if t is None else t.to(cuda)  # noqa: E731
    numd, residd, dyd = (t.to(cuda, dtype) for t in (num, resid, dy))
    gd = None
    if gbuf is not None:
        gd = gbuf.to(cuda, dtype)[..., H * d:].view(B, T, H, d).transpose(1, 2)
    y = torch.empty(B, T, H * d, dtype=dtype, device=cuda).view(B, T, H, d).transpose(1, 2)
    fused.read_fwd(numd, dev(mass), residd, gd, y, s, eps, gbias=dev(gbias))
    assert rel_err(y, ref[0]) < tol
    dg = torch.empty(B, T, H, d, dtype=dtype, device=cuda).transpose(1, 2) if gate else None
    dnum, dmass, (dresid, _), dg, dgb = fused.read_bwd(numd, dev(mass), residd, gd, dyd, s, eps, dg=dg,
                                                       gbias=dev(gbias),
                                                       gbias_grad=torch.float32 if bias else None)
    assert rel_err(dnum, ref[1]) < tol
    assert rel_err(dresid, ref[3]) < tol
    if normalize:
        assert rel_err(dmass, ref[2]) < tol
    if gate:
        assert rel_err(dg, ref[4]) < tol
    if bias:
        assert rel_err(dgb, ref[5]) < tol
