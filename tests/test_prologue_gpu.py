"""Query/key prologue kernels (ts_qknorm_fwd / ts_qknorm_bwd) against float64
autograd of the reference's input RoPE and L2 norm (rope.py:41-49 with fp32
angles, norms.py:11-12): strided views of a token-major projection, full,
partial and no rotation, a row below eps, fp32 (rel 1e-3) and bf16 (rel 2e-2).
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def reference(x, rot, base, eps):
    x = x.double().cpu().requires_grad_(True)
    y = x
    if rot:
        T = x.shape[2]
        inv = 1.0 / (base ** (torch.arange(0, rot, 2, dtype=torch.float32) / rot))
        ang = torch.outer(torch.arange(T, dtype=torch.float32), inv).double()
        cos, sin = ang.cos(), ang.sin()
        x1, x2 = x[..., :rot:2], x[..., 1:rot:2]
        out = torch.stack((x1 * cos - x2 * sin, x1 * sin + x2 * cos), dim=-1).flatten(-2)
        y = torch.cat((out, x[..., rot:]), dim=-1)
    return y / y.norm(dim=-1, keepdim=True).clamp_min(eps), x


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("B,H,T,d,rot", [(2, 3, 37, 64, 32), (1, 2, 300, 64, 64), (2, 2, 129, 48, 0),
                                         (1, 1, 5, 16, 2)])
def test_qk_norm_matches_autograd(cuda, dtype, tol, B, H, T, d, rot):
    from thetascan_amd._core.ops import prologue

    vec = 16 // torch.tensor([], dtype=dtype).element_size()
    if d % vec:
        pytest.skip("width must be a multiple of 16 bytes")
    g = torch.Generator().manual_seed(B * 100 + T + d + rot)
    proj = torch.randn(B, T, 3, H, d, generator=g)
    proj[0, 0, 1, 0] = 1e-9  # one key row below eps
    eps = 1e-6
    dy = torch.randn(B, H, T, d, generator=g)
    for part in (0, 1):  # q, k views of the token-major projection
        x = proj.to(dtype)[:, :, part].permute(0, 2, 1, 3)
        y_ref, x64 = reference(x.float(), rot, 10000.0, eps)
        (y_ref * dy.double()).sum().backward()
        xd = proj.to(cuda, dtype)[:, :, part].permute(0, 2, 1, 3).detach().requires_grad_(True)
        y = prologue.qk_norm(xd, rot, 10000.0, eps)
        assert y is not None, "the strided projection view must take the kernel"
        assert rel_err(y, y_ref) < tol
        y.backward(dy.to(cuda, dtype))
        assert rel_err(xd.grad, x64.grad) < tol
