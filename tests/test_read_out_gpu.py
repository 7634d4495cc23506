"""Read fused with the output projection (ts_read_out_fwd / ts_read_out_bwd).

out = y W^T with y = (resid + s * num / (mass + eps)) * silu(g + g_bias)
(block.py:718-724, gates.py:34-40, engine.py:440-442, 526-528).  Checked:

- the y the forward keeps equals ts_read_fwd's bit for bit;
- out against the fp32 product of that y and W (the kernel's only rounding is
  the bf16 store of out: rel 4e-3);
- the whole chain, forward and every gradient (num, mass, resid, g, g_bias),
  against float64 autograd of the same bf16 inputs at rel 2e-2;
- ragged T, one token, head widths 32 / 64 / 128, output widths 128 - 1024
  (several row slices per token tile), with and without the gate, the key-mass
  normalization, the gate bias and the residual.
Metric: max-abs error over max-abs reference.
"""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def chain_reference(num, mass, resid, g, gbias, w, dout, s, eps):
    """float64 autograd of out = read(...) @ w^T on the CPU."""
    leaves = {}

    def leaf(name, t):
        if t is None:
            return None
        x = t.double().cpu().requires_grad_(True)
        leaves[name] = x
        return x

    num_, mass_, resid_, g_, gb_ = leaf("num", num), leaf("mass", mass), leaf("resid", resid), leaf("g", g), \
        leaf("gbias", gbias)
    B, H, T, d = num_.shape
    mem = num_ if mass_ is None else num_ / (mass_.unsqueeze(-1) + eps)
    y = s * mem if resid_ is None else resid_ + s * mem
    if g_ is not None:
        pre = g_ if gb_ is None else g_ + gb_.view(1, H, 1, d)
        y = y * torch.nn.functional.silu(pre)
    y2 = y.transpose(1, 2).reshape(B * T, H * d)
    out = y2 @ w.double().cpu().t()
    out.backward(dout.double().cpu())
    return out.detach(), {k: v.grad for k, v in leaves.items()}


CASES = [
    # B, H, T, d, N
    (2, 8, 300, 64, 512),
    (1, 8, 64, 64, 512),
    (1, 4, 1, 64, 256),
    (2, 4, 130, 32, 128),
    (1, 4, 97, 128, 384),
    (1, 8, 70, 64, 1024),
]
FLAGS = [
    # normalize, gate, bias, resid
    (False, True, True, True),
    (True, True, False, True),
    (True, False, False, True),
    (False, False, False, False),
    (True, True, True, True),
]


@pytest.mark.parametrize("B,H,T,d,N", CASES)
@pytest.mark.parametrize("normalize,gate,bias,has_resid", FLAGS)
def test_read_out_matches_the_read_and_the_product(cuda, B, H, T, d, N, normalize, gate, bias, has_resid):
    from thetascan_amd._core.ops import fused

    dt = torch.bfloat16
    g0 = torch.Generator().manual_seed(B * 7919 + T * 31 + d + N)
    K = H * d
    num = torch.randn(B, H, T, d, generator=g0).to(dt)
    resid = torch.randn(B, H, T, d, generator=g0).to(dt) if has_resid else None
    mass = torch.rand(B, H, T, generator=g0) * 3 + 0.1 if normalize else None
    # the gate as a strided view of a token-major [B, T, 2K] projection buffer
    gbuf = (torch.randn(B, T, 2 * K, generator=g0) * 2).to(dt) if gate else None
    gview = None if gbuf is None else gbuf[..., K:].reshape(B, T, H, d).transpose(1, 2)
    gbias = torch.randn(K, generator=g0) * 0.5 if bias else None
    w = (torch.randn(N, K, generator=g0) / K ** 0.5).to(dt)
    dout = (torch.randn(B * T, N, generator=g0) * 0.1).to(dt)
    s, eps = 0.7, 1e-6
    ref_out, ref_grads = chain_reference(num, mass, resid, gview, gbias, w, dout, s, eps)

    dev = lambda t: None if t is None else t.to(cuda)  # noqa: E731
    num_d, resid_d, mass_d, gbias_d, w_d, dout_d = map(dev, (num, resid, mass, gbias, w, dout))
    gbuf_d = dev(gbuf)
    g_d = None if gbuf_d is None else gbuf_d[..., K:].reshape(B, T, H, d).transpose(1, 2)
    assert fused.read_out_supported(B, H, T, d, N, dt)

    out = torch.full((B * T, N), float("nan"), dtype=dt, device=cuda)
    y = torch.full((B * T, K), float("nan"), dtype=dt, device=cuda)
    fused.read_out_fwd(num_d, mass_d, resid_d, g_d, w_d, out, y, s, eps, gbias=gbias_d)
    # y equals the read kernel's
    y_read = torch.empty(B, T, H, d, dtype=dt, device=cuda)
    fused.read_fwd(num_d, mass_d, resid_d, g_d, y_read.transpose(1, 2), s, eps, gbias=gbias_d)
    assert torch.equal(y.view(B, T, H, d), y_read)
    # out is y W^T up to the bf16 rounding of out
    prod = (y.float() @ w_d.float().t())
    assert rel_err(out.float(), prod) < 4e-3
    assert rel_err(out.float().cpu(), ref_out) < 2e-2

    w_t = w_d.t().contiguous()
    dnum, dmass, (dresid, _), dg, dgb = fused.read_out_bwd(
        num_d, mass_d, resid_d, g_d, w_t, dout_d, s, eps, gbias=gbias_d,
        gbias_grad=torch.float32 if (gate and bias) else None)
    torch.cuda.synchronize()
    assert rel_err(dnum.float().cpu(), ref_grads["num"]) < 2e-2
    if has_resid:
        assert rel_err(dresid.float().cpu(), ref_grads["resid"]) < 2e-2
    if normalize:
        assert rel_err(dmass.cpu(), ref_grads["mass"]) < 2e-2
    if gate:
        assert rel_err(dg.float().cpu(), ref_grads["g"]) < 2e-2
    if gate and bias:
        assert rel_err(dgb.float().cpu(), ref_grads["gbias"]) < 2e-2


def test_read_out_backward_matches_the_unfused_backward(cuda):
    """Against ts_read_bwd fed with dy = dout W formed in fp32: the two differ
    only by dy's bf16 rounding in the unfused path."""
    from thetascan_amd._core.ops import fused

    dt = torch.bfloat16
    B, H, T, d, N = 2, 8, 200, 64, 512
    K = H * d
    g0 = torch.Generator().manual_seed(5)
    num = torch.randn(B, H, T, d, generator=g0).to(dt).to(cuda)
    resid = torch.randn(B, H, T, d, generator=g0).to(dt).to(cuda)
    mass = (torch.rand(B, H, T, generator=g0) * 3 + 0.1).to(cuda)
    gbuf = (torch.randn(B, T, K, generator=g0) * 2).to(dt).to(cuda)
    g = gbuf.view(B, T, H, d).transpose(1, 2)
    gbias = (torch.randn(K, generator=g0) * 0.5).to(cuda)
    w = (torch.randn(N, K, generator=g0) / K ** 0.5).to(dt).to(cuda)
    dout = (torch.randn(B * T, N, generator=g0) * 0.1).to(dt).to(cuda)
    dy = (dout.float() @ w.float()).to(dt).view(B, T, H, d).transpose(1, 2)
    a = fused.read_bwd(num, mass, resid, g, dy, 0.7, 1e-6, gbias=gbias, gbias_grad=torch.float32)
    b = fused.read_out_bwd(num, mass, resid, g, w.t().contiguous(), dout, 0.7, 1e-6, gbias=gbias,
                           gbias_grad=torch.float32)
    for x, z in ((a[0], b[0]), (a[1], b[1]), (a[2][0], b[2][0]), (a[3], b[3]), (a[4], b[4])):
        assert rel_err(z.float(), x.float()) < 1e-2


def test_read_out_rejects_shapes_it_does_not_tile(cuda):
    from thetascan_amd._core.ops import fused

    assert not fused.read_out_supported(1, 3, 64, 64, 512, torch.bfloat16)   # H*d = 192
    assert not fused.read_out_supported(1, 8, 64, 64, 500, torch.bfloat16)   # N not a multiple of 128
    assert not fused.read_out_supported(1, 8, 64, 64, 512, torch.float32)    # bf16 only
    assert not fused.read_out_supported(1, 16, 64, 64, 512, torch.bfloat16)  # H*d > 512
