"""The decayed prefix (ts_wcumsum) against the oracle (GPU tests).

The key-mass prefixes of the feature-mass read (src/thetascan/_core/ops/
interface.py:58-107, 216-230): the plain prefix, the static-retention
``ema_cumsum`` and the per-token decayed stream, causal and anti-causal, at
T = 80, 4096 and 32768 (one to thousands of time segments), with rows taken
four features at a time and, for unaligned rows, one at a time, plus the
gradients of the prefix input and of the retention through the autograd op.
fp32 throughout; rel 1e-4 forward, rel 1e-3 for gradients.
"""
from __future__ import annotations

import pytest
import torch

from oracle import scans as oracle
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, F, kind, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, T, F, generator=g, dtype=torch.float64).float().double()
    ret = None
    if kind == "static":
        ret = torch.log(torch.rand(H, generator=g, dtype=torch.float64) * 0.099 + 0.9).float().double()
    elif kind == "stream":
        ret = (-torch.rand(B, H, T, 1, generator=g, dtype=torch.float64) * 0.05).float().double()
    return x, ret


def _oracle(x, ret, reverse):
    """z_t = a_t z_{t-1} + x_t in float64 (anti-causal: a flipped scan whose
    step into t uses the decay of t + 1)."""
    if reverse:
        x = x.flip(2)
        if ret is not None and ret.ndim == 4:
            shifted = torch.zeros_like(ret)
            shifted[:, :, 1:] = ret.flip(2)[:, :, :-1]
            ret = shifted
    if ret is None:
        out = oracle.causal_prefix_sum(x)
    elif ret.ndim == 1:
        out = oracle.ema_cumsum(x, ret)
    else:
        ones = torch.ones(*x.shape[:3], 1, dtype=x.dtype)
        out = oracle.linattn_chunk(ones, ones, x, ret)
    return out.flip(2) if reverse else out


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
@pytest.mark.parametrize("T", [80, 4096, 32768])
def test_decayed_prefix_matches_oracle(cuda, T, kind, reverse):
    from thetascan_amd._core.ops import fused

    B, H, F = 2, 3, 40
    x, ret = _inputs(B, H, T, F, kind, seed=T + (7 if reverse else 0))
    expected = _oracle(x, ret, reverse)
    r_dev = None if ret is None else ret.to(cuda, torch.float32)
    got = fused.wcumsum(x.to(cuda, torch.float32), r_dev, reverse)
    print(f"wcumsum T={T} {kind} reverse={reverse}", flush=True)
    assert got.dtype == torch.float32 and got.shape == expected.shape
    assert rel_err(got, expected) < 1e-4


@pytest.mark.parametrize("layout", ["six_features", "unaligned_view"])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_decayed_prefix_one_feature_per_thread(cuda, kind, layout):
    """Rows that are not 16-byte aligned (a feature count that is not a
    multiple of four, or a view starting one float into its storage) take the
    one-feature-per-thread kernels; same bar as above."""
    from thetascan_amd._core.ops import fused

    B, H, T = 2, 3, 4096
    F = 6 if layout == "six_features" else 40
    x, ret = _inputs(B, H, T, F, kind, seed=31)
    expected = _oracle(x, ret, False)
    r_dev = None if ret is None else ret.to(cuda, torch.float32)
    if layout == "unaligned_view":
        wide = torch.zeros(B, H, T, F + 1, device=cuda, dtype=torch.float32)
        wide[..., 1:] = x.to(cuda, torch.float32)
        xd = wide[..., 1:]
        assert xd.data_ptr() % 16 != 0 and xd.stride(-1) == 1
    else:
        xd = x.to(cuda, torch.float32)
    got = fused.wcumsum(xd, r_dev, False)
    print(f"wcumsum {layout} {kind}", flush=True)
    assert rel_err(got, expected) < 1e-4


@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_decayed_prefix_gradients(cuda, kind):
    """Gradients of x and of the retention through interface.ema_cumsum /
    causal_prefix_sum / decayed_prefix against float64 autograd."""
    from thetascan_amd._core.ops import interface

    B, H, T, F = 2, 3, 4096, 24
    x, ret = _inputs(B, H, T, F, kind, seed=99)
    dy = torch.randn(B, H, T, F, generator=torch.Generator().manual_seed(98), dtype=torch.float64)
    x64 = x.clone().requires_grad_(True)
    r64 = None if ret is None else ret.clone().requires_grad_(True)
    (_oracle(x64, r64, False) * dy).sum().backward()
    xd = x.to(cuda, torch.float32).requires_grad_(True)
    rd = None if ret is None else ret.to(cuda, torch.float32).requires_grad_(True)
    if kind == "none":
        out = interface.causal_prefix_sum(xd)
    elif kind == "static":
        out = interface.ema_cumsum(xd, rd)
    else:
        out = interface.decayed_prefix(xd, rd)
    (out * dy.to(cuda, torch.float32)).sum().backward()
    assert rel_err(out, _oracle(x, ret, False)) < 1e-4
    assert rel_err(xd.grad, x64.grad) < 1e-3
    if rd is not None:
        g_ref = r64.grad
        if kind == "stream":
            g_ref = g_ref.clone()
            g_ref[:, :, 0] = 0.0  # the first token's decay multiplies no stored state
        assert rel_err(rd.grad, g_ref) < 1e-3


def test_decayed_prefix_reads_strided_views(cuda):
    """A [B,T,H,F] buffer viewed as [B,H,T,F] (non-contiguous head stride) and
    an output view with padded rows give the same prefix."""
    from thetascan_amd._core.ops import fused

    B, H, T, F = 2, 4, 700, 16
    g = torch.Generator().manual_seed(5)
    base = torch.randn(B, T, H, F, generator=g)
    view = base.to(cuda).transpose(1, 2)
    la = torch.log(torch.tensor([0.9, 0.95, 0.99, 0.5])).to(cuda)
    got = fused.wcumsum(view, la, False)
    expected = oracle.ema_cumsum(base.transpose(1, 2).double(), la.double().cpu())
    assert rel_err(got, expected) < 1e-4
