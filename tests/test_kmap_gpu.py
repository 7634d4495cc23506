"""Kernel feature maps with their learned controls (ts_kmap_fwd / ts_kmap_bwd).

phi = map(rmsnorm(a) - tau) with the softmax partition (scalar, per-head or
per-feature gain; score bias; relative_soft / relative_st / relative_st_blend
sparsity) or the ReLU^2 ridge (score bias, threshold), against the float64
oracle (oracle/mixer.py: rmsnorm, softmax_partition, relu2_ridge, restated
from kernel_features.py:43-135 and pinned by the golden feature-map vectors).
Forward and the gradients of a, tau, the score bias, the gain, rho and alpha;
ragged T, feature widths 16 / 32 / 48 / 64, bf16 and fp32.  Tolerances: rel
1e-3 (fp32), 2e-2 (bf16) on the map and every gradient (measured at most 2.6e-5
and 3.7e-3); max-abs error over max-abs reference.
"""
from __future__ import annotations

import types

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

CASES = [
    # kind, gain_mode, sparsity, score_bias, tau, relu2_threshold
    ("softmax_partition", "fixed", "none", False, False, False),
    ("softmax_partition", "head", "none", True, True, False),
    ("softmax_partition", "feature", "none", True, False, False),
    ("softmax_partition", "head", "relative_soft", False, True, False),
    ("softmax_partition", "fixed", "relative_st", True, False, False),
    ("softmax_partition", "head", "relative_st_blend", False, False, False),
    ("softmax_partition", "feature", "relative_st_blend", True, True, False),
    ("relu2_ridge", "fixed", "none", True, False, False),
    ("relu2_ridge", "fixed", "none", False, True, True),
]


def oracle_map(a, cfg, tau, gain, bias, rthr, rho, alpha):
    from oracle import mixer as om

    z, _ = om.rmsnorm(a)
    if tau is not None:
        z = z - tau.view(1, tau.shape[0], 1, tau.shape[1])
    if cfg.kernel_kind == "relu2_ridge":
        return om.relu2_ridge(z, score_bias=bias, tau=rthr)
    return om.softmax_partition(z, gain if gain is not None else cfg.softmax_gain, score_bias=bias,
                                sparsity=cfg.kernel_sparsity, rho=rho, blend=alpha,
                                temperature=cfg.kernel_threshold_temperature)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("m", [16, 48, 64])
@pytest.mark.parametrize("case", CASES)
def test_kmap_matches_the_oracle(cuda, dtype, tol, m, case):
    from thetascan_amd._core.ops import kernel_features as kf

    kind, gain_mode, sparsity, has_bias, has_tau, has_rthr = case
    B, H, T = 2, 3, 300
    g0 = torch.Generator().manual_seed(m * 13 + len(sparsity) + (7 if has_bias else 0))
    cfg = types.SimpleNamespace(kernel_kind=kind, softmax_gain=8.0, kernel_sparsity=sparsity,
                                kernel_threshold_temperature=0.25, eps=1e-6)
    a = torch.randn(B, H, T, m, generator=g0).to(dtype).double()
    tau = torch.randn(H, m, generator=g0) * 0.3 if has_tau else None
    bias = torch.randn(H, m, generator=g0) * 0.3 if has_bias else None
    rthr = torch.rand(H, generator=g0) * 0.5 if has_rthr else None
    gain = None
    if gain_mode == "head":
        gain = torch.rand(H, generator=g0) * 6 + 2
    elif gain_mode == "feature":
        gain = torch.rand(H, m, generator=g0) * 6 + 2
    rho = torch.rand(H, generator=g0) * 0.2 + 0.01 if sparsity != "none" else None
    alpha = torch.rand(H, generator=g0) if sparsity == "relative_st_blend" else None
    dphi = torch.randn(B, H, T, m, generator=g0)

    ctl = {"tau": tau, "gain": gain, "bias": bias, "rthr": rthr, "rho": rho, "alpha": alpha}
    ref_leaves = {k: (None if v is None else v.double().requires_grad_(True)) for k, v in ctl.items()}
    a64 = a.clone().requires_grad_(True)
    ref = oracle_map(a64, cfg, ref_leaves["tau"], ref_leaves["gain"], ref_leaves["bias"], ref_leaves["rthr"],
                     ref_leaves["rho"], ref_leaves["alpha"])
    ref.backward(dphi.to(dtype).double())

    dev = {k: (None if v is None else v.to(cuda).requires_grad_(True)) for k, v in ctl.items()}
    ad = a.to(dtype).to(cuda).requires_grad_(True)
    phi = kf.kmap(ad, cfg, rms=True, tau=dev["tau"], softmax_gain=dev["gain"], score_bias=dev["bias"],
                  relu2_threshold=dev["rthr"], relative_threshold=dev["rho"], sparse_blend_alpha=dev["alpha"])
    phi.backward(dphi.to(dtype).to(cuda))
    torch.cuda.synchronize()
    assert phi.dtype == dtype
    assert rel_err(phi.float(), ref) < tol
    assert rel_err(ad.grad.float(), a64.grad) < tol
    for name, leaf in ref_leaves.items():
        if leaf is None:
            continue
        assert rel_err(dev[name].grad, leaf.grad) < tol, name
