"""The long-context workload: a B-spline memory expanded 2x on its projection
rows (8 trainable projections -> 16 -> 16 x 8 basis = 128 features) read
through a bank of four recency rates {0.9, 0.99, 0.999, 0.9999} (GPU tests).

Both are extensions of this build's core config (the reference caps a bank at
two branches and expands only the ReLU^2 map; its public config, like this
one, rejects them).  Checked:
* five retentions (the plain sum and four rates) run as two multi-view passes
  whose outputs equal one-view scans bit for bit;
* the mixer at d_model 512, H8, T 1000 against the float64 oracle, whose
  four-rate blend is pinned by the one-rate identity of
  tests/test_oracle_bank_expansion.py (fp32 rel 1e-3, bf16 rel 2e-2);
* at the workload's T = 32768: deterministic replay and exact causality.
"""
from __future__ import annotations

import dataclasses

import pytest
import torch

from oracle import mixer as oracle_mixer
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

RATES = (0.9, 0.99, 0.999, 0.9999)


def bank4_module(cuda, dtype, seed=0):
    """The workload's mixer (core config) and the oracle's flat config."""
    import thetascan_amd as ts
    from thetascan_amd._core.modules.block import ThetaScan as CoreMixer

    public = ts.ThetaScanConfig(
        d_model=512, n_heads=8, memory_multiplier=2, family="kernel",
        kernel=ts.KernelConfig(feature_map="projected_bspline", read_normalization="key_mass"),
        temporal=ts.TemporalConfig(mode="bank", bank_mode="fast", recency_branches=2, retention_inits=(0.9, 0.999)),
        runtime=ts.RuntimeConfig(backend="hip", scan_chunk=128),
    )
    cfg = dataclasses.replace(public._to_core_config(), feature_expansion=2, fade_branches=4, fade_alpha_inits=RATES)
    torch.manual_seed(seed)
    module = CoreMixer(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.startswith("W2.") or name == "fade_eta":
                p.copy_(torch.randn(p.shape, generator=g) * (0.3 if name == "fade_eta" else 0.02))
    core = dict(oracle_mixer.core_config(public.to_dict()), feature_expansion=2, fade_branches=4)
    return module.to(cuda, dtype), core


@pytest.mark.parametrize("mass", [False, True])
def test_five_retentions_equal_one_view_scans(cuda, mass):
    from thetascan_amd._core.ops import scan_hip

    g = torch.Generator().manual_seed(11)
    B, H, T, dk, dv = 2, 8, 1000, 128, 64
    q = torch.rand(B, H, T, dk, generator=g).to(cuda, torch.bfloat16)
    k = torch.rand(B, H, T, dk, generator=g).to(cuda, torch.bfloat16)
    v = torch.randn(B, H, T, dv, generator=g).to(cuda, torch.bfloat16)
    rets = (None,) + tuple(torch.full((H,), r).log().to(cuda) for r in RATES)
    if mass:
        views = scan_hip.linattn_views_mass(q, k, v, rets)
        for r, (num, m) in zip(rets, views):
            (num1, m1), = scan_hip.linattn_views_mass(q, k, v, (r,))
            assert torch.equal(num, num1) and torch.equal(m, m1)
    else:
        views = scan_hip.linattn_views(q, k, v, rets)
        for r, out in zip(rets, views):
            assert torch.equal(out, scan_hip.linattn(q, k, v, log_alpha=r))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bank4_bspline_mixer_matches_oracle(cuda, dtype):
    module, core = bank4_module(cuda, dtype, seed=7)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 1000, 512, generator=g, dtype=torch.float64).to(dtype).double()
    params = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module.named_parameters()}
    x64 = x.clone().requires_grad_(True)
    y64 = oracle_mixer.forward(core, params, x64, backend="chunk")
    dy = torch.randn(y64.shape, generator=g, dtype=torch.float64) * 0.1
    (y64 * dy).sum().backward()
    xd = x.to(cuda, dtype).requires_grad_(True)
    y = module(xd)
    (y.float() * dy.to(cuda, torch.float32)).sum().backward()
    print(f"bank4 bspline mixer {dtype}: path={module.last_path}", flush=True)
    tol = 1e-3 if dtype == torch.float32 else 2e-2
    assert rel_err(y, y64) < tol
    assert rel_err(xd.grad, x64.grad) < tol
    assert rel_err(module.fade_eta.grad, params["fade_eta"].grad) < tol


def test_bank4_bspline_long_context_determinism_and_causality(cuda):
    module, _ = bank4_module(cuda, torch.bfloat16, seed=3)
    g = torch.Generator().manual_seed(4)
    T, t0 = 32768, 20000
    x = torch.randn(1, T, 512, generator=g).to(cuda, torch.bfloat16)
    with torch.no_grad():
        y1 = module(x)
        y2 = module(x)
        x2 = x.clone()
        x2[:, t0] += 1.0
        y3 = module(x2)
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(y1, y2)
    assert torch.equal(y3[:, :t0], y1[:, :t0])
    assert not torch.equal(y3[:, t0:], y1[:, t0:])
