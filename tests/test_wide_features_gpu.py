"""Feature widths of 192 and 384 on the chunked feature kernels (GPU tests).

The published expanded kernel preset has m = 384 (192 trainable projection
rows, sign-expanded twice); a memory multiplier of 3 at head width 64, or of
6 at head width 32, gives m = 192.  These widths run the chunked kernels in
bf16 (the feature axis walked 64 features at a time).  Each mixer below runs
them on the multi-view path and is checked against the float64 oracle, across
both feature maps, input and feature RoPE, the learned ReLU^2 threshold,
shared key/query, banks, the ema stream and the plain sum, with a ragged last
tile.  ReLU^2 mixers take the bf16 bar, rel 2e-2, on outputs, dx and every
parameter gradient (measured at most 1.6e-2).  The softmax partition at
sharpness 8 multiplies the bf16 rounding of its pre-activations by 8: on the
same configurations the 64- and 128-wide feature kernels reach 2.4-2.5 % in dx
and the composed bf16 path 5-7 %, so the softmax mixers take 3e-2 (outputs,
dx) and 4e-2 (parameters); measured at most 2.9e-2 (m = 192) and 3.3e-2
(m = 384).
"""
from __future__ import annotations

import pytest
import torch

import thetascan_amd as ts
from oracle import mixer as oracle_mixer
from tests.conftest import rel_err
from tests.test_mixer_gpu import _headline_config, _seeded, build_module

pytestmark = pytest.mark.gpu


def _preset(d_model=128, heads=2):
    """kernel_expanded_reference_v0_1 at a small model width (head width 64, m = 384)."""
    pub = ts.ThetaScanConfig.kernel_expanded_reference_v0_1(d_model=d_model, n_heads=heads).to_dict()
    pub["runtime"].update(backend="hip", scan_chunk=64)
    return pub


def _case(name):
    if name == "preset_m384":
        return _preset()
    if name == "softmax_m192_feature_rope_ema":
        pub = _headline_config("feature", "none", "softmax_partition", d_model=128, heads=2, mult=3)
        pub["temporal"]["mode"] = "ema"
        return pub
    if name == "relu2_m192_d32_input_rope_sum":
        return _headline_config("input", "key_mass", "relu2_ridge", d_model=128, heads=4, mult=6)
    if name == "softmax_m384_stale_bank":
        pub = _headline_config("input", "key_mass", "softmax_partition", d_model=128, heads=2, mult=6)
        pub["temporal"].update(mode="bank", bank_mode="stale", recency_branches=2, retention_inits=[0.9, 0.99])
        return pub
    raise KeyError(name)


@pytest.mark.parametrize("name", ["preset_m384", "softmax_m192_feature_rope_ema", "relu2_m192_d32_input_rope_sum",
                                  "softmax_m384_stale_bank"])
def test_wide_feature_mixer_matches_float64_oracle(cuda, name):
    pub = _case(name)
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 5)
    with torch.no_grad():
        for pname, p in module._core.named_parameters():
            if pname in ("fade_eta", "kernel_relu2_threshold"):
                p.copy_(torch.randn(p.shape, generator=torch.Generator().manual_seed(6)) * 0.3)
    core = oracle_mixer.core_config(pub)
    assert core["mem_hidden"] in (192, 384)
    params64 = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module._core.named_parameters()}
    g = torch.Generator().manual_seed(7)
    B, T, D = 2, 150, pub["d_model"]
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, D, generator=g, dtype=torch.float64) * 0.1
    x64 = x.clone().requires_grad_(True)
    y64 = oracle_mixer.forward(core, params64, x64)
    (y64 * dy).sum().backward()

    module = module.to(torch.bfloat16)
    xb = x.to(cuda, torch.bfloat16).requires_grad_(True)
    yb = module(xb)
    print(f"wide {name}: m={core['mem_hidden']} path={module._core.last_path}", flush=True)
    assert module._core.last_path == "fused"
    (yb.float() * dy.to(cuda, torch.float32)).sum().backward()
    tol, ptol = (3e-2, 4e-2) if "softmax" in name else (2e-2, 2e-2)
    assert rel_err(yb, y64) < tol
    assert rel_err(xb.grad, x64.grad) < tol
    for pname, p in module._core.named_parameters():
        if params64[pname].grad is not None and params64[pname].grad.abs().max() > 0:
            assert rel_err(p.grad, params64[pname].grad) < ptol, pname


def test_wide_widths_stay_on_the_composed_path_in_fp32(cuda):
    """The chunked kernels are bf16 only: an fp32 mixer at m = 384 takes the
    composed path and still matches the oracle at the fp32 bar."""
    pub = _preset()
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 5)
    core = oracle_mixer.core_config(pub)
    params64 = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module._core.named_parameters()}
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 70, pub["d_model"], generator=g, dtype=torch.float64)
    y64 = oracle_mixer.forward(core, params64, x)
    y = module(x.to(cuda, torch.float32))
    assert module._core.last_path == "composed"
    assert rel_err(y, y64) < 1e-3
