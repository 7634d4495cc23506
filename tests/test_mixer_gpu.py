"""Mixer parity on the GPU (hip backend) against the reference.

* Every golden case (written from the reference, float64) is loaded into the
  MI355X module by state dict and run in fp32 on the GPU: outputs, the input
  gradient and every parameter gradient must match the reference within rel
  1e-3 (fp32 bar; measured at most 2.3e-5, 2.8e-4 and 3.2e-4, all in the
  sparse straight-through blend case).
* The fused three-kernel path and the composed path agree with each other.
* bf16 runs at benchmark-like widths match the float64 CPU oracle within rel
  2e-2 (the bf16 bar), forward and backward.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import mixer as oracle_mixer
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "mixer_cases.json").read_text())


def build_module(pub: dict, device, dtype=torch.float32):
    import thetascan_amd as ts

    pub = json.loads(json.dumps(pub))
    pub["runtime"]["backend"] = "hip"
    # the initial weights do not depend on which tests ran before
    torch.manual_seed(0)
    return ts.ThetaScan(ts.ThetaScanConfig.from_dict(pub)).to(device=device, dtype=dtype)


def load_golden(name):
    data = np.load(GOLDEN / f"mixer_{name}.npz", allow_pickle=False)
    state = {k[len("param:"):]: torch.from_numpy(data[k]) for k in data.files if k.startswith("param:")}
    for k in data.files:
        if k.startswith("buffer:"):
            state[k[len("buffer:"):]] = torch.from_numpy(data[k])
    grads = {k[len("grad:"):]: torch.from_numpy(data[k]) for k in data.files
             if k.startswith("grad:") and k != "grad:x"}
    return state, grads, {k: torch.from_numpy(data[k]) for k in ("x", "dy", "y", "grad:x")}


@pytest.mark.parametrize("name", sorted(CASES))
def test_mixer_matches_reference_golden(cuda, name):
    state, grads, arr = load_golden(name)
    module = build_module(CASES[name]["config"], cuda)
    module.load_state_dict({k: v.to(torch.float32) if v.is_floating_point() else v for k, v in state.items()},
                           strict=True)
    x = arr["x"].to(cuda, torch.float32).requires_grad_(True)
    from thetascan_amd import _lib

    with _lib.record_launches() as launches:
        y = module(x)
        (y * arr["dy"].to(cuda, torch.float32)).sum().backward()
        torch.cuda.synchronize()
    print(f"{name}: path={module._core.last_path}", flush=True)
    assert rel_err(y, arr["y"]) < 1e-3, name
    if CASES[name]["config"]["family"] == "gn":
        # every GN write runs its nonlinear core in a HIP kernel: the fused
        # depth-1 write, or the per-row activation (any depth, two steps, SwiGLU)
        names = {r[0] for r in launches}
        assert names & {"ts_gn_write_fwd", "ts_gn_act_fwd"}, (name, sorted(names))
        assert names & {"ts_gn_write_bwd", "ts_gn_act_bwd"}, (name, sorted(names))
    params = dict(module.named_parameters())
    worst = max((rel_err(params[p].grad, g), p) for p, g in grads.items() if params[p].grad is not None)
    print(f"errors {name}: y {rel_err(y, arr['y']):.2e} dx {rel_err(x.grad, arr['grad:x']):.2e} "
          f"worst parameter gradient {worst[0]:.2e} ({worst[1]})", flush=True)
    assert rel_err(x.grad, arr["grad:x"]) < 1e-3, name
    for pname, g in grads.items():
        assert params[pname].grad is not None, (name, pname)
        assert rel_err(params[pname].grad, g) < 1e-3, (name, pname)


def _headline_config(placement: str, normalization: str, feature_map="relu2_ridge", d_model=512, heads=8,
                     mult=1):
    return {
        "d_model": d_model, "n_heads": heads, "head_dim": None, "memory_multiplier": mult,
        "feature_expansion": 1, "expansion_key": "thetascan", "depth": 1, "share_key_query": False,
        "key_value_heads": None, "output_gate": True, "family": "kernel",
        "gn": {"nonlinearity": "relu2", "jacobian_steps": 1, "read_normalization": "none"},
        "kernel": {"feature_map": feature_map, "value_representation": "raw", "value_anchors": 8,
                   "value_mlp_multiplier": 1.0, "kernel_sharpness": 8.0, "kernel_sharpness_mode": "fixed",
                   "score_bias": False, "relu2_threshold_mode": "none", "sparsity": "none",
                   "sparse_blend_init": 0.0, "relative_threshold_init": 0.01, "threshold_temperature": 0.25,
                   "bspline_basis_count": 8, "bspline_degree": 3, "bspline_bound": 3.0, "bspline_scale": 1.0,
                   "bspline_scale_mode": "fixed", "feature_parameters_trainable": True,
                   "read_normalization": normalization},
        "rope": {"mode": "partial", "fraction": 0.5, "base": 10000.0, "placement": placement},
        "temporal": {"mode": "sum", "bank_mode": "fast", "retention_init": 0.9, "recency_branches": 1,
                     "retention_inits": None, "half_life_inits": None, "blend_mode": "free"},
        "regularization": {"feature_weight": 0.0, "head_weight": 0.0, "value_mlp_weight": 0.0},
        "runtime": {"backend": "hip", "scan_chunk": 64},
    }


def _seeded(module, seed=0, w2_std=0.02):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters()):
            if name.endswith("W2.0"):
                p.copy_(torch.randn(p.shape, generator=g) * w2_std)
            elif name.endswith("ogate.g.lin.weight"):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)


@pytest.mark.parametrize("variant", [("feature", "none"), ("input", "key_mass"), ("input", "none")])
@pytest.mark.parametrize("feature_map", ["relu2_ridge", "softmax_partition"])
def test_fused_and_composed_paths_agree(cuda, variant, feature_map):
    placement, normalization = variant
    pub = _headline_config(placement, normalization, feature_map, d_model=256, heads=4)
    module = build_module(pub, cuda)
    _seeded(module, 1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 200, 256, generator=g).to(cuda)
    dy = torch.randn(2, 200, 256, generator=g).to(cuda)
    outs, grads = [], []
    for force_composed in (False, True):
        module.zero_grad()
        xi = x.clone().requires_grad_(True)
        if force_composed:
            module._core.fused_eligible = lambda _x: False
        y = module(xi)
        assert module._core.last_path == ("composed" if force_composed else "fused")
        (y * dy).sum().backward()
        outs.append(y.detach())
        grads.append([xi.grad] + [p.grad.clone() for p in module.parameters()])
    assert rel_err(outs[0], outs[1]) < 1e-4
    for a, b in zip(grads[0], grads[1]):
        assert rel_err(a, b) < 1e-3


@pytest.mark.parametrize("case", ["input_full_d128", "feature_full_m128"])
def test_fused_and_composed_agree_with_full_rotations(cuda, case):
    """Rotations wider than 64 dims or features: the feature kernels preload
    the factors of the first four 16-wide blocks and read the tables of the
    others where they are applied; both parts against the composed path."""
    if case == "input_full_d128":
        pub = _headline_config("input", "key_mass", d_model=512, heads=4)  # head width 128, m = 128
    else:
        pub = _headline_config("feature", "none", d_model=256, heads=4, mult=2)  # head width 64, m = 128
    pub["rope"]["fraction"] = 1.0
    module = build_module(pub, cuda)
    _seeded(module, 3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 150, pub["d_model"], generator=g).to(cuda)
    dy = torch.randn(2, 150, pub["d_model"], generator=g).to(cuda)
    outs, grads = [], []
    for force_composed in (False, True):
        module.zero_grad()
        xi = x.clone().requires_grad_(True)
        if force_composed:
            module._core.fused_eligible = lambda _x: False
        y = module(xi)
        print(f"full rotation {case}: path={module._core.last_path}", flush=True)
        assert module._core.last_path == ("composed" if force_composed else "fused")
        (y * dy).sum().backward()
        outs.append(y.detach())
        grads.append([xi.grad] + [p.grad.clone() for p in module.parameters()])
    assert rel_err(outs[0], outs[1]) < 1e-4
    for a, b in zip(grads[0], grads[1]):
        assert rel_err(a, b) < 1e-3


@pytest.mark.parametrize("variant", [("feature", "none"), ("input", "key_mass")])
def test_headline_bf16_matches_float64_oracle(cuda, variant):
    """The benchmark mixer (kernel, ReLU^2 ridge, m=d=64, H=8, d_model=512) in
    bf16 on the GPU against the float64 oracle, at T=256 (rel 2e-2)."""
    placement, normalization = variant
    pub = _headline_config(placement, normalization)
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 3)
    core = oracle_mixer.core_config(pub)
    params64 = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module._core.named_parameters()}
    g = torch.Generator().manual_seed(4)
    B, T = 2, 256
    x = torch.randn(B, T, 512, generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, 512, generator=g, dtype=torch.float64) * 0.1
    x64 = x.clone().requires_grad_(True)
    y64 = oracle_mixer.forward(core, params64, x64)
    (y64 * dy).sum().backward()

    module = module.to(torch.bfloat16)
    xb = x.to(cuda, torch.bfloat16).requires_grad_(True)
    yb = module(xb)
    assert module._core.last_path == "fused"
    (yb.float() * dy.to(cuda, torch.float32)).sum().backward()
    assert rel_err(yb, y64) < 2e-2
    assert rel_err(xb.grad, x64.grad) < 2e-2
    for name, p in module._core.named_parameters():
        if params64[name].grad is not None and params64[name].grad.abs().max() > 0:
            assert rel_err(p.grad, params64[name].grad) < 3e-2, name


def test_cpu_input_raises_instead_of_falling_back(cuda):
    import thetascan_amd as ts

    module = ts.ThetaScan(ts.ThetaScanConfig(d_model=64, n_heads=2, family="kernel"))
    with pytest.raises(RuntimeError, match="GPU"):
        module(torch.randn(1, 8, 64))


@pytest.mark.parametrize("variant", [("feature", "none"), ("input", "key_mass")])
@pytest.mark.parametrize("feature_map", ["relu2_ridge", "softmax_partition"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_call_memory_matches_per_entry_calls(cuda, variant, feature_map, dtype, monkeypatch):
    """ts_memory_fwd / ts_memory_bwd run the same kernels as the per-entry-point
    calls (used while launches are recorded): outputs and every gradient are
    bit-identical, and the one-call path is the one a plain step takes."""
    from thetascan_amd import _lib
    from thetascan_amd._core.ops import fused

    placement, normalization = variant
    pub = _headline_config(placement, normalization, feature_map, d_model=256, heads=4)
    module = build_module(pub, cuda, dtype)
    _seeded(module, 5)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 300, 256, generator=g).to(cuda, dtype)
    dy = torch.randn(2, 300, 256, generator=g).to(cuda, dtype)
    native = []
    real = fused._native_forward
    monkeypatch.setattr(fused, "_native_forward", lambda *a, **k: (native.append(1), real(*a, **k))[1])
    results = []
    for per_entry in (False, True):
        module.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        if per_entry:
            with _lib.record_launches():
                y = module(xi)
                y.backward(dy)
                torch.cuda.synchronize()
        else:
            y = module(xi)
            y.backward(dy)
        assert module._core.last_path == "fused"
        results.append([y.detach(), xi.grad] + [p.grad for p in module.parameters() if p.grad is not None])
    assert native == [1], "the plain step must take the one-call path"
    assert len(results[0]) == len(results[1])
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_native_backward_survives_rope_table_eviction(cuda):
    """The one-call backward reads the RoPE tables its forward named: they stay
    alive with the autograd node when the table cache drops them between the
    forward and the backward (sequences of many lengths), so the gradients
    equal those of an undisturbed step bit for bit."""
    from thetascan_amd._core.ops import fused

    pub = _headline_config("feature", "none", d_model=256, heads=4)
    module = build_module(pub, cuda, torch.bfloat16)
    _seeded(module, 9)
    g = torch.Generator().manual_seed(10)
    T = 300
    x = torch.randn(2, T, 256, generator=g).to(cuda, torch.bfloat16)
    dy = torch.randn(2, T, 256, generator=g).to(cuda, torch.bfloat16)
    runs = []
    for evict in (False, True):
        module.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        y = module(xi)
        if evict:
            for t in range(1, 80):
                fused.rope_tables(1000 + t, 16, 10000.0, cuda)
            assert not any(key[0] == T for key in fused._TABLES)
            torch.cuda.empty_cache()
            junk = torch.full((1 << 22,), float("nan"), device=cuda)
            del junk
        y.backward(dy)
        runs.append([xi.grad] + [p.grad for p in module.parameters() if p.grad is not None])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def _views_config(layout: str, temporal: str, feature_map: str):
    pub = _headline_config("input", "key_mass", feature_map, d_model=256, heads=4)
    if layout == "share_kq":
        pub.update(share_key_query=True, output_gate=False)
        pub["kernel"]["relu2_threshold_mode"] = "learned_per_head" if feature_map == "relu2_ridge" else "none"
        pub["kernel"]["value_representation"] = "value_mlp"
    elif layout == "gqa":
        pub.update(key_value_heads=2)
        pub["rope"]["placement"] = "feature"
        pub["kernel"]["read_normalization"] = "none"
    t = pub["temporal"]
    if temporal == "ema":
        t["mode"] = "ema"
    elif temporal.startswith("bank"):
        t.update(mode="bank", bank_mode=temporal.split("_")[1], recency_branches=2, retention_inits=[0.9, 0.99])
    return pub


@pytest.mark.parametrize("layout,temporal", [("qkv", "bank_fast"), ("qkv", "bank_stale"), ("qkv", "ema"),
                                             ("share_kq", "sum"), ("share_kq", "bank_fast"), ("gqa", "ema")])
@pytest.mark.parametrize("feature_map", ["relu2_ridge", "softmax_partition"])
def test_views_path_agrees_with_composed(cuda, layout, temporal, feature_map):
    """Temporal banks, the ema stream and the shared-key/query and grouped
    layouts run the feature kernels on the multi-view path; in fp32 it agrees
    with the composed path (its maps in ts_kmap) at rel 1e-4 (3e-4 for the
    stale bank), gradients 1e-3, retention gradients 3e-3."""
    pub = _views_config(layout, temporal, feature_map)
    module = build_module(pub, cuda)
    _seeded(module, 11)
    with torch.no_grad():
        for name, p in module._core.named_parameters():
            if name in ("fade_eta", "kernel_relu2_threshold") or name.startswith(("vmlp_out.", "kq_bias")):
                p.copy_(torch.randn(p.shape, generator=torch.Generator().manual_seed(12)) * 0.3)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 200, 256, generator=g).to(cuda)
    dy = torch.randn(2, 200, 256, generator=g).to(cuda)
    outs, grads = [], []
    for force_composed in (False, True):
        module.zero_grad()
        xi = x.clone().requires_grad_(True)
        if force_composed:
            module._core.fused_eligible = lambda _x: False
        y = module(xi)
        assert module._core.last_path == ("composed" if force_composed else "fused")
        assert force_composed or not module._core._fused_cfg
        (y * dy).sum().backward()
        outs.append(y.detach())
        grads.append([(n, p.grad.clone()) for n, p in module.named_parameters()] + [("x", xi.grad)])
    # a stale bank reads the difference of two memories, which amplifies fp32
    # rounding: at this shape the softmax stale bank sits 1.3e-4 from the
    # float64 oracle on either path and the paths 1.7e-4 from each other
    assert rel_err(outs[0], outs[1]) < (3e-4 if temporal == "bank_stale" else 1e-4)
    for (name, a), (_, b) in zip(grads[0], grads[1]):
        # an fp32 retention gradient sums t (q.dq - k.dk) over t, terms that
        # cancel, so the last bits of the features decide it: for the softmax
        # stale bank the two paths sit 6.4e-4 and 3.6e-3 from the float64
        # oracle (5.4e-4 with the composed map in torch fp32); bf16 static
        # retentions take the pair-sum kernel instead
        assert rel_err(a, b) < (6e-3 if name.endswith("fade_alpha") else 1e-3), name
