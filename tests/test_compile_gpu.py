"""The hip backend under torch.compile (GPU tests).

Mirrors the reference's compile-stability tests
(tests/test_scan_chunk.py:663-738) on the ``hip`` backend: every HIP entry
point is a torch.library custom op with a fake implementation and an autograd
formula, so TorchDynamo traces the mixer forward once (one unique graph over
six training steps) for the sum, EMA and bank temporal modes, and the retained
modes trace as one full graph, forward and backward.  The headline fused path
traces as one full graph too, and the compiled steps equal the eager ones.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _mixer(cuda, temporal: dict, blend: float, preset="kernel_expanded_reference_v0_1"):
    from thetascan_amd import ThetaScan, ThetaScanConfig

    config = ThetaScanConfig.from_dict({
        "preset": preset, "d_model": 64, "n_heads": 2, "temporal": temporal,
        "runtime": {"backend": "hip", "scan_chunk": 16},
    })
    torch.manual_seed(11)
    mixer = ThetaScan(config).to(cuda)
    with torch.no_grad():
        if mixer._core.fade_eta is not None:
            mixer._core.fade_eta.fill_(blend)
    return mixer


@pytest.mark.parametrize("label,temporal,blend", [("sum", {"mode": "sum"}, 0.0), ("ema", {"mode": "ema"}, 0.0),
                                                  ("bank", {}, 0.3)])
def test_every_temporal_mode_traces_once(cuda, label, temporal, blend):
    import torch._dynamo as dynamo

    mixer = _mixer(cuda, temporal, blend)
    dynamo.reset()
    dynamo.utils.counters.clear()
    compiled = torch.compile(mixer, backend="eager", dynamic=False)
    x = torch.randn(1, 32, 64, device=cuda)
    for _ in range(6):
        compiled(x).square().mean().backward()
        compiled.zero_grad(set_to_none=True)
    print(f"compile {label}: {dict(dynamo.utils.counters['stats'])}", flush=True)
    assert dynamo.utils.counters["stats"].get("unique_graphs", 0) == 1, label


@pytest.mark.parametrize("label,temporal,blend", [("ema", {"mode": "ema"}, 0.0), ("bank", {}, 0.3)])
def test_retained_modes_are_one_full_forward_graph(cuda, label, temporal, blend):
    import torch._dynamo as dynamo

    mixer = _mixer(cuda, temporal, blend)
    dynamo.reset()
    compiled = torch.compile(mixer, backend="eager", dynamic=False, fullgraph=True)
    x = torch.randn(1, 32, 64, device=cuda)
    compiled(x).square().mean().backward()
    assert all(p.grad is not None for p in mixer.parameters() if p.requires_grad), label


def _headline(cuda, dtype):
    from tests.test_mixer_gpu import _headline_config, _seeded, build_module

    module = build_module(_headline_config("feature", "none", d_model=256, heads=4), cuda, dtype)
    _seeded(module, 5)
    return module


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_path_compiles_to_one_graph_equal_to_eager(cuda, dtype):
    """The fused three-kernel mixer under fullgraph compile: one graph, and
    outputs and every gradient bit-identical to the eager step."""
    import torch._dynamo as dynamo

    module = _headline(cuda, dtype)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 300, 256, generator=g).to(cuda, dtype)
    dy = torch.randn(2, 300, 256, generator=g).to(cuda, dtype)
    dynamo.reset()
    dynamo.utils.counters.clear()
    compiled = torch.compile(module, backend="eager", dynamic=False, fullgraph=True)
    runs = []
    for fn in (module, compiled, compiled):
        module.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        y = fn(xi)
        y.backward(dy)
        runs.append([y.detach(), xi.grad] + [p.grad for p in module.parameters()])
    assert module._core.last_path == "fused"
    assert dynamo.utils.counters["stats"].get("unique_graphs", 0) == 1
    for run in runs[1:]:
        for a, b in zip(runs[0], run):
            assert torch.equal(a, b)


@pytest.mark.parametrize("preset", ["kernel_expanded_reference_v0_1", "gn_reference_v0_1"])
def test_stacked_qkv_under_aot_autograd_equals_eager(cuda, preset):
    """The stacked qkv projection (share_key_query=False) and the custom ops'
    autograd registrations through AOTAutograd (fullgraph, aot_eager): the
    output and every parameter gradient equal the eager step's."""
    import torch._dynamo as dynamo
    from thetascan_amd import ThetaScan, ThetaScanConfig

    config = ThetaScanConfig.from_dict({
        "preset": preset, "d_model": 64, "n_heads": 2, "share_key_query": False,
        "runtime": {"backend": "hip", "scan_chunk": 16},
    })
    torch.manual_seed(12)
    mixer = ThetaScan(config).to(cuda)
    with torch.no_grad():
        for name, p in mixer.named_parameters():
            if "W2" in name or "fade_eta" in name:
                p.copy_(torch.randn_like(p) * 0.1)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(2, 40, 64, generator=g).to(cuda)
    dy = torch.randn(2, 40, 64, generator=g).to(cuda)
    dynamo.reset()
    compiled = torch.compile(mixer, backend="aot_eager", dynamic=False, fullgraph=True)
    runs = []
    for fn in (mixer, compiled):
        mixer.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        y = fn(xi)
        y.backward(dy)
        runs.append([y.detach(), xi.grad] + [p.grad for p in mixer.parameters()])
    print(f"aot_eager {preset}: path={mixer._core.last_path}", flush=True)
    for a, b in zip(*runs):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)
