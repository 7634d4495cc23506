"""The fused mixer step captured as HIP graphs (torch.cuda.make_graphed_callables)
replays exactly like eager execution (GPU tests).

Every replay is compared with the eager result, with eager work and device
synchronisations between replays, so a graph node that only behaves on its
first replay is caught."""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _module(cuda, placement, normalization):
    import thetascan_amd as ts

    rope = ts.RoPEConfig(mode="partial", fraction=0.5, placement=placement)
    cfg = ts.ThetaScanConfig(
        d_model=256, n_heads=4, memory_multiplier=1, family="kernel",
        kernel=ts.KernelConfig(feature_map="relu2_ridge", read_normalization=normalization),
        rope=rope, temporal=ts.TemporalConfig(mode="sum"),
        runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64),
    )
    torch.manual_seed(3)
    module = ts.ThetaScan(cfg)
    with torch.no_grad():
        for p in module.parameters():
            p.add_(torch.randn_like(p) * 0.02)
    return module.to(cuda, torch.bfloat16)


@pytest.mark.parametrize("variant", [("feature", "none"), ("input", "key_mass")])
def test_graphed_step_replays_match_eager(cuda, variant):
    module = _module(cuda, *variant)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 320, 256, generator=g).to(cuda, torch.bfloat16)
    dys = [(torch.randn(2, 320, 256, generator=g) * 0.1).to(cuda, torch.bfloat16) for _ in range(3)]

    def eager(dy):
        module.zero_grad(set_to_none=True)
        y = module(x)
        y.backward(dy)
        return y.detach().clone(), [p.grad.detach().clone() for p in module.parameters()]

    expected = [eager(dy) for dy in dys]
    assert module._core.last_path == "fused"
    graphed = torch.cuda.make_graphed_callables(module, (x,), num_warmup_iters=3)
    for replay in range(6):
        dy = dys[replay % 3]
        module.zero_grad(set_to_none=True)
        y = graphed(x)
        y.backward(dy)
        torch.cuda.synchronize()
        y_ref, g_ref = expected[replay % 3]
        assert rel_err(y, y_ref) < 1e-6, replay
        for p, ref in zip(module.parameters(), g_ref):
            assert rel_err(p.grad, ref) < 1e-6, replay
        # eager work between replays
        _ = (x.float() * 2).sum().item()
