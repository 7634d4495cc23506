"""The hybrid language model on the GPU: a bf16 training step through both
ThetaScan layers, and the per-row int8 round trip of a partly trained model
(eval loss within 1e-3 relative of the bf16 weights' loss).  The host model
is defined by this build (its upstream script is not available), so the int8
figure has no reference number: parity unpinned."""
from __future__ import annotations

import pytest
import torch

from thetascan_amd import hybrid_lm as lm

pytestmark = pytest.mark.gpu


def _affine_batches(g, dev, B, T):
    """A learnable stream: token_{t+1} = (5 token_t + 3) mod 1024."""
    start = torch.randint(0, lm.VOCAB, (B, 1), generator=g)
    seq = [start]
    for _ in range(T):
        seq.append((seq[-1] * 5 + 3) % lm.VOCAB)
    s = torch.cat(seq, 1).to(dev)
    return s[:, :-1], s[:, 1:]


def test_training_step_and_int8_round_trip(cuda):
    torch.manual_seed(0)
    model = lm.HybridLM().to(cuda, torch.bfloat16)
    assert lm.parameter_count(model) == 17_059_976
    g = torch.Generator().manual_seed(1)
    opt = torch.optim.Adam(model.parameters(), lr=2e-3)
    losses = []
    for step in range(12):
        x, y = _affine_batches(g, cuda, 16, 256)
        loss = model(x, y)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        for name, p in model.named_parameters():
            assert p.grad is None or torch.isfinite(p.grad.float()).all(), name
        opt.step()
        losses.append(float(loss.detach()))
    print(f"hybrid LM losses {losses[0]:.3f} -> {losses[-1]:.3f}; path={model.blocks[4].attn._core.last_path}",
          flush=True)
    assert losses[-1] < 0.5 * losses[0]
    theta = model.blocks[4].attn._core
    assert theta.W2[0].abs().max() > 0 and theta.proj_out.weight.abs().max() > 0
    model.eval()
    with torch.no_grad():
        x, y = _affine_batches(g, cuda, 32, 512)
        base = float(model(x, y))
        model.load_state_dict(lm.int8_round_trip(model))
        quant = float(model(x, y))
    print(f"eval loss bf16 {base:.6f} int8 round trip {quant:.6f}", flush=True)
    assert abs(quant - base) / base < 1e-3
