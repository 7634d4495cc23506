"""What the HIP path keeps alive for backward, and the peak memory of a step
(GPU tests; the reference's footprint tests are tests/test_scan_chunk.py:
30-51, 343-405).

* The scan retains its inputs only: no score tile of any size survives the
  forward, so the largest retained tensor is one [B,H,T,max(dk,dv)] stream
  and doubling T doubles the retained bytes (the reference's bar: less than
  2.4x).
* The headline mixer (fwd+bwd, bf16) retains bytes linear in T, and the peak
  memory of a training step above the parameters grows linearly in T.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


class SavedBytes:
    """Bytes autograd keeps for backward inside the block (every tensor packed
    by a saved-tensor hook, counted once per pack)."""

    def __init__(self) -> None:
        self.total = 0
        self.largest = 0

    def __enter__(self):
        def pack(t: torch.Tensor) -> torch.Tensor:
            n = t.numel() * t.element_size()
            self.total += n
            self.largest = max(self.largest, n)
            return t

        self._hooks = torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t)
        self._hooks.__enter__()
        return self

    def __exit__(self, *exc) -> None:
        self._hooks.__exit__(*exc)


def _scan_saved(cuda, T: int, dtype=torch.float32):
    from thetascan_amd._core.ops import scan_hip

    B, H, dk, dv = 1, 2, 64, 33
    g = torch.Generator().manual_seed(5)
    q, k = (torch.randn(B, H, T, dk, generator=g).to(cuda, dtype).requires_grad_(True) for _ in range(2))
    v = torch.randn(B, H, T, dv, generator=g).to(cuda, dtype).requires_grad_(True)
    log_alpha = torch.full((H,), -0.1, device=cuda, requires_grad=True)
    with SavedBytes() as saved:
        out = scan_hip.linattn(q, k, v, log_alpha=log_alpha)
    out.sum().backward()
    return saved, (B * H * T * max(dk, dv) * q.element_size())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_retains_no_score_tiles(cuda, dtype):
    saved, stream_bytes = _scan_saved(cuda, 512, dtype)
    score_bytes = 1 * 2 * 512 * 512 * 4  # a [B,H,T,T] fp32 score tensor
    assert saved.largest <= stream_bytes
    assert saved.largest < score_bytes
    doubled, _ = _scan_saved(cuda, 1024, dtype)
    assert doubled.total < 2.4 * saved.total


def _mixer_step(cuda, T: int):
    import bench

    module = bench.seeded_module(bench.headline_config("feature_rope"), 0).to(cuda, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, T, 512, generator=g).to(cuda, torch.bfloat16)
    dy = (torch.randn(2, T, 512, generator=g) * 1e-2).to(cuda, torch.bfloat16)
    y = module(x)
    y.backward(dy)  # warm caches (RoPE tables, workspaces) outside the measurement
    del y
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    with SavedBytes() as saved:
        y = module(x)
    y.backward(dy)
    torch.cuda.synchronize()
    return saved.total, torch.cuda.max_memory_allocated() - base


def test_mixer_footprint_is_linear_in_sequence_length(cuda):
    saved1, peak1 = _mixer_step(cuda, 1024)
    saved2, peak2 = _mixer_step(cuda, 2048)
    saved4, peak4 = _mixer_step(cuda, 4096)
    print(f"retained bytes {saved1} {saved2} {saved4}; peak above resident {peak1} {peak2} {peak4}", flush=True)
    assert saved2 < 2.2 * saved1 and saved4 < 2.2 * saved2
    assert peak2 < 2.2 * peak1 and peak4 < 2.2 * peak2
