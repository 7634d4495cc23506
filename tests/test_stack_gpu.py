"""ts_stack_heads: three [B,H,T,d] stream gradients gathered into the
[B,T,3,H,d] layout of a stacked q/k/v projection's gradient (the backward of
the split at block.py:593-594), against torch.stack of the transposed streams.
A copy: results must be bit-identical, zeros where a stream has no gradient."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _reference(grads):
    like = next(g for g in grads if g is not None)
    parts = [torch.zeros_like(like) if g is None else g for g in grads]
    return torch.stack([g.transpose(1, 2) for g in parts], dim=2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,T,d,missing", [(2, 8, 300, 64, None), (1, 3, 17, 16, 1), (3, 2, 64, 128, 0),
                                             (2, 4, 1, 32, 2)])
def test_stack_heads_equals_torch_stack(cuda, dtype, B, H, T, d, missing):
    from thetascan_amd import _lib
    from thetascan_amd._core.ops.linear import stack_heads

    g = torch.Generator().manual_seed(B * 1000 + T)
    grads = []
    for s in range(3):
        if s == missing:
            grads.append(None)
            continue
        if s == 1:
            # a head-major view of token-major memory, like the q/k prologue's output
            t = torch.randn(B, T, H, d, generator=g).to(cuda, dtype).transpose(1, 2)
        else:
            t = torch.randn(B, H, T, d, generator=g).to(cuda, dtype)
        grads.append(t)
    with _lib.record_launches() as recs:
        out = stack_heads(grads)
        torch.cuda.synchronize()
    print(f"stack B{B} H{H} T{T} d{d} missing={missing} {dtype}", flush=True)
    assert [r[0] for r in recs] == ["ts_stack_heads"]
    assert out.shape == (B, T, 3, H, d) and out.is_contiguous()
    assert torch.equal(out, _reference(grads))


def test_stack_heads_refuses_unaligned_rows(cuda):
    """Rows that are not 16-byte aligned are refused on the host (no launch)."""
    from thetascan_amd import _lib

    lib = _lib.load()
    x = torch.zeros(1, 2, 8, 20, dtype=torch.bfloat16, device=cuda)  # 40-byte rows
    out = torch.empty(1, 8, 1, 2, 20, dtype=torch.bfloat16, device=cuda)
    desc = _lib.StackDesc(1, 2, 8, 20, 1, _lib.TS_BF16)
    src = (_lib.Strided * 1)(_lib.strided(x))
    rc = lib.ts_stack_heads(ctypes.byref(desc), src, out.data_ptr(), _lib.stream_handle(x.device))
    assert rc == _lib.TS_ERR_VALUE
    desc = _lib.StackDesc(1, 2, 8, 16, 5, _lib.TS_BF16)  # more than four streams
    assert lib.ts_stack_heads(ctypes.byref(desc), src, out.data_ptr(), None) == _lib.TS_ERR_VALUE
