"""The gradient reductions (ts_sum_slots, ts_col_sums) against torch (GPU tests)."""
from __future__ import annotations

import pytest
import torch

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("slots,n", [(1, 1), (3, 100), (64, 32768), (128, 4096), (256, 512), (7, 70000)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_slot_sum_matches_torch(cuda, slots, n, dtype):
    from thetascan_amd._core.ops.linear import slot_sum

    g = torch.Generator().manual_seed(slots * 7 + n)
    parts = torch.randn(slots, n, generator=g).to(cuda)
    out = slot_sum(parts, dtype, (n,))
    assert out.dtype == dtype
    assert rel_err(out, parts.double().sum(0)) < (1e-6 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("rows,cols,stride", [(1, 8, 8), (200, 64, 72), (32768, 512, 2048), (5000, 256, 256)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_column_sum_matches_torch(cuda, rows, cols, stride, dtype):
    from thetascan_amd._core.ops.linear import column_sum

    g = torch.Generator().manual_seed(rows + cols)
    base = torch.randn(rows, stride, generator=g).to(cuda, dtype)
    x = base[:, stride - cols:]
    out = column_sum(x, torch.float32)
    assert rel_err(out, x.double().sum(0)) < 1e-5


def test_two_slot_buffers_sum_together(cuda):
    from thetascan_amd import _lib

    a = torch.randn(5, 1000, device=cuda)
    b = torch.randn(9, 1000, device=cuda)
    out = torch.empty(1000, device=cuda)
    lib = _lib.load()
    _lib.check(lib.ts_sum_slots(a.data_ptr(), 5, b.data_ptr(), 9, 1000, out.data_ptr(), _lib.TS_F32, 0.5,
                                _lib.stream_handle(a.device)), "sum")
    expected = 0.5 * (a.double().sum(0) + b.double().sum(0))
    assert rel_err(out, expected) < 1e-6


@pytest.mark.parametrize("G,N,p,q", [(8, 2048, 128, 64), (2, 1000, 64, 128), (3, 37, 16, 32), (1, 4096, 128, 128),
                                     (4, 64, 48, 80)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_token_contraction_matches_float64(cuda, G, N, p, q, dtype):
    """ts_contract_tokens (the GN weight-gradient contractions) against a
    float64 einsum on the same rounded inputs, including token counts that
    leave a ragged last tile and operand views with a group stride."""
    from thetascan_amd._core.ops.gn import contract_tokens

    g = torch.Generator().manual_seed(G * 7 + N + p + q)
    a = torch.randn(G, N, p, generator=g).to(dtype)
    b_full = torch.randn(2, G, N, q, generator=g).to(dtype)
    b = b_full[1]
    expected = torch.einsum("gnp,gnq->gpq", a.double(), b.double())
    out = contract_tokens(a.to(cuda), b_full.to(cuda)[1])
    assert out.dtype == torch.float32 and out.shape == (G, p, q)
    assert rel_err(out, expected) < 1e-5
