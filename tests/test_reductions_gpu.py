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
