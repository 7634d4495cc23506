"""The measured GEMM solution table (thetascan_amd.gemm_solutions).

With the table in force, the projection GEMMs of the benchmark shape replay
the recorded hipBLASLt / rocBLAS solutions; their results must agree with the
libraries' heuristic choice to the rounding of bf16 outputs (both accumulate
in fp32; only the kernel, and with it the summation order, changes), and the
switch must turn off again.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def test_measured_solutions_agree_with_the_heuristic_choice(cuda):
    from thetascan_amd import gemm_solutions

    g = torch.Generator().manual_seed(0)
    x = torch.randn(32768, 512, generator=g).to(cuda, torch.bfloat16)
    w_in = (torch.randn(2048, 512, generator=g) / 512 ** 0.5).to(cuda, torch.bfloat16)
    w_out = (torch.randn(512, 512, generator=g) / 512 ** 0.5).to(cuda, torch.bfloat16)
    dout = torch.randn(32768, 512, generator=g).to(cuda, torch.bfloat16)

    def products():
        return [F.linear(x, w_in), F.linear(x, w_out), dout @ w_out]

    gemm_solutions.use_measured_gemms(False)
    ref = products()
    try:
        assert gemm_solutions.use_measured_gemms(True), "the table's library versions match this image"
        assert gemm_solutions.in_force()
        got = products()
        torch.cuda.synchronize()
    finally:
        gemm_solutions.use_measured_gemms(False)
    assert not gemm_solutions.in_force()
    for a, b in zip(got, ref):
        assert rel_err(a.float(), b.float().double()) < 1e-2
