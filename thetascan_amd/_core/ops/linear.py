"""Projection GEMMs with split-K weight gradients.

The mixer's weight gradients contract over every token of the batch
(K = B*T = 32768 at the benchmark shape) into small outputs (512x512,
1536x512, or 64x64 per head).  A single GEMM of that shape launches only a
few dozen workgroups on MI355X's 256 CUs; splitting K into S slices turns it
into one batched GEMM of S independent slices (fp32 outputs) plus a small
sum, which fills the chip.  Forward and input-gradient GEMMs are unchanged
library GEMMs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _slices(rows: int, target: int = 2048, max_slices: int = 16) -> int:
    s = 1
    while s < max_slices and rows % (2 * s) == 0 and rows // (2 * s) >= target:
        s *= 2
    return s


def split_k_outer(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """sum_n a[..., n, :]^T b[..., n, :] in fp32 for [G, N, A] x [G, N, B] -> [G, A, B]."""
    G, N, A = a.shape
    s = _slices(N)
    a_s = a.reshape(G * s, N // s, A)
    b_s = b.reshape(G * s, N // s, b.shape[-1])
    if a.dtype in (torch.bfloat16, torch.float16) and a.is_cuda:
        out = torch.bmm(a_s.transpose(1, 2), b_s, out_dtype=torch.float32)
    else:
        out = torch.bmm(a_s.transpose(1, 2).float(), b_s.float())
    return out.view(G, s, A, -1).sum(1)


class _Linear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        n_out, n_in = weight.shape
        dy2 = dy.reshape(-1, n_out)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = (dy2 @ weight).view(x.shape)
        if ctx.needs_input_grad[1]:
            x2 = x.reshape(-1, n_in)
            dw = split_k_outer(dy2.unsqueeze(0), x2.unsqueeze(0))[0].to(weight.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            rows = dy2.shape[0]
            s = _slices(rows, 256, 64)
            db = dy2.view(s, rows // s, n_out).sum(1, dtype=torch.float32).sum(0).to(dy.dtype)
        return dx, dw, db


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear`` whose weight gradient is a split-K batched GEMM."""
    if not x.is_cuda:
        return F.linear(x, weight, bias)
    return _Linear.apply(x, weight, bias)
