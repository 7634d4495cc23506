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

import ctypes

import torch
import torch.nn.functional as F

from ... import _lib


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


def slot_sum(parts: torch.Tensor, dtype: torch.dtype, shape) -> torch.Tensor:
    """sum over the leading (slot) axis of fp32 ``parts`` -> ``shape`` in ``dtype``
    (one ts_sum_slots launch on the GPU)."""
    if not parts.is_cuda or dtype not in (torch.bfloat16, torch.float32):
        return parts.sum(0).view(shape).to(dtype)
    parts = parts.contiguous()
    out = torch.empty(shape, dtype=dtype, device=parts.device)
    lib = _lib.load()
    _lib.check(lib.ts_sum_slots(parts.data_ptr(), parts.shape[0], None, 0, parts[0].numel(), out.data_ptr(),
                                _lib.dtype_code(dtype), 1.0, _lib.stream_handle(parts.device)), "ts_sum_slots")
    return out


def weight_grad(dy2: torch.Tensor, x2: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """dy2^T x2 over all rows -> [n_out, n_in] in ``dtype`` (split-K GEMM + slot sum)."""
    rows = dy2.shape[0]
    s = _slices(rows)
    while s > 1 and s * dy2.shape[1] * x2.shape[1] > (8 << 20):  # partial slots stay within 32 MiB
        s //= 2
    if not (dy2.is_cuda and dy2.dtype in (torch.bfloat16, torch.float16)):
        return split_k_outer(dy2.unsqueeze(0), x2.unsqueeze(0))[0].to(dtype)
    parts = torch.bmm(dy2.reshape(s, rows // s, -1).transpose(1, 2), x2.reshape(s, rows // s, -1),
                      out_dtype=torch.float32)
    return slot_sum(parts, dtype, (dy2.shape[1], x2.shape[1]))


def column_sum(x2: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Sum of the rows of a [rows, cols] matrix (any row stride) -> [cols] in ``dtype``."""
    rows, cols = x2.shape
    ok = (x2.is_cuda and x2.dtype in (torch.bfloat16, torch.float32) and x2.stride(1) == 1 and cols % 8 == 0
          and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0)
    if not ok:
        return x2.float().sum(0).to(dtype)
    slices = max(1, min(256, rows // 128))
    parts = torch.empty(slices, cols, dtype=torch.float32, device=x2.device)
    lib = _lib.load()
    _lib.check(lib.ts_col_sums(x2.data_ptr(), _lib.dtype_code(x2.dtype), rows, cols, x2.stride(0),
                               parts.data_ptr(), slices, _lib.stream_handle(x2.device)), "ts_col_sums")
    return slot_sum(parts, dtype, (cols,))


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
            dw = weight_grad(dy2, x.reshape(-1, n_in), weight.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = column_sum(dy2, dy.dtype)
        return dx, dw, db


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear`` whose weight gradient is a split-K batched GEMM."""
    if not x.is_cuda:
        return F.linear(x, weight, bias)
    return _Linear.apply(x, weight, bias)


class _HeadMatmul(torch.autograd.Function):
    """y[b, h] = x[b, h] @ M[h] for a [B,H,T,K] stream and per-head (or shared)
    matrices M [H or 1, K, N] (M = W^T or W): the fast-network GEMVs of the
    composed path (engine.py:117-158, 180-195) as one batched GEMM per call,
    without the permute copies of an einsum.  Both GEMMs take contiguous right
    operands; the weight gradient is a token contraction per (batch, head)
    (ts_contract_tokens) summed over the batch."""

    @staticmethod
    def forward(ctx, x, W, trans: bool):
        B, H, T, K = x.shape
        M = (W.transpose(-1, -2) if trans else W).to(x.dtype)
        N = M.shape[-1]
        Mb = M.expand(B, H, K, N).reshape(B * H, K, N).contiguous()
        x3 = x.reshape(B * H, T, K)
        if not x3.is_contiguous():
            x3 = x3.contiguous()
        y = torch.bmm(x3, Mb).view(B, H, T, N)
        ctx.save_for_backward(x3, Mb)
        ctx.meta = (B, H, T, K, N, W.shape[0], trans, W.dtype)
        return y

    @staticmethod
    def backward(ctx, dy):
        from .gn import contract_tokens

        x3, Mb = ctx.saved_tensors
        B, H, T, K, N, Hw, trans, wdtype = ctx.meta
        dy3 = dy.to(x3.dtype).reshape(B * H, T, N).contiguous()
        dx = dW = None
        if ctx.needs_input_grad[0]:
            dx = torch.bmm(dy3, Mb.transpose(1, 2).contiguous()).view(B, H, T, K)
        if ctx.needs_input_grad[1]:
            dM = contract_tokens(x3, dy3).view(B, H, K, N).sum(0)  # fp32 [H, K, N]
            if Hw == 1:
                dM = dM.sum(0, keepdim=True)
            dW = (dM.transpose(-1, -2) if trans else dM).to(wdtype)
        return dx, dW, None


def head_matmul(x: torch.Tensor, W: torch.Tensor, trans: bool) -> torch.Tensor:
    """x [B,H,T,K] times W^T (``trans``, W [H|1, N, K]) or W (W [H|1, K, N]) per head."""
    return _HeadMatmul.apply(x, W, trans)
