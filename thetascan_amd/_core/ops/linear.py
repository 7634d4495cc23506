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
from .dispatch import HipOp


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


def stack_heads(grads) -> torch.Tensor:
    """[B,T,n,H,d] from n stream gradients [B,H,T,d] (None: zeros), the
    layout of a stacked projection's output gradient: one ts_stack_heads
    launch on the GPU for bf16 / fp32 rows that are 16-byte aligned, else (and
    while torch.compile traces, which cannot enter a ctypes call) the torch
    stack of the transposed streams."""
    like = next(g for g in grads if g is not None)
    es = like.element_size()
    vec = 16 // es

    def fits(g):
        return g is None or (g.is_cuda and g.dtype == like.dtype and g.shape == like.shape and g.stride(-1) == 1
                             and g.data_ptr() % 16 == 0 and all(st % vec == 0 for st in g.stride()[:3]))

    B, H, T, d = like.shape
    if (torch.compiler.is_compiling() or not (like.dtype in (torch.bfloat16, torch.float32) and d % vec == 0
                                              and len(grads) <= 4 and all(fits(g) for g in grads))):
        parts = [torch.zeros_like(like) if g is None else g for g in grads]
        return torch.stack([g.transpose(1, 2) for g in parts], dim=2)
    out = torch.empty(B, T, len(grads), H, d, dtype=like.dtype, device=like.device)
    src = (_lib.Strided * len(grads))(*[_lib.strided(g) for g in grads])
    desc = _lib.StackDesc(B, H, T, d, len(grads), _lib.dtype_code(like.dtype))
    lib = _lib.load()
    with _lib.timed("ts_stack_heads", lambda: 2 * out.numel() * es):
        status = lib.ts_stack_heads(ctypes.byref(desc), src, out.data_ptr(), _lib.stream_handle(like.device))
    _lib.check(status, "ts_stack_heads")
    return out


# F.linear whose backward forms the weight gradient as a split-K GEMM, and the
# per-head GEMMs of the composed path, as autograd nodes (dispatch.HipOp: a
# torch.library custom op under torch.compile -- their backward reaches the
# HIP reductions through ctypes, which a traced graph cannot contain -- and an
# autograd.Function in eager mode).

def _linear_forward(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    return F.linear(x, weight, bias)


def _linear_fake(x, weight, bias):
    return x.new_empty(*x.shape[:-1], weight.shape[0])


def _linear_backward_impl(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, need: list[bool]
                          ) -> list[torch.Tensor]:
    n_out, n_in = weight.shape
    dy2 = dy.reshape(-1, n_out)
    dx = (dy2 @ weight).view(x.shape) if need[0] else dy.new_empty(0)
    dw = weight_grad(dy2, x.reshape(-1, n_in), weight.dtype) if need[1] else dy.new_empty(0)
    db = column_sum(dy2, dy.dtype) if need[2] else dy.new_empty(0)
    return [dx, dw, db]


def _linear_backward_fake(dy, x, weight, need):
    return [x.new_empty(x.shape) if need[0] else dy.new_empty(0),
            weight.new_empty(weight.shape) if need[1] else dy.new_empty(0),
            dy.new_empty(weight.shape[0]) if need[2] else dy.new_empty(0)]


def _linear_setup(ctx, inputs, output):
    x, weight, bias = inputs
    ctx.need = [x.requires_grad, weight.requires_grad, bias is not None and bias.requires_grad]
    ctx.save_for_backward(x, weight)


def _linear_backward(ctx, dy, bwd):
    x, weight = ctx.saved_tensors
    dx, dw, db = bwd(dy, x, weight, ctx.need)
    return (dx if ctx.need[0] else None, dw if ctx.need[1] else None, db if ctx.need[2] else None)


_linear_op = HipOp("linear", forward=_linear_forward, forward_fake=_linear_fake,
                   backward_impl=_linear_backward_impl, backward_fake=_linear_backward_fake,
                   setup=_linear_setup, backward=_linear_backward)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear`` whose weight gradient is a split-K batched GEMM."""
    if not x.is_cuda:
        return F.linear(x, weight, bias)
    return _linear_op(x, weight, bias)


def _head_operand(W: torch.Tensor, B: int, H: int, K: int, trans: bool, dtype) -> torch.Tensor:
    M = (W.transpose(-1, -2) if trans else W).to(dtype)
    return M.expand(B, H, K, M.shape[-1]).reshape(B * H, K, M.shape[-1]).contiguous()


def _head_matmul_forward(x: torch.Tensor, W: torch.Tensor, trans: bool) -> torch.Tensor:
    B, H, T, K = x.shape
    Mb = _head_operand(W, B, H, K, trans, x.dtype)
    x3 = x.reshape(B * H, T, K)
    if not x3.is_contiguous():
        x3 = x3.contiguous()
    return torch.bmm(x3, Mb).view(B, H, T, Mb.shape[-1])


def _head_matmul_fake(x, W, trans):
    N = W.shape[-2] if trans else W.shape[-1]
    return x.new_empty(*x.shape[:3], N)


def _head_matmul_backward_impl(dy: torch.Tensor, x: torch.Tensor, W: torch.Tensor, trans: bool, need: list[bool]
                               ) -> list[torch.Tensor]:
    from .gn import contract_tokens

    B, H, T, K = x.shape
    Mb = _head_operand(W, B, H, K, trans, x.dtype)
    N = Mb.shape[-1]
    x3 = x.reshape(B * H, T, K)
    if not x3.is_contiguous():
        x3 = x3.contiguous()
    dy3 = dy.to(x.dtype).reshape(B * H, T, N).contiguous()
    dx, dW = dy.new_empty(0), dy.new_empty(0)
    if need[0]:
        dx = torch.bmm(dy3, Mb.transpose(1, 2).contiguous()).view(B, H, T, K)
    if need[1]:
        dM = contract_tokens(x3, dy3).view(B, H, K, N).sum(0)  # fp32 [H, K, N]
        if W.shape[0] == 1:
            dM = dM.sum(0, keepdim=True)
        dW = (dM.transpose(-1, -2) if trans else dM).to(W.dtype).contiguous()
    return [dx, dW]


def _head_matmul_backward_fake(dy, x, W, trans, need):
    return [x.new_empty(x.shape) if need[0] else dy.new_empty(0), W.new_empty(W.shape) if need[1] else dy.new_empty(0)]


def _head_matmul_setup(ctx, inputs, output):
    x, W, trans = inputs
    ctx.trans = trans
    ctx.need = [x.requires_grad, W.requires_grad]
    ctx.save_for_backward(x, W)


def _head_matmul_backward(ctx, dy, bwd):
    x, W = ctx.saved_tensors
    dx, dW = bwd(dy, x, W, ctx.trans, ctx.need)
    return (dx if ctx.need[0] else None, dW if ctx.need[1] else None, None)


_head_matmul_op = HipOp("head_matmul", forward=_head_matmul_forward, forward_fake=_head_matmul_fake,
                        backward_impl=_head_matmul_backward_impl, backward_fake=_head_matmul_backward_fake,
                        setup=_head_matmul_setup, backward=_head_matmul_backward)


def head_matmul(x: torch.Tensor, W: torch.Tensor, trans: bool) -> torch.Tensor:
    """x [B,H,T,K] times W^T (``trans``, W [H|1, N, K]) or W (W [H|1, K, N]) per
    head: the fast-network GEMVs of the composed path (engine.py:117-158,
    180-195) as one batched GEMM per call, without the permute copies of an
    einsum.  Both GEMMs take contiguous right operands; the weight gradient is
    a token contraction per (batch, head) (ts_contract_tokens) summed over the
    batch."""
    return _head_matmul_op(x, W, bool(trans))
