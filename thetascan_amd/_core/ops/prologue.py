"""Query/key prologue of the composed mixer path on the GPU.

``qk_norm(x, rot, base, eps)`` is the input RoPE followed by the query/key L2
norm of block.py:595-599 (rope.py:41-49 pairs (2i, 2i+1) of the first ``rot``
channels, fp32 angles; norms.py:11-12 ``x / max(|x|, eps)``) as one HIP kernel
each way (ts_qknorm_fwd / ts_qknorm_bwd).  It reads the strided [B,H,T,d]
views the qkv projection leaves and writes contiguous rows.
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from .dispatch import HipOp
from .fused import rope_tables


def _eligible(x: torch.Tensor) -> bool:
    """Shape and dtype the kernel covers (layout is fixed up inside the op)."""
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float32) or x.ndim != 4:
        return False
    vec = 16 // x.element_size()
    d = x.shape[-1]
    return d % vec == 0 and d // vec <= 64


def _readable(x: torch.Tensor) -> torch.Tensor:
    """x itself when its rows are 16-byte aligned with a contiguous feature
    axis, else an aligned copy."""
    vec = 16 // x.element_size()
    if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(s % vec == 0 for s in x.stride()[:3]):
        return x
    return x.clone(memory_format=torch.contiguous_format)


def _tables(T: int, rot: int, base: float, device):
    if not rot:
        return None, None
    return rope_tables(T, rot, base, device)


def _qknorm_forward(x: torch.Tensor, rot: int, base: float, eps: float) -> torch.Tensor:
    B, H, T, d = x.shape
    x = _readable(x)
    lib = _lib.load()
    desc = _lib.QkNormDesc(B, H, T, d, _lib.dtype_code(x.dtype), int(rot), float(eps))
    cs, sn = _tables(T, rot, base, x.device)
    y = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device)
    with _lib.timed("ts_qknorm_fwd", lambda: _lib.nbytes(x, y)):
        status = lib.ts_qknorm_fwd(ctypes.byref(desc), _lib.strided(x), _lib.strided(y), _lib.ptr(cs),
                                   _lib.ptr(sn), _lib.stream_handle(x.device))
    _lib.check(status, "ts_qknorm_fwd")
    return y


def _qknorm_fake(x, rot, base, eps):
    return x.new_empty(x.shape)


def _qknorm_backward_impl(x: torch.Tensor, dy: torch.Tensor, rot: int, base: float, eps: float) -> torch.Tensor:
    B, H, T, d = x.shape
    x = _readable(x)
    lib = _lib.load()
    dy = _readable(dy.to(x.dtype))
    desc = _lib.QkNormDesc(B, H, T, d, _lib.dtype_code(x.dtype), int(rot), float(eps))
    cs, sn = _tables(T, rot, base, x.device)
    dx = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device)
    with _lib.timed("ts_qknorm_bwd", lambda: _lib.nbytes(x, dy, dx)):
        status = lib.ts_qknorm_bwd(ctypes.byref(desc), _lib.strided(x), _lib.strided(dy), _lib.strided(dx),
                                   _lib.ptr(cs), _lib.ptr(sn), _lib.stream_handle(x.device))
    _lib.check(status, "ts_qknorm_bwd")
    return dx


def _qknorm_backward_fake(x, dy, rot, base, eps):
    return x.new_empty(x.shape)


def _qknorm_setup(ctx, inputs, output):
    x, rot, base, eps = inputs
    ctx.args = (rot, base, eps)
    ctx.save_for_backward(x)


def _qknorm_backward(ctx, dy, bwd):
    (x,) = ctx.saved_tensors
    return bwd(x, dy, *ctx.args), None, None, None


_qknorm_op = HipOp("qknorm", forward=_qknorm_forward, forward_fake=_qknorm_fake,
                   backward_impl=_qknorm_backward_impl, backward_fake=_qknorm_backward_fake,
                   setup=_qknorm_setup, backward=_qknorm_backward)


def qk_norm(x: torch.Tensor, rot: int, base: float, eps: float) -> torch.Tensor | None:
    """rope(x) / max(|rope(x)|, eps) over the last axis of a [B,H,T,d] view,
    or None for a width or dtype the kernel does not cover."""
    if not _eligible(x):
        return None
    return _qknorm_op(x, int(rot), float(base), float(eps))
