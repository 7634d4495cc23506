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
from .fused import rope_tables


def _eligible(x: torch.Tensor) -> bool:
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float32) or x.ndim != 4:
        return False
    vec = 16 // x.element_size()
    d = x.shape[-1]
    return (x.stride(-1) == 1 and d % vec == 0 and d // vec <= 64 and x.data_ptr() % 16 == 0
            and all(s % vec == 0 for s in x.stride()[:3]))


class _QkNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, rot: int, base: float, eps: float):
        B, H, T, d = x.shape
        lib = _lib.load()
        desc = _lib.QkNormDesc(B, H, T, d, _lib.dtype_code(x.dtype), int(rot), float(eps))
        cs = sn = None
        if rot:
            cs, sn = rope_tables(T, rot, base, x.device)
        y = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device)
        with _lib.timed("ts_qknorm_fwd", lambda: _lib.nbytes(x, y)):
            status = lib.ts_qknorm_fwd(ctypes.byref(desc), _lib.strided(x), _lib.strided(y), _lib.ptr(cs),
                                       _lib.ptr(sn), _lib.stream_handle(x.device))
        _lib.check(status, "ts_qknorm_fwd")
        ctx.save_for_backward(x)
        ctx.rot, ctx.base, ctx.eps = rot, base, eps
        return y

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        B, H, T, d = x.shape
        lib = _lib.load()
        dy = dy.to(x.dtype)
        if not _eligible(dy):
            dy = dy.contiguous()
        desc = _lib.QkNormDesc(B, H, T, d, _lib.dtype_code(x.dtype), int(ctx.rot), float(ctx.eps))
        cs = sn = None
        if ctx.rot:
            cs, sn = rope_tables(T, ctx.rot, ctx.base, x.device)
        dx = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device)
        with _lib.timed("ts_qknorm_bwd", lambda: _lib.nbytes(x, dy, dx)):
            status = lib.ts_qknorm_bwd(ctypes.byref(desc), _lib.strided(x), _lib.strided(dy), _lib.strided(dx),
                                       _lib.ptr(cs), _lib.ptr(sn), _lib.stream_handle(x.device))
        _lib.check(status, "ts_qknorm_bwd")
        return dx, None, None, None


def qk_norm(x: torch.Tensor, rot: int, base: float, eps: float) -> torch.Tensor | None:
    """rope(x) / max(|rope(x)|, eps) over the last axis of a [B,H,T,d] view,
    or None when the view cannot be read by the kernel (unaligned rows)."""
    if not _eligible(x):
        return None
    return _QkNorm.apply(x, rot, base, eps)
