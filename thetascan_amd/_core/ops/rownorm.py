"""RMS-normed rows with an optional rotary turn and per-head gain (ts_rownorm).

The hybrid language model around the ThetaScan layers normalizes every
token's residual stream and, in its softmax-attention layers, each head's
query and key rows before a half-split rotary turn and a per-head query gain
(the upstream training script's ``rms_norm`` + rotate + gain, written there as
a chain of torch operations).  :func:`rms_rows` is one HIP launch per
direction: fp32 arithmetic with one rounding at the store, the row's 1/rms
kept for the backward, the gain's gradient summed per head from one fp32 sum
per row.
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from .dispatch import HipOp

WIDTHS = (8, 16, 32, 64, 128, 256, 512)


def _desc(x: torch.Tensor, rope: bool, eps: float) -> _lib.RowNormDesc:
    B, H, T, W = x.shape
    return _lib.RowNormDesc(B, H, T, W, _lib.dtype_code(x.dtype), int(rope), float(eps))


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x with 16-byte aligned rows (a copy only where the view does not give them)."""
    es = x.element_size()
    ok = x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in x.stride()[:-1])
    return x if ok else x.contiguous()


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else t.detach().to(torch.float32).contiguous()


def _forward(x: torch.Tensor, cos: torch.Tensor | None, sin: torch.Tensor | None, gain: torch.Tensor | None,
             rope: bool, eps: float) -> list[torch.Tensor]:
    lib = _lib.load()
    x4 = _rows(x)
    B, H, T, W = x4.shape
    c, s, g = _f32(cos), _f32(sin), _f32(gain)
    y = torch.empty(B, H, T, W, dtype=x.dtype, device=x.device)
    rstd = torch.empty(B, H, T, dtype=torch.float32, device=x.device)
    desc = _desc(x4, rope, eps)
    with _lib.timed("ts_rownorm_fwd", lambda: _lib.nbytes(x4, y, rstd)):
        status = lib.ts_rownorm_fwd(ctypes.byref(desc), _lib.strided(x4), _lib.ptr(c), _lib.ptr(s), _lib.ptr(g),
                                    y.data_ptr(), rstd.data_ptr(), _lib.stream_handle(x.device))
    _lib.check(status, "ts_rownorm_fwd")
    return [y, rstd]


def _forward_fake(x, cos, sin, gain, rope, eps):
    return [x.new_empty(x.shape), x.new_empty(x.shape[:3], dtype=torch.float32)]


def _backward_impl(dy: torch.Tensor, x: torch.Tensor, cos: torch.Tensor | None, sin: torch.Tensor | None,
                   gain: torch.Tensor | None, rstd: torch.Tensor, rope: bool, eps: float,
                   need_gain: bool) -> list[torch.Tensor]:
    lib = _lib.load()
    x4 = _rows(x)
    d4 = _rows(dy.to(x.dtype))
    c, s, g = _f32(cos), _f32(sin), _f32(gain)
    dx = torch.empty(x4.shape, dtype=x.dtype, device=x.device)
    dg_row = torch.empty(x4.shape[:3], dtype=torch.float32, device=x.device) if need_gain else None
    desc = _desc(x4, rope, eps)
    with _lib.timed("ts_rownorm_bwd", lambda: _lib.nbytes(x4, d4, rstd, dx)):
        status = lib.ts_rownorm_bwd(ctypes.byref(desc), _lib.strided(x4), _lib.strided(d4), _lib.ptr(c),
                                    _lib.ptr(s), _lib.ptr(g), rstd.data_ptr(), dx.data_ptr(), _lib.ptr(dg_row),
                                    _lib.stream_handle(x.device))
    _lib.check(status, "ts_rownorm_bwd")
    dgain = dg_row.sum(dim=(0, 2)).to(gain.dtype) if need_gain else x.new_empty(0)
    return [dx, dgain]


def _backward_fake(dy, x, cos, sin, gain, rstd, rope, eps, need_gain):
    return [x.new_empty(x.shape), gain.new_empty(gain.shape) if need_gain else x.new_empty(0)]


def _setup(ctx, inputs, output):
    x, cos, sin, gain, rope, eps = inputs
    ctx.rope, ctx.eps = rope, eps
    ctx.need_gain = gain is not None and gain.requires_grad
    ctx.save_for_backward(x, cos, sin, gain, output[1])


def _backward(ctx, grads, bwd):
    x, cos, sin, gain, rstd = ctx.saved_tensors
    dy = grads[0]
    if dy is None:
        return None, None, None, None, None, None
    dx, dgain = bwd(dy, x, cos, sin, gain, rstd, ctx.rope, ctx.eps, ctx.need_gain)
    return dx, None, None, dgain if ctx.need_gain else None, None, None


_rownorm_op = HipOp("rownorm", forward=_forward, forward_fake=_forward_fake, backward_impl=_backward_impl,
                    backward_fake=_backward_fake, setup=_setup, backward=_backward)


def supported(x: torch.Tensor, rope: bool = False) -> bool:
    """Whether :func:`rms_rows` takes ``x`` (a host query)."""
    return (x.is_cuda and x.ndim == 4 and x.dtype in (torch.bfloat16, torch.float32) and x.shape[-1] in WIDTHS
            and (not rope or x.shape[-1] >= 16))


def rms_rows(x: torch.Tensor, cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
             gain: torch.Tensor | None = None, eps: float | None = None) -> torch.Tensor:
    """``gain[h] * rotate(rms_norm(x))`` for x [B,H,T,W] (any row strides):
    the rotary turn of the halves by ``cos``/``sin`` [T, W/2] when given, the
    per-head ``gain`` [H] when given; ``eps`` defaults to what F.rms_norm
    uses, the machine epsilon of its fp32 arithmetic (also for bf16 rows)."""
    if not x.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    rope = cos is not None
    if not supported(x, rope):
        raise NotImplementedError(f"ts_rownorm: rows of shape {tuple(x.shape)} and dtype {x.dtype}")
    if eps is None:
        eps = float(torch.finfo(torch.float32).eps)
    return _rownorm_op(x, cos, sin, gain, rope, float(eps))[0]
