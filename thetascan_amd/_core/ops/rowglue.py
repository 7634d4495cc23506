"""Row-wise glue of the hybrid language model's blocks on the GPU.

The host model around the ThetaScan layers mixes its residual stream with
the embedding (``mix0 * x + mix1 * x0``), adds each sublayer's output with a
learned per-channel scale (``x + scale * f(x)``) and squares the ReLU of its
MLP's hidden layer (the upstream training script's torch elementwise chain).
:func:`scale_add` is one HIP launch per direction for the first two
(``ts_scale_add_*``: fp32 arithmetic, one rounding, the factors read in the
rows' dtype; the factors' gradients
from per-workgroup column partials summed in slot order), :func:`relu2` one
for the third (``ts_relu2_*``).
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from .dispatch import HipOp
from .linear import slot_sum


def _desc(t: torch.Tensor) -> _lib.RowsDesc:
    return _lib.RowsDesc(t.numel() // t.shape[-1], t.shape[-1], _lib.dtype_code(t.dtype))


def _factor(t: torch.Tensor | None, like: torch.Tensor) -> torch.Tensor | None:
    """A per-channel factor in the rows' dtype (no conversion launch when it
    already is: the parameters of a model in that dtype)."""
    if t is None:
        return None
    t = t.detach()
    if t.dtype != like.dtype:
        t = t.to(like.dtype)
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def supported(*tensors: torch.Tensor) -> bool:
    """Whether the HIP row glue takes these tensors (a host query): CUDA,
    bf16 or fp32 of one dtype and shape, contiguous, 16-byte aligned, the
    last axis a multiple of 8 and at most 2048."""
    first = tensors[0]
    return all(t.is_cuda and t.dtype == first.dtype and t.shape == first.shape and t.is_contiguous()
               and t.data_ptr() % 16 == 0 for t in tensors) and first.dtype in (torch.bfloat16, torch.float32) \
        and first.ndim >= 1 and first.shape[-1] % 8 == 0 and first.shape[-1] <= 2048


# ---------------------------------------------------------------- scale-add

def _scale_add_forward(x: torch.Tensor, u: torch.Tensor, a: torch.Tensor | None,
                       b: torch.Tensor | None) -> torch.Tensor:
    lib = _lib.load()
    y = torch.empty_like(x)
    fa, fb = _factor(a, x), _factor(b, x)
    with _lib.timed("ts_scale_add_fwd", lambda: _lib.nbytes(x, u, y)):
        status = lib.ts_scale_add_fwd(ctypes.byref(_desc(x)), x.data_ptr(), u.data_ptr(), _lib.ptr(fa), _lib.ptr(fb),
                                      y.data_ptr(), _lib.stream_handle(x.device))
    _lib.check(status, "ts_scale_add_fwd")
    return y


def _scale_add_fake(x, u, a, b):
    return torch.empty_like(x)


def _scale_add_backward_impl(g: torch.Tensor, x: torch.Tensor, u: torch.Tensor, a: torch.Tensor | None,
                             b: torch.Tensor | None, need: list[bool]) -> list[torch.Tensor]:
    lib = _lib.load()
    g = g.contiguous()
    desc = _desc(x)
    W = x.shape[-1]
    n = ctypes.c_int32()
    _lib.check(lib.ts_scale_add_parts(ctypes.byref(desc), ctypes.byref(n)), "ts_scale_add_parts")
    dx = torch.empty_like(x) if need[0] else None
    du = torch.empty_like(u) if need[1] else None
    pa = torch.empty(n.value, W, dtype=torch.float32, device=x.device) if need[2] else None
    pb = torch.empty(n.value, W, dtype=torch.float32, device=x.device) if need[3] else None
    fa, fb = _factor(a, x), _factor(b, x)
    with _lib.timed("ts_scale_add_bwd", lambda: _lib.nbytes(g, x if need[2] else None, u if need[3] else None,
                                                            dx, du)):
        status = lib.ts_scale_add_bwd(ctypes.byref(desc), g.data_ptr(), x.data_ptr(), u.data_ptr(), _lib.ptr(fa),
                                      _lib.ptr(fb), _lib.ptr(dx), _lib.ptr(du), _lib.ptr(pa), _lib.ptr(pb),
                                      _lib.stream_handle(x.device))
    _lib.check(status, "ts_scale_add_bwd")
    empty = x.new_empty(0)
    return [empty if dx is None else dx, empty if du is None else du,
            empty if pa is None else slot_sum(pa, a.dtype, (W,)),
            empty if pb is None else slot_sum(pb, b.dtype, (W,))]


def _scale_add_backward_fake(g, x, u, a, b, need):
    empty = x.new_empty(0)
    return [torch.empty_like(x) if need[0] else empty, torch.empty_like(u) if need[1] else empty,
            a.new_empty(a.shape) if need[2] else empty, b.new_empty(b.shape) if need[3] else empty]


def _scale_add_setup(ctx, inputs, output):
    x, u, a, b = inputs
    ctx.need = [x.requires_grad, u.requires_grad, a is not None and a.requires_grad,
                b is not None and b.requires_grad]
    ctx.save_for_backward(x, u, a, b)


def _scale_add_backward(ctx, g, bwd):
    x, u, a, b = ctx.saved_tensors
    if g is None:
        return None, None, None, None
    dx, du, da, db = bwd(g, x, u, a, b, ctx.need)
    return tuple(t if w else None for t, w in zip((dx, du, da, db), ctx.need))


_scale_add_op = HipOp("scale_add", forward=_scale_add_forward, forward_fake=_scale_add_fake,
                      backward_impl=_scale_add_backward_impl, backward_fake=_scale_add_backward_fake,
                      setup=_scale_add_setup, backward=_scale_add_backward)


def scale_add(x: torch.Tensor, u: torch.Tensor, a: torch.Tensor | None = None,
              b: torch.Tensor | None = None) -> torch.Tensor:
    """``a * x + b * u`` over the last axis (a, b: [W] per-channel factors,
    None: 1) in one HIP launch per direction; the torch expression where the
    tensors are not :func:`supported`."""
    W = x.shape[-1]
    if supported(x, u) and all(f is None or (f.shape == (W,) and f.is_cuda) for f in (a, b)):
        return _scale_add_op(x, u, a, b)
    ax = x if a is None else a.to(x.dtype) * x
    return ax + (u if b is None else b.to(u.dtype) * u)


# ---------------------------------------------------------------- relu^2

def _relu2_forward(z: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    h = torch.empty_like(z)
    with _lib.timed("ts_relu2_fwd", lambda: _lib.nbytes(z, h)):
        status = lib.ts_relu2_fwd(ctypes.byref(_desc(z)), z.data_ptr(), h.data_ptr(), _lib.stream_handle(z.device))
    _lib.check(status, "ts_relu2_fwd")
    return h


def _relu2_fake(z):
    return torch.empty_like(z)


def _relu2_backward_impl(g: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    g = g.contiguous()
    dz = torch.empty_like(z)
    with _lib.timed("ts_relu2_bwd", lambda: _lib.nbytes(z, g, dz)):
        status = lib.ts_relu2_bwd(ctypes.byref(_desc(z)), z.data_ptr(), g.data_ptr(), dz.data_ptr(),
                                  _lib.stream_handle(z.device))
    _lib.check(status, "ts_relu2_bwd")
    return dz


def _relu2_backward_fake(g, z):
    return torch.empty_like(z)


def _relu2_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])


def _relu2_backward(ctx, g, bwd):
    (z,) = ctx.saved_tensors
    return (None if g is None else bwd(g, z),)


_relu2_op = HipOp("relu2", forward=_relu2_forward, forward_fake=_relu2_fake, backward_impl=_relu2_backward_impl,
                  backward_fake=_relu2_backward_fake, setup=_relu2_setup, backward=_relu2_backward)


def relu2(z: torch.Tensor) -> torch.Tensor:
    """``relu(z)^2`` in one HIP launch per direction; the torch expression
    where ``z`` is not :func:`supported`."""
    if supported(z):
        return _relu2_op(z)
    return torch.relu(z).square()


# ---------------------------------------------------------------- softcapped cross entropy

def _xent_forward(z: torch.Tensor, target: torch.Tensor, cap: float) -> list[torch.Tensor]:
    lib = _lib.load()
    rows = z.shape[0]
    loss = torch.empty(rows, dtype=torch.float32, device=z.device)
    lse = torch.empty(rows, dtype=torch.float32, device=z.device)
    with _lib.timed("ts_softcap_xent_fwd", lambda: _lib.nbytes(z, target, loss, lse)):
        status = lib.ts_softcap_xent_fwd(ctypes.byref(_desc(z)), z.data_ptr(), target.data_ptr(), float(cap),
                                         loss.data_ptr(), lse.data_ptr(), _lib.stream_handle(z.device))
    _lib.check(status, "ts_softcap_xent_fwd")
    return [loss.mean(), lse]


def _xent_fake(z, target, cap):
    return [z.new_empty((), dtype=torch.float32), z.new_empty(z.shape[0], dtype=torch.float32)]


def _xent_backward_impl(g: torch.Tensor, z: torch.Tensor, target: torch.Tensor, lse: torch.Tensor,
                        cap: float) -> torch.Tensor:
    lib = _lib.load()
    dz = torch.empty_like(z)
    g32 = g.detach().to(torch.float32).reshape(1).contiguous()
    with _lib.timed("ts_softcap_xent_bwd", lambda: _lib.nbytes(z, target, lse, dz)):
        status = lib.ts_softcap_xent_bwd(ctypes.byref(_desc(z)), z.data_ptr(), target.data_ptr(), float(cap),
                                         lse.data_ptr(), g32.data_ptr(), 1.0 / max(z.shape[0], 1), dz.data_ptr(),
                                         _lib.stream_handle(z.device))
    _lib.check(status, "ts_softcap_xent_bwd")
    return dz


def _xent_backward_fake(g, z, target, lse, cap):
    return torch.empty_like(z)


def _xent_setup(ctx, inputs, output):
    z, target, cap = inputs
    ctx.cap = cap
    ctx.save_for_backward(z, target, output[1])


def _xent_backward(ctx, grads, bwd):
    z, target, lse = ctx.saved_tensors
    g = grads[0]
    return (None if g is None else bwd(g, z, target, lse, ctx.cap)), None, None


_xent_op = HipOp("softcap_xent", forward=_xent_forward, forward_fake=_xent_fake, backward_impl=_xent_backward_impl,
                 backward_fake=_xent_backward_fake, setup=_xent_setup, backward=_xent_backward)


def xent_supported(z: torch.Tensor, target: torch.Tensor) -> bool:
    """Whether :func:`softcap_cross_entropy` runs the HIP kernels (a host
    query): [rows, W] bf16 / fp32 logits (W at most 512 and a multiple of 8,
    or a multiple of 512 up to 4096) and int64 targets on the GPU."""
    W = z.shape[-1]
    return (z.ndim == 2 and supported(z) and target.is_cuda and target.dtype == torch.int64
            and target.shape == z.shape[:1] and target.is_contiguous() and (W <= 512 or (W % 512 == 0 and W <= 4096)))


def softcap_cross_entropy(z: torch.Tensor, target: torch.Tensor, cap: float) -> torch.Tensor:
    """Mean over rows of ``cross_entropy(cap * tanh(z / cap), target)`` for
    logits z [rows, W] (targets in [0, W), no ignored index) in one HIP
    launch per direction; torch's fp32 chain where the tensors are not
    :func:`xent_supported`."""
    if xent_supported(z, target):
        return _xent_op(z, target, float(cap))[0]
    c = cap * torch.tanh(z.float() / cap)
    return torch.nn.functional.cross_entropy(c, target)
