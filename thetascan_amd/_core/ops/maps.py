"""HIP B-spline feature map and temporal-bank blend (autograd wrappers).

``bspline_features`` replaces the tensor form of
src/thetascan/_core/ops/kernel_features.py:138-230 (open-uniform basis and
the projected feature map) with ``ts_bspline_fwd`` / ``ts_bspline_bwd``.
``bank_blend`` replaces the fast / stale fade blends of
src/thetascan/_core/modules/block.py:667-718 with ``ts_blend_fwd`` /
``ts_blend_bwd``.  Both run on the caller's current stream; a CPU tensor or a
missing library raises (no fallback).
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from .dispatch import HipOp

_KERNEL_DTYPES = (torch.bfloat16, torch.float32)


def _on_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A view whose last axis is contiguous and whose rows start on 16 bytes
    where the storage allows (otherwise the kernels take the scalar path)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _as4d(t: torch.Tensor) -> torch.Tensor:
    if t.ndim == 4:
        return t
    if t.ndim < 1:
        raise ValueError("expected at least one axis")
    return t.reshape(1, 1, -1, t.shape[-1])


# ------------------------------------------------------------------ B-spline


def _spline_desc(pre4, n_basis, degree, bound, scale):
    B, H, T, P = pre4.shape
    return _lib.BsplineDesc(B, H, T, P, int(n_basis), int(degree), _lib.dtype_code(pre4.dtype), float(bound),
                            float(scale))


def _bspline_forward(pre: torch.Tensor, scale_h: torch.Tensor | None, n_basis: int, degree: int, bound: float,
                scale: float) -> torch.Tensor:
    lib = _lib.load()
    shape = pre.shape
    pre4 = _rows(_as4d(pre))
    desc = _spline_desc(pre4, n_basis, degree, bound, scale)
    out = torch.empty(*pre4.shape[:3], pre4.shape[3] * n_basis, dtype=pre.dtype, device=pre.device)
    sh = None if scale_h is None else scale_h.detach().to(torch.float32).contiguous()
    with _lib.timed("ts_bspline_fwd", lambda: _lib.nbytes(pre4, out)):
        status = lib.ts_bspline_fwd(ctypes.byref(desc), _lib.strided(pre4), _lib.ptr(sh), _lib.strided(out),
                                    _lib.stream_handle(pre.device))
    _lib.check(status, "ts_bspline_fwd")
    return out.reshape(*shape[:-1], shape[-1] * n_basis)


def _bspline_fake(pre, scale_h, n_basis, degree, bound, scale):
    return pre.new_empty(*pre.shape[:-1], pre.shape[-1] * n_basis)


def _bspline_backward_impl(dout: torch.Tensor, pre: torch.Tensor, scale_h: torch.Tensor | None, n_basis: int, degree: int,
                    bound: float, scale: float) -> list[torch.Tensor]:
    lib = _lib.load()
    shape = pre.shape
    pre4 = _rows(_as4d(pre))
    desc = _spline_desc(pre4, n_basis, degree, bound, scale)
    sh = None if scale_h is None else scale_h.detach().to(torch.float32).contiguous()
    d4 = _rows(dout.to(pre4.dtype).reshape(*pre4.shape[:3], pre4.shape[3] * n_basis))
    dpre = torch.empty_like(pre4)
    parts = None
    if sh is not None:
        n = ctypes.c_int32()
        _lib.check(lib.ts_bspline_parts(ctypes.byref(desc), ctypes.byref(n)), "ts_bspline_parts")
        parts = torch.empty(pre4.shape[1], n.value, dtype=torch.float32, device=pre4.device)
    with _lib.timed("ts_bspline_bwd", lambda: _lib.nbytes(pre4, d4, dpre)):
        status = lib.ts_bspline_bwd(ctypes.byref(desc), _lib.strided(pre4), _lib.ptr(sh), _lib.strided(d4),
                                    _lib.strided(dpre), _lib.ptr(parts), _lib.stream_handle(pre4.device))
    _lib.check(status, "ts_bspline_bwd")
    dscale = dout.new_empty(0) if parts is None else parts.sum(-1).to(scale_h.dtype)
    return [dpre.reshape(shape), dscale]


def _bspline_backward_fake(dout, pre, scale_h, n_basis, degree, bound, scale):
    return [pre.new_empty(pre.shape), dout.new_empty(0) if scale_h is None else scale_h.new_empty(scale_h.shape)]


def _bspline_setup(ctx, inputs, output):
    pre, scale_h, n_basis, degree, bound, scale = inputs
    ctx.args = (n_basis, degree, bound, scale)
    ctx.save_for_backward(pre, scale_h)


def _bspline_backward(ctx, dout, bwd):
    pre, scale_h = ctx.saved_tensors
    dpre, dscale = bwd(dout, pre, scale_h, *ctx.args)
    return dpre, (dscale if scale_h is not None else None), None, None, None, None


_bspline_op = HipOp("bspline", forward=_bspline_forward, forward_fake=_bspline_fake,
                    backward_impl=_bspline_backward_impl, backward_fake=_bspline_backward_fake,
                    setup=_bspline_setup, backward=_bspline_backward)


def bspline_features(pre: torch.Tensor, *, n_basis: int, degree: int, bound: float, scale) -> torch.Tensor:
    """``basis(pre * scale).flatten(-2) / P`` (kernel_features.py:208-230).

    ``scale`` is a float (fixed scale) or a per-head tensor ``[H]`` for a
    head-major ``[B,H,T,P]`` input (the learned per-head scale).
    """
    _on_gpu(pre)
    if pre.dtype not in _KERNEL_DTYPES:
        raise NotImplementedError(f"hip B-spline features support bf16 and fp32, got {pre.dtype}")
    if degree < 0:
        raise ValueError("B-spline degree must be non-negative")
    if n_basis <= degree:
        raise ValueError("B-spline basis count must exceed its degree")
    if bound <= 0.0:
        raise ValueError("B-spline bound must be positive")
    if torch.is_tensor(scale):
        if pre.ndim != 4 or scale.ndim != 1 or scale.shape[0] != pre.shape[1]:
            raise ValueError(
                "kernel control must have shape [n_heads] or [n_heads, n_features], "
                f"got {tuple(scale.shape)} for reference {tuple(pre.shape)}"
            )
        _on_gpu(scale)
        return _bspline_op(pre, scale, int(n_basis), int(degree), float(bound), 1.0)
    return _bspline_op(pre, None, int(n_basis), int(degree), float(bound), float(scale))


# ---------------------------------------------------- B-spline of RMS-normed inputs


def _bspline_norm_forward(a: torch.Tensor, shift: torch.Tensor | None, scale_h: torch.Tensor | None, n_basis: int,
                          degree: int, bound: float, scale: float, eps: float) -> torch.Tensor:
    lib = _lib.load()
    a4 = _rows(a)
    desc = _spline_desc(a4, n_basis, degree, bound, scale)
    out = torch.empty(*a4.shape[:3], a4.shape[3] * n_basis, dtype=a.dtype, device=a.device)
    sh = None if scale_h is None else scale_h.detach().to(torch.float32).contiguous()
    sf = None if shift is None else shift.detach().to(torch.float32).contiguous()
    with _lib.timed("ts_bspline_norm_fwd", lambda: _lib.nbytes(a4, out)):
        status = lib.ts_bspline_norm_fwd(ctypes.byref(desc), _lib.strided(a4), _lib.ptr(sf), float(eps), _lib.ptr(sh),
                                         _lib.strided(out), _lib.stream_handle(a.device))
    _lib.check(status, "ts_bspline_norm_fwd")
    return out


def _bspline_norm_fake(a, shift, scale_h, n_basis, degree, bound, scale, eps):
    return a.new_empty(*a.shape[:-1], a.shape[-1] * n_basis)


def _bspline_norm_backward_impl(dout: torch.Tensor, a: torch.Tensor, shift: torch.Tensor | None,
                                scale_h: torch.Tensor | None, n_basis: int, degree: int, bound: float, scale: float,
                                eps: float) -> list[torch.Tensor]:
    lib = _lib.load()
    a4 = _rows(a)
    B, H, T, P = a4.shape
    desc = _spline_desc(a4, n_basis, degree, bound, scale)
    sh = None if scale_h is None else scale_h.detach().to(torch.float32).contiguous()
    sf = None if shift is None else shift.detach().to(torch.float32).contiguous()
    d4 = _rows(dout.to(a4.dtype).reshape(B, H, T, P * n_basis))
    da = torch.empty_like(a4)
    n = ctypes.c_int32()
    _lib.check(lib.ts_bspline_parts(ctypes.byref(desc), ctypes.byref(n)), "ts_bspline_parts")
    sparts = None if sh is None else torch.empty(H, n.value, dtype=torch.float32, device=a.device)
    hparts = None if sf is None else torch.empty(H, n.value, P, dtype=torch.float32, device=a.device)
    with _lib.timed("ts_bspline_norm_bwd", lambda: _lib.nbytes(a4, d4, da)):
        status = lib.ts_bspline_norm_bwd(ctypes.byref(desc), _lib.strided(a4), _lib.ptr(sf), float(eps), _lib.ptr(sh),
                                         _lib.strided(d4), _lib.strided(da), _lib.ptr(sparts), _lib.ptr(hparts),
                                         _lib.stream_handle(a.device))
    _lib.check(status, "ts_bspline_norm_bwd")
    dshift = dout.new_empty(0) if hparts is None else hparts.sum(1).to(shift.dtype)
    dscale = dout.new_empty(0) if sparts is None else sparts.sum(-1).to(scale_h.dtype)
    return [da, dshift, dscale]


def _bspline_norm_backward_fake(dout, a, shift, scale_h, n_basis, degree, bound, scale, eps):
    like = lambda t: dout.new_empty(0) if t is None else t.new_empty(t.shape)  # noqa: E731
    return [a.new_empty(a.shape), like(shift), like(scale_h)]


def _bspline_norm_setup(ctx, inputs, output):
    a, shift, scale_h, *args = inputs
    ctx.args = args
    ctx.save_for_backward(a, shift, scale_h)


def _bspline_norm_backward(ctx, dout, bwd):
    a, shift, scale_h = ctx.saved_tensors
    da, dshift, dscale = bwd(dout, a, shift, scale_h, *ctx.args)
    return (da, dshift if shift is not None else None, dscale if scale_h is not None else None,
            *([None] * len(ctx.args)))


_bspline_norm_op = HipOp("bspline_norm", forward=_bspline_norm_forward, forward_fake=_bspline_norm_fake,
                         backward_impl=_bspline_norm_backward_impl, backward_fake=_bspline_norm_backward_fake,
                         setup=_bspline_norm_setup, backward=_bspline_norm_backward)


def bspline_norm_supported(a: torch.Tensor) -> bool:
    """Whether ts_bspline_norm_* take this stream: P a power of two up to 64."""
    P = a.shape[-1]
    return a.is_cuda and a.ndim == 4 and a.dtype in _KERNEL_DTYPES and P <= 64 and (P & (P - 1)) == 0


def bspline_norm_features(a: torch.Tensor, *, shift, eps: float, n_basis: int, degree: int, bound: float,
                          scale) -> torch.Tensor:
    """``basis((rmsnorm(a) + shift) * scale).flatten(-2) / P`` for the raw W1
    products ``a`` [B,H,T,P] (engine.py:117-158 with kernel_features.py:208-230):
    one ts_bspline_norm_fwd / _bwd pair.  ``shift`` is None or [H, P]."""
    _on_gpu(a)
    if degree < 0:
        raise ValueError("B-spline degree must be non-negative")
    if n_basis <= degree:
        raise ValueError("B-spline basis count must exceed its degree")
    if bound <= 0.0:
        raise ValueError("B-spline bound must be positive")
    if torch.is_tensor(scale):
        return _bspline_norm_op(a, shift, scale, int(n_basis), int(degree), float(bound), 1.0, float(eps))
    return _bspline_norm_op(a, shift, None, int(n_basis), int(degree), float(bound), float(scale), float(eps))


# ---------------------------------------------------------------- bank blend


def _blend_desc(first, n_in):
    B, H, T, d = first.shape
    return _lib.BlendDesc(B, H, T, d, n_in, _lib.dtype_code(first.dtype))


def _blend_forward(coef: torch.Tensor, inputs: list[torch.Tensor]) -> torch.Tensor:
    lib = _lib.load()
    ins = [_rows(t) for t in inputs]
    desc = _blend_desc(ins[0], len(ins))
    cf = coef.detach().to(torch.float32).contiguous()
    # token-major: the output gate and the projection read it as [B,T,H*d]
    # without a transposing copy
    B, H, T, d = ins[0].shape
    y = torch.empty(B, T, H, d, dtype=ins[0].dtype, device=ins[0].device).transpose(1, 2)
    arr = (_lib.Strided * len(ins))(*[_lib.strided(t) for t in ins])
    with _lib.timed("ts_blend_fwd", lambda: _lib.nbytes(*ins, y)):
        status = lib.ts_blend_fwd(ctypes.byref(desc), arr, _lib.ptr(cf), _lib.strided(y),
                                  _lib.stream_handle(y.device))
    _lib.check(status, "ts_blend_fwd")
    return y


def _blend_fake(coef, inputs):
    B, H, T, d = inputs[0].shape
    return inputs[0].new_empty(B, T, H, d).transpose(1, 2)


def _blend_backward_impl(dy: torch.Tensor, coef: torch.Tensor, inputs: list[torch.Tensor], need: list[bool]
                  ) -> list[torch.Tensor]:
    lib = _lib.load()
    ins = [_rows(t) for t in inputs]
    n = len(ins)
    desc = _blend_desc(ins[0], n)
    cf = coef.detach().to(torch.float32).contiguous()
    g = _rows(dy.to(ins[0].dtype))
    dins = [torch.empty_like(t) if need[1 + i] else None for i, t in enumerate(ins)]
    count = ctypes.c_int32()
    _lib.check(lib.ts_blend_parts(ctypes.byref(desc), ctypes.byref(count)), "ts_blend_parts")
    parts = torch.empty(n, ins[0].shape[1], count.value, dtype=torch.float32, device=g.device)
    arr = (_lib.Strided * n)(*[_lib.strided(t) for t in ins])
    darr = (_lib.Strided * n)(*[_lib.strided(t) for t in dins])
    with _lib.timed("ts_blend_bwd", lambda: _lib.nbytes(*ins, g, *dins)):
        status = lib.ts_blend_bwd(ctypes.byref(desc), arr, _lib.ptr(cf), _lib.strided(g), darr, _lib.ptr(parts),
                                  _lib.stream_handle(g.device))
    _lib.check(status, "ts_blend_bwd")
    dcoef = parts.sum(-1).to(coef.dtype) if need[0] else dy.new_empty(0)
    return [dcoef] + [dy.new_empty(0) if t is None else t for t in dins]


def _blend_backward_fake(dy, coef, inputs, need):
    empty = dy.new_empty(0)
    return [coef.new_empty(coef.shape) if need[0] else empty] + \
        [t.new_empty(t.shape) if w else empty for t, w in zip(inputs, need[1:])]


def _blend_setup(ctx, inputs, output):
    coef, ins = inputs
    ctx.need = [coef.requires_grad] + [t.requires_grad for t in ins]
    ctx.save_for_backward(coef, *ins)


def _blend_backward(ctx, dy, bwd):
    coef, *ins = ctx.saved_tensors
    res = bwd(dy, coef, list(ins), ctx.need)
    grads = [g if w else None for g, w in zip(res, ctx.need)]
    return grads[0], grads[1:]


_blend_op = HipOp("blend", forward=_blend_forward, forward_fake=_blend_fake, backward_impl=_blend_backward_impl,
                  backward_fake=_blend_backward_fake, setup=_blend_setup, backward=_blend_backward)


def bank_blend(inputs, coef: torch.Tensor) -> torch.Tensor:
    """``sum_i coef[i, h] * inputs[i]`` over ``[B,H,T,d]`` views (1 to 8 of
    them), returned as a [B,H,T,d] view of token-major [B,T,H,d] memory."""
    if not 1 <= len(inputs) <= 8:
        raise ValueError("bank blend takes 1 to 8 views")
    _on_gpu(coef, *inputs)
    first = inputs[0]
    if first.dtype not in _KERNEL_DTYPES or first.ndim != 4:
        raise NotImplementedError("hip bank blend takes bf16 or fp32 [B,H,T,d] views")
    for t in inputs:
        if t.shape != first.shape or t.dtype != first.dtype:
            raise ValueError("bank blend views must share shape and dtype")
    if coef.shape != (len(inputs), first.shape[1]):
        raise ValueError(f"bank blend coefficients must be [{len(inputs)}, {first.shape[1]}]")
    return _blend_op(coef, list(inputs))


def bank_blend_gated(inputs, coef: torch.Tensor, gate: torch.Tensor, gate_bias: torch.Tensor | None) -> torch.Tensor:
    """``bank_blend(inputs, coef) * silu(gate + gate_bias)`` in one launch
    (ts_blend_gated_fwd), written token-major like :func:`bank_blend`.
    Inference only: nothing here records autograd (the caller runs it with
    grad disabled); ``gate`` is the [B,H,T,d] view of the output gate's
    pre-activation x W_g^T in the inputs' dtype, ``gate_bias`` [H*d]."""
    if torch.is_grad_enabled():
        raise RuntimeError("bank_blend_gated is a forward-only epilogue: call it with grad disabled")
    first = inputs[0]
    if not (1 <= len(inputs) <= 8 and first.is_cuda and first.dtype in _KERNEL_DTYPES and first.ndim == 4
            and gate.shape == first.shape and gate.dtype == first.dtype
            and all(t.shape == first.shape and t.dtype == first.dtype for t in inputs)):
        raise NotImplementedError("bank_blend_gated: views and gate must share shape and a kernel dtype")
    lib = _lib.load()
    ins = [_rows(t) for t in inputs]
    g = _rows(gate)
    B, H, T, d = first.shape
    y = torch.empty(B, T, H, d, dtype=first.dtype, device=first.device).transpose(1, 2)
    cf = coef.detach().to(torch.float32).contiguous()
    gb = None if gate_bias is None else gate_bias.detach().to(torch.float32).contiguous()
    arr = (_lib.Strided * len(ins))(*[_lib.strided(t) for t in ins])
    with _lib.timed("ts_blend_fwd", lambda: _lib.nbytes(*ins, g, y)):
        status = lib.ts_blend_gated_fwd(ctypes.byref(_blend_desc(ins[0], len(ins))), arr, _lib.ptr(cf),
                                        _lib.strided(g), _lib.ptr(gb), _lib.strided(y), _lib.stream_handle(y.device))
    _lib.check(status, "ts_blend_gated_fwd")
    return y


def fast_coefficients(etas) -> torch.Tensor:
    """(1 - sum_j eta_j, eta_1 .. eta_J) over (R_0, R_1 .. R_J) (block.py:683-695)."""
    eta = torch.stack([e.reshape(-1) for e in etas]).to(torch.float32)
    return torch.cat([(1.0 - eta.sum(0)).unsqueeze(0), eta])


def stale_coefficients(etas) -> torch.Tensor:
    """(1, -eta_1 .. -eta_J, sum_j eta_j) over (R_0, R_stale_1 .. R_stale_J, R_null) (block.py:697-717)."""
    eta = torch.stack([e.reshape(-1) for e in etas]).to(torch.float32)
    return torch.cat([torch.ones_like(eta[:1]), -eta, eta.sum(0, keepdim=True)])


# ------------------------------------------------------------------ value anchors


def _anchor_desc(v4, V, c_heads, gain, eps):
    B, H, T, d = v4.shape
    return _lib.AnchorDesc(B, H, T, d, int(V), int(c_heads), _lib.dtype_code(v4.dtype), float(gain), float(eps))


def _anchor_forward(v: torch.Tensor, codebook: torch.Tensor, gain: float, eps: float) -> torch.Tensor:
    lib = _lib.load()
    v4 = _rows(v)
    c = codebook.detach().to(torch.float32).contiguous()
    desc = _anchor_desc(v4, c.shape[1], c.shape[0], gain, eps)
    r = torch.empty(*v4.shape[:3], c.shape[1], dtype=v.dtype, device=v.device)
    with _lib.timed("ts_anchor_fwd", lambda: _lib.nbytes(v4, r)):
        status = lib.ts_anchor_fwd(ctypes.byref(desc), _lib.strided(v4), c.data_ptr(), _lib.strided(r),
                                   _lib.stream_handle(v.device))
    _lib.check(status, "ts_anchor_fwd")
    return r


def _anchor_fake(v, codebook, gain, eps):
    return v.new_empty(*v.shape[:3], codebook.shape[1])


def _anchor_backward_impl(dr: torch.Tensor, v: torch.Tensor, codebook: torch.Tensor, gain: float,
                          eps: float) -> list[torch.Tensor]:
    from .gn import contract_tokens

    lib = _lib.load()
    v4 = _rows(v)
    B, H, T, d = v4.shape
    c = codebook.detach().to(torch.float32).contiguous()
    V = c.shape[1]
    desc = _anchor_desc(v4, V, c.shape[0], gain, eps)
    vp = ctypes.c_int32()
    _lib.check(lib.ts_anchor_width(ctypes.byref(desc), ctypes.byref(vp)), "ts_anchor_width")
    dr4 = dr.to(v.dtype)
    dv = torch.empty(B, H, T, d, dtype=v.dtype, device=v.device)
    dls = torch.empty(H, B * T, vp.value, dtype=v.dtype, device=v.device)
    with _lib.timed("ts_anchor_bwd", lambda: _lib.nbytes(v4, dr4, dv, dls)):
        status = lib.ts_anchor_bwd(ctypes.byref(desc), _lib.strided(v4), c.data_ptr(), _lib.strided(dr4),
                                   _lib.strided(dv), dls.data_ptr(), _lib.stream_handle(v.device))
    _lib.check(status, "ts_anchor_bwd")
    # dC[h] = sum over tokens of dls^T v: the values as head-major token rows
    vt = v4.transpose(0, 1)
    if not (vt.stride(1) == T * vt.stride(2)):
        vt = vt.contiguous()
    dc = contract_tokens(dls, vt.reshape(H, B * T, d))[:, :V]
    if c.shape[0] == 1:
        dc = dc.sum(0, keepdim=True)
    return [dv, dc.to(codebook.dtype)]


def _anchor_backward_fake(dr, v, codebook, gain, eps):
    return [v.new_empty(v.shape), codebook.new_empty(codebook.shape)]


def _anchor_setup(ctx, inputs, output):
    v, codebook, gain, eps = inputs
    ctx.args = (gain, eps)
    ctx.save_for_backward(v, codebook)


def _anchor_backward(ctx, dr, bwd):
    v, codebook = ctx.saved_tensors
    dv, dc = bwd(dr, v, codebook, *ctx.args)
    return dv, dc, None, None


_anchor_op = HipOp("anchor_code", forward=_anchor_forward, forward_fake=_anchor_fake,
                   backward_impl=_anchor_backward_impl, backward_fake=_anchor_backward_fake,
                   setup=_anchor_setup, backward=_anchor_backward)


def anchor_code(v: torch.Tensor, codebook: torch.Tensor, *, gain: float, eps: float) -> torch.Tensor:
    """softmax(gain * C (v / max(||v||, eps))) over the anchors of a value
    codebook ``codebook`` [1|H, V, d] for head-major values ``v`` [B,H,T,d]
    (engine.py:284-296), in v's dtype."""
    _on_gpu(v, codebook)
    if v.dtype not in _KERNEL_DTYPES:
        raise NotImplementedError(f"hip value anchors support bf16 and fp32, got {v.dtype}")
    if v.ndim != 4 or codebook.ndim != 3 or codebook.shape[-1] != v.shape[-1]:
        raise ValueError("value anchors need v [B,H,T,d] and a codebook [1|H,V,d]")
    return _anchor_op(v, codebook, float(gain), float(eps))
