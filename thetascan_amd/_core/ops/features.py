"""The kernel-family feature map as one autograd node per stream.

``kernel_features(x, w1, w2, tau, spec, want_resid)`` runs ts_feature_fwd on
a raw [B,H,T,d] key or query stream: input RoPE and L2 norm
(block.py:595-618), a = W1 xn, RMSNorm, the per-head threshold, the ReLU^2
ridge or softmax partition (kernel_features.py:73-135), feature RoPE
(engine.py:74-86) and, for queries, the residual read xn + s W2 h
(engine.py:522-528).  Its backward is ts_feature_bwd with the weight
gradients contracted inside the kernel.  Any temporal view set (plain sum,
ema stream, recency banks) scans the features it returns.
"""
from __future__ import annotations

import torch

from .dispatch import HipOp
from .fused import FeatureSpec, feature_bwd, feature_fwd, sum_grads


def _spec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps) -> FeatureSpec:
    return FeatureSpec(int(kind), int(m), float(gain), int(in_rot), int(feat_rot), float(rope_base),
                       float(resid_scale), float(eps))


def _placeholder(like: torch.Tensor) -> torch.Tensor:
    return like.new_empty(0)


def _or_none(t: torch.Tensor):
    return None if t.numel() == 0 and t.ndim == 1 else t


def _rows(t: torch.Tensor) -> torch.Tensor:
    """t itself when its rows are 16-byte aligned with a contiguous feature
    axis, else a contiguous copy."""
    vec = 16 // t.element_size()
    if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % vec == 0 for s in t.stride()[:3]):
        return t
    return t.contiguous()


def _weights(x, w1, w2, tau, want_w2: bool):
    dt = x.dtype
    w1c = w1.detach().to(dt).contiguous()
    w2c = w2.detach().to(dt).contiguous() if want_w2 else None
    tauf = None if tau is None else tau.detach().to(torch.float32).contiguous()
    return w1c, w2c, tauf


def _features_forward(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, tau: torch.Tensor, kind: int, m: int,
                      gain: float, in_rot: int, feat_rot: int, rope_base: float, resid_scale: float, eps: float,
                      want_resid: bool) -> list[torch.Tensor]:
    spec = _spec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps)
    xk = _rows(x)
    w1c, w2c, tauf = _weights(xk, w1, _or_none(w2), _or_none(tau), want_resid)
    phi, resid = feature_fwd(spec, xk, w1c, w2c, tauf, want_resid)
    return [phi, resid if resid is not None else _placeholder(x)]


def _features_fake(x, w1, w2, tau, kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps, want_resid):
    B, H, T, d = x.shape
    return [x.new_empty(B, H, T, m), x.new_empty(B, H, T, d) if want_resid else _placeholder(x)]


def _features_backward_impl(dphi: torch.Tensor, dresid: torch.Tensor, x: torch.Tensor, w1: torch.Tensor,
                            w2: torch.Tensor, tau: torch.Tensor, kind: int, m: int, gain: float, in_rot: int,
                            feat_rot: int, rope_base: float, resid_scale: float, eps: float, want_resid: bool,
                            need: list[bool]) -> list[torch.Tensor]:
    spec = _spec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps)
    B, H, T, d = x.shape
    xk = _rows(x)
    dres = _or_none(dresid)
    w2_, tau_ = _or_none(w2), _or_none(tau)
    w1c, w2c, tauf = _weights(xk, w1, w2_, tau_, dres is not None)
    dphi = _or_none(dphi)
    dphi = torch.zeros(B, H, T, m, dtype=x.dtype, device=x.device) if dphi is None else _rows(dphi.to(x.dtype))
    if dres is not None:
        dres = _rows(dres.to(x.dtype))
    dx = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device)
    want_w = need[1] or need[2] or need[3]
    dw1, dw2, dtau = feature_bwd(spec, xk, w1c, tauf, dphi, dres, dx, w2=w2c, want_weights=want_w)
    out = [dx,
           sum_grads(dw1, None, w1.dtype, w1.shape) if need[1] else None,
           sum_grads(dw2, None, w2.dtype, w2.shape) if (need[2] and dw2 is not None) else None,
           sum_grads(dtau, None, tau.dtype, tau.shape) if (need[3] and dtau is not None) else None]
    like = [x, w1, w2, tau]
    return [_placeholder(t) if g is None else g for g, t in zip(out, like)]


def _features_backward_fake(dphi, dresid, x, w1, w2, tau, kind, m, gain, in_rot, feat_rot, rope_base,
                            resid_scale, eps, want_resid, need):
    like = [x, w1, w2, tau]
    return [torch.empty_like(t) if (n and _or_none(t) is not None) else _placeholder(t) for t, n in zip(like, need)]


def _features_setup(ctx, inputs, output):
    x, w1, w2, tau, *args = inputs
    ctx.args = tuple(args)
    ctx.need = [x.requires_grad, w1.requires_grad, w2.requires_grad and _or_none(w2) is not None,
                tau.requires_grad and _or_none(tau) is not None]
    ctx.save_for_backward(x, w1, w2, tau)


def _features_backward(ctx, grads, bwd):
    x, w1, w2, tau = ctx.saved_tensors
    dphi, dresid = grads
    dphi = _placeholder(x) if dphi is None else dphi
    dresid = _placeholder(x) if dresid is None else dresid
    res = bwd(dphi, dresid, x, w1, w2, tau, *ctx.args, ctx.need)
    out = [None if not n else _or_none(g) for g, n in zip(res, ctx.need)]
    return (*out, *([None] * len(ctx.args)))


_features_op = HipOp("kernel_features", forward=_features_forward, forward_fake=_features_fake,
                     backward_impl=_features_backward_impl, backward_fake=_features_backward_fake,
                     setup=_features_setup, backward=_features_backward)


def kernel_features(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor | None, tau: torch.Tensor | None,
                    spec: FeatureSpec, want_resid: bool):
    """(phi [B,H,T,m], resid [B,H,T,d] or None) of one raw key/query stream
    ``x`` [B,H,T,d] (``w2`` is read only with ``want_resid``)."""
    w2_ = w2 if (want_resid and w2 is not None) else _placeholder(w1)
    tau_ = tau if tau is not None else _placeholder(w1)
    phi, resid = _features_op(x, w1, w2_, tau_, int(spec.kind), int(spec.m), float(spec.gain), int(spec.in_rot),
                              int(spec.feat_rot), float(spec.rope_base), float(spec.resid_scale), float(spec.eps),
                              bool(want_resid))
    return phi, (resid if want_resid else None)
