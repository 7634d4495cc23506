"""Positive feature maps of the kernel memory (GPU tensor form).

Same maps and numerical safeguards as src/thetascan/_core/ops/kernel_features.py:
softmax partition with optional relative-to-max sparsity (73-113, 43-70) and
ReLU^2 ridge with uniform fallback (116-135).  The clamped open-uniform
B-spline map (138-230) runs in its own HIP kernel (ts_bspline_fwd/bwd).  The
depth-1 kernel-memory hot path evaluates the softmax/ReLU^2 maps inside the
fused HIP write kernel (ts_feature_fwd); these tensor forms serve the
configurations that kernel does not cover (sparse softmax, score biases,
learned sharpness, GN reads).
"""
from __future__ import annotations

import ctypes

import torch

from . import maps
from .dispatch import HipOp


def head_parameter(value: torch.Tensor, reference: torch.Tensor) -> torch.Tensor:
    """Broadcast a [H] or [H,M] control over a head-major [B,H,...,M] tensor."""
    value = value.to(device=reference.device, dtype=reference.dtype)
    if value.ndim == 1 and value.shape[0] == reference.shape[1]:
        return value.view(1, value.shape[0], *([1] * (reference.ndim - 2)))
    if value.ndim == 2 and value.shape[0] == reference.shape[1] and value.shape[1] == reference.shape[-1]:
        return value.view(1, value.shape[0], *([1] * (reference.ndim - 3)), value.shape[1])
    raise ValueError(
        "kernel control must have shape [n_heads] or [n_heads, n_features], "
        f"got {tuple(value.shape)} for reference {tuple(reference.shape)}"
    )


def _gain(value, fallback: float, reference: torch.Tensor):
    if value is None:
        return fallback
    if not torch.is_tensor(value):
        return float(value)
    return head_parameter(value, reference)


def relative_threshold_features(logits, rho, *, temperature: float, straight_through: bool, eps: float):
    if temperature <= 0.0:
        raise ValueError("relative threshold temperature must be positive")
    shifted = logits - logits.amax(dim=-1, keepdim=True)
    margin = shifted - head_parameter(rho, logits).clamp(min=eps, max=1.0 - eps).log()
    soft = torch.sigmoid(margin / temperature)
    if straight_through:
        gate = (margin >= 0.0).to(soft.dtype) + soft - soft.detach()
    else:
        gate = soft
    weights = shifted.exp() * gate
    return weights / weights.sum(dim=-1, keepdim=True).clamp_min(eps)


def softmax_partition_features(pre, *, gain, fallback_gain: float, score_bias, sparsity: str,
                               relative_threshold, sparse_blend_alpha=None, threshold_temperature: float,
                               eps: float):
    scores = pre if score_bias is None else pre + head_parameter(score_bias, pre)
    logits = scores * _gain(gain, fallback_gain, scores)
    dense = torch.softmax(logits, dim=-1)
    if sparsity == "none":
        return dense
    if relative_threshold is None:
        raise RuntimeError("relative kernel sparsity requires a threshold tensor")
    if sparsity not in ("relative_soft", "relative_st", "relative_st_blend"):
        raise ValueError(f"unknown kernel sparsity: {sparsity!r}")
    sparse = relative_threshold_features(
        logits, relative_threshold, temperature=threshold_temperature,
        straight_through=sparsity != "relative_soft", eps=eps,
    )
    if sparsity != "relative_st_blend":
        return sparse
    if sparse_blend_alpha is None:
        raise RuntimeError("relative_st_blend requires a learned sparse blend tensor")
    return dense + head_parameter(sparse_blend_alpha, logits) * (sparse - dense)


def relu2_ridge_features(pre, *, score_bias, relu2_threshold=None, eps: float):
    if score_bias is not None:
        pre = pre + head_parameter(score_bias, pre)
    if relu2_threshold is not None:
        pre = pre - head_parameter(relu2_threshold, pre)
    features = torch.relu(pre).square()
    mass = features.sum(dim=-1, keepdim=True)
    uniform = torch.full_like(features, 1.0 / features.shape[-1])
    return torch.where(mass > eps, features / mass.clamp_min(eps), uniform)


def projected_bspline_features(pre, *, n_basis: int, degree: int, bound: float, scale, fallback_scale: float):
    """The projected B-spline map on the GPU (ts_bspline_fwd / ts_bspline_bwd)."""
    return maps.bspline_features(pre, n_basis=n_basis, degree=degree, bound=bound,
                                 scale=fallback_scale if scale is None else scale)


def feature_map(pre, cfg, *, softmax_gain=None, spline_scale=None, score_bias=None, relu2_threshold=None,
                relative_threshold=None, sparse_blend_alpha=None):
    """Dispatch the configured positive feature map (kernel_features.py:233-273)."""
    if cfg.kernel_kind == "softmax_partition":
        return softmax_partition_features(
            pre, gain=softmax_gain, fallback_gain=cfg.softmax_gain, score_bias=score_bias,
            sparsity=cfg.kernel_sparsity, relative_threshold=relative_threshold,
            sparse_blend_alpha=sparse_blend_alpha, threshold_temperature=cfg.kernel_threshold_temperature,
            eps=cfg.eps,
        )
    if cfg.kernel_kind == "relu2_ridge":
        return relu2_ridge_features(pre, score_bias=score_bias, relu2_threshold=relu2_threshold, eps=cfg.eps)
    if cfg.kernel_kind == "projected_bspline":
        return projected_bspline_features(
            pre, n_basis=cfg.bspline_basis_count, degree=cfg.bspline_degree, bound=cfg.bspline_bound,
            scale=spline_scale, fallback_scale=cfg.bspline_scale,
        )
    raise ValueError(f"unknown kernel kind: {cfg.kernel_kind!r}")


# ------------------------------------------------------------------ HIP maps with controls

_SPARSITY = {"none": 0, "relative_soft": 1, "relative_st": 2, "relative_st_blend": 3}
KMAP_SOFTMAX, KMAP_RELU2 = 0, 1
KMAP_WIDTHS = (16, 32, 48, 64)


def _kmap_desc(a, kind, rms, gain_mode, sparsity, gain, temp, eps):
    from ... import _lib

    B, H, T, m = a.shape
    return _lib.KmapDesc(B, H, T, m, _lib.dtype_code(a.dtype), int(kind), int(rms), int(gain_mode), int(sparsity),
                         float(gain), float(temp), float(eps))


def _kmap_params(shift, gainv, rho, alpha):
    from ... import _lib

    f = lambda t: None if t is None else t.detach().to(torch.float32).contiguous()  # noqa: E731
    held = [f(t) for t in (shift, gainv, rho, alpha)]
    return _lib.KmapParams(*[_lib.ptr(t) for t in held]), held


def _kmap_forward(a: torch.Tensor, shift: torch.Tensor | None, gainv: torch.Tensor | None, rho: torch.Tensor | None,
                  alpha: torch.Tensor | None, kind: int, rms: bool, gain_mode: int, sparsity: int, gain: float,
                  temp: float, eps: float) -> torch.Tensor:
    from ... import _lib

    lib = _lib.load()
    a4 = a if a.stride(-1) == 1 else a.contiguous()
    desc = _kmap_desc(a4, kind, rms, gain_mode, sparsity, gain, temp, eps)
    prm, _held = _kmap_params(shift, gainv, rho, alpha)
    phi = torch.empty(a4.shape, dtype=a.dtype, device=a.device)
    with _lib.timed("ts_kmap_fwd", lambda: _lib.nbytes(a4, phi)):
        status = lib.ts_kmap_fwd(ctypes.byref(desc), ctypes.byref(prm), _lib.strided(a4), _lib.strided(phi),
                                 _lib.stream_handle(a.device))
    _lib.check(status, "ts_kmap_fwd")
    return phi


def _kmap_fake(a, shift, gainv, rho, alpha, kind, rms, gain_mode, sparsity, gain, temp, eps):
    return a.new_empty(a.shape)


def _kmap_backward_impl(dphi: torch.Tensor, a: torch.Tensor, shift: torch.Tensor | None,
                        gainv: torch.Tensor | None, rho: torch.Tensor | None, alpha: torch.Tensor | None, kind: int,
                        rms: bool, gain_mode: int, sparsity: int, gain: float, temp: float,
                        eps: float) -> list[torch.Tensor]:
    from ... import _lib
    from .linear import slot_sum

    lib = _lib.load()
    a4 = a if a.stride(-1) == 1 else a.contiguous()
    B, H, T, m = a4.shape
    desc = _kmap_desc(a4, kind, rms, gain_mode, sparsity, gain, temp, eps)
    prm, _held = _kmap_params(shift, gainv, rho, alpha)
    d4 = dphi.to(a.dtype)
    d4 = d4 if d4.stride(-1) == 1 else d4.contiguous()
    da = torch.empty(a4.shape, dtype=a.dtype, device=a.device)
    n = ctypes.c_int32()
    _lib.check(lib.ts_kmap_parts(ctypes.byref(desc), ctypes.byref(prm), ctypes.byref(n)), "ts_kmap_parts")
    P = n.value
    dev = a.device
    new = lambda *shape: torch.empty(*shape, dtype=torch.float32, device=dev)  # noqa: E731
    dshift = new(P, H, m) if shift is not None else None
    dgain = (new(P, H) if gain_mode == 1 else new(P, H, m)) if gain_mode else None
    drho = new(P, H) if sparsity else None
    dalpha = new(P, H) if sparsity == 3 else None
    grads = _lib.KmapGrads(_lib.strided(da), _lib.ptr(dshift), _lib.ptr(dgain), _lib.ptr(drho), _lib.ptr(dalpha))
    with _lib.timed("ts_kmap_bwd", lambda: _lib.nbytes(a4, d4, da)):
        status = lib.ts_kmap_bwd(ctypes.byref(desc), ctypes.byref(prm), _lib.strided(a4), _lib.strided(d4),
                                 ctypes.byref(grads), _lib.stream_handle(dev))
    _lib.check(status, "ts_kmap_bwd")
    empty = a.new_empty(0)
    out = [da]
    for parts, like in ((dshift, shift), (dgain, gainv), (drho, rho), (dalpha, alpha)):
        out.append(empty if parts is None else slot_sum(parts, torch.float32, like.shape).to(like.dtype))
    return out


def _kmap_backward_fake(dphi, a, shift, gainv, rho, alpha, kind, rms, gain_mode, sparsity, gain, temp, eps):
    return [a.new_empty(a.shape)] + [a.new_empty(0) if t is None else t.new_empty(t.shape)
                                     for t in (shift, gainv, rho, alpha)]


def _kmap_setup(ctx, inputs, output):
    a, shift, gainv, rho, alpha, *args = inputs
    ctx.args = args
    ctx.save_for_backward(a, shift, gainv, rho, alpha)


def _kmap_backward(ctx, dphi, bwd):
    a, shift, gainv, rho, alpha = ctx.saved_tensors
    da, ds, dg, dr, dal = bwd(dphi, a, shift, gainv, rho, alpha, *ctx.args)
    keep = lambda g, t: g if t is not None else None  # noqa: E731
    return (da, keep(ds, shift), keep(dg, gainv), keep(dr, rho), keep(dal, alpha), *([None] * len(ctx.args)))


_kmap_op = HipOp("kmap", forward=_kmap_forward, forward_fake=_kmap_fake, backward_impl=_kmap_backward_impl,
                 backward_fake=_kmap_backward_fake, setup=_kmap_setup, backward=_kmap_backward)


def _as_head_feature(value, H: int, m: int):
    """A [H] or [H, m] control as [H, m] (a differentiable broadcast)."""
    if value.ndim == 1:
        return value.view(-1, 1).expand(H, m)
    return value.reshape(-1, m).expand(H, m)


def kmap_eligible(a: torch.Tensor, cfg) -> bool:
    """Whether ts_kmap_fwd takes this map and stream (softmax partition or ReLU^2
    ridge, feature width 16 / 32 / 48 / 64, bf16 or fp32 on the GPU)."""
    return (a.is_cuda and a.ndim == 4 and a.shape[-1] in KMAP_WIDTHS and a.dtype in (torch.bfloat16, torch.float32)
            and cfg.kernel_kind in ("softmax_partition", "relu2_ridge"))


def kmap(a, cfg, *, rms: bool, tau=None, softmax_gain=None, score_bias=None, relu2_threshold=None,
         relative_threshold=None, sparse_blend_alpha=None):
    """The configured kernel feature map of ``rmsnorm(a) - tau`` (``rms``) or of
    ``a`` on the GPU, with every learned control (kernel_features.py:43-135):
    one ts_kmap_fwd / ts_kmap_bwd pair.  ``tau`` is the block's learned
    threshold [H, m]; the score bias and the ReLU^2 threshold join it as one
    additive shift."""
    B, H, T, m = a.shape
    kind = KMAP_SOFTMAX if cfg.kernel_kind == "softmax_partition" else KMAP_RELU2
    terms = []
    if tau is not None:
        terms.append(-_as_head_feature(tau, H, m))
    if score_bias is not None:
        terms.append(_as_head_feature(score_bias, H, m))
    if kind == KMAP_RELU2 and relu2_threshold is not None:
        terms.append(-_as_head_feature(relu2_threshold, H, m))
    shift = None
    for t in terms:
        shift = t.float() if shift is None else shift + t.float()
    gain_mode, gainv, gain = 0, None, float(cfg.softmax_gain)
    sparsity, rho, alpha = 0, None, None
    if kind == KMAP_SOFTMAX:
        if softmax_gain is not None and torch.is_tensor(softmax_gain):
            gainv = softmax_gain
            gain_mode = 1 if softmax_gain.ndim == 1 else 2
        elif softmax_gain is not None:
            gain = float(softmax_gain)
        sparsity = _SPARSITY[cfg.kernel_sparsity]
        if sparsity:
            if relative_threshold is None:
                raise RuntimeError("relative kernel sparsity requires a threshold tensor")
            if cfg.kernel_threshold_temperature <= 0.0:
                raise ValueError("relative threshold temperature must be positive")
            rho = relative_threshold
        if sparsity == 3:
            if sparse_blend_alpha is None:
                raise RuntimeError("relative_st_blend requires a learned sparse blend tensor")
            alpha = sparse_blend_alpha
    return _kmap_op(a, shift, gainv, rho, alpha, int(kind), bool(rms), int(gain_mode), int(sparsity), gain,
                 float(cfg.kernel_threshold_temperature), float(cfg.eps))
