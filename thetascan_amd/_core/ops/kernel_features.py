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

import torch

from . import maps


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
