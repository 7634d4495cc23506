"""Flat core configuration of the mixer (field names and defaults of
src/thetascan/_core/config.py:24-199, with ``"hip"`` added to the backend
list).  Cross-field rules follow src/thetascan/_core/config.py:218-432."""
from __future__ import annotations

from dataclasses import dataclass

# tanh is an extension of this build (the reference's GN nonlinearities are
# relu2, silu and swiglu): sigma' = 1 - tanh^2, signed features
NONLINS = ("relu2", "silu", "swiglu", "softmax_hidden", "tanh")
FADE_MODES = ("stale", "fast")
FADE_BLEND_MODES = ("free", "tanh")
ACCUMS = ("sum", "ema_gate")
WRITE_RULES = ("gn", "kernel")
ROPES = ("none", "full", "partial")
ROPE_PLACEMENTS = ("input", "feature")
DECAYS = ("off", "scalar")
BACKENDS = ("auto", "naive", "quad", "chunk", "cumsum", "fla", "hip")
PARAM_DTYPES = ("fp32", "fp16", "bf16", "fp8_e4m3")
SOFTMAX_GAIN_MODES = ("fixed", "learned_per_head", "learned_per_feature")
KERNEL_KINDS = ("softmax_partition", "relu2_ridge", "projected_bspline")
KERNEL_SPARSITY_MODES = ("none", "relative_soft", "relative_st", "relative_st_blend")
KERNEL_RELU2_THRESHOLD_MODES = ("none", "learned_per_head")
READ_NORM_MODES = ("key_mass", "feature_mass")
BSPLINE_SCALE_MODES = ("fixed", "learned_per_head")
# recency branches of a bank: the reference allows 1 or 2; this build's core
# config up to 6 (a stale bank blends J + 2 views, the blend kernel up to 8)
MAX_FADE_BRANCHES = 6


@dataclass
class ThetaScanConfig:
    d_model: int = 512
    n_heads: int = 8
    head_dim: int | None = None
    mem_mult: int = 2
    depth: int = 1
    nonlin: str = "relu2"
    fast_w1: bool = True
    write_iters: int = 1
    write_rule: str = "gn"
    kernel_kind: str = "softmax_partition"
    kernel_score_bias: bool = False
    kernel_relu2_threshold_mode: str = "none"
    kernel_sparsity: str = "none"
    kernel_sparse_blend_init: float = 0.0
    kernel_relative_threshold_init: float = 0.01
    kernel_threshold_temperature: float = 0.25
    bspline_basis_count: int = 8
    bspline_degree: int = 3
    bspline_bound: float = 3.0
    bspline_scale: float = 1.0
    bspline_scale_mode: str = "fixed"
    value_centers: int = 0
    value_mlp_mult: float = 0.0
    read_fade: bool = False
    read_fade_mode: str = "stale"
    fade_alpha_init: float = 0.9
    fade_branches: int = 1
    fade_alpha_inits: tuple | None = None
    fade_blend_mode: str = "free"
    learn_thresh: bool = False
    feature_expansion: int = 1
    expansion_key: str = "thetascan"
    accumulation: str = "sum"
    read_norm: bool = False
    read_norm_mode: str = "key_mass"
    read_norm_w1: bool = False
    rope: str = "partial"
    rope_frac: float = 0.5
    rope_base: float = 10000.0
    rope_placement: str = "input"
    qk_norm: bool = True
    act_norm: bool = True
    decay_gate: str = "off"
    out_gate: bool = True
    share_kq: bool = False
    key_value_heads: int | None = None
    param_dtype: str = "fp32"
    compute_dtype: str = "fp32"
    backend: str = "auto"
    softmax_gain: float = 1.0
    softmax_gain_mode: str = "fixed"
    ortho_intra: float = 0.0
    ortho_inter: float = 0.0
    value_mlp_ortho: float = 0.0
    eps: float = 1e-6
    scan_chunk: int = 512
    # Extension of this build: the damping of the GN Jacobi diagonal.  None
    # keeps the reference's damping, eps (engine.py:255).
    gn_damping: float | None = None

    def __post_init__(self):
        if self.head_dim is None:
            self.head_dim = self.d_model // self.n_heads
        self.validate()

    @property
    def mem_hidden(self) -> int:
        return self.mem_mult * self.head_dim

    @property
    def resolved_fade_alphas(self) -> tuple:
        if self.fade_alpha_inits is not None:
            return tuple(float(v) for v in self.fade_alpha_inits)
        if self.fade_branches == 2:
            return (float(self.fade_alpha_init), 0.99)
        return (float(self.fade_alpha_init),)

    def validate(self):
        def one_of(value, allowed, name):
            if value not in allowed:
                raise ValueError(f"{name}={value!r} not in {allowed}")

        one_of(self.nonlin, NONLINS, "nonlin")
        one_of(self.accumulation, ACCUMS, "accumulation")
        one_of(self.rope, ROPES, "rope")
        one_of(self.rope_placement, ROPE_PLACEMENTS, "rope_placement")
        one_of(self.decay_gate, DECAYS, "decay_gate")
        one_of(self.backend, BACKENDS, "backend")
        one_of(self.param_dtype, PARAM_DTYPES, "param_dtype")
        one_of(self.softmax_gain_mode, SOFTMAX_GAIN_MODES, "softmax_gain_mode")
        one_of(self.kernel_kind, KERNEL_KINDS, "kernel_kind")
        one_of(self.kernel_sparsity, KERNEL_SPARSITY_MODES, "kernel_sparsity")
        one_of(self.kernel_relu2_threshold_mode, KERNEL_RELU2_THRESHOLD_MODES, "kernel_relu2_threshold_mode")
        one_of(self.read_norm_mode, READ_NORM_MODES, "read_norm_mode")
        one_of(self.bspline_scale_mode, BSPLINE_SCALE_MODES, "bspline_scale_mode")
        one_of(self.write_rule, WRITE_RULES, "write_rule")
        if not isinstance(self.scan_chunk, int) or self.scan_chunk < 1:
            raise ValueError("scan_chunk must be a positive integer")
        if self.learn_thresh and self.nonlin == "swiglu":
            raise ValueError("learn_thresh and swiglu are mutually exclusive")
        if self.compute_dtype != "fp32":
            raise ValueError("v1 supports compute_dtype='fp32' only")
        if self.write_iters not in (1, 2):
            raise ValueError("write_iters must be 1 or 2")
        if self.depth < 1:
            raise ValueError("depth >= 1")
        if self.d_model % self.n_heads:
            raise ValueError("d_model % n_heads != 0")
        if self.write_rule == "kernel":
            if self.fast_w1:
                raise ValueError("write_rule='kernel' has no dW1: set fast_w1=False")
            if self.write_iters != 1:
                raise ValueError("write_rule='kernel' requires write_iters=1")
            if self.depth != 1:
                raise ValueError("write_rule='kernel' requires depth=1")
            if self.kernel_kind == "projected_bspline":
                if self.mem_hidden % self.bspline_basis_count:
                    raise ValueError("projected_bspline requires mem_hidden divisible by bspline_basis_count")
                if self.kernel_score_bias:
                    raise ValueError("kernel_score_bias is not defined for projected_bspline")
                if self.rope_placement == "feature" and self.rope != "none":
                    raise ValueError("projected_bspline excludes feature-space RoPE")
        if self.value_mlp_mult < 0:
            raise ValueError("value_mlp_mult must be >= 0 (0 = disabled)")
        if self.value_centers:
            if self.value_centers < 2:
                raise ValueError("value_centers must be >= 2")
            if self.write_rule != "kernel" or not self.read_norm:
                raise ValueError("value_centers requires write_rule='kernel' and read_norm")
        if self.read_fade:
            one_of(self.read_fade_mode, FADE_MODES, "read_fade_mode")
            one_of(self.fade_blend_mode, FADE_BLEND_MODES, "fade_blend_mode")
            if self.accumulation != "sum":
                raise ValueError("read_fade requires accumulation='sum'")
            if type(self.fade_branches) is not int or not 1 <= self.fade_branches <= MAX_FADE_BRANCHES:
                raise ValueError(f"fade_branches must be between 1 and {MAX_FADE_BRANCHES}")
            alphas = self.resolved_fade_alphas
            if len(alphas) != self.fade_branches:
                raise ValueError("fade_alpha_inits must contain exactly fade_branches values")
            if any(not 0.0 < a < 1.0 for a in alphas):
                raise ValueError("all fade alpha initializers must be in (0, 1)")
            if self.fade_branches == 2 and alphas[0] == alphas[1]:
                raise ValueError("two fade branches require distinct initial timescales")
            if len(set(alphas)) != len(alphas):
                raise ValueError("fade branches require distinct initial timescales")
        if type(self.feature_expansion) is not int or self.feature_expansion < 1:
            raise ValueError("feature_expansion must be an integer >= 1")
        if self.feature_expansion > 1:
            if self.mem_hidden % self.feature_expansion:
                raise ValueError("feature_expansion must divide the effective memory width")
            if self.nonlin != "relu2":
                raise ValueError("feature_expansion requires nonlin='relu2'")
            if self.write_rule == "kernel" and self.kernel_kind not in ("relu2_ridge", "projected_bspline"):
                raise ValueError("kernel feature_expansion requires kernel_kind='relu2_ridge' "
                                 "(or this build's projected_bspline, expanded on projection rows)")
            if (self.write_rule == "kernel" and self.kernel_kind == "projected_bspline"
                    and (self.mem_hidden // self.feature_expansion) % self.bspline_basis_count):
                raise ValueError("projected_bspline feature_expansion requires mem_hidden / feature_expansion "
                                 "divisible by bspline_basis_count")
        if self.key_value_heads is not None:
            if not 1 <= self.key_value_heads <= self.n_heads or self.n_heads % self.key_value_heads:
                raise ValueError("key_value_heads must divide n_heads")
            if self.share_kq:
                raise ValueError("key_value_heads and share_kq=True are mutually exclusive")
        if self.accumulation == "ema_gate" and self.decay_gate == "off":
            raise ValueError("accumulation='ema_gate' requires decay_gate != 'off'")
        if self.decay_gate != "off" and self.accumulation != "ema_gate":
            raise ValueError("decay_gate is only used by accumulation='ema_gate'")
        if not (0.0 < self.rope_frac <= 1.0):
            raise ValueError("rope_frac in (0,1]")
        if self.softmax_gain <= 0:
            raise ValueError("softmax_gain must be > 0")
        if self.gn_damping is not None and not self.gn_damping > 0.0:
            raise ValueError("gn_damping must be > 0")
        if self.read_norm:
            if self.rope != "none" and self.rope_placement == "feature":
                raise ValueError("feature-space RoPE makes the read_norm denominator signed")
            if self.write_rule == "gn" and self.nonlin not in ("relu2", "tanh"):
                raise ValueError("GN read_norm requires nonlin='relu2' (or this build's signed-mass tanh)")
        elif self.read_norm_mode != "key_mass":
            raise ValueError("read_norm_mode is active only when read_norm=True")
        if self.read_norm_w1:
            if (not self.read_norm or self.write_rule != "gn" or not self.fast_w1
                    or self.nonlin not in ("relu2", "tanh")):
                raise ValueError("read_norm_w1 requires read_norm, GN, fast W1 and relu2 (or tanh)")
