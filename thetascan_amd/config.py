"""Public configuration surface (drop-in for src/thetascan/config.py).

Same dataclasses, field names, defaults, validation rules, manifests
(``to_dict`` / ``from_dict``) and versioned presets as the reference
(src/thetascan/config.py:58-890).  The only addition is the ``"hip"`` scan
backend in ``RuntimeConfig.backend``; ``"auto"`` resolves to it in this
package.
"""
from __future__ import annotations

import math
from copy import deepcopy
from dataclasses import asdict, dataclass, field
from numbers import Real
from typing import Any, Literal, Mapping

Family = Literal["gn", "kernel"]
GNNonlinearity = Literal["relu2", "relu2_threshold", "silu", "swiglu"]
GNReadNormalization = Literal["none", "w2_feature_mass", "both_feature_mass"]
KernelFeatureMap = Literal["softmax_partition", "relu2_ridge", "projected_bspline"]
KernelValueRepresentation = Literal["raw", "value_anchors", "value_mlp"]
KernelSparsity = Literal["none", "relative_soft", "relative_st", "relative_st_blend"]
KernelReadNormalization = Literal["none", "key_mass", "feature_mass"]
KernelSharpnessMode = Literal["fixed", "learned_per_head", "learned_per_feature"]
KernelReLU2ThresholdMode = Literal["none", "learned_per_head"]
KernelBSplineScaleMode = Literal["fixed", "learned_per_head"]
TemporalMode = Literal["sum", "ema", "bank"]
BankMode = Literal["fast", "stale"]
BlendMode = Literal["free", "tanh"]
Backend = Literal["auto", "naive", "quad", "chunk", "cumsum", "fla", "hip"]
RoPEMode = Literal["none", "partial", "full"]
RoPEPlacement = Literal["input", "feature"]

BACKENDS = ("auto", "naive", "quad", "chunk", "cumsum", "fla", "hip")


def _strict_int(name: str, value: object) -> None:
    if type(value) is not int:
        raise TypeError(f"{name} must be an integer")


def _strict_bool(name: str, value: object) -> None:
    if type(value) is not bool:
        raise TypeError(f"{name} must be a boolean")


def _finite(name: str, value: object) -> None:
    if isinstance(value, bool) or not isinstance(value, Real):
        raise TypeError(f"{name} must be a real number")
    if not math.isfinite(float(value)):
        raise ValueError(f"{name} must be finite")


def _choice(name: str, value, allowed) -> None:
    if value not in allowed:
        raise ValueError(f"unknown {name}: {value!r}")


@dataclass
class GNConfig:
    """Gauss--Newton fast-weight memory options (config.py:58-94)."""

    nonlinearity: GNNonlinearity = "relu2"
    jacobian_steps: int = 1
    read_normalization: GNReadNormalization = "none"

    def validate(self) -> None:
        _strict_int("GNConfig.jacobian_steps", self.jacobian_steps)
        _choice("GN nonlinearity", self.nonlinearity, ("relu2", "relu2_threshold", "silu", "swiglu"))
        if self.jacobian_steps not in (1, 2):
            raise ValueError("GNConfig.jacobian_steps must be 1 or 2")
        _choice("GN read normalization", self.read_normalization, ("none", "w2_feature_mass", "both_feature_mass"))
        if self.read_normalization != "none" and self.nonlinearity not in ("relu2", "relu2_threshold"):
            raise ValueError("GN feature-mass normalization requires non-negative relu2 or relu2_threshold features")
        if self.read_normalization != "none" and self.jacobian_steps != 1:
            raise ValueError("GN feature-mass normalization requires jacobian_steps=1")


@dataclass
class KernelConfig:
    """Normalized positive-feature kernel memory options (config.py:97-263)."""

    feature_map: KernelFeatureMap = "softmax_partition"
    value_representation: KernelValueRepresentation = "raw"
    value_anchors: int = 8
    value_mlp_multiplier: float = 1.0
    kernel_sharpness: float = 8.0
    kernel_sharpness_mode: KernelSharpnessMode = "fixed"
    score_bias: bool = False
    relu2_threshold_mode: KernelReLU2ThresholdMode = "none"
    sparsity: KernelSparsity = "none"
    sparse_blend_init: float = 0.0
    relative_threshold_init: float = 0.01
    threshold_temperature: float = 0.25
    bspline_basis_count: int = 8
    bspline_degree: int = 3
    bspline_bound: float = 3.0
    bspline_scale: float = 1.0
    bspline_scale_mode: KernelBSplineScaleMode = "fixed"
    feature_parameters_trainable: bool = True
    read_normalization: KernelReadNormalization = "key_mass"

    def validate(self) -> None:
        _strict_bool("KernelConfig.score_bias", self.score_bias)
        _strict_bool("KernelConfig.feature_parameters_trainable", self.feature_parameters_trainable)
        for name in ("value_anchors", "bspline_basis_count", "bspline_degree"):
            _strict_int(f"KernelConfig.{name}", getattr(self, name))
        for name in ("value_mlp_multiplier", "kernel_sharpness", "sparse_blend_init", "relative_threshold_init",
                     "threshold_temperature", "bspline_bound", "bspline_scale"):
            _finite(f"KernelConfig.{name}", getattr(self, name))
        _choice("kernel feature map", self.feature_map, ("softmax_partition", "relu2_ridge", "projected_bspline"))
        _choice("kernel value representation", self.value_representation, ("raw", "value_anchors", "value_mlp"))
        _choice("kernel read normalization", self.read_normalization, ("none", "key_mass", "feature_mass"))
        if self.value_representation == "value_anchors" and self.value_anchors < 2:
            raise ValueError("KernelConfig.value_anchors must be at least 2")
        if self.value_representation == "value_mlp" and self.value_mlp_multiplier <= 0:
            raise ValueError("KernelConfig.value_mlp_multiplier must be positive")
        if self.kernel_sharpness <= 0:
            raise ValueError("KernelConfig.kernel_sharpness must be positive")
        if self.kernel_sharpness_mode not in ("fixed", "learned_per_head", "learned_per_feature"):
            raise ValueError("KernelConfig.kernel_sharpness_mode must be 'fixed', 'learned_per_head', "
                             "or 'learned_per_feature'")
        _choice("kernel sparsity", self.sparsity, ("none", "relative_soft", "relative_st", "relative_st_blend"))
        if not 0.0 <= self.sparse_blend_init <= 1.0:
            raise ValueError("KernelConfig.sparse_blend_init must be in [0, 1]")
        if self.sparsity != "relative_st_blend" and self.sparse_blend_init != 0.0:
            raise ValueError("KernelConfig.sparse_blend_init is active only with sparsity='relative_st_blend'")
        if self.relu2_threshold_mode not in ("none", "learned_per_head"):
            raise ValueError("KernelConfig.relu2_threshold_mode must be 'none' or 'learned_per_head'")
        if self.relu2_threshold_mode != "none" and self.feature_map != "relu2_ridge":
            raise ValueError("learned relu2_threshold_mode requires feature_map='relu2_ridge'")
        if self.relu2_threshold_mode != "none" and self.score_bias:
            raise ValueError("relu2_threshold_mode and score_bias are redundant affine controls; enable only one")
        if not 0.0 < self.relative_threshold_init < 1.0:
            raise ValueError("KernelConfig.relative_threshold_init must be in (0, 1)")
        if self.threshold_temperature <= 0.0:
            raise ValueError("KernelConfig.threshold_temperature must be positive")
        if self.sparsity != "none" and self.feature_map != "softmax_partition":
            raise ValueError("learned relative sparsity is currently defined for feature_map='softmax_partition' only")
        if self.kernel_sharpness_mode != "fixed" and self.feature_map != "softmax_partition":
            raise ValueError("learned kernel_sharpness_mode is defined for feature_map='softmax_partition' only")
        if self.bspline_basis_count <= self.bspline_degree:
            raise ValueError("kernel B-spline basis count must exceed its degree")
        if self.bspline_degree != 3:
            raise ValueError("kernel projected_bspline currently supports degree=3 only")
        if self.bspline_bound <= 0.0 or self.bspline_scale <= 0.0:
            raise ValueError("kernel B-spline bound and scale must be positive")
        if self.bspline_scale_mode not in ("fixed", "learned_per_head"):
            raise ValueError("KernelConfig.bspline_scale_mode must be 'fixed' or 'learned_per_head'")
        if self.feature_map != "projected_bspline" and self.bspline_scale_mode != "fixed":
            raise ValueError("learned bspline_scale_mode requires feature_map='projected_bspline'")


@dataclass
class RoPEConfig:
    """Rotary positional features of memory keys and queries (config.py:266-294)."""

    mode: RoPEMode = "none"
    fraction: float = 0.5
    base: float = 10_000.0
    placement: RoPEPlacement = "input"

    def validate(self) -> None:
        _finite("RoPEConfig.fraction", self.fraction)
        _finite("RoPEConfig.base", self.base)
        _choice("RoPE mode", self.mode, ("none", "partial", "full"))
        _choice("RoPE placement", self.placement, ("input", "feature"))
        if not 0.0 < self.fraction <= 1.0:
            raise ValueError("RoPEConfig.fraction must be in (0, 1]")
        if self.base <= 0.0:
            raise ValueError("RoPEConfig.base must be positive")


@dataclass
class TemporalConfig:
    """How writes combine over time: sum, EMA or a recency bank (config.py:297-385)."""

    mode: TemporalMode = "sum"
    bank_mode: BankMode = "fast"
    retention_init: float = 0.9
    recency_branches: int = 1
    retention_inits: tuple | None = None
    half_life_inits: tuple | None = None
    blend_mode: BlendMode = "free"

    def resolved_retentions(self) -> tuple:
        if self.retention_inits is not None:
            return tuple(float(v) for v in self.retention_inits)
        if self.half_life_inits is not None:
            return tuple(math.pow(2.0, -1.0 / float(v)) for v in self.half_life_inits)
        if self.recency_branches == 2:
            return (float(self.retention_init), 0.99)
        return (float(self.retention_init),)

    def validate(self) -> None:
        _strict_int("TemporalConfig.recency_branches", self.recency_branches)
        _finite("TemporalConfig.retention_init", self.retention_init)
        _choice("temporal mode", self.mode, ("sum", "ema", "bank"))
        _choice("bank mode", self.bank_mode, ("fast", "stale"))
        if not 0.0 < self.retention_init < 1.0:
            raise ValueError("TemporalConfig.retention_init must be in (0, 1)")
        if self.recency_branches not in (1, 2):
            raise ValueError("TemporalConfig.recency_branches must be 1 or 2")
        if self.blend_mode not in ("free", "tanh"):
            raise ValueError("TemporalConfig.blend_mode must be 'free' or 'tanh'")
        if self.retention_inits is not None and self.half_life_inits is not None:
            raise ValueError("set only one of retention_inits and half_life_inits")
        for name in ("retention_inits", "half_life_inits"):
            values = getattr(self, name)
            if values is not None:
                for i, v in enumerate(values):
                    _finite(f"TemporalConfig.{name}[{i}]", v)
        if self.half_life_inits is not None and any(v <= 0.0 for v in self.half_life_inits):
            raise ValueError("half-lives must be positive")
        retentions = self.resolved_retentions()
        if len(retentions) != self.recency_branches:
            raise ValueError("retention/half-life initializers must contain exactly recency_branches values")
        if any(not 0.0 < v < 1.0 for v in retentions):
            raise ValueError("retentions must be in (0, 1)")
        if self.recency_branches == 2 and retentions[0] == retentions[1]:
            raise ValueError("two recency branches require distinct initial timescales")


@dataclass
class RegularizationConfig:
    """Optional cosine-orthogonality penalty weights (config.py:388-406)."""

    feature_weight: float = 0.0
    head_weight: float = 0.0
    value_mlp_weight: float = 0.0

    def validate(self) -> None:
        for name in ("feature_weight", "head_weight", "value_mlp_weight"):
            _finite(f"RegularizationConfig.{name}", getattr(self, name))
            if getattr(self, name) < 0.0:
                raise ValueError("regularization weights must be non-negative")


@dataclass
class RuntimeConfig:
    """Execution selection.  ``auto`` and ``hip`` run the MI355X kernels;
    ``scan_chunk`` is validated exactly like the reference (config.py:409-468)
    and only changes the reference backends' rounding, since the scan is exact
    for any tiling."""

    backend: Backend = "auto"
    scan_chunk: int = 512

    def validate(self) -> None:
        if self.backend not in BACKENDS:
            raise ValueError("RuntimeConfig.backend must be one of " + ", ".join(repr(b) for b in BACKENDS))
        if not isinstance(self.scan_chunk, bool) and isinstance(self.scan_chunk, int):
            if self.scan_chunk < 1:
                raise ValueError("RuntimeConfig.scan_chunk must be >= 1")
        else:
            raise TypeError("RuntimeConfig.scan_chunk must be an int")


_NESTED = {
    "gn": GNConfig,
    "kernel": KernelConfig,
    "rope": RoPEConfig,
    "temporal": TemporalConfig,
    "regularization": RegularizationConfig,
    "runtime": RuntimeConfig,
}


@dataclass
class ThetaScanConfig:
    """Public ThetaScan configuration (config.py:471-890)."""

    d_model: int = 512
    n_heads: int = 8
    head_dim: int | None = None
    memory_multiplier: int = 2
    feature_expansion: int = 1
    expansion_key: str = "thetascan"
    depth: int = 1
    share_key_query: bool = False
    key_value_heads: int | None = None
    output_gate: bool = True
    family: Family = "gn"
    gn: GNConfig = field(default_factory=GNConfig)
    kernel: KernelConfig = field(default_factory=KernelConfig)
    rope: RoPEConfig = field(default_factory=RoPEConfig)
    temporal: TemporalConfig = field(default_factory=TemporalConfig)
    regularization: RegularizationConfig = field(default_factory=RegularizationConfig)
    runtime: RuntimeConfig = field(default_factory=RuntimeConfig)

    @property
    def resolved_head_dim(self) -> int:
        return self.head_dim or self.d_model // self.n_heads

    def validate(self) -> None:
        _strict_bool("ThetaScanConfig.share_key_query", self.share_key_query)
        _strict_bool("ThetaScanConfig.output_gate", self.output_gate)
        for name in ("d_model", "n_heads", "memory_multiplier", "feature_expansion", "depth"):
            _strict_int(f"ThetaScanConfig.{name}", getattr(self, name))
        if self.head_dim is not None:
            _strict_int("ThetaScanConfig.head_dim", self.head_dim)
        if self.family not in ("gn", "kernel"):
            raise ValueError("ThetaScanConfig.family must be 'gn' or 'kernel'")
        if self.d_model <= 0 or self.n_heads <= 0 or self.memory_multiplier <= 0:
            raise ValueError("d_model, n_heads, and memory_multiplier must be positive")
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if self.head_dim is not None and self.head_dim * self.n_heads != self.d_model:
            raise ValueError("head_dim * n_heads must equal d_model")
        if self.key_value_heads is not None:
            if type(self.key_value_heads) is not int:
                raise TypeError("ThetaScanConfig.key_value_heads must be an integer or None")
            if not 1 <= self.key_value_heads <= self.n_heads:
                raise ValueError("key_value_heads must be in [1, n_heads]")
            if self.n_heads % self.key_value_heads:
                raise ValueError("n_heads must be divisible by key_value_heads")
            if self.share_key_query:
                raise ValueError("key_value_heads and share_key_query=True are mutually exclusive")
        if self.depth < 1:
            raise ValueError("depth must be at least 1")
        if self.feature_expansion < 1:
            raise ValueError("ThetaScanConfig.feature_expansion must be >= 1")
        memory_features = self.memory_multiplier * self.resolved_head_dim
        if self.feature_expansion > 1:
            if not isinstance(self.expansion_key, str) or not self.expansion_key:
                raise ValueError("ThetaScanConfig.expansion_key must be a non-empty string")
            if memory_features % self.feature_expansion:
                raise ValueError("feature_expansion must divide the effective memory width "
                                 "(memory_multiplier * head_dim)")
            if self.family == "gn" and self.gn.nonlinearity not in ("relu2", "relu2_threshold"):
                raise ValueError("GN feature_expansion requires nonlinearity 'relu2' or 'relu2_threshold'")
            if self.family == "kernel" and self.kernel.feature_map != "relu2_ridge":
                raise ValueError("kernel feature_expansion requires feature_map='relu2_ridge'")
        self.temporal.validate()
        self.rope.validate()
        self.regularization.validate()
        self.runtime.validate()
        if self.runtime.backend == "cumsum" and self.temporal.mode != "sum":
            raise ValueError("backend='cumsum' supports temporal.mode='sum' only")
        if self.family == "gn":
            self.gn.validate()
            if (self.rope.mode != "none" and self.rope.placement == "feature"
                    and self.gn.read_normalization != "none"):
                raise ValueError("feature-space RoPE makes the GN feature-mass denominator signed")
            return
        kernel = self.kernel
        kernel.validate()
        if (self.rope.mode != "none" and self.rope.placement == "feature"
                and kernel.read_normalization in ("key_mass", "feature_mass")):
            raise ValueError("feature-space RoPE makes the kernel normalization denominator signed; use "
                             "placement='input', mode='none', or read_normalization='none'")
        if self.depth != 1:
            raise ValueError("kernel memory currently supports depth=1 only")
        if kernel.feature_map == "projected_bspline":
            if memory_features % kernel.bspline_basis_count:
                raise ValueError("projected_bspline requires memory_multiplier * head_dim to be divisible by "
                                 "bspline_basis_count")
            if kernel.score_bias:
                raise ValueError("score_bias is an affine-score axis and is not used by projected_bspline")
            if self.rope.placement == "feature" and self.rope.mode != "none":
                raise ValueError("projected_bspline requires input-space RoPE")
        if kernel.value_representation == "value_anchors" and kernel.read_normalization != "key_mass":
            raise ValueError("kernel value_anchors requires read_normalization='key_mass'")

    def to_dict(self) -> dict[str, Any]:
        return deepcopy(asdict(self))

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> "ThetaScanConfig":
        if not isinstance(data, Mapping):
            raise TypeError("ThetaScanConfig.from_dict expects a mapping")
        payload: dict[str, Any] = deepcopy(dict(data))

        def merge(base: dict, override: Mapping) -> dict:
            for key, value in override.items():
                if isinstance(value, Mapping) and isinstance(base.get(key), dict):
                    base[key] = merge(dict(base[key]), value)
                else:
                    base[key] = deepcopy(value)
            return base

        preset = payload.pop("preset", None)
        if preset is not None:
            presets = {
                "gn_reference_v0_1": cls.gn_reference_v0_1,
                "gn_expanded_reference_v0_1": cls.gn_expanded_reference_v0_1,
                "kernel_expanded_reference_v0_1": cls.kernel_expanded_reference_v0_1,
            }
            if preset not in presets:
                raise ValueError(f"unknown ThetaScan preset: {preset!r}")
            d_model = payload.pop("d_model", 512)
            n_heads = payload.pop("n_heads", 8)
            payload = merge(presets[preset](d_model=d_model, n_heads=n_heads).to_dict(), payload)
        for name, constructor in _NESTED.items():
            value = payload.get(name)
            if isinstance(value, Mapping):
                item = dict(value)
                if name == "temporal":
                    for tuple_name in ("retention_inits", "half_life_inits"):
                        if item.get(tuple_name) is not None:
                            item[tuple_name] = tuple(item[tuple_name])
                payload[name] = constructor(**item)
        config = cls(**payload)
        config.validate()
        return config

    def _to_core_config(self):
        """Public hierarchy -> flat core config (config.py:703-796)."""
        self.validate()
        from ._core.config import ThetaScanConfig as CoreConfig

        common: dict[str, object] = {
            "d_model": self.d_model, "n_heads": self.n_heads, "head_dim": self.head_dim,
            "mem_mult": self.memory_multiplier, "feature_expansion": self.feature_expansion,
            "expansion_key": self.expansion_key, "depth": self.depth, "backend": self.runtime.backend,
            "scan_chunk": self.runtime.scan_chunk, "rope": self.rope.mode, "rope_frac": self.rope.fraction,
            "rope_base": self.rope.base, "rope_placement": self.rope.placement, "qk_norm": True,
            "act_norm": True, "out_gate": self.output_gate, "share_kq": self.share_key_query,
            "key_value_heads": self.key_value_heads, "ortho_intra": self.regularization.feature_weight,
            "ortho_inter": self.regularization.head_weight,
            "value_mlp_ortho": self.regularization.value_mlp_weight,
        }
        if self.temporal.mode == "ema":
            common.update(accumulation="ema_gate", decay_gate="scalar")
        else:
            common.update(accumulation="sum", decay_gate="off")
        if self.temporal.mode == "bank":
            common.update(
                read_fade=True, read_fade_mode=self.temporal.bank_mode,
                fade_alpha_init=self.temporal.retention_init, fade_branches=self.temporal.recency_branches,
                fade_alpha_inits=self.temporal.resolved_retentions(), fade_blend_mode=self.temporal.blend_mode,
            )
        if self.family == "gn":
            nonlin = "relu2" if self.gn.nonlinearity == "relu2_threshold" else self.gn.nonlinearity
            common.update(
                write_rule="gn", nonlin=nonlin, learn_thresh=self.gn.nonlinearity == "relu2_threshold",
                write_iters=self.gn.jacobian_steps, fast_w1=True,
                read_norm=self.gn.read_normalization != "none",
                read_norm_w1=self.gn.read_normalization == "both_feature_mass",
            )
        else:
            k = self.kernel
            common.update(
                write_rule="kernel",
                nonlin="softmax_hidden" if k.feature_map == "softmax_partition" else "relu2",
                kernel_kind=k.feature_map, kernel_score_bias=k.score_bias,
                kernel_relu2_threshold_mode=k.relu2_threshold_mode, kernel_sparsity=k.sparsity,
                kernel_sparse_blend_init=k.sparse_blend_init,
                kernel_relative_threshold_init=k.relative_threshold_init,
                kernel_threshold_temperature=k.threshold_temperature,
                bspline_basis_count=k.bspline_basis_count, bspline_degree=k.bspline_degree,
                bspline_bound=k.bspline_bound, bspline_scale=k.bspline_scale,
                bspline_scale_mode=k.bspline_scale_mode, softmax_gain=k.kernel_sharpness,
                softmax_gain_mode=k.kernel_sharpness_mode, fast_w1=False, write_iters=1,
                read_norm=k.read_normalization != "none",
                read_norm_mode=k.read_normalization if k.read_normalization != "none" else "key_mass",
                value_centers=k.value_anchors if k.value_representation == "value_anchors" else 0,
                value_mlp_mult=k.value_mlp_multiplier if k.value_representation == "value_mlp" else 0.0,
            )
        return CoreConfig(**common)

    # ---- versioned presets (config.py:804-890); validated at head_dim = 64

    @classmethod
    def gn_reference_v0_1(cls, d_model: int = 512, n_heads: int = 8) -> "ThetaScanConfig":
        return cls(
            d_model=d_model, n_heads=n_heads, memory_multiplier=3, share_key_query=True, output_gate=False,
            family="gn",
            gn=GNConfig(nonlinearity="relu2", jacobian_steps=1, read_normalization="both_feature_mass"),
            rope=RoPEConfig(mode="partial", fraction=0.5, base=10_000.0),
            temporal=TemporalConfig(mode="bank", bank_mode="fast", retention_init=0.9, recency_branches=1,
                                    retention_inits=(0.9,), blend_mode="free"),
        )

    @classmethod
    def gn_expanded_reference_v0_1(cls, d_model: int = 512, n_heads: int = 8) -> "ThetaScanConfig":
        return cls(
            d_model=d_model, n_heads=n_heads, memory_multiplier=6, feature_expansion=2, share_key_query=True,
            output_gate=False, family="gn",
            gn=GNConfig(nonlinearity="relu2_threshold", jacobian_steps=1, read_normalization="both_feature_mass"),
            rope=RoPEConfig(mode="partial", fraction=0.5, base=10_000.0),
            temporal=TemporalConfig(mode="bank", bank_mode="fast", recency_branches=1, retention_inits=(0.9,),
                                    blend_mode="free"),
        )

    @classmethod
    def kernel_expanded_reference_v0_1(cls, d_model: int = 512, n_heads: int = 8) -> "ThetaScanConfig":
        return cls(
            d_model=d_model, n_heads=n_heads, memory_multiplier=6, feature_expansion=2, share_key_query=True,
            output_gate=False, family="kernel",
            kernel=KernelConfig(feature_map="relu2_ridge", relu2_threshold_mode="learned_per_head",
                                read_normalization="key_mass"),
            rope=RoPEConfig(mode="partial", fraction=0.5, base=10_000.0),
            temporal=TemporalConfig(mode="bank", bank_mode="fast", recency_branches=2, half_life_inits=(8.0, 64.0),
                                    blend_mode="free"),
        )
