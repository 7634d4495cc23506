"""ThetaScan on MI355X: the public API of the reference package with a
hand-written gfx950 ``hip`` scan backend underneath."""
from .api import ThetaScan
from .state import ThetaScanState
from .decode import DecodeGraph
from .config import (
    Backend,
    BankMode,
    BlendMode,
    Family,
    GNConfig,
    GNNonlinearity,
    GNReadNormalization,
    KernelBSplineScaleMode,
    KernelConfig,
    KernelFeatureMap,
    KernelReLU2ThresholdMode,
    KernelReadNormalization,
    KernelSharpnessMode,
    KernelSparsity,
    KernelValueRepresentation,
    RegularizationConfig,
    RoPEConfig,
    RoPEMode,
    RoPEPlacement,
    RuntimeConfig,
    TemporalConfig,
    TemporalMode,
    ThetaScanConfig,
)

__version__ = "0.1.0"

__all__ = [
    "Backend", "BankMode", "BlendMode", "Family", "GNConfig", "GNNonlinearity", "GNReadNormalization",
    "DecodeGraph", "KernelBSplineScaleMode", "KernelConfig", "KernelFeatureMap", "KernelReLU2ThresholdMode",
    "KernelReadNormalization", "KernelSharpnessMode", "KernelSparsity", "KernelValueRepresentation",
    "RegularizationConfig", "RoPEConfig", "RoPEMode", "RoPEPlacement", "RuntimeConfig", "TemporalConfig",
    "TemporalMode", "ThetaScan", "ThetaScanConfig", "ThetaScanState",
]
